"""bf16 -> fp16 cast with round-toward-zero (reference kernel/convert.py:24-34).

Same signature and preconditions as the reference's `bf16_to_fp16`; the
conversion runs in a HIP kernel (v_cvt_pkrtz_f16_f32) behind the C++ torch op
feather_ops::bf16_to_fp16: values beyond the fp16 range saturate to +-65504, and
values below fp16's subnormal grid truncate.

`bf16_to_fp16_rne` (no counterpart in the reference's module) is the library's
round-to-nearest-even cast: the values of x.to(torch.float16) (overflow to inf),
the pass the any-M entry runs before the large GEMM tiles for bf16 activations.
"""

from __future__ import annotations

import torch

from .hip import _lib


def bf16_to_fp16(x: torch.Tensor) -> torch.Tensor:
    assert x.dtype == torch.bfloat16
    assert x.is_contiguous()
    assert x.numel() % 2 == 0
    _lib.require_cuda(x)
    _lib.load_torch_ops()
    return torch.ops.feather_ops.bf16_to_fp16.default(x, False)


def bf16_to_fp16_rne(x: torch.Tensor) -> torch.Tensor:
    assert x.dtype == torch.bfloat16
    assert x.is_contiguous()
    _lib.require_cuda(x)
    _lib.load_torch_ops()
    return torch.ops.feather_ops.bf16_to_fp16.default(x, True)
