"""bf16 -> fp16 cast with round-toward-zero (reference kernel/convert.py:24-34).

Same signature and preconditions as the reference's `bf16_to_fp16`; the
conversion runs in a HIP kernel (v_cvt_pkrtz_f16_f32): values beyond the fp16
range saturate to +-65504, and values below fp16's subnormal grid truncate.
"""

from __future__ import annotations

import torch

from .hip import _lib


def bf16_to_fp16(x: torch.Tensor) -> torch.Tensor:
    assert x.dtype == torch.bfloat16
    assert x.is_contiguous()
    assert x.numel() % 2 == 0
    dev = _lib.require_cuda(x)
    out = torch.empty(x.shape, dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().feather_bf16_to_fp16(x.data_ptr(), out.data_ptr(), x.numel(), _lib.stream_ptr(dev)),
                   "bf16_to_fp16")
    return out
