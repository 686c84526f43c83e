"""The C5 workload end to end on the device: the 40-block DiT linear stack at hidden size 5120,
FFN 13824, M = 32768. Every one of the 240 weights is quantized and prepacked on the device by
the load path (comfy_feather/quant.py:116-136 of the reference) and checked bit for bit against
torch's e5m2 cast of the same fp32 product (the cast the oracle's encoder is pinned to); every
GEMM output is checked over the whole tensor by row and column checksums against float64
arithmetic, and block 0's six outputs elementwise against a float64 evaluation under the
north-star gate as written (max-abs 2e-2, rel-Frobenius 1e-3)."""

import numpy as np
import pytest
import torch

from gpu_util import assert_gemm_close_dev, assert_row_col_checksums, torch_ref_dev

pytestmark = pytest.mark.gpu

M = 32768
# (name, K, N) of one block's linears, applied to ~N(0,1) inputs (no unnormalised chaining)
LINEARS = [("q", 5120, 5120), ("k", 5120, 5120), ("v", 5120, 5120), ("o", 5120, 5120),
           ("up", 5120, 13824), ("down", 13824, 5120)]
BLOCKS = 40


def _expected_codes(w: torch.Tensor, scale: float) -> torch.Tensor:
    """(N, K) e5m2 codes of the load path: fp32(w) * fp32(1/scale), cast to e5m2 by torch."""
    inv = float(np.float32(1.0) / np.float32(scale))
    return (w.float() * inv).to(torch.float8_e5m2).view(torch.uint8)


def test_config5_forty_blocks(cuda, quant, hk):
    gd = torch.Generator(device=cuda).manual_seed(5)
    xs = {K: torch.randn(M, K, generator=gd, device=cuda).half() for K in (5120, 13824)}
    pinned = False
    for blk in range(BLOCKS):
        print(f"config 5 block {blk}", flush=True)
        for name, K, N in LINEARS:
            w = (torch.randn(N, K, generator=gd, device=cuda) * 0.02).half()
            bias = (torch.randn(N, generator=gd, device=cuda) * 0.01).half()
            qt = quant.make_feather_quantized_weight(w, None, torch.float16)
            bp, scale = quant.get_feather_plain_tensors(qt)
            s = float(scale.item())
            amax = np.float32(w.abs().max().float().item())
            assert np.float32(s) == amax / np.float32(57344.0), (blk, name)
            want = _expected_codes(w, s)
            if not pinned:
                # torch's device cast equals its CPU cast (the one the oracle is pinned to)
                assert torch.equal(want.cpu(), _expected_codes(w.cpu(), s)), "device e5m2 cast differs from CPU"
                pinned = True
            got = quant.unprepack_transpose(bp).view(torch.uint8)
            assert torch.equal(got, want), f"block {blk} {name}: quantized codes differ"
            del got, want
            sd = scale.reshape(1).float().contiguous()
            y = hk.scaled_mm_hip_any_m(xs[K], bp, sd, bias, torch.float16)
            assert_row_col_checksums(xs[K], bp, sd, bias, y, label=f"block {blk} {name}")
            if blk == 0:
                ref = torch_ref_dev(xs[K], bp, sd, bias, torch.float16)
                assert_gemm_close_dev(y, ref, torch.float16, f"block 0 {name}", literal=True)
                del ref
            del y, w, bp, qt
    torch.cuda.synchronize()
