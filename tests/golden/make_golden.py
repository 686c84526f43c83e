"""Writes the golden fixtures in this folder (run from the repo root: python tests/golden/make_golden.py).

Every fixture is produced by the numpy oracle and, where torch implements the
same operation, cross-checked against torch's CPU result before it is
written. The reference ships no vectors of its own for this path, so these
are the committed known answers the GPU tests compare against:

  e5m2_codes.npz    fp8 e5m2 code of every fp16 and every bf16 bit pattern
                    (torch's float -> float8_e5m2 cast, equal to the oracle)
  bf16_rtz.npz      fp16 bits of every bf16 pattern under round-toward-zero
  quant_c1.npz      the C1 workload's weight (N=K=1024, ~N(0, 0.02), seed 0)
                    quantized on the load path (fp32) and the patch path
                    (fp16 with the reciprocal clamp, bf16): sha256 of the
                    prepacked bytes, the scale, 32 sampled rows
  gemm_small.npz    A (64x256 fp16), prepacked e5m2 B (16x128x16), scale,
                    bias and the fp16 / bf16 outputs of the kernel contract
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import feather_oracle as O  # noqa: E402


def _all16() -> np.ndarray:
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def e5m2_codes() -> None:
    bits = _all16()
    from_f16 = O.e5m2_encode(bits.view(np.float16).astype(np.float32))
    from_bf16 = O.e5m2_encode(O.bf16_bits_to_f32(bits))
    t16 = torch.from_numpy(bits.view(np.float16).copy()).to(torch.float8_e5m2).view(torch.uint8).numpy()
    tbf = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(torch.float8_e5m2)
    assert np.array_equal(from_f16, t16) and np.array_equal(from_bf16, tbf.view(torch.uint8).numpy())
    np.savez_compressed(HERE / "e5m2_codes.npz", from_fp16=from_f16, from_bf16=from_bf16)


def bf16_rtz() -> None:
    np.savez_compressed(HERE / "bf16_rtz.npz", fp16_bits=O.bf16_to_fp16_rtz(_all16()))


def config1_weight() -> torch.Tensor:
    g = torch.Generator().manual_seed(0)
    return torch.randn(1024, 1024, generator=g) * 0.02  # (N, K) float32


def quant_c1() -> None:
    w32 = config1_weight()
    rows = np.arange(0, 1024, 32)
    out = {}
    cases = {
        "load_f16": (w32.half().numpy(), O.DT_F16, "load"),
        "native_f16": (w32.half().numpy(), O.DT_F16, "native"),
        "native_bf16": (w32.bfloat16().view(torch.int16).numpy().view(np.uint16), O.DT_BF16, "native"),
        "load_f32": (w32.numpy(), O.DT_F32, "load"),
    }
    for name, (w, dt, path) in cases.items():
        codes, s = (O.quantize_load if path == "load" else O.quantize_native)(w, dt)
        packed = O.prepack_transpose(codes)
        out[f"{name}_sha256"] = np.frombuffer(hashlib.sha256(packed.tobytes()).digest(), dtype=np.uint8)
        out[f"{name}_scale"] = np.array([s], dtype=np.float32)
        out[f"{name}_rows"] = codes[rows]
    out["rows"] = rows
    np.savez_compressed(HERE / "quant_c1.npz", **out)


def gemm_small() -> None:
    g = torch.Generator().manual_seed(1)
    M, N, K = 64, 128, 256
    a = torch.randn(M, K, generator=g).half().numpy()
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    codes, s = O.quantize_load(w, O.DT_F32)
    packed = O.prepack_transpose(codes)
    bias16 = (torch.randn(N, generator=g) * 0.01).half().numpy()
    bias_bf = O.f32_to_bf16_rne(bias16.astype(np.float32))
    y16 = O.scaled_mm_ref(a, packed, s, bias16, O.DT_F16)
    ybf = O.scaled_mm_ref(a, packed, s, bias_bf, O.DT_BF16)
    np.savez_compressed(HERE / "gemm_small.npz", a=a, b_prepacked=packed, scale=np.array([s], np.float32),
                        bias_f16=bias16, bias_bf16=bias_bf, out_f16=y16, out_bf16=ybf,
                        exact_f32=O.scaled_mm_ref_f32(a, packed, s).astype(np.float32))


if __name__ == "__main__":
    e5m2_codes()
    bf16_rtz()
    quant_c1()
    gemm_small()
    print("fixtures written to", HERE)
