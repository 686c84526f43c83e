"""CPU oracle for the FeatherOps scaled_mm hot path -- TEST INFRASTRUCTURE ONLY.

This module is a numpy restatement of the reference's arithmetic. It exists to
check the HIP kernels: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and never as the thing measured or shipped.
The product path (comfyui-featherops_amd/) never imports it.

Every function cites the reference code it restates (paths relative to the
reference checkout). The formulations are deliberately different from the
kernels' bit tricks: fp8 encoding is a nearest-value search over the code
table, bf16 rounding picks between the two neighbouring bf16 values, and the
GEMM accumulates in float64.

Pinning (what each function is checked against, in tests/test_oracle.py):
  e5m2_decode       exhaustive vs torch's float8_e5m2 -> float32 cast, and the
                    known-answer table of cpp_benchmarks/benchmark_scaled_mm_hip.cpp:127-137
  e5m2_encode       exhaustive over all fp16 and bf16 bit patterns, plus
                    ~2^22 fp32 patterns around every code boundary, vs torch's cast
  bf16_rne / fp16   vs torch's float32 -> bfloat16 / float16 casts (exhaustive
                    over sampled fp32 patterns)
  bf16_to_fp16_rtz  exhaustive 65,536 bf16 patterns: closed form (fp16-exact
                    values unchanged and equal to torch's cast, saturation, RTZ
                    in the fp16 subnormal range)
  prepack / unprepack / prepack_kn   brute-force index identity and round trips
  quantize_*        torch step-by-step evaluation and closed-form invariants
                    (max element -> code 0x7b, amax 0 -> scale 1, fp16 clamp
                    -> scale 1/65504, dequant error <= half a code step)
  scaled_mm_*       brute-force float64 loops on tiny shapes, all-ones weight
                    -> row sums, identity weight, naive == ref when no fp16
                    overflow; lora= : zero factors == no term, constant
                    factors -> closed-form R*t*u added before the rounding
                    (a term that moves a value across an fp16 tie)
"""

from __future__ import annotations

import numpy as np

E5M2_MAX = 57344.0
FP16_MAX = 65504.0

# ---------------------------------------------------------------------------
# fp8 e5m2 code table: [s:1][e:5][m:2], bias 15
# ---------------------------------------------------------------------------


def _e5m2_value(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 2) & 0x1F
    m = code & 0x3
    if e == 0x1F:
        return s * np.inf if m == 0 else np.nan
    if e == 0:
        return s * (m / 4.0) * 2.0**-14
    return s * (1.0 + m / 4.0) * 2.0 ** (e - 15)


E5M2_TABLE = np.array([_e5m2_value(c) for c in range(256)], dtype=np.float64)
# positive finite codes 0x00..0x7b in increasing value
_POS_VALUES = E5M2_TABLE[:0x7C]


def e5m2_decode(codes: np.ndarray) -> np.ndarray:
    """fp8 e5m2 code -> float32 (exact). Used by kernel/naive.py:20-22 (b.to(fp16))."""
    return E5M2_TABLE[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


def e5m2_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> fp8 e5m2 code, as torch's `.to(torch.float8_e5m2)`.

    Nearest representable value, ties to the code with an even mantissa;
    magnitudes at or above the midpoint 61440 between the largest finite code
    (57344) and 2^16 become infinity; NaN -> 0x7f with the sign bit kept.
    Used by comfy_feather/quant.py:73.
    """
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        ax = np.abs(x.astype(np.float64))
    hi = np.searchsorted(_POS_VALUES, ax, side="left")  # first value >= ax
    hi_c = np.minimum(hi, 0x7B)
    lo_c = np.maximum(hi - 1, 0)
    d_hi = np.abs(_POS_VALUES[hi_c] - ax)
    d_lo = np.abs(ax - _POS_VALUES[lo_c])
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((hi_c & 1) == 0))
    code = np.where(pick_hi, hi_c, lo_c).astype(np.uint8)
    code = np.where(ax >= 61440.0, np.uint8(0x7C), code)
    code = np.where(np.isnan(x), np.uint8(0x7F), code)
    sign = np.signbit(x).astype(np.uint8) << 7
    return (code | sign).astype(np.uint8)


# ---------------------------------------------------------------------------
# 16-bit float helpers (bf16 carried as uint16 bit patterns)
# ---------------------------------------------------------------------------


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (torch's conversion); NaN -> 0x7fc0."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    lo = (u & np.uint32(0xFFFF0000)).astype(np.uint32)
    step_bits = (lo + np.uint32(0x10000)).astype(np.uint32)  # next magnitude (may reach inf)
    with np.errstate(invalid="ignore"):
        lo_v = lo.view(np.float32).astype(np.float64)
        hi_v = step_bits.view(np.float32).astype(np.float64)
        # stepping past the largest finite bf16 lands on +-inf; its rounding
        # neighbour is +-2^128
        hi_v = np.where(np.isinf(hi_v), np.copysign(2.0**128, hi_v), hi_v)
        xv = x.astype(np.float64)
        d_lo = np.abs(xv - lo_v)
        d_hi = np.abs(hi_v - xv)
    lo_even = ((lo >> 16) & 1) == 0
    take_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ~lo_even)
    with np.errstate(invalid="ignore"):
        out = np.where(take_hi, step_bits >> 16, lo >> 16).astype(np.uint16)
    # exact values (including +-inf and zeros) keep their pattern
    out = np.where((u & np.uint32(0xFFFF)) == 0, (u >> 16).astype(np.uint16), out)
    out = np.where(np.isnan(x), np.uint16(0x7FC0), out)
    return out.astype(np.uint16)


def f32_to_fp16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> float16, round to nearest even, overflow to inf (IEEE)."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16)


_FP16_POS = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)  # +0 .. 65504


def bf16_to_fp16_rtz(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp16 bits, rounding toward zero (kernel/convert.py:12-18:
    v_cvt_pkrtz_f16_f32). Magnitudes above 65504 saturate to 65504, +-inf stay
    infinite, NaN stays NaN (returned as 0x7e00 | sign)."""
    b = np.asarray(bits, dtype=np.uint16)
    with np.errstate(invalid="ignore"):
        v = bf16_bits_to_f32(b).astype(np.float64)
    av = np.abs(v)
    with np.errstate(invalid="ignore"):
        idx = np.searchsorted(_FP16_POS, av, side="right") - 1  # largest fp16 <= |v|
    idx = np.clip(idx, 0, len(_FP16_POS) - 1)
    mag = idx.astype(np.uint16)
    mag = np.where(np.isinf(v), np.uint16(0x7C00), mag)
    mag = np.where(np.isnan(v), np.uint16(0x7E00), mag)
    sign = (b & np.uint16(0x8000)).astype(np.uint16)
    return (mag | sign).astype(np.uint16)


# ---------------------------------------------------------------------------
# layouts
# ---------------------------------------------------------------------------


def prepack_transpose(w_nk: np.ndarray) -> np.ndarray:
    """(N, K) -> (K/16, N, 16): P[i, n, j] = W[n, 16 i + j] (comfy_feather/quant.py:11-13)."""
    n, k = w_nk.shape
    out = np.empty((k // 16, n, 16), dtype=w_nk.dtype)
    for i in range(k // 16):
        out[i] = w_nk[:, 16 * i : 16 * i + 16]
    return out


def unprepack_transpose(p: np.ndarray) -> np.ndarray:
    """(K/16, N, 16) -> (N, K) (comfy_feather/quant.py:17-19)."""
    kg, n, _ = p.shape
    out = np.empty((n, kg * 16), dtype=p.dtype)
    for i in range(kg):
        out[:, 16 * i : 16 * i + 16] = p[i]
    return out


def prepack_kn(b_kn: np.ndarray) -> np.ndarray:
    """(K, N) -> (K/16, N, 16): P[i, n, j] = B[16 i + j, n] (kernel/hip/hip_kernel.py:170-171)."""
    k, n = b_kn.shape
    out = np.empty((k // 16, n, 16), dtype=b_kn.dtype)
    for i in range(k // 16):
        out[i] = b_kn[16 * i : 16 * i + 16, :].T
    return out


def unprepack_kn(p: np.ndarray) -> np.ndarray:
    """(K/16, N, 16) -> (K, N) (kernel/naive.py:13-16)."""
    kg, n, _ = p.shape
    out = np.empty((kg * 16, n), dtype=p.dtype)
    for i in range(kg):
        out[16 * i : 16 * i + 16, :] = p[i].T
    return out


# ---------------------------------------------------------------------------
# quantize (comfy_feather/quant.py:52-74, 116-146)
# ---------------------------------------------------------------------------

DT_F16, DT_BF16, DT_F32 = "f16", "bf16", "f32"


def _to_f32(w: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == DT_F16:
        return np.asarray(w, dtype=np.float16).astype(np.float32)
    if dtype == DT_BF16:
        return bf16_bits_to_f32(w)
    return np.asarray(w, dtype=np.float32)


def _round_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to `dtype` and return them as float32."""
    if dtype == DT_F16:
        return f32_to_fp16_rne(x).astype(np.float32)
    if dtype == DT_BF16:
        return bf16_bits_to_f32(f32_to_bf16_rne(x))
    return np.asarray(x, dtype=np.float32)


def _scale_from_amax(amax: np.float32, dtype: str) -> np.float32:
    """quant.py:54-58: s = amax / 57344 (fp32 division); 0 -> 1; fp16 clamps 1/s."""
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        s = np.float32(amax) / np.float32(E5M2_MAX)
        if s == 0:
            s = np.float32(1.0)
        if dtype == DT_F16:
            r = np.float32(1.0) / s
            if not np.isnan(r):
                r = np.float32(min(max(float(r), -FP16_MAX), FP16_MAX))
            s = np.float32(1.0) / r
    return np.float32(s)


def quantize_native(w: np.ndarray, dtype: str, scale: float | None = None) -> tuple[np.ndarray, np.float32]:
    """quantize_fp8e5m2_scaled(x) with x in its own dtype (quant.py:52-74), as
    called by the patch path (quant.py:81-96,139-146). Returns the (N, K) codes
    (unprepacked) and the fp32 scale."""
    x = _to_f32(w, dtype)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        if scale is None:
            amax = np.float32(np.max(np.abs(x))) if x.size else np.float32(0)
            if np.isnan(x).any():
                amax = np.float32(np.nan)
            s = _scale_from_amax(amax, dtype)
        else:
            s = np.float32(scale)
        inv = _round_dtype(np.array([np.float32(1.0) / s], dtype=np.float32), dtype)[0]
        xs = _round_dtype(x * inv, dtype)
    return e5m2_encode(xs), np.float32(s)


def quantize_load(w: np.ndarray, dtype: str, ckpt_scale: float | None = None) -> tuple[np.ndarray, np.float32]:
    """make_feather_quantized_weight for a non-e5m2 weight (quant.py:116-136):
    quantize_fp8e5m2_scaled(weight.to(float32) * scale) -- all fp32."""
    x = _to_f32(w, dtype) * np.float32(1.0 if ckpt_scale is None else ckpt_scale)
    return quantize_native(x.astype(np.float32), DT_F32)


def dequantize(codes_nk: np.ndarray, scale: float, dtype: str) -> np.ndarray:
    """quant.py:99-102: (float32(q) * scale).to(orig_dtype). Returns float32 values
    for f32, float16 for f16, bf16 bits for bf16."""
    v = e5m2_decode(codes_nk) * np.float32(scale)
    if dtype == DT_F16:
        return f32_to_fp16_rne(v)
    if dtype == DT_BF16:
        return f32_to_bf16_rne(v)
    return v.astype(np.float32)


# ---------------------------------------------------------------------------
# GEMM (kernel/naive.py:4-41 and kernel/hip/hip_kernel.cu:366-419)
# ---------------------------------------------------------------------------


def _finish(acc32: np.ndarray, scale, bias, out_dtype: str, term=None) -> np.ndarray:
    """scale in fp32 -> (+ term, one fp32 rounding) -> round to out dtype ->
    bias added in out dtype."""
    with np.errstate(over="ignore", invalid="ignore"):
        c = acc32.astype(np.float32)
        if scale is not None:
            c = c * np.float32(scale)
        if term is not None:
            c = (c.astype(np.float64) + term).astype(np.float32)
        if out_dtype == DT_F16:
            y = f32_to_fp16_rne(c)
            if bias is not None:
                y = f32_to_fp16_rne(y.astype(np.float32) + np.asarray(bias, dtype=np.float16).astype(np.float32))
            return y
        y = f32_to_bf16_rne(c)
        if bias is not None:
            y = f32_to_bf16_rne(bf16_bits_to_f32(y) + bf16_bits_to_f32(bias))
        return y


def _decode_b(b_prepacked: np.ndarray, b_dtype: str) -> np.ndarray:
    codes = unprepack_kn(np.asarray(b_prepacked, dtype=np.uint8))
    if b_dtype == "e5m2":
        return e5m2_decode(codes)
    return e4m3fn_decode(codes)


def scaled_mm_ref(a: np.ndarray, b_prepacked: np.ndarray, scale, bias, out_dtype: str,
                  b_dtype: str = "e5m2", lora=None) -> np.ndarray:
    """The kernel contract (hip_kernel.cu:366-419 with a round-to-nearest bf16
    epilogue): sum in float64 then float32, scale on the float32 value, round
    to the output type, add bias in the output type. fp16 out -> float16 array,
    bf16 out -> uint16 bits.

    lora=(T, U): the fused unmerged-LoRA epilogue -- T (M, R) . U (N, R)^T,
    summed in float64, is added to the scaled float32 value before the output
    rounding. This is the build's own contract for that path: the reference
    (comfy_feather/lora.py:4-35) instead adds F.linear(F.linear(x, A), B) * s
    to the finished output with a rounding to x's dtype after every step, so
    the two agree to those roundings, not bit for bit."""
    a64 = np.asarray(a, dtype=np.float16).astype(np.float64)
    b64 = _decode_b(b_prepacked, b_dtype).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        acc = (a64 @ b64).astype(np.float32)
    term = None
    if lora is not None:
        t, u = (np.asarray(f, dtype=np.float64) for f in lora)
        term = t @ u.T
    return _finish(acc, scale, bias, out_dtype, term)


def scaled_mm_ref_f32(a: np.ndarray, b_prepacked: np.ndarray, scale, b_dtype: str = "e5m2") -> np.ndarray:
    """float64 value of (A @ dec(B)) * scale before any output rounding."""
    a64 = np.asarray(a, dtype=np.float16).astype(np.float64)
    b64 = _decode_b(b_prepacked, b_dtype).astype(np.float64)
    acc = a64 @ b64
    return acc * (1.0 if scale is None else float(np.float32(scale)))


def scaled_mm_naive(a: np.ndarray, b_prepacked: np.ndarray, scale, bias, out_dtype: str,
                    b_dtype: str = "e5m2") -> np.ndarray:
    """kernel/naive.py:4-41 as written: the product is rounded to fp16 *before*
    the scale (naive.py:20-23), which overflows to inf once |A @ B| > 65504."""
    a32 = np.asarray(a, dtype=np.float16).astype(np.float32)
    b32 = _decode_b(b_prepacked, b_dtype)
    with np.errstate(over="ignore", invalid="ignore"):
        c16 = f32_to_fp16_rne(a32 @ b32)
    return _finish(c16.astype(np.float32), scale, bias, out_dtype)


def e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    """fp8 e4m3fn code -> float32: [s:1][e:4][m:3], bias 7, no inf, 0x7f/0xff NaN."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, (m / 8.0) * 2.0**-6, (1.0 + m / 8.0) * np.power(2.0, e - 7))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(np.float32)


def scaled_mm_naive_torch(a, b_prepacked, scale, bias, out_dtype):
    """kernel/naive.py:4-41 (b_prepacked=True, per-tensor scale) on host torch, for the CPU
    baseline: the (K/16, N, 16) codes are unpacked to (K, N) and decoded to fp16, the product is
    torch's fp16 CPU matmul (rounded to fp16, naive.py:20-23), then scale in fp32, cast to
    out_dtype, bias added in out_dtype. a: fp16 (M, K) tensor; b_prepacked: uint8 or fp8
    (K/16, N, 16) tensor; scale: 0-d/1-element fp32 tensor or None; bias: (N,) tensor or None."""
    import torch

    k16, n, _ = b_prepacked.shape
    codes = b_prepacked.view(torch.uint8).transpose(1, 2).reshape(k16 * 16, n)
    w16 = codes.view(torch.float8_e5m2).to(torch.float16)
    prod = torch.matmul(a.to(torch.float16), w16)
    if scale is not None:
        prod = prod.float() * scale.float().reshape(())
    y = prod.to(out_dtype)
    if bias is not None:
        y = y + bias.to(out_dtype)
    return y


def lora_down_ref(x: np.ndarray, d: np.ndarray, dtype: str) -> np.ndarray:
    """T = F.linear(x, lora_A), the first step of the reference's LoRA side path
    (comfy_feather/lora.py:27-30): x (M, K) and d (R, K) in dtype (float16 arrays,
    or uint16 bf16 bits), the products summed in float64, rounded to float32 and
    then to dtype (nearest even). Returns float16 for f16, uint16 bf16 bits for bf16."""
    if dtype == DT_F16:
        x64 = np.asarray(x, dtype=np.float16).astype(np.float64)
        d64 = np.asarray(d, dtype=np.float16).astype(np.float64)
    else:
        x64 = bf16_bits_to_f32(np.asarray(x, dtype=np.uint16)).astype(np.float64)
        d64 = bf16_bits_to_f32(np.asarray(d, dtype=np.uint16)).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        acc = (x64 @ d64.T).astype(np.float32)
    return f32_to_fp16_rne(acc) if dtype == DT_F16 else f32_to_bf16_rne(acc)
