"""CPU checks that pin the numpy oracle (oracle/feather_oracle.py).

Ground truths: torch's own fp8/bf16/fp16 casts (the reference's arithmetic is
those casts), the reference's e5m2 known-answer table, closed forms and brute
force on tiny shapes. The golden fixtures are checked to still equal the
oracle."""

import hashlib

import numpy as np
import pytest
import torch

from oracle import feather_oracle as O

from conftest import GOLDEN

ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_e5m2_decode_exhaustive_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes).view(torch.float8_e5m2).to(torch.float32).numpy()
    o = O.e5m2_decode(codes)
    assert np.array_equal(np.isnan(t), np.isnan(o))
    assert np.array_equal(t[~np.isnan(t)], o[~np.isnan(o)])


def test_e4m3fn_decode_exhaustive_vs_torch():
    # reference kernel/hip/hip_kernel.py:37 routes float8_e4m3fn weights to the same GEMM and
    # test_scaled_mm_hip.py:53-54 builds them with torch's cast: torch's decode is the ground truth
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    o = O.e4m3fn_decode(codes)
    assert np.array_equal(np.isnan(t), np.isnan(o))
    assert np.array_equal(np.isnan(o).nonzero()[0], [0x7F, 0xFF])
    fin = ~np.isnan(t)
    assert np.array_equal(t[fin].view(np.uint32), o[fin].view(np.uint32))  # signed zeros included


def test_e4m3fn_known_answers():
    # values fixed by the OCP fp8 definition: max normal 448, min normal 2^-6, min subnormal 2^-9
    kat = {0x00: 0.0, 0x38: 1.0, 0xB8: -1.0, 0x7E: 448.0, 0xFE: -448.0, 0x08: 2.0**-6,
           0x01: 2.0**-9, 0x07: 7 * 2.0**-9, 0x3C: 1.5, 0x40: 2.0, 0x30: 0.5}
    for code, val in kat.items():
        assert O.e4m3fn_decode(np.array([code], np.uint8))[0] == val
    # the encode direction through torch round-trips every finite code
    codes = np.arange(256, dtype=np.uint8)
    vals = O.e4m3fn_decode(codes)
    fin = ~np.isnan(vals)
    back = torch.from_numpy(vals[fin]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(back, codes[fin])


def test_e5m2_known_answers():
    # cpp_benchmarks/benchmark_scaled_mm_hip.cpp:127-137 of the reference
    kat = {0xBC: -1.0, 0xBA: -0.75, 0xB8: -0.5, 0xB4: -0.25, 0x00: 0.0, 0x34: 0.25, 0x38: 0.5, 0x3A: 0.75, 0x3C: 1.0}
    for code, val in kat.items():
        assert O.e5m2_decode(np.array([code], np.uint8))[0] == val
        assert O.e5m2_encode(np.array([val], np.float32))[0] == (0x80 if code == 0x00 and val < 0 else code)
    # fp16 bits are the code shifted into the high byte for every code (the kernel's widen)
    codes = np.arange(256, dtype=np.uint16)
    widened = (codes << 8).astype(np.uint16).view(np.float16).astype(np.float32)
    o = O.e5m2_decode(codes.astype(np.uint8))
    assert np.array_equal(np.isnan(widened), np.isnan(o))
    assert np.array_equal(widened[~np.isnan(o)], o[~np.isnan(o)])


def test_e5m2_encode_exhaustive_fp16_bf16_vs_torch():
    f16 = ALL16.view(np.float16)
    t = torch.from_numpy(f16.copy()).to(torch.float8_e5m2).view(torch.uint8).numpy()
    assert np.array_equal(O.e5m2_encode(f16.astype(np.float32)), t)
    tb = torch.from_numpy(ALL16.view(np.int16).copy()).view(torch.bfloat16).to(torch.float8_e5m2)
    assert np.array_equal(O.e5m2_encode(O.bf16_bits_to_f32(ALL16)), tb.view(torch.uint8).numpy())


def test_e5m2_encode_fp32_boundaries_vs_torch():
    # every code value and every midpoint, +-64 ulps around each, both signs
    vals = O.E5M2_TABLE[np.isfinite(O.E5M2_TABLE)]
    vals = np.unique(np.abs(vals))
    mids = (vals[1:] + vals[:-1]) / 2
    pts = np.concatenate([vals, mids, [61440.0, 65536.0, 2.0**-17, 2.0**-16 * 1.5]]).astype(np.float32)
    bits = pts.view(np.uint32)[:, None].astype(np.int64) + np.arange(-64, 65)[None, :]
    bits = np.clip(bits, 0, 0x7FFFFFFF).astype(np.uint32).reshape(-1)
    x = np.concatenate([bits.view(np.float32), -bits.view(np.float32)])
    rng = np.random.default_rng(0)
    x = np.concatenate([x, rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    t = torch.from_numpy(x.copy()).to(torch.float8_e5m2).view(torch.uint8).numpy()
    assert np.array_equal(O.e5m2_encode(x), t)


def test_bf16_and_fp16_rounding_vs_torch():
    rng = np.random.default_rng(1)
    x = rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # include exact ties for bf16
    ties = (rng.integers(0, 2**16, 4096, dtype=np.uint64).astype(np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, np.array([3.4028235e38, -3.4028235e38, 0.0, -0.0], np.float32)])
    tb = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ob = O.f32_to_bf16_rne(x)
    nan = np.isnan(x)
    assert np.array_equal(ob[~nan], tb[~nan])
    assert np.all(ob[nan] == 0x7FC0)
    th = torch.from_numpy(x.copy()).to(torch.float16).numpy()
    oh = O.f32_to_fp16_rne(x)
    assert np.array_equal(oh[~nan].view(np.uint16), th[~nan].view(np.uint16))


def test_bf16_to_fp16_rtz_closed_form():
    out = O.bf16_to_fp16_rtz(ALL16)
    v = O.bf16_bits_to_f32(ALL16).astype(np.float64)
    o = out.view(np.float16).astype(np.float64)
    fin = np.isfinite(v)
    normal = fin & (np.abs(v) >= 2.0**-14) & (np.abs(v) <= 65504)
    # every bf16 value in fp16's normal range is exact in fp16: RTZ == RNE == torch
    t = torch.from_numpy(ALL16.view(np.int16).copy()).view(torch.bfloat16).to(torch.float16).numpy()
    assert np.array_equal(out[normal], t[normal].view(np.uint16))
    # saturation instead of inf
    big = fin & (np.abs(v) > 65504)
    assert np.all(np.abs(o[big]) == 65504) and np.array_equal(np.sign(o[big]), np.sign(v[big]))
    # subnormal range: truncation, |o| <= |v| < |o| + 2^-24, same sign
    small = fin & (np.abs(v) < 2.0**-14)
    assert np.all(np.abs(o[small]) <= np.abs(v[small]))
    assert np.all(np.abs(v[small]) - np.abs(o[small]) < 2.0**-24)
    assert np.array_equal(np.signbit(o[small]), np.signbit(v[small]))
    assert np.all(np.isinf(o[np.isinf(v)])) and np.all(np.isnan(o[np.isnan(v)]))


@pytest.mark.parametrize("n,k", [(1, 16), (3, 32), (5, 48), (64, 64)])
def test_prepack_index_identity(n, k):
    w = np.random.default_rng(n).integers(0, 256, (n, k), dtype=np.uint8)
    p = O.prepack_transpose(w)
    for i in range(k // 16):
        for r in range(n):
            for j in range(16):
                assert p[i, r, j] == w[r, 16 * i + j]
    assert np.array_equal(O.unprepack_transpose(p), w)
    b = w.T.copy()  # (K, N)
    pb = O.prepack_kn(b)
    assert np.array_equal(pb, p)  # (K,N) prepack of W^T == (N,K) prepack of W
    assert np.array_equal(O.unprepack_kn(pb), b)


def _torch_quant_steps(x: torch.Tensor, clamp_fp16: bool):
    """quant.py:52-74 evaluated with torch CPU ops, one step per line."""
    s = torch.amax(x.abs()).to(torch.float32) / 57344.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    if clamp_fp16:
        s = 1.0 / torch.clamp(1.0 / s, min=-65504.0, max=65504.0)
    inv = (1.0 / s).to(x.dtype)
    return (x * inv).to(torch.float8_e5m2).view(torch.uint8).numpy(), np.float32(s.item())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("std", [0.02, 1.0, 300.0])
def test_quantize_native_vs_torch_steps(dtype, std):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(64, 128, generator=g) * std).to(dtype)
    t_codes, t_s = _torch_quant_steps(x, dtype == torch.float16)
    if dtype == torch.bfloat16:
        xin, dt = x.view(torch.int16).numpy().view(np.uint16), O.DT_BF16
    else:
        xin, dt = x.numpy(), {torch.float16: O.DT_F16, torch.float32: O.DT_F32}[dtype]
    codes, s = O.quantize_native(xin, dt)
    assert s == t_s
    assert np.array_equal(codes, t_codes)


def test_quantize_load_invariants():
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(256, 512, generator=g) * 0.02).numpy()
    codes, s = O.quantize_load(w, O.DT_F32)
    amax = np.float32(np.abs(w).max())
    assert s == np.float32(amax / np.float32(57344.0))
    # the largest element lands exactly on the largest finite code
    idx = np.unravel_index(np.argmax(np.abs(w)), w.shape)
    assert codes[idx] & 0x7F == 0x7B
    assert np.all((codes & 0x7F) <= 0x7B)  # nothing overflows
    # dequantized values are within half a code step (relative 2^-3) of w
    deq = O.e5m2_decode(codes).astype(np.float64) * s
    big = np.abs(w) > 2.0**-14 * s
    assert np.all(np.abs(deq[big] - w[big]) <= np.abs(w[big]) * 2.0**-3 + 1e-30)
    # checkpoint scale multiplies first: quantizing w*2 with ckpt 1 == w with ckpt 2
    c2, s2 = O.quantize_load(w, O.DT_F32, ckpt_scale=2.0)
    c3, s3 = O.quantize_load((w * np.float32(2.0)).astype(np.float32), O.DT_F32)
    assert np.array_equal(c2, c3) and s2 == s3


def test_quantize_special_cases():
    z = np.zeros((16, 32), np.float16)
    codes, s = O.quantize_native(z, O.DT_F16)
    assert s == 1.0 and np.all(codes == 0)
    # fp16 clamp: amax < 57344/65504 gives scale 1/65504 rather than amax/57344
    w = np.full((16, 32), 0.09, np.float16)
    _, s16 = O.quantize_native(w, O.DT_F16)
    assert s16 == np.float32(1.0) / np.float32(65504.0)
    _, s32 = O.quantize_load(w, O.DT_F16)
    assert s32 == np.float32(np.float32(np.float16(0.09)) / np.float32(57344.0))


def test_scaled_mm_oracle_brute_force():
    rng = np.random.default_rng(5)
    M, N, K = 3, 16, 32
    a = rng.standard_normal((M, K)).astype(np.float16)
    codes = rng.integers(0, 0x7C, (K, N), dtype=np.uint8) | (rng.integers(0, 2, (K, N), dtype=np.uint8) << 7)
    bp = O.prepack_kn(codes)
    s = np.float32(0.37)
    exact = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            exact[m, n] = sum(float(a[m, k]) * float(O.E5M2_TABLE[codes[k, n]]) for k in range(K))
    got = O.scaled_mm_ref_f32(a, bp, s)
    assert np.allclose(got, exact * float(s), rtol=1e-12, atol=0)
    y = O.scaled_mm_ref(a, bp, s, None, O.DT_F16)
    assert np.array_equal(y, (np.float32(exact) * s).astype(np.float16))


def test_scaled_mm_oracle_special_weights():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((8, 64)).astype(np.float16)
    ones = np.full((64, 16), 0x3C, np.uint8)  # 1.0
    y = O.scaled_mm_ref_f32(a, O.prepack_kn(ones), None)
    assert np.allclose(y, a.astype(np.float64).sum(1, keepdims=True).repeat(16, 1))
    eye = np.zeros((64, 64), np.uint8)
    eye[np.arange(64), np.arange(64)] = 0x3C
    y = O.scaled_mm_ref(a, O.prepack_kn(eye), None, None, O.DT_F16)
    assert np.array_equal(y, a)
    # naive (fp16 product then scale) equals the fp32 path when nothing overflows and scale is a power of 2
    b = rng.integers(0x30, 0x3C, (64, 16), dtype=np.uint8)
    yn = O.scaled_mm_naive(a, O.prepack_kn(b), np.float32(0.5), None, O.DT_F16)
    yr = O.scaled_mm_ref(a, O.prepack_kn(b), np.float32(0.5), None, O.DT_F16)
    assert np.array_equal(yn, yr)


def test_scaled_mm_oracle_lora_term():
    """lora=(T, U) adds T . U^T to the scaled float32 value before the output
    rounding: zero factors change nothing; constant factors give R*t*u, placed
    so that only the before-rounding order moves the result across an fp16 tie."""
    rng = np.random.default_rng(7)
    a = rng.standard_normal((8, 64)).astype(np.float16)
    b = O.prepack_kn(rng.integers(0x30, 0x3C, (64, 32), dtype=np.uint8))
    z_t, z_u = np.zeros((8, 32)), np.zeros((32, 32))
    for od in (O.DT_F16, O.DT_BF16):
        assert np.array_equal(O.scaled_mm_ref(a, b, np.float32(0.5), None, od, lora=(z_t, z_u)),
                              O.scaled_mm_ref(a, b, np.float32(0.5), None, od))
    eye = np.zeros((64, 64), np.uint8)
    eye[np.arange(64), np.arange(64)] = 0x3C
    ones = np.ones((1, 64), np.float16)
    s = np.float32(1 + 2.0**-11 - 2.0**-20)  # alone: just below the tie 1 + 2^-11 -> rounds to 1.0
    t = np.full((1, 32), 2.0**-12)
    u = np.full((64, 32), 2.0**-12)  # R * t * u = 2^-19 lifts it past the tie
    y = O.scaled_mm_ref(ones, O.prepack_kn(eye), s, None, O.DT_F16, lora=(t, u))
    assert np.all(y == np.float16(1 + 2.0**-10))
    assert np.all(O.scaled_mm_ref(ones, O.prepack_kn(eye), s, None, O.DT_F16) == np.float16(1.0))


def test_golden_fixtures_match_oracle():
    z = np.load(GOLDEN / "e5m2_codes.npz")
    assert np.array_equal(z["from_fp16"], O.e5m2_encode(ALL16.view(np.float16).astype(np.float32)))
    r = np.load(GOLDEN / "bf16_rtz.npz")
    assert np.array_equal(r["fp16_bits"], O.bf16_to_fp16_rtz(ALL16))
    q = np.load(GOLDEN / "quant_c1.npz")
    g = torch.Generator().manual_seed(0)
    w32 = torch.randn(1024, 1024, generator=g) * 0.02
    codes, s = O.quantize_load(w32.half().numpy(), O.DT_F16)
    assert s == q["load_f16_scale"][0]
    packed = O.prepack_transpose(codes)
    assert hashlib.sha256(packed.tobytes()).digest() == q["load_f16_sha256"].tobytes()
    assert np.array_equal(codes[q["rows"]], q["load_f16_rows"])
    # the patch path on fp16 hits the reciprocal clamp (amax ~0.1 < 0.875)
    assert q["native_f16_scale"][0] == np.float32(1.0) / np.float32(65504.0)
    gm = np.load(GOLDEN / "gemm_small.npz")
    y = O.scaled_mm_ref(gm["a"], gm["b_prepacked"], gm["scale"][0], gm["bias_f16"], O.DT_F16)
    assert np.array_equal(y, gm["out_f16"])


def test_naive_torch_matches_numpy_naive():
    """The host-torch restatement of kernel/naive.py (the CPU baseline) against the numpy one:
    both round A @ B to fp16 before the scale; torch's fp16 CPU matmul sums in another order,
    so they agree to the fp16 rounding of the product, not bit for bit. A wrong unpack or a
    transposed operand would be off by O(1)."""
    g = torch.Generator().manual_seed(3)
    for M, N, K in [(64, 128, 256), (256, 1024, 1024), (33, 80, 4096)]:
        a = torch.randn(M, K, generator=g).half()
        w = (torch.randn(K, N, generator=g) * 0.05).to(torch.float8_e5m2).view(torch.uint8).numpy()
        packed = O.prepack_kn(w)
        s = np.float32(0.75)
        bias = (torch.randn(N, generator=g) * 0.01).half()
        y = O.scaled_mm_naive_torch(a, torch.from_numpy(packed), torch.tensor(s), bias, torch.float16)
        r = O.scaled_mm_naive(a.numpy(), packed, s, bias.numpy(), O.DT_F16).astype(np.float32)
        assert y.dtype == torch.float16 and y.shape == (M, N)
        y = y.float().numpy()
        assert np.allclose(y, r, rtol=2e-3, atol=1e-3 * np.abs(r).max())
        ref = O.scaled_mm_ref(a.numpy(), packed, s, bias.numpy(), O.DT_F16).astype(np.float32)
        assert np.allclose(y, ref, rtol=2e-3, atol=1e-3 * np.abs(ref).max())


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_lora_down_ref_brute_force_and_selection(dtype):
    """lora_down_ref against explicit per-element loops on a tiny case, and a selection
    matrix (d rows = unit vectors) that must return columns of x exactly."""
    rng = np.random.default_rng(5)
    M, K, R = 3, 16, 4
    xf = rng.standard_normal((M, K)).astype(np.float32)
    df = rng.standard_normal((R, K)).astype(np.float32)
    if dtype == "f16":
        x, d = xf.astype(np.float16), df.astype(np.float16)
        xv, dv = x.astype(np.float64), d.astype(np.float64)
    else:
        x, d = O.f32_to_bf16_rne(xf), O.f32_to_bf16_rne(df)
        xv, dv = O.bf16_bits_to_f32(x).astype(np.float64), O.bf16_bits_to_f32(d).astype(np.float64)
    t = O.lora_down_ref(x, d, dtype)
    for m in range(M):
        for r in range(R):
            s = 0.0
            for k in range(K):
                s += xv[m, k] * dv[r, k]
            want = np.float32(s)
            got = float(t[m, r]) if dtype == "f16" else float(O.bf16_bits_to_f32(np.array([t[m, r]]))[0])
            want_r = float(np.float16(want)) if dtype == "f16" else float(
                O.bf16_bits_to_f32(O.f32_to_bf16_rne(np.array([want], np.float32)))[0])
            assert got == want_r
    sel = np.zeros((K, K), np.float32)
    sel[np.arange(K), rng.permutation(K)] = 1.0
    ds = sel.astype(np.float16) if dtype == "f16" else O.f32_to_bf16_rne(sel)
    cols = O.lora_down_ref(x, ds, dtype)
    perm = sel.argmax(1)
    assert np.array_equal(np.asarray(cols).view(np.uint16), np.asarray(x)[:, perm].view(np.uint16))
