"""GPU parity of the scaled_mm kernels against the oracle (through the C ABI
and the drop-in Python API)."""

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import (assert_gemm_close, assert_gemm_close_dev, assert_row_col_checksums, capi_scaled_mm, lib,
                      stream, to_dev_codes, torch_ref_dev, weight_like)
from oracle import feather_oracle as O

pytestmark = pytest.mark.gpu

TILE_CFGS = [(2, 4, 4, 8, 4), (4, 2, 4, 4, 8), (4, 2, 4, 4, 4), (2, 4, 4, 8, 3), (2, 4, 4, 4, 6), (2, 4, 4, 4, 4), (4, 2, 4, 2, 4), (1, 8, 4, 8, 2), (1, 1, 2, 2, 2)]


def _bias_for(out_dtype, n, gen):
    b16 = (torch.randn(n, generator=gen) * 0.01).half()
    if out_dtype == torch.float16:
        return b16, b16.numpy()
    bb = b16.float().bfloat16()
    return bb, bb.view(torch.int16).numpy().view(np.uint16)


def test_golden_small_all_kernels(cuda, hk):
    z = np.load(GOLDEN / "gemm_small.npz")
    a = torch.from_numpy(z["a"]).to(cuda)
    bp = to_dev_codes(z["b_prepacked"], cuda)
    s = torch.from_numpy(z["scale"]).to(cuda)
    b16 = torch.from_numpy(z["bias_f16"]).to(cuda)
    bbf = torch.from_numpy(z["bias_bf16"].view(np.int16)).view(torch.bfloat16).to(cuda)
    for cfg in hk._CONFIGS:
        print("golden cfg", cfg, flush=True)
        y = capi_scaled_mm(a, bp, s, b16, torch.float16, cfg)
        assert_gemm_close(y, z["out_f16"], torch.float16, f"f16 {cfg}")
        y = capi_scaled_mm(a, bp, s, bbf, torch.bfloat16, cfg)
        assert_gemm_close(y, z["out_bf16"], torch.bfloat16, f"bf16 {cfg}")


@pytest.mark.parametrize("M,N,K", [(16, 128, 128), (48, 256, 1024), (64, 512, 4096), (128, 128, 128),
                                   (256, 256, 512), (512, 256, 256), (100, 384, 320), (300, 512, 1040),
                                   (1024, 1024, 1024)])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("splitk", ["default", "0"])
def test_shapes_and_tiles(cuda, monkeypatch, M, N, K, out_dtype, splitk):
    """Every tile config on each shape; FEATHEROPS_SPLITK=0 keeps small shapes on
    the tuple's tile kernel instead of the split-K tiles they are routed to."""
    if splitk != "default":
        monkeypatch.setenv("FEATHEROPS_SPLITK", splitk)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    a = torch.randn(M, K, generator=g).half()
    packed, s = weight_like(N, K, g)
    bias, bias_np = _bias_for(out_dtype, N, g)
    od = O.DT_F16 if out_dtype == torch.float16 else O.DT_BF16
    ref = O.scaled_mm_ref(a.numpy(), packed, s, bias_np, od)
    ad, bd = a.to(cuda), to_dev_codes(packed, cuda)
    sd = torch.tensor([s], device=cuda)
    for cfg in TILE_CFGS:
        print("shape", M, N, K, out_dtype, cfg, flush=True)
        y = capi_scaled_mm(ad, bd, sd, bias.to(cuda), out_dtype, cfg)
        assert_gemm_close(y, ref, out_dtype, f"{M}x{N}x{K} {cfg}")


@pytest.mark.parametrize("b_dtype", [torch.float8_e5m2, torch.float8_e4m3fn])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
def test_reference_style_inputs(cuda, hk, b_dtype, out_dtype):
    """The reference test's data (test_scaled_mm_hip.py:10-13): B = randn cast to
    fp8, scale 2.34, bias randn in the output type, every compatible config."""
    g = torch.Generator().manual_seed(11)
    for M, N, K in [(16, 128, 128), (256, 256, 256), (512, 512, 512)]:
        a = torch.randn(M, K, generator=g).half()
        b = torch.randn(K, N, generator=g).to(b_dtype)
        bias = torch.randn(N, generator=g).to(out_dtype)
        codes_kn = b.view(torch.uint8).numpy()
        packed = O.prepack_kn(codes_kn)
        bias_np = bias.numpy() if out_dtype == torch.float16 else bias.view(torch.int16).numpy().view(np.uint16)
        od = O.DT_F16 if out_dtype == torch.float16 else O.DT_BF16
        ref = O.scaled_mm_ref(a.numpy(), packed, np.float32(2.34), bias_np, od,
                              "e5m2" if b_dtype == torch.float8_e5m2 else "e4m3")
        bp = hk.prepack_b_for_scaled_mm(b.to(cuda))
        assert np.array_equal(bp.view(torch.uint8).cpu().numpy(), packed)
        s = torch.tensor(2.34, device=cuda)
        for cfg in hk._CONFIGS:
            bm, bn, ck = 16 * cfg[0] * cfg[3], 16 * cfg[1] * cfg[4], 16 * cfg[2]
            if M % bm or N % bn or K % ck:
                continue
            y = hk.scaled_mm_hip_configured(a.to(cuda), bp, s, bias.to(cuda), out_dtype, *cfg)
            torch.cuda.synchronize()
            assert_gemm_close(y, ref, out_dtype, f"{M}x{N}x{K} {cfg} {b_dtype}")


def test_special_weights(cuda):
    g = torch.Generator().manual_seed(2)
    M, K, N = 192, 256, 128
    a = torch.randn(M, K, generator=g).half()
    ad = a.to(cuda)
    ones_np = O.prepack_kn(np.full((K, N), 0x3C, np.uint8))
    ones = to_dev_codes(ones_np, cuda)
    for cfg in [(2, 4, 4, 8, 4), (1, 1, 2, 1, 2)]:
        for m in (M, 16):
            y = capi_scaled_mm(ad[:m].contiguous(), ones, None, None, torch.float16, cfg)
            assert (y == y[:, :1]).all(), "all-ones weight: every column is the row sum"
            ref = O.scaled_mm_ref(a.numpy()[:m], ones_np, None, None, O.DT_F16)
            assert_gemm_close(y, ref, torch.float16, f"row sums {cfg} m={m}")
    eye = np.zeros((K, K), np.uint8)
    eye[np.arange(K), np.arange(K)] = 0x3C
    y = capi_scaled_mm(ad, to_dev_codes(O.prepack_kn(eye), cuda), None, None, torch.float16)
    assert torch.equal(y.cpu(), a)
    # scale only, no bias; bias only, no scale
    packed, s = weight_like(N, K, g)
    bd = to_dev_codes(packed, cuda)
    ref = O.scaled_mm_ref(a.numpy(), packed, s, None, O.DT_F16)
    assert_gemm_close(capi_scaled_mm(ad, bd, torch.tensor([s], device=cuda), None, torch.float16), ref,
                      torch.float16)
    bias = (torch.randn(N, generator=g)).half()
    ref = O.scaled_mm_ref(a.numpy(), packed, None, bias.numpy(), O.DT_F16)
    assert_gemm_close(capi_scaled_mm(ad, bd, None, bias.to(cuda), torch.float16), ref, torch.float16)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,cfg", [(256, 256, (2, 4, 4, 8, 4)), (16, 256, (1, 1, 2, 1, 2)),
                                     (64, 256, (1, 8, 4, 8, 2)), (256, 272, (2, 4, 4, 8, 4))])
def test_signed_zero_outputs(cuda, M, K, cfg, out_dtype):
    """Zero rows of A under a negative scale: the oracle's fp32 product 0 * s
    is -0, so every output of those rows is -0 (sign bit set) on every path:
    LDS tiles, small-M kernel, split-K tiles, register-staged tile (K % 64)."""
    g = torch.Generator().manual_seed(11)
    N = 256
    a = torch.randn(M, K, generator=g).half()
    a[::3] = 0.0
    packed, _ = weight_like(N, K, g)
    s = -0.75
    ref = O.scaled_mm_ref(a.numpy(), packed, np.float32(s), None, O.DT_F16 if out_dtype == torch.float16 else O.DT_BF16)
    y = capi_scaled_mm(a.to(cuda), to_dev_codes(packed, cuda), torch.tensor([s], device=cuda), None, out_dtype, cfg)
    bits = y.view(torch.int16).cpu().numpy().view(np.uint16)
    ref_bits = ref.view(np.uint16) if ref.dtype == np.float16 else ref
    assert (ref_bits[::3] == 0x8000).all(), "oracle: 0 * negative scale is -0"
    assert np.array_equal(bits[::3], ref_bits[::3]), f"signed zeros {M}x{K} {cfg}"
    assert_gemm_close(y, ref, out_dtype, f"negative scale {M}x{K} {cfg}")


def test_inf_nan_propagation(cuda):
    M, K, N = 64, 128, 64
    a = torch.ones(M, K, dtype=torch.float16)
    a[3, 5] = float("inf")
    a[7, 9] = float("nan")
    codes = np.full((K, N), 0x3C, np.uint8)
    codes[5, 10] = 0xBC  # -1 meets +inf -> -inf in column 10
    ref = O.scaled_mm_ref(a.numpy(), O.prepack_kn(codes), None, None, O.DT_F16)
    for cfg in [(2, 4, 4, 8, 4), (1, 1, 2, 1, 2)]:
        y = capi_scaled_mm(a.to(cuda), to_dev_codes(O.prepack_kn(codes), cuda), None, None, torch.float16, cfg)
        assert_gemm_close(y, ref, torch.float16, "inf/nan")
    for m in (80, 16):  # overflow to inf in the fp16 output
        big = torch.full((m, K), 60000.0, dtype=torch.float16)
        y = capi_scaled_mm(big.to(cuda), to_dev_codes(O.prepack_kn(np.full((K, N), 0x3C, np.uint8)), cuda),
                           None, None, torch.float16)
        assert torch.isinf(y).all()


@pytest.mark.parametrize("splitk", ["0", ""])
@pytest.mark.parametrize("cfg", [(2, 4, 4, 8, 4), (2, 4, 4, 4, 6), (2, 4, 4, 8, 3), (1, 1, 2, 1, 2)])
def test_bf16_output_nan_is_canonical(cuda, monkeypatch, cfg, splitk):
    """bf16 outputs: NaN results carry torch's canonical 0x7fc0 (its float -> bfloat16 cast), from a
    NaN activation, from inf - inf in the sum and from a NaN bias; every other element matches the
    oracle; rows without non-finite inputs are unaffected (the epilogue redoes a wave's conversion
    only when that wave produced a NaN)."""
    M, K, N = 256, 128, 384
    g = torch.Generator().manual_seed(3)
    a = torch.randn(M, K, generator=g).half()
    a[3, 5] = float("nan")
    a[70, 9] = float("inf")
    a[70, 10] = float("inf")
    codes = np.full((K, N), 0x3C, np.uint8)
    codes[9, 200] = 0xBC  # +inf * -1 meets +inf * +1 in column 200 of row 70: NaN (+inf elsewhere)
    packed = O.prepack_kn(codes)
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    bias[17] = float("nan")
    bias_np = bias.view(torch.int16).numpy().view(np.uint16)
    ref = O.scaled_mm_ref(a.numpy(), packed, None, bias_np, O.DT_BF16)
    if splitk:  # the tuple's own tile instead of the split-K route this size takes by default
        monkeypatch.setenv("FEATHEROPS_SPLITK", splitk)
    y = capi_scaled_mm(a.to(cuda), to_dev_codes(packed, cuda), None, bias.to(cuda), torch.bfloat16, cfg)
    bits = y.view(torch.int16).cpu().numpy().view(np.uint16)
    nan = (ref & 0x7FFF) > 0x7F80
    assert nan[3].all() and nan[:, 17].all() and nan[70, 200]
    assert np.array_equal((bits & 0x7FFF) > 0x7F80, nan), cfg
    assert (bits[nan] == 0x7FC0).all(), sorted(set(bits[nan].tolist()))[:8]
    assert_gemm_close(y, ref, torch.bfloat16, f"bf16 nan {cfg}")


def test_deterministic(cuda):
    g = torch.Generator().manual_seed(9)
    a = torch.randn(512, 1024, generator=g).half().to(cuda)
    packed, s = weight_like(768, 1024, g)
    bd = to_dev_codes(packed, cuda)
    sd = torch.tensor([s], device=cuda)
    for cfg in [(2, 4, 4, 8, 4), (1, 1, 2, 1, 2)]:
        y1 = capi_scaled_mm(a, bd, sd, None, torch.float16, cfg)
        y2 = capi_scaled_mm(a, bd, sd, None, torch.float16, cfg)
        assert torch.equal(y1, y2)
    # every tile kernel sums K in the same order: bit-identical across tiles
    ys = [capi_scaled_mm(a, bd, sd, None, torch.float16, c) for c in TILE_CFGS]
    for y in ys[1:]:
        assert torch.equal(ys[0], y)


def _sampled_rows_check(cuda, M, N, K, out_dtype, cfg, nrows=24, seed=0):
    """Full-size run; the oracle recomputes a random subset of output rows."""
    g = torch.Generator().manual_seed(seed)
    packed, s = weight_like(N, K, g)
    bias, bias_np = _bias_for(out_dtype, N, g)
    gd = torch.Generator(device=cuda).manual_seed(seed)
    a = torch.randn(M, K, generator=gd, device=cuda).half()
    y = capi_scaled_mm(a, to_dev_codes(packed, cuda), torch.tensor([s], device=cuda), bias.to(cuda),
                       out_dtype, cfg)
    rows = np.sort(np.random.default_rng(seed).choice(M, size=min(nrows, M), replace=False))
    od = O.DT_F16 if out_dtype == torch.float16 else O.DT_BF16
    ref = O.scaled_mm_ref(a[torch.from_numpy(rows).to(cuda)].cpu().numpy(), packed, s, bias_np, od)
    literal = out_dtype == torch.float16  # the north-star gate as written (fp16 outputs)
    assert_gemm_close(y[torch.from_numpy(rows).to(cuda)], ref, out_dtype, f"{M}x{N}x{K}", literal=literal)
    assert torch.isfinite(y).all()
    # the whole output: elementwise against a torch fp32 matmul of the same operands, and row and
    # column checksums against float64 arithmetic
    bd, sd, bsd = to_dev_codes(packed, cuda), torch.tensor([s], device=cuda), bias.to(cuda)
    assert_gemm_close_dev(y, torch_ref_dev(a, bd, sd, bsd, out_dtype), out_dtype, f"full {M}x{N}x{K}",
                          literal=literal)
    assert_row_col_checksums(a, bd, sd, bsd, y, label=f"{M}x{N}x{K}")


def test_baseline_config2_small_m(cuda):
    _sampled_rows_check(cuda, 16, 4096, 4096, torch.float16, (1, 1, 2, 1, 2), nrows=16)


@pytest.mark.parametrize("K,N", [(3072, 12288), (12288, 3072), (3072, 3072)])
def test_baseline_config3_image_dit(cuda, K, N):
    _sampled_rows_check(cuda, 4096, N, K, torch.bfloat16, (2, 4, 4, 8, 4))


@pytest.mark.parametrize("K,N", [(5120, 13824), (13824, 5120), (5120, 5120)])
def test_baseline_config4_video_dit(cuda, K, N):
    _sampled_rows_check(cuda, 32768, N, K, torch.float16, (2, 4, 4, 8, 4), nrows=16)


@pytest.mark.parametrize("M,N,K", [(16, 4096, 4096), (16, 3072, 3072), (1, 1040, 2048), (33, 2000, 4096),
                                   (64, 4096, 4096), (48, 12288, 2048), (16, 128, 128), (16, 5120, 13824),
                                   (1, 3072, 12288), (8, 2048, 12288), (32, 5120, 13824), (7, 2000, 8192)])
def test_small_m_split_k_workspace(cuda, M, N, K):
    """feather_launch_scaled_mm_ws: K split across workgroups through the
    workspace; twice in a row (the arrival counters must come back to zero)."""
    from gpu_util import lib, stream

    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).half()
    packed, s = weight_like(N, K, g)
    bias, bias_np = _bias_for(torch.float16, N, g)
    ref = O.scaled_mm_ref(a.numpy(), packed, s, bias_np, O.DT_F16)
    cfg = (1, 1, 2, 1, 2)
    nbytes = lib().feather_scaled_mm_workspace_size(M, N, K, *cfg)
    ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=cuda)
    ad, bd, sd, bsd = a.to(cuda), to_dev_codes(packed, cuda), torch.tensor([s], device=cuda), bias.to(cuda)
    outs = []
    for _ in range(2):
        c = torch.full((M, N), float("nan"), dtype=torch.float16, device=cuda)
        ok = lib().feather_launch_scaled_mm_ws(ad.data_ptr(), bd.data_ptr(), sd.data_ptr(), bsd.data_ptr(),
                                               c.data_ptr(), M, N, K, 1, 1, *cfg, 1, 0, ws.data_ptr(), ws.numel(),
                                               stream(cuda))
        assert ok
        torch.cuda.synchronize()
        assert_gemm_close(c, ref, torch.float16, f"ws {M}x{N}x{K}")
        outs.append(c)
    assert torch.equal(outs[0], outs[1]), "split-K reduction must be deterministic"
    if nbytes:
        # split across workgroups: the workspace starts with one arrival counter
        # per 64-column tile (LDS split-K path) or per 32- or 64-column strip
        # (small-M kernel); the first (N + 63) // 64 are counters either way
        tiles = (N + 63) // 64
        assert (ws[: tiles * 4] == 0).all(), "arrival counters must be left at zero"


def test_workspace_shared_across_shapes(cuda):
    """One workspace, zeroed once, serves a sequence of K-split calls of
    different shapes: a call with more tiles than the one before must not read
    that call's leftover partials as arrival counters. Small-M kernel and
    split-K LDS tiles, each shape twice, fewer tiles before more."""
    from gpu_util import lib, stream

    seq = [(16, 3072, 12288), (16, 5120, 13824), (8, 2048, 12288), (256, 1024, 2112), (512, 560, 2048),
           (64, 4096, 4096), (48, 6144, 2048), (16, 5120, 13824), (512, 560, 2048)]
    cfg = (2, 2, 4, 4, 4)
    need = max(lib().feather_scaled_mm_workspace_size(M, N, K, *cfg) for M, N, K in seq)
    ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
    for i, (M, N, K) in enumerate(seq):
        g = torch.Generator().manual_seed(i)
        a = torch.randn(M, K, generator=g).half()
        packed, s = weight_like(N, K, g)
        ref = O.scaled_mm_ref(a.numpy(), packed, s, None, O.DT_F16)
        assert lib().feather_scaled_mm_workspace_size(M, N, K, *cfg) > 0, "every shape here splits K"
        ad, bd, sd = a.to(cuda), to_dev_codes(packed, cuda), torch.tensor([s], device=cuda)
        for rep in range(2):
            c = torch.full((M, N), float("nan"), dtype=torch.float16, device=cuda)
            assert lib().feather_launch_scaled_mm_ws(ad.data_ptr(), bd.data_ptr(), sd.data_ptr(), None, c.data_ptr(),
                                                     M, N, K, 1, 0, *cfg, 1, 0, ws.data_ptr(), ws.numel(),
                                                     stream(cuda))
            torch.cuda.synchronize()
            assert_gemm_close(c, ref, torch.float16, f"shared workspace step {i} {M}x{N}x{K} rep {rep}")
        assert (ws[:65536] == 0).all(), "the counter region is left zero"


@pytest.mark.parametrize("M,N,K", [(16, 4096, 1024), (16, 12288, 512), (48, 1024, 2048), (64, 1024, 1024),
                                   (256, 768, 512), (1024, 4096, 1024), (100, 512, 1040), (4096, 4096, 4096),
                                   (4096, 3072, 3072), (1000, 5120, 640), (4608, 3072, 3072), (2048, 2048, 64),
                                   (1024, 1536, 128), (3000, 2304, 320)])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
def test_bf16_activations(cuda, hk, M, N, K, out_dtype):
    """bf16 A through the any-M entry: rounded to fp16 inside the kernel (or cast
    first where the kernel has no bf16 variant) -- bit-identical to passing
    a.to(float16), and within the gate of the oracle on the fp16-rounded A.
    Includes values that overflow fp16 (1e6 -> inf), fp16 subnormals and zeros."""
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).bfloat16()
    a[0, :4] = torch.tensor([3.0e-6, -5.0e-8, 1.0e-9, 0.0]).bfloat16()
    a[M - 1, 3] = 1.0e6 if M > 1 else a[M - 1, 3]
    packed, s = weight_like(N, K, g)
    bias, bias_np = _bias_for(out_dtype, N, g)
    ad = a.to(cuda)
    bd = to_dev_codes(packed, cuda).view(torch.float8_e5m2)
    sd = torch.tensor(s, device=cuda)
    y = hk.scaled_mm_hip_any_m(ad, bd, sd, bias.to(cuda), out_dtype)
    y16 = hk.scaled_mm_hip_any_m(ad.to(torch.float16), bd, sd, bias.to(cuda), out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y16.view(torch.int16)), "bf16 A must equal the fp16 cast of A"
    od = O.DT_F16 if out_dtype == torch.float16 else O.DT_BF16
    ref = O.scaled_mm_ref(a.to(torch.float16).numpy(), packed, s, bias_np, od)
    assert_gemm_close(y, ref, out_dtype, f"bf16 A {M}x{N}x{K}")


def test_validation_fast_path_matches_full(cuda, hk):
    """The one-expression fast path of validate_scaled_mm accepts valid CUDA
    arguments and rejects every argument the full checks reject (which then
    raise the reference's message)."""
    M, N, K = 64, 128, 256

    def good():
        return dict(a=torch.empty(M, K, dtype=torch.float16, device=cuda),
                    b=torch.empty(K // 16, N, 16, dtype=torch.float8_e5m2, device=cuda),
                    scale=torch.ones((), dtype=torch.float32, device=cuda),
                    bias=torch.zeros(N, dtype=torch.float16, device=cuda),
                    c=torch.empty(M, N, dtype=torch.float16, device=cuda), cfg=(1, 1, 2, 1, 2), b_dtype=1)

    def fast(x, **kw):
        return hk._valid_fast(x["a"], x["b"], x["scale"], x["bias"], x["c"], *x["cfg"], x["b_dtype"],
                              kw.get("block_divisible", True), kw.get("allow_bf16_a", False))

    x = good()
    assert fast(x)
    misaligned = torch.empty(M * K + 1, dtype=torch.float16, device=cuda)[1:].view(M, K)
    mutations = [
        (dict(a=x["a"].float()), "a must be float16"),
        (dict(a=x["a"].bfloat16()), "a must be float16"),
        (dict(c=x["c"].float()), "c must be float16 or bfloat16"),
        (dict(b=x["b"].view(torch.uint8)), "b_prepacked must be float8_e5m2"),
        (dict(b_dtype=0), "b_prepacked must be float8_e4m3fn"),
        (dict(a=x["a"][:, :128]), r"b_prepacked.shape\[0\] must equal K/16"),
        (dict(c=torch.empty(32, N, dtype=torch.float16, device=cuda)), r"c.shape\[0\] must equal M"),
        (dict(a=torch.empty(K, M, dtype=torch.float16, device=cuda).t()), r"a.stride\(0\) must equal K"),
        (dict(c=torch.empty(N, M, dtype=torch.float16, device=cuda).t()), r"c.stride\(0\) must equal N"),
        (dict(scale=torch.ones(2, device=cuda)), "scale must have one element"),
        (dict(scale=torch.ones((), dtype=torch.float16, device=cuda)), "scale must be float32"),
        (dict(scale=torch.ones((), dtype=torch.float32)), "scale must be a CUDA tensor"),
        (dict(bias=torch.zeros(N, dtype=torch.bfloat16, device=cuda)), "bias must have the same dtype as c"),
        (dict(bias=torch.zeros(64, dtype=torch.float16, device=cuda)), "bias must have N elements"),
        (dict(a=misaligned), "a data pointer must be 16-byte aligned"),
        (dict(cfg=(1, 1, 2, 8, 2)), r"M \(64\) must be divisible by kBlockM \(128\)"),
        (dict(cfg=(1, 8, 4, 1, 2)), r"N \(128\) must be divisible by kBlockN \(256\)"),
    ]
    for change, msg in mutations:
        y = good()
        y.update(change)
        assert not fast(y), msg
        with pytest.raises(RuntimeError, match=msg):
            hk.validate_scaled_mm(y["a"], y["b"], y["scale"], y["bias"], y["c"], *y["cfg"], y["b_dtype"])
        # the C++ op (csrc/torch_op.cpp) raises the same message before launching anything
        with pytest.raises(RuntimeError, match=msg):
            torch.ops.feather_ops.scaled_mm.default(y["a"], y["b"], y["scale"], y["bias"], y["c"], *y["cfg"],
                                                    y["b_dtype"])
    # the any-M entry's relaxed rules: no block divisibility, bf16 activations
    y = good()
    y.update(cfg=(1, 1, 2, 8, 2), a=x["a"].bfloat16())
    assert fast(y, block_divisible=False, allow_bf16_a=True)
    assert not fast(y, block_divisible=True, allow_bf16_a=True)
    assert not fast(y, block_divisible=False, allow_bf16_a=False)


def test_size_one_dims_any_stride(cuda, hk):
    """A dimension of size 1 may carry any stride (torch leaves it arbitrary,
    e.g. after .contiguous() of a permuted (1, N, 16) weight): M = 1
    activations/outputs and K = 16 weights with odd size-1 strides run and
    match the oracle."""
    g = torch.Generator().manual_seed(21)
    M, N, K = 1, 96, 16
    a = torch.randn(M, K, generator=g).half()
    packed, s = weight_like(N, K, g)
    ref = O.scaled_mm_ref(a.numpy(), packed, s, None, O.DT_F16)
    ad = a.to(cuda).as_strided((M, K), (999, 1))
    bd = to_dev_codes(packed, cuda).as_strided((1, N, 16), (7, 16, 1))
    assert ad.stride(0) != K and bd.stride(0) != N * 16
    y = hk.scaled_mm_hip_any_m(ad, bd, torch.tensor(s, device=cuda), None, torch.float16)
    torch.cuda.synchronize()
    assert_gemm_close(y, ref, torch.float16, "size-1 strides any_m")
    # the op's validation also accepts an M = 1 output with any row stride
    c = torch.empty((1, N), dtype=torch.float16, device=cuda).as_strided((1, N), (5, 1))
    hk.validate_scaled_mm(ad, bd, torch.tensor(s, device=cuda), None, c, 1, 1, 1, 1, 2, 1, block_divisible=False)


@pytest.mark.parametrize("b_dtype", [torch.float8_e5m2, torch.float8_e4m3fn])
@pytest.mark.parametrize("route", ["small_m", "tile", "lds", "split_k"])
def test_every_fp8_code_decodes_exactly(cuda, b_dtype, route):
    """All 256 weight codes through each kernel family: column n of B holds
    code n in its first K row and zeros below, A's rows are e_0, so C[:, n]
    is exactly the decoded code (NaN codes NaN, e5m2 infinities inf; -0
    comes out as +0 because the accumulator starts at +0)."""
    import os

    M, K, splitk = {"small_m": (16, 16, None), "tile": (256, 16, "0"), "lds": (256, 64, "0"),
                    "split_k": (256, 64, "1")}[route]
    cfg = (1, 1, 2, 1, 2) if route == "small_m" else (2, 4, 4, 8, 4) if route == "lds" else (2, 2, 2, 4, 4)
    N = 256
    codes = torch.zeros(K, N, dtype=torch.uint8)
    codes[0] = torch.arange(256, dtype=torch.uint8)
    bp = codes.view(K // 16, 16, N).permute(0, 2, 1).contiguous().to(cuda)
    a = torch.zeros(M, K, dtype=torch.float16)
    a[:, 0] = 1.0
    a = a.to(cuda)
    c = torch.full((M, N), 7.0, dtype=torch.float16, device=cuda)
    L = lib()
    b_code = 0 if b_dtype == torch.float8_e4m3fn else 1
    old = os.environ.get("FEATHEROPS_SPLITK")
    try:
        if splitk is not None:
            os.environ["FEATHEROPS_SPLITK"] = splitk
        kid = L.feather_scaled_mm_kernel_id(M, N, K, *cfg)
        want_kid = {"small_m": (10, 10), "tile": (1, 9), "lds": (20, 29), "split_k": (30, 39)}[route]
        assert want_kid[0] <= kid <= want_kid[1], f"{route}: kernel id {kid}"
        ws_bytes = L.feather_scaled_mm_workspace_size(M, N, K, *cfg)
        ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=cuda)
        ok = L.feather_launch_scaled_mm_ws(a.data_ptr(), bp.data_ptr(), None, None, c.data_ptr(), M, N, K, 0, 0, *cfg,
                                           b_code, 0, ws.data_ptr(), ws.numel(), stream(cuda))
        torch.cuda.synchronize()
    finally:
        if old is None:
            os.environ.pop("FEATHEROPS_SPLITK", None)
        else:
            os.environ["FEATHEROPS_SPLITK"] = old
    assert ok
    dec = O.e4m3fn_decode(np.arange(256)) if b_code == 0 else O.e5m2_decode(np.arange(256, dtype=np.uint8))
    want = torch.from_numpy(dec.astype(np.float32)).to(torch.float16).expand(M, N)
    got = c.cpu()
    assert torch.equal(torch.isnan(got), torch.isnan(want)), route
    fin = ~torch.isnan(want)
    assert torch.equal(got[fin], want[fin]), route


def test_baseline_config1_gemm(cuda, hk, quant):
    """The C1 workload (the reference's CPU-runnable case) end to end: A (256,1024) ~N(0,1) fp16, W (1024,1024) ~N(0,0.02) in fp16
    quantized on the load path (its bytes and scale equal the golden fixture), fp16 out with a
    bias; the GEMM through the C ABI on every config tuple that takes M=256, through the
    reference's torch op and through the drop-in Python entries, each against the oracle over
    the whole output."""
    z = np.load(GOLDEN / "quant_c1.npz")
    g = torch.Generator().manual_seed(0)
    w32 = torch.randn(1024, 1024, generator=g) * 0.02  # the golden fixture's weight
    a = torch.randn(256, 1024, generator=g).half()
    bias = (torch.randn(1024, generator=g) * 0.01).half()
    qt = quant.make_feather_quantized_weight(w32.half().to(cuda), None, torch.float16)
    bp, sd = quant.get_feather_plain_tensors(qt)
    assert np.float32(sd.item()) == z["load_f16_scale"][0]
    import hashlib

    packed = bp.view(torch.uint8).cpu().numpy()
    assert hashlib.sha256(packed.tobytes()).digest() == z["load_f16_sha256"].tobytes()
    ad, bsd = a.to(cuda), bias.to(cuda)
    sd = sd.reshape(1).contiguous()
    ref = O.scaled_mm_ref(a.numpy(), packed, np.float32(sd.item()), bias.numpy(), O.DT_F16)
    ran = 0
    for cfg in hk._CONFIGS:
        wm, wn, u, rm, rn = cfg
        if 256 % (16 * wm * rm) or 1024 % (16 * wn * rn) or 1024 % (16 * u):
            continue
        print("C1 cfg", cfg, flush=True)
        y = capi_scaled_mm(ad, bp, sd, bsd, torch.float16, cfg)
        assert_gemm_close(y, ref, torch.float16, f"C1 capi {cfg}", literal=True)
        ran += 1
    assert ran >= 20
    c = torch.empty(256, 1024, dtype=torch.float16, device=cuda)
    torch.ops.feather_ops.scaled_mm(ad, bp, sd, bsd, c, 2, 4, 4, 8, 4, 1)
    torch.cuda.synchronize()
    assert_gemm_close(c, ref, torch.float16, "C1 torch op", literal=True)
    y = hk.scaled_mm_hip(ad, bp, sd, bsd, torch.float16)
    assert_gemm_close(y, ref, torch.float16, "C1 scaled_mm_hip", literal=True)
    y = hk.scaled_mm_hip_any_m(ad, bp, sd, bsd, torch.float16)
    assert_gemm_close(y, ref, torch.float16, "C1 any-M", literal=True)
    # the route the C1 workload takes by default (the 64x64 split-K-route tiles, unsplit at K=1024) is deterministic
    assert torch.equal(y, hk.scaled_mm_hip_any_m(ad, bp, sd, bsd, torch.float16))


@pytest.mark.parametrize("M,N,K,out_dtype", [(4100, 4112, 1024, torch.float16), (2304, 9232, 512, torch.bfloat16),
                                             (8192, 2064, 256, torch.float16)])
def test_multi_wave_grids_ragged(cuda, M, N, K, out_dtype):
    """Grids with more output tiles than CUs and ragged edges, through the reference ABI and
    the workspace entry: every tile config gives the same bits (all sum K in the same order),
    and the whole output matches a float64 evaluation and the checksums."""
    g = torch.Generator().manual_seed(M + N)
    packed, s = weight_like(N, K, g)
    bias, _ = _bias_for(out_dtype, N, g)
    gd = torch.Generator(device=cuda).manual_seed(M)
    a = torch.randn(M, K, generator=gd, device=cuda).half()
    bd, sd, bsd = to_dev_codes(packed, cuda), torch.tensor([s], device=cuda), bias.to(cuda)
    ref = torch_ref_dev(a, bd, sd, bsd, out_dtype)
    first = None
    L = lib()
    for cfg in [(2, 4, 4, 8, 4), (4, 2, 4, 4, 8), (2, 4, 4, 8, 3), (2, 4, 4, 4, 6), (2, 4, 4, 4, 4), (4, 2, 4, 4, 4),
                (2, 2, 4, 4, 4)]:
        print("multi-wave", M, N, K, cfg, "kernel", L.feather_scaled_mm_kernel_id(M, N, K, *cfg), flush=True)
        y = capi_scaled_mm(a, bd, sd, bsd, out_dtype, cfg)
        assert_gemm_close_dev(y, ref, out_dtype, f"{M}x{N}x{K} {cfg}")
        if first is None:
            first = y
            assert_row_col_checksums(a, bd, sd, bsd, y, label=f"{M}x{N}x{K}")
        else:
            assert torch.equal(y.view(torch.int16), first.view(torch.int16)), f"{cfg} differs from the first config"
        nbytes = L.feather_scaled_mm_workspace_size(M, N, K, *cfg)
        ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=cuda)
        y2 = torch.full((M, N), float("nan"), dtype=out_dtype, device=cuda)
        assert L.feather_launch_scaled_mm_ws(a.data_ptr(), bd.data_ptr(), sd.data_ptr(), bsd.data_ptr(), y2.data_ptr(),
                                             M, N, K, 1, 1, *cfg, 1, 0 if out_dtype == torch.float16 else 1,
                                             ws.data_ptr(), nbytes, stream(cuda))
        torch.cuda.synchronize()
        assert torch.equal(y2.view(torch.int16), first.view(torch.int16)), f"{cfg} workspace entry differs"


def _lean_call(ad, bd, sd, bsd, M, N, K, a_bf16, b_e4m3, out_dtype, has_scale=1, has_bias=1):
    c = torch.full((M, N), float("nan"), dtype=out_dtype, device=ad.device)
    ok = lib().feather_launch_scaled_mm_ex(ad.data_ptr(), int(a_bf16), bd.data_ptr(),
                                           sd.data_ptr() if has_scale else None,
                                           bsd.data_ptr() if has_bias else None, c.data_ptr(), M, N, K, has_scale,
                                           has_bias, 1, 1, 2, 1, 2, 0 if b_e4m3 else 1,
                                           0 if out_dtype == torch.float16 else 1, None, 0, stream(ad.device))
    assert ok
    torch.cuda.synchronize()
    return c


@pytest.mark.parametrize("M", [1, 3, 8, 9, 16, 17, 24, 31, 32])
@pytest.mark.parametrize("variant", ["f16_e5m2_f16", "f16_e4m3_bf16", "bf16_e5m2_f16", "bf16_e5m2_bf16",
                                     "noscale_nobias"])
def test_small_m_lean_route(cuda, M, variant):
    """M <= 32 with K % 64 == 0 and one K range per 16-column strip runs the lean small-M
    kernel (one or two 16-row tiles), which copies only the A rows below M into LDS: rows >= M
    of its LDS slabs hold whatever the previous workgroup on that CU left there. A call with
    M = 16 or 32 and an all-NaN A runs first on the same shape, so every slab row past M holds
    NaN bits when the M-row call runs; its output must still equal the oracle (an output row
    reads only its own A row) and carry no NaN."""
    N, K = 4096, 2048
    a_bf16 = variant.startswith("bf16")
    b_e4m3 = "e4m3" in variant
    out_dtype = torch.bfloat16 if variant.endswith("bf16") else torch.float16
    has_scale = has_bias = 0 if variant == "noscale_nobias" else 1
    g = torch.Generator().manual_seed(1000 + M)
    a = torch.randn(M, K, generator=g)
    if not has_scale:
        a = a * 1e-3  # unscaled codes reach 57344: keep |C| far below fp16's range
    a_t = a.bfloat16() if a_bf16 else a.half()
    if b_e4m3:
        w = torch.randn(N, K, generator=g) * 0.02
        s = np.float32(w.abs().max().item()) / np.float32(448.0)
        codes = (w * float(np.float32(1.0) / s)).to(torch.float8_e4m3fn).view(torch.uint8)
        packed = codes.view(N, K // 16, 16).permute(1, 0, 2).contiguous().numpy()
        bd = to_dev_codes(packed, cuda, torch.float8_e4m3fn)
    else:
        packed, s = weight_like(N, K, g)
        bd = to_dev_codes(packed, cuda)
    bias, bias_np = _bias_for(out_dtype, N, g)
    sd = torch.tensor([s], device=cuda)
    bsd = bias.to(cuda)
    # fill the LDS slabs with NaN rows: an M = 16 call on an all-NaN A of the same dtype
    Mp = 16 if M <= 16 else 32
    poison = torch.full((Mp, K), float("nan"), dtype=a_t.dtype, device=cuda)
    yp = _lean_call(poison, bd, sd, bsd, Mp, N, K, a_bf16, b_e4m3, out_dtype)
    assert torch.isnan(yp).all()
    y = _lean_call(a_t.to(cuda), bd, sd, bsd, M, N, K, a_bf16, b_e4m3, out_dtype, has_scale, has_bias)
    od = O.DT_F16 if out_dtype == torch.float16 else O.DT_BF16
    ref = O.scaled_mm_ref(a_t.to(torch.float16).numpy(), packed, s if has_scale else None,
                          bias_np if has_bias else None, od, "e4m3fn" if b_e4m3 else "e5m2")
    assert_gemm_close(y, ref, out_dtype, f"lean {variant} M={M}")


@pytest.mark.parametrize("M", [5, 16, 20, 32])
@pytest.mark.parametrize("N,K", [(1040, 64), (2048, 1088), (1024, 4160), (4096, 64 * 129)])
def test_small_m_lean_stage_counts(cuda, M, N, K):
    """The lean small-M kernel over stage counts that do not fill its rounds (one 64-K stage; 17,
    65 and 129 stages against 16 waves x 4 or 2 stages per round) and N a multiple of 16 only:
    whole output against the oracle, through the workspace entry (same route as the torch op)."""
    g = torch.Generator().manual_seed(M * 7 + N + K)
    a = torch.randn(M, K, generator=g).half()
    packed, s = weight_like(N, K, g)
    bias, bias_np = _bias_for(torch.float16, N, g)
    cfg = (1, 1, 2, 1, 2)
    nbytes = lib().feather_scaled_mm_workspace_size(M, N, K, *cfg)
    ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=cuda)
    ad, bd, sd, bsd = a.to(cuda), to_dev_codes(packed, cuda), torch.tensor([s], device=cuda), bias.to(cuda)
    c = torch.full((M, N), float("nan"), dtype=torch.float16, device=cuda)
    print("lean stages", M, N, K, flush=True)
    assert lib().feather_launch_scaled_mm_ws(ad.data_ptr(), bd.data_ptr(), sd.data_ptr(), bsd.data_ptr(),
                                             c.data_ptr(), M, N, K, 1, 1, *cfg, 1, 0, ws.data_ptr(), ws.numel(),
                                             stream(cuda))
    torch.cuda.synchronize()
    ref = O.scaled_mm_ref(a.numpy(), packed, s, bias_np, O.DT_F16)
    assert_gemm_close(c, ref, torch.float16, f"lean {M}x{N}x{K}")



LARGE_TILE_CFGS = [(2, 4, 4, 8, 4), (4, 2, 4, 4, 8), (4, 2, 4, 4, 4), (2, 4, 4, 8, 3), (2, 4, 4, 4, 6), (2, 4, 4, 4, 4),
                   (2, 2, 4, 4, 4)]


@pytest.mark.parametrize("K", [64, 128, 192, 256, 320, 1088])
@pytest.mark.parametrize("b_dtype", [torch.float8_e5m2, torch.float8_e4m3fn])
def test_large_tiles_every_stage_count(cuda, monkeypatch, K, b_dtype):
    """Every large LDS tile from one 64-K stage up: the first stage, the steady three-stage
    loop and its 1-, 2- and 3-stage tails take different code, and on e5m2 weights the
    widening and MFMAs there are ordered by hand (each K half's first two weight columns
    widened during the previous half's last repeat, none after the last stage). All configs
    must give the same bits (the K order of every sum is the same), M and N not multiples of
    the tiles, and match a float64 evaluation of the whole output."""
    monkeypatch.setenv("FEATHEROPS_SPLITK", "0")  # this grid would otherwise take the split-K tiles
    M, N = 777, 1152
    g = torch.Generator().manual_seed(K)
    a = torch.randn(M, K, generator=g).half().to(cuda)
    fmax = 448.0 if b_dtype == torch.float8_e4m3fn else 57344.0
    w = torch.randn(N, K, generator=g) * 0.02
    s = (w.abs().max() / fmax).float().reshape(1)
    bp = (w / s).to(b_dtype).view(N, K // 16, 16).permute(1, 0, 2).contiguous().to(cuda)
    sd = s.to(cuda)
    bias = (torch.randn(N, generator=g) * 0.1).half().to(cuda)
    ref = torch_ref_dev(a, bp, sd, bias, torch.float16, b_dtype=b_dtype)
    first = None
    for cfg in LARGE_TILE_CFGS:
        kid = lib().feather_scaled_mm_kernel_id(M, N, K, *cfg)
        print("large tile", M, N, K, cfg, "kernel", kid, b_dtype, flush=True)
        assert 20 <= kid <= 26, f"{cfg} maps to kernel {kid}, not a large LDS tile"
        y = capi_scaled_mm(a, bp.view(torch.uint8), sd, bias, torch.float16, cfg,
                           b_dtype=0 if b_dtype == torch.float8_e4m3fn else 1)
        assert_gemm_close_dev(y, ref, torch.float16, f"{cfg} K={K}")
        if first is None:
            first = y
        else:
            assert torch.equal(y.view(torch.int16), first.view(torch.int16)), f"{cfg} K={K} differs from {LARGE_TILE_CFGS[0]}"


# (M, N, K, kernel id, K splits, stage ring depth): every split-K tile width with both ring depths,
# the ring deeper than a split's stage count (its copies past the end repeat the last stage),
# ragged M and N
SPLITK_RING_CASES = [
    (64, 13824, 5120, 30, 1, 6),
    (40, 1008, 2048, 30, 16, 5),     # two stages per split, ring of five
    (1000, 1008, 1024, 30, 1, 5),
    (512, 3008, 12288, 31, 1, 6),
    (100, 5120, 5120, 31, 3, 5),
    (24, 5008, 5120, 34, 6, 5),
    (32, 13824, 8192, 34, 2, 6),
    (17, 528, 8192, 34, 32, 5),      # four stages per split
]


@pytest.mark.parametrize("M,N,K,kid,ks,stages", SPLITK_RING_CASES)
@pytest.mark.parametrize("b_dtype,out_dtype", [(torch.float8_e5m2, torch.float16), (torch.float8_e4m3fn, torch.bfloat16)])
def test_split_k_tiles_every_width_and_ring(cuda, monkeypatch, M, N, K, kid, ks, stages, b_dtype, out_dtype):
    """The split-K LDS tiles (64 x 64, 64 x 128, 32 x 128) on five- and six-stage copy rings,
    through the workspace entry, against a float64 evaluation of the whole output, twice in a
    row (deterministic, counters back at zero). The kernel id and the split count (read back
    from the workspace size) are the plan's; the ring depth follows from them (six from 64 K
    stages per split)."""
    from gpu_util import stream

    monkeypatch.setenv("FEATHEROPS_SPLITK", "1")
    cfg = (2, 2, 4, 4, 4)
    assert lib().feather_scaled_mm_kernel_id(M, N, K, *cfg) == kid
    bm, bn = {30: (64, 64), 31: (64, 128), 34: (32, 128)}[kid]
    tiles = (M + bm - 1) // bm * ((N + bn - 1) // bn)
    nbytes = lib().feather_scaled_mm_workspace_size(M, N, K, *cfg)
    assert nbytes == (0 if ks == 1 else 65536 + tiles * ks * bm * bn * 4)
    per = (K // 64 + ks - 1) // ks
    assert (6 if (K // 64) // ks >= 64 else 5) == stages and per >= 1
    print("split-K tile", M, N, K, "kernel", kid, "splits", ks, "stages", stages, b_dtype, out_dtype, flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    a = torch.randn(M, K, generator=g).half().to(cuda)
    fmax = 448.0 if b_dtype == torch.float8_e4m3fn else 57344.0
    w = torch.randn(N, K, generator=g) * 0.02
    s = (w.abs().max() / fmax).float().reshape(1)
    bp = (w / s).to(b_dtype).view(N, K // 16, 16).permute(1, 0, 2).contiguous().to(cuda)
    del w
    sd = s.to(cuda)
    bias = (torch.randn(N, generator=g) * 0.1).to(out_dtype).to(cuda)
    ref = torch_ref_dev(a, bp, sd, bias, out_dtype, b_dtype=b_dtype)
    ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=cuda)
    outs = []
    for _ in range(2):
        c = torch.full((M, N), float("nan"), dtype=out_dtype, device=cuda)
        assert lib().feather_launch_scaled_mm_ws(a.data_ptr(), bp.data_ptr(), sd.data_ptr(), bias.data_ptr(),
                                                 c.data_ptr(), M, N, K, 1, 1, *cfg,
                                                 0 if b_dtype == torch.float8_e4m3fn else 1,
                                                 0 if out_dtype == torch.float16 else 1, ws.data_ptr(), ws.numel(),
                                                 stream(cuda))
        torch.cuda.synchronize()
        assert_gemm_close_dev(c, ref, out_dtype, f"split-K {M}x{N}x{K} kernel {kid}")
        outs.append(c)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), "split-K reduction must be deterministic"
    assert (ws[:65536] == 0).all(), "arrival counters must be left at zero"
