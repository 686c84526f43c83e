"""Seeded random parity sweep over shapes, output dtypes, bias/scale presence,
bf16 activations, every config and both fp8 weight formats, against the
oracle (the reference kernel contract, hip_kernel.cu:366-419). Calls of
different shapes run back to back through the torch ops, so the K-split
workspace they share is exercised across shape changes (a regression guard
for counters that once overlapped an earlier call's partials)."""

import numpy as np
import pytest
import torch

from gpu_util import assert_gemm_close, to_dev_codes, weight_like
from oracle import feather_oracle as O

pytestmark = pytest.mark.gpu

M_CHOICES = [1, 2, 7, 15, 16, 17, 31, 32, 33, 47, 48, 63, 64, 65, 100, 129, 255, 256, 300]


def _bias_np(bias, out):
    return bias.view(torch.int16).numpy().view(np.uint16) if out == torch.bfloat16 else bias.numpy()


@pytest.mark.parametrize("seed", [0, 1])
def test_random_any_m(cuda, hk, seed):
    rng = np.random.default_rng(seed)
    for case in range(30):
        M = int(rng.choice(M_CHOICES))
        N = 16 * int(rng.integers(1, 48))
        K = 16 * int(rng.integers(1, 96))
        out = torch.float16 if rng.random() < 0.5 else torch.bfloat16
        a_bf16 = rng.random() < 0.3
        has_s, has_b = rng.random() < 0.8, rng.random() < 0.6
        g = torch.Generator().manual_seed(1000 * seed + case)
        a = torch.randn(M, K, generator=g).half()
        if has_s:
            packed, s = weight_like(N, K, g)
        else:  # unscaled codes of a ~N(0, 0.5) weight
            w8 = (torch.randn(N, K, generator=g) * 0.5).to(torch.float8_e5m2).view(torch.uint8)
            packed, s = w8.view(N, K // 16, 16).permute(1, 0, 2).contiguous().numpy(), None
        bias = (torch.randn(N, generator=g) * 0.5).to(out)
        x = a.bfloat16() if a_bf16 else a
        # bf16 activations: the reference Linear casts them to fp16 first (ops.py:88)
        ref = O.scaled_mm_ref(x.half().numpy(), packed, s, _bias_np(bias, out) if has_b else None,
                              O.DT_F16 if out == torch.float16 else O.DT_BF16)
        y = hk.scaled_mm_hip_any_m(x.to(cuda), to_dev_codes(packed, cuda),
                                   torch.tensor(s, device=cuda) if has_s else None,
                                   bias.to(cuda) if has_b else None, out)
        torch.cuda.synchronize()
        assert_gemm_close(y, ref, out, f"seed {seed} case {case}: M={M} N={N} K={K} {out} bf16a={a_bf16}")


@pytest.mark.parametrize("seed", [0, 1])
def test_random_configured(cuda, hk, seed):
    rng = np.random.default_rng(100 + seed)
    for case in range(25):
        cfg = hk._CONFIGS[int(rng.integers(0, len(hk._CONFIGS)))]
        wm, wn, u, rm, rn = cfg
        bm, bn, ck = 16 * wm * rm, 16 * wn * rn, 16 * u
        M = bm * int(rng.integers(1, max(2, 512 // bm + 1)))
        N = bn * int(rng.integers(1, max(2, 768 // bn + 1)))
        K = ck * int(rng.integers(1, max(2, 1024 // ck + 1)))
        out = torch.float16 if rng.random() < 0.5 else torch.bfloat16
        e4 = rng.random() < 0.3
        has_s, has_b = rng.random() < 0.8, rng.random() < 0.6
        g = torch.Generator().manual_seed(5000 + 1000 * seed + case)
        a = torch.randn(M, K, generator=g).half()
        wdt = torch.float8_e4m3fn if e4 else torch.float8_e5m2
        codes = (torch.randn(N, K, generator=g) * 0.5).to(wdt).view(torch.uint8)
        packed = codes.view(N, K // 16, 16).permute(1, 0, 2).contiguous().numpy()
        s = np.float32(0.37)
        bias = (torch.randn(N, generator=g) * 0.5).to(out)
        ref = O.scaled_mm_ref(a.numpy(), packed, s if has_s else None, _bias_np(bias, out) if has_b else None,
                              O.DT_F16 if out == torch.float16 else O.DT_BF16, "e4m3fn" if e4 else "e5m2")
        y = hk.scaled_mm_hip_configured(a.to(cuda), to_dev_codes(packed, cuda, wdt),
                                        torch.tensor(s, device=cuda) if has_s else None,
                                        bias.to(cuda) if has_b else None, out, *cfg)
        torch.cuda.synchronize()
        assert_gemm_close(y, ref, out, f"seed {seed} case {case}: cfg={cfg} M={M} N={N} K={K} {out} e4m3={e4}")


@pytest.mark.parametrize("seed", [0, 1])
def test_random_any_m_lora(cuda, hk, seed):
    """scaled_mm_hip_any_m_lora over random shapes (fused LDS-tile route and
    the fallback routes), ranks, factor and output dtypes: the fused route
    against the oracle's lora= contract (term added before the output
    rounding), the others against the GEMM output plus the term rounded to the
    output type."""
    rng = np.random.default_rng(200 + seed)
    for case in range(16):
        M = int(rng.choice([17, 64, 300, 1024, 2048]))
        N = int(rng.choice([256, 768, 2048, 3072]))
        K = int(rng.choice([256, 512, 1040]))
        R = 32 * int(rng.integers(1, 5))
        out = torch.float16 if rng.random() < 0.5 else torch.bfloat16
        fdt = torch.float16 if rng.random() < 0.5 else torch.bfloat16
        g = torch.Generator().manual_seed(3000 * seed + case)
        a = torch.randn(M, K, generator=g).half()
        packed, s = weight_like(N, K, g)
        bias = (torch.randn(N, generator=g) * 0.5).to(out)
        t = (torch.randn(M, R, generator=g) * 0.2).to(fdt)
        u = (torch.randn(N, R, generator=g) * 0.05).to(fdt)
        y = hk.scaled_mm_hip_any_m_lora(a.to(cuda), to_dev_codes(packed, cuda), torch.tensor(s, device=cuda),
                                        bias.to(cuda), out, t.to(cuda), u.to(cuda))
        torch.cuda.synchronize()
        od = O.DT_F16 if out == torch.float16 else O.DT_BF16
        kid = hk.kernel_id(M, N, K, hk.any_m_config(M, N, K))
        label = f"seed {seed} case {case}: M={M} N={N} K={K} R={R} {out} {fdt} kid={kid}"
        if 20 <= kid < 30:
            ref = O.scaled_mm_ref(a.numpy(), packed, s, _bias_np(bias, out), od,
                                  lora=(t.double().numpy(), u.double().numpy()))
        else:
            base = O.scaled_mm_ref(a.numpy(), packed, s, _bias_np(bias, out), od)
            base = torch.from_numpy(O.bf16_bits_to_f32(base) if base.dtype == np.uint16 else base.astype(np.float32))
            yr = base.to(out) + torch.mm(t, u.t()).to(out)
            ref = yr.numpy() if out == torch.float16 else yr.view(torch.int16).numpy().view(np.uint16)
        assert_gemm_close(y, ref, out, label)


@pytest.mark.parametrize("seed", [0, 1])
def test_random_lora_down(cuda, hk, seed):
    """The LoRA down-projection over random row counts, K and ranks (K split across workgroups
    or not, rank chunks of 128 plus a remainder), both dtypes, back to back on one stream
    through the torch op (one shared workspace), against the oracle's lora_down_ref."""
    rng = np.random.default_rng(200 + seed)
    for case in range(24):
        M = int(rng.choice([1, 5, 64, 65, 300, 1000, 2048, 4100, 9000]))
        K = 8 * int(rng.integers(1, 700))
        R = 32 * int(rng.integers(1, 9))
        dt = torch.float16 if rng.random() < 0.5 else torch.bfloat16
        g = torch.Generator().manual_seed(5000 * seed + case)
        x = torch.randn(M, K, generator=g).to(dt)
        d = (torch.randn(R, K, generator=g) * 0.05).to(dt)
        t = torch.ops.feather_ops.lora_down.default(x.to(cuda), d.to(cuda))
        torch.cuda.synchronize()
        if dt == torch.float16:
            ref = O.lora_down_ref(x.numpy(), d.numpy(), O.DT_F16)
        else:
            ref = O.lora_down_ref(x.view(torch.int16).numpy().view(np.uint16),
                                  d.view(torch.int16).numpy().view(np.uint16), O.DT_BF16)
        assert_gemm_close(t, ref, dt, f"seed {seed} case {case}: M={M} K={K} R={R} {dt}")


def test_random_large_shapes(cuda, hk):
    """Seeded shapes of the size the large tiles serve (M 1000-6000, N often a multiple of 384 so the
    128x384 pick appears, ragged M and N), fp16 and bf16 outputs, bias on or off, an occasional NaN
    activation or bias entry: the any-M op over the whole output against a float64 evaluation on
    the device, canonical bf16 NaNs, and the 128x384 tile through the C ABI where its blocks divide."""
    from gpu_util import assert_gemm_close_dev, capi_scaled_mm, torch_ref_dev

    rng = np.random.default_rng(42)
    gd = torch.Generator(device=cuda).manual_seed(42)
    for case in range(12):
        M = int(rng.integers(1000, 6000))
        N = 384 * int(rng.integers(1, 12)) if rng.random() < 0.5 else 16 * int(rng.integers(20, 700))
        K = 64 * int(rng.integers(1, 60)) if rng.random() < 0.8 else 16 * int(rng.integers(10, 300))
        out = torch.bfloat16 if rng.random() < 0.5 else torch.float16
        has_b = rng.random() < 0.7
        a = torch.randn(M, K, generator=gd, device=cuda).half()
        w = torch.randn(N, K, generator=gd, device=cuda) * 0.02
        s = (w.abs().max() / 57344.0).float().reshape(1)
        bp = (w / s).to(torch.float8_e5m2).view(N, K // 16, 16).permute(1, 0, 2).contiguous()
        bias = (torch.randn(N, generator=gd, device=cuda) * 0.1).to(out) if has_b else None
        if rng.random() < 0.3:
            a[int(rng.integers(0, M)), int(rng.integers(0, K))] = float("nan")
        if has_b and rng.random() < 0.3:
            bias[int(rng.integers(0, N))] = float("nan")
        cfg = hk.any_m_config(M, N, K)
        print("large", case, M, N, K, out, has_b, cfg, flush=True)
        ref = torch_ref_dev(a, bp, s, bias, out)
        y = hk.scaled_mm_hip_any_m(a, bp, s, bias, out)
        assert_gemm_close_dev(y, ref, out, f"large {case} {cfg}")
        if out == torch.bfloat16:
            assert bool((y.view(torch.int16)[torch.isnan(y)] == 0x7FC0).all()), "non-canonical bf16 NaN"
        if M % 128 == 0 and N % 384 == 0 and K % 64 == 0:
            assert_gemm_close_dev(capi_scaled_mm(a, bp, s, bias, out, (2, 4, 4, 4, 6)), ref, out, f"128x384 {case}")
        del ref, y



def test_random_large_shapes_e4m3_bf16_activations(cuda, hk):
    """The large-shape sweep with e4m3fn weights and bf16 activations mixed in: the any-M op
    (bf16 activations are rounded to fp16 by the library's cast, as ops.py:88's x.to(float16))
    over the whole output against a float64 evaluation of the same fp16 activations."""
    from gpu_util import assert_gemm_close_dev, torch_ref_dev

    rng = np.random.default_rng(7)
    gd = torch.Generator(device=cuda).manual_seed(7)
    for case in range(8):
        M = int(rng.integers(1000, 5000))
        N = 384 * int(rng.integers(1, 10)) if rng.random() < 0.5 else 16 * int(rng.integers(20, 600))
        K = 64 * int(rng.integers(1, 50))
        out = torch.bfloat16 if rng.random() < 0.5 else torch.float16
        e4m3 = rng.random() < 0.5
        a_bf16 = rng.random() < 0.5
        fmt = torch.float8_e4m3fn if e4m3 else torch.float8_e5m2
        fmax = 448.0 if e4m3 else 57344.0
        x = torch.randn(M, K, generator=gd, device=cuda)
        a = x.to(torch.bfloat16) if a_bf16 else x.half()
        w = torch.randn(N, K, generator=gd, device=cuda) * 0.02
        s = (w.abs().max() / fmax).float().reshape(1)
        bp = (w / s).to(fmt).view(N, K // 16, 16).permute(1, 0, 2).contiguous()
        bias = (torch.randn(N, generator=gd, device=cuda) * 0.1).to(out)
        print("large e4m3/bf16", case, M, N, K, out, e4m3, a_bf16, hk.any_m_config(M, N, K), flush=True)
        ref = torch_ref_dev(a.to(torch.float16), bp, s, bias, out, b_dtype=fmt)
        y = hk.scaled_mm_hip_any_m(a, bp, s, bias, out)
        assert_gemm_close_dev(y, ref, out, f"large e4m3/bf16 {case}")
        del ref, y


@pytest.mark.parametrize("seed", [0, 1])
def test_random_split_k_region(cuda, hk, seed):
    """Random shapes around the split-K routes (17 <= M <= 2048, N and K 1024..10240) through the
    any-M entry with its default routing: the small-M kernel, the split-K tiles (64 x 64, 64 x 128,
    32 x 128 on five- or six-stage rings, K splits from one to many) or the tile kernels, whichever
    the shape takes; the whole output against a float64 evaluation on the device, and the kernel
    each case took is printed."""
    from gpu_util import assert_gemm_close_dev, torch_ref_dev

    rng = np.random.default_rng(100 + seed)
    for case in range(16):
        M = int(rng.choice([17, 24, 33, 40, 48, 56, 64, 77, 154, 256, 512, 1024, 2048]))
        N = 16 * int(rng.integers(64, 641))
        K = 64 * int(rng.integers(16, 161))
        out = torch.float16 if rng.random() < 0.5 else torch.bfloat16
        b_dtype = torch.float8_e4m3fn if rng.random() < 0.3 else torch.float8_e5m2
        kid = hk.kernel_id(M, N, K, hk.any_m_config(M, N, K))
        print(f"seed {seed} case {case}: M={M} N={N} K={K} {out} {b_dtype} kernel {kid}", flush=True)
        g = torch.Generator(device=cuda).manual_seed(1000 * seed + case)
        a = torch.randn(M, K, generator=g, device=cuda).half()
        fmax = 448.0 if b_dtype == torch.float8_e4m3fn else 57344.0
        w = torch.randn(N, K, generator=g, device=cuda) * 0.02
        s = (w.abs().max() / fmax).float().reshape(())
        bp = (w / s).to(b_dtype).view(N, K // 16, 16).permute(1, 0, 2).contiguous()
        del w
        bias = (torch.randn(N, generator=g, device=cuda) * 0.1).to(out)
        y = hk.scaled_mm_hip_any_m(a, bp, s, bias, out)
        ref = torch_ref_dev(a, bp, s, bias, out, b_dtype=b_dtype)
        assert_gemm_close_dev(y, ref, out, f"seed {seed} case {case}: M={M} N={N} K={K} kernel {kid}")
