"""GPU tests of the unmerged-LoRA path (reference comfy_feather/lora.py:4-35):
the term fused into the LDS tiles' epilogue, the fallback routes, and
FeatherOps.Linear with LoRA patches attached."""

import numpy as np
import pytest
import torch

from gpu_util import assert_gemm_close
from lora_util import make_patches
from oracle import feather_oracle as O

pytestmark = pytest.mark.gpu


def _setup(cuda, hk, M, N, K, seed, x_dtype, out_dtype, ranks=(16, 8)):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(x_dtype).to(cuda)
    w = torch.randn(K, N, generator=g).to(torch.float8_e5m2)
    bp = hk.prepack_b_for_scaled_mm(w.to(cuda))
    s = torch.tensor(0.04, device=cuda)
    bias = (torch.randn(N, generator=g) * 0.1).to(out_dtype).to(cuda)
    wf, expect = make_patches(N, K, list(ranks), g, device=cuda, dtype=x_dtype)
    return x, bp, s, bias, wf, expect


def _bias_np(bias, out_dtype):
    return bias.cpu().numpy() if out_dtype == torch.float16 else bias.cpu().view(torch.int16).numpy().view(np.uint16)


def _od(out_dtype):
    return O.DT_F16 if out_dtype == torch.float16 else O.DT_BF16


def _fused_ref(x, bp, s, bias, out_dtype, t, u):
    """The fused epilogue's contract: T . U^T joins the scaled fp32 value before
    the output rounding (oracle scaled_mm_ref(lora=...)), with the factors the
    kernel was given."""
    return O.scaled_mm_ref(x.to(torch.float16).cpu().numpy(), bp.view(torch.uint8).cpu().numpy(),
                           np.float32(s.item()), _bias_np(bias, out_dtype), _od(out_dtype),
                           lora=(t.double().cpu().numpy(), u.double().cpu().numpy()))


def _separate_ref(x, bp, s, bias, out_dtype, t, u):
    """The other routes: the GEMM's output, then C += (T @ U^T) in the factors'
    dtype rounded to the output type (torch on the host for the term)."""
    base = O.scaled_mm_ref(x.to(torch.float16).cpu().numpy(), bp.view(torch.uint8).cpu().numpy(),
                           np.float32(s.item()), _bias_np(bias, out_dtype), _od(out_dtype))
    base = torch.from_numpy(O.bf16_bits_to_f32(base) if base.dtype == np.uint16 else base.astype(np.float32))
    y = base.to(out_dtype) + torch.mm(t.cpu(), u.cpu().t()).to(out_dtype)
    return _as_oracle(y, out_dtype)


def _exact(x, bp, s, bias, out_dtype, expect):
    """fp64 value of the whole layer with no rounding anywhere: (A @ dec(B)) * s
    + bias + every patch's F.linear(F.linear(x, A), B) * s."""
    acc = O.scaled_mm_ref_f32(x.to(torch.float16).cpu().numpy(), bp.view(torch.uint8).cpu().numpy(),
                              np.float32(s.item()))
    xd = x.double().cpu()
    term = sum((xd @ d.double().cpu().T) @ u.double().cpu().T * sc for d, u, sc in expect)
    return torch.from_numpy(acc) + bias.double().cpu() + term


def _as_oracle(ref: torch.Tensor, dtype):
    r = ref.to(dtype)
    return r.numpy() if dtype == torch.float16 else r.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("x_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(2048, 2048, 512), (1000, 4096, 1024), (37, 384, 256), (300, 384, 256),
                                   (64, 2048, 512)])
def test_any_m_lora_matches_reference(cuda, hk, pkg, M, N, K, x_dtype, out_dtype):
    from featherops_amd.comfy_feather import lora

    x, bp, s, bias, wf, expect = _setup(cuda, hk, M, N, K, M + N, x_dtype, out_dtype)
    t, u = lora.lora_factors(x, wf)
    y = hk.scaled_mm_hip_any_m_lora(x, bp, s, bias, out_dtype, t, u)
    torch.cuda.synchronize()
    kid = hk.kernel_id(M, N, K, hk.any_m_config(M, N, K))
    fused = 20 <= kid < 30
    ref = (_fused_ref if fused else _separate_ref)(x, bp, s, bias, out_dtype, t, u)
    assert_gemm_close(y, ref, out_dtype, f"lora {M}x{N}x{K} {x_dtype} {out_dtype} fused={fused}")
    if fused:  # the same GEMM with zero factors is the plain any-M result
        y0 = hk.scaled_mm_hip_any_m_lora(x, bp, s, bias, out_dtype, torch.zeros_like(t), torch.zeros_like(u))
        assert torch.equal(y0, hk.scaled_mm_hip_any_m(x, bp, s, bias, out_dtype))


def test_fused_route_is_taken_and_deterministic(cuda, hk, pkg):
    from featherops_amd.comfy_feather import lora

    M, N, K = 2048, 2048, 512
    assert 20 <= hk.kernel_id(M, N, K, hk.any_m_config(M, N, K)) < 30
    x, bp, s, bias, wf, expect = _setup(cuda, hk, M, N, K, 9, torch.bfloat16, torch.bfloat16, ranks=(64, 32))
    t, u = lora.lora_factors(x, wf)
    assert t.shape[1] == 96
    # C ABI: the fused entry launches for this route (returns true)
    c = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    x16 = x.to(torch.float16)
    L = hk._lib.lib()
    ok = L.feather_launch_scaled_mm_lora(x16.data_ptr(), bp.data_ptr(), s.data_ptr(), bias.data_ptr(), c.data_ptr(),
                                         M, N, K, 1, 1, t.data_ptr(), u.data_ptr(), 96, 1, *hk.any_m_config(M, N, K),
                                         1, 1, torch.cuda.current_stream().cuda_stream)
    assert ok
    y = hk.scaled_mm_hip_any_m_lora(x, bp, s, bias, torch.bfloat16, t, u)
    torch.cuda.synchronize()
    assert torch.equal(c, y)
    for _ in range(3):
        assert torch.equal(hk.scaled_mm_hip_any_m_lora(x, bp, s, bias, torch.bfloat16, t, u), y)
    # refused (false, nothing launched): rank not a multiple of 32, e4m3 weights, small-M route
    assert not L.feather_launch_scaled_mm_lora(x16.data_ptr(), bp.data_ptr(), s.data_ptr(), None, c.data_ptr(), M, N,
                                               K, 1, 0, t.data_ptr(), u.data_ptr(), 48, 1,
                                               *hk.any_m_config(M, N, K), 1, 1, 0)
    assert not L.feather_launch_scaled_mm_lora(x16.data_ptr(), bp.data_ptr(), s.data_ptr(), None, c.data_ptr(), M, N,
                                               K, 1, 0, t.data_ptr(), u.data_ptr(), 96, 1,
                                               *hk.any_m_config(M, N, K), 0, 1, 0)
    assert not L.feather_launch_scaled_mm_lora(x16.data_ptr(), bp.data_ptr(), s.data_ptr(), None, c.data_ptr(), 16, N,
                                               K, 1, 0, t.data_ptr(), u.data_ptr(), 96, 1,
                                               *hk.any_m_config(16, N, K), 1, 1, 0)


def test_fused_route_when_the_pick_has_no_lora_epilogue(cuda, hk, pkg):
    """At M=4096, N=3072 the any-M pick is the 128x384 tile, which has no rank-R epilogue: the C ABI
    refuses it, and the LoRA op runs the fused epilogue on the 256x192 tile (same 256-tile grid)."""
    from featherops_amd.comfy_feather import lora

    M, N, K = 4096, 3072, 512
    assert hk.any_m_config(M, N, K) == (2, 4, 4, 4, 6)
    x, bp, s, bias, wf, expect = _setup(cuda, hk, M, N, K, 11, torch.bfloat16, torch.bfloat16, ranks=(32,))
    t, u = lora.lora_factors(x, wf)
    x16 = x.to(torch.float16)
    c = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    L = hk._lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    args = (x16.data_ptr(), bp.data_ptr(), s.data_ptr(), bias.data_ptr(), c.data_ptr(), M, N, K, 1, 1, t.data_ptr(),
            u.data_ptr(), t.shape[1], 1)
    assert not L.feather_launch_scaled_mm_lora(*args, 2, 4, 4, 4, 6, 1, 1, st)
    assert L.feather_launch_scaled_mm_lora(*args, 2, 4, 4, 8, 3, 1, 1, st)
    y = hk.scaled_mm_hip_any_m_lora(x, bp, s, bias, torch.bfloat16, t, u)
    torch.cuda.synchronize()
    assert torch.equal(c, y)
    rows = torch.tensor([0, 1, 255, 256, 2047, 4095], device=cuda)
    ref = _fused_ref(x[rows], bp, s, bias, torch.bfloat16, t[rows], u)
    assert_gemm_close(y[rows], ref, torch.bfloat16, "4096x3072 fused LoRA")


def test_any_m_lora_argument_checks(cuda, hk, pkg):
    M, N, K = 256, 512, 256
    x = torch.zeros(M, K, dtype=torch.float16, device=cuda)
    bp = torch.zeros(K // 16, N, 16, dtype=torch.float8_e5m2, device=cuda)
    t = torch.zeros(M, 32, dtype=torch.float16, device=cuda)
    u = torch.zeros(N, 32, dtype=torch.float16, device=cuda)
    op = hk.scaled_mm_hip_any_m_lora
    with pytest.raises(RuntimeError, match="multiple of 32"):
        op(x, bp, None, None, torch.float16, t[:, :16].contiguous(), u[:, :16].contiguous())
    with pytest.raises(RuntimeError, match="must both be float16 or both bfloat16"):
        op(x, bp, None, None, torch.float16, t, u.bfloat16())
    with pytest.raises(RuntimeError, match=r"\(M, R\)"):
        op(x, bp, None, None, torch.float16, t[:100], u)
    with pytest.raises(RuntimeError, match="contiguous"):
        op(x, bp, None, None, torch.float16, torch.zeros(64, M, dtype=torch.float16, device=cuda).t()[:, :32], u)


@pytest.mark.parametrize("m", [37, 2048])
def test_linear_with_lora_patches(cuda, pkg, m):
    """FeatherOps.Linear with basic LoRA patches: the fused path (fuse_lora,
    default) and the reference's separate pass agree within the output gate."""
    from featherops_amd.comfy_feather import ops, quant

    g = torch.Generator().manual_seed(m)
    K, N = 512, 2048
    lin = ops.feather_ops(out_dtype=torch.bfloat16).Linear(K, N)
    sd = {"weight": (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16),
          "bias": (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)}
    lin._load_from_state_dict(sd, "", {}, True, [], [], [])
    lin.weight = lin.weight.to(cuda) if not isinstance(lin.weight, torch.Tensor) else lin.weight
    lin.bias = torch.nn.Parameter(lin.bias.to(cuda), requires_grad=False)
    wf, expect = make_patches(N, K, [16, 32], g, device=cuda, dtype=torch.bfloat16)
    lin.weight_function = wf
    x = torch.randn(1, m, K, generator=g).to(torch.bfloat16).to(cuda)
    y_fused = lin(x)
    lin.fuse_lora = False
    y_sep = lin(x)
    torch.cuda.synchronize()
    assert y_fused.shape == (1, m, N) and y_fused.dtype == torch.bfloat16
    qdata, scale = quant.get_feather_plain_tensors(lin.weight)
    exact = _exact(x.reshape(m, K), qdata.to(cuda), torch.tensor(scale.item()), lin.bias, torch.bfloat16, expect)
    # Both paths against the unrounded value. The reference's own arithmetic
    # rounds to bf16 after the GEMM, each F.linear, the scaling and the add
    # (about 2^-9 relative per step), so the gate here is the bf16 chain's:
    # rel-Fro <= 4e-3, every element within max(2e-2, 4 ulp of bf16 at |exact|).
    for name, y in (("fused", y_fused), ("separate", y_sep)):
        d = (y.reshape(m, N).double().cpu() - exact).abs()
        fro = d.norm().item() / exact.norm().item()
        ulp = torch.exp2(torch.floor(torch.log2(exact.abs().clamp_min(2.0**-14))) - 7)
        worst = (d / torch.maximum(torch.full_like(ulp, 2e-2), 4 * ulp)).max().item()
        assert fro <= 4e-3 and worst <= 1.0, f"{name} linear m={m}: rel-Fro {fro:.3g}, worst {worst:.3g}"
    if m < 2048:
        return
    # on the fused route the result is the more exact of the two (one rounding of the sum)
    d_f = (y_fused.reshape(m, N).double().cpu() - exact).norm().item()
    d_s = (y_sep.reshape(m, N).double().cpu() - exact).norm().item()
    assert d_f <= d_s * 1.05, (d_f, d_s)
