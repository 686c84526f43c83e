"""GPU tests of the drop-in callers: FeatherOps.Linear, scaled_mm_hip autotune,
and the torch.compile contract (reference test_scaled_mm_hip_autotune_compile.py)."""

import numpy as np
import pytest
import torch

from gpu_util import assert_gemm_close
from oracle import feather_oracle as O

pytestmark = pytest.mark.gpu


def _linear_ref(x: torch.Tensor, qdata: torch.Tensor, scale: float, bias, out_dtype):
    a = x.reshape(-1, x.shape[-1]).to(torch.float16).cpu().numpy()
    od = O.DT_F16 if out_dtype == torch.float16 else O.DT_BF16
    b = None
    if bias is not None:
        b = bias.cpu().numpy() if out_dtype == torch.float16 else bias.cpu().view(torch.int16).numpy().view(np.uint16)
    return O.scaled_mm_ref(a, qdata.view(torch.uint8).cpu().numpy(), np.float32(scale), b, od)


@pytest.mark.parametrize("pad_m", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 37, 130, 300])
def test_feather_linear_forward(cuda, pkg, out_dtype, m, pad_m):
    from featherops_amd.comfy_feather import ops, quant

    g = torch.Generator().manual_seed(m)
    K, N = 256, 384
    ops_cls = ops.feather_ops(out_dtype=out_dtype)
    lin = ops_cls.Linear(K, N)
    lin.pad_m = pad_m
    sd = {"weight": (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16),
          "bias": (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)}
    lin._load_from_state_dict(sd, "", {}, True, [], [], [])
    assert lin.is_quantized
    lin.weight = lin.weight.to(cuda) if not isinstance(lin.weight, torch.Tensor) else lin.weight
    lin.bias = torch.nn.Parameter(lin.bias.to(cuda), requires_grad=False)
    qdata, scale = quant.get_feather_plain_tensors(lin.weight)
    x = torch.randn(2, m, K, generator=g).to(torch.bfloat16).to(cuda)
    y = lin(x)
    torch.cuda.synchronize()
    assert y.shape == (2, m, N) and y.dtype == torch.bfloat16
    ref = _linear_ref(x, qdata, scale.item(), lin.bias, out_dtype)
    # the layer casts its out_dtype result back to the input dtype (bf16)
    ref_t = torch.from_numpy(O.bf16_bits_to_f32(ref) if ref.dtype == np.uint16 else ref.astype(np.float32))
    ref_bf = ref_t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert_gemm_close(y.reshape(-1, N), ref_bf, torch.bfloat16, f"linear m={m} pad_m={pad_m}")


def test_feather_linear_excluded_and_patch(cuda, pkg):
    from featherops_amd.comfy_feather import ops, quant

    ops_cls = ops.feather_ops(out_dtype=torch.float16, excluded_names=("proj_out",))
    lin = ops_cls.Linear(64, 32)
    w = torch.randn(32, 64) * 0.1
    lin._load_from_state_dict({"proj_out.weight": w.clone()}, "proj_out.", {}, True, [], [], [])
    assert not lin.is_quantized
    lin2 = ops_cls.Linear(64, 32)
    lin2._load_from_state_dict({"blocks.0.weight": w.clone().to(cuda)}, "blocks.0.", {}, True, [], [], [])
    assert lin2.is_quantized
    deq = lin2.convert_weight(lin2.weight)
    assert deq.shape == (32, 64) and deq.dtype == torch.float16
    assert (deq.float().cpu() - w).abs().max().item() <= w.abs().max().item() * 2**-3
    lin2.set_weight(deq)
    assert quant.is_feather_quantized_weight(lin2.weight)
    y = lin2(torch.zeros(0, 64, device=cuda))
    assert y.shape == (0, 32)


def test_scaled_mm_hip_autotune_eager(cuda, hk):
    g = torch.Generator().manual_seed(0)
    a = torch.randn(512, 512, generator=g).half()
    b = torch.randn(512, 512, generator=g).to(torch.float8_e5m2)
    bias = torch.randn(512, generator=g).half()
    bp = hk.prepack_b_for_scaled_mm(b.to(cuda))
    s = torch.tensor(2.34, device=cuda)
    y = hk.scaled_mm_hip(a.to(cuda), bp, s, bias.to(cuda), torch.float16)
    ref = O.scaled_mm_ref(a.numpy(), bp.view(torch.uint8).cpu().numpy(), np.float32(2.34), bias.numpy(), O.DT_F16)
    assert_gemm_close(y, ref, torch.float16, "autotuned")
    y2 = hk.scaled_mm_hip(a.to(cuda), bp, None, None, torch.float16)  # no scale, no bias
    ref2 = O.scaled_mm_ref(a.numpy(), bp.view(torch.uint8).cpu().numpy(), None, None, O.DT_F16)
    assert_gemm_close(y2, ref2, torch.float16, "autotuned no scale")


def test_torch_compile_configured_and_autotuned(cuda, hk):
    g = torch.Generator().manual_seed(1)
    a = torch.randn(512, 512, generator=g).half().to(cuda)
    b = torch.randn(512, 512, generator=g).to(torch.float8_e5m2)
    bias = torch.randn(512, generator=g).half().to(cuda)
    bp = hk.prepack_b_for_scaled_mm(b.to(cuda))
    s = torch.tensor(2.34, device=cuda)
    ref = O.scaled_mm_ref(a.cpu().numpy(), bp.view(torch.uint8).cpu().numpy(), np.float32(2.34),
                          bias.cpu().numpy(), O.DT_F16)

    @torch.compile(fullgraph=True)
    def configured(a, bp, s, bias):
        return hk.scaled_mm_hip_configured(a, bp, s, bias, torch.float16, 1, 1, 2, 1, 2)

    assert_gemm_close(configured(a, bp, s, bias), ref, torch.float16, "compile configured")

    @torch.compile(fullgraph=True)
    def autotuned(x, bp, bias):
        x = x.to(torch.float16).view(-1, x.shape[-1])
        return hk.scaled_mm_hip(x, bp, None, bias, torch.float16)

    xv = a.view(2, 256, 512).to(torch.bfloat16)
    y = autotuned(xv, bp, bias)
    ref2 = O.scaled_mm_ref(xv.to(torch.float16).view(-1, 512).cpu().numpy(), bp.view(torch.uint8).cpu().numpy(),
                           None, bias.cpu().numpy(), O.DT_F16)
    assert_gemm_close(y, ref2, torch.float16, "compile autotuned view input no scale")


def test_torch_compile_any_m(cuda, hk):
    """The any-M op (C++, Meta kernel for tracing) under torch.compile with
    fullgraph: bf16 activations of a ragged M, the op traced as one call."""
    g = torch.Generator().manual_seed(5)
    K, N = 512, 384
    b = torch.randn(K, N, generator=g).to(torch.float8_e5m2)
    bp = hk.prepack_b_for_scaled_mm(b.to(cuda))
    s = torch.tensor(0.75, device=cuda)
    bias = torch.randn(N, generator=g).to(torch.bfloat16).to(cuda)

    @torch.compile(fullgraph=True)
    def f(x, bp, s, bias):
        return hk.scaled_mm_hip_any_m(x.view(-1, x.shape[-1]), bp, s, bias, torch.bfloat16)

    for m in (37, 300):
        x = torch.randn(1, m, K, generator=g).to(torch.bfloat16).to(cuda)
        y = f(x, bp, s, bias)
        assert y.shape == (m, N) and y.dtype == torch.bfloat16
        ref = O.scaled_mm_ref(x.view(m, K).to(torch.float16).cpu().numpy(), bp.view(torch.uint8).cpu().numpy(),
                              np.float32(0.75), bias.cpu().view(torch.int16).numpy().view(np.uint16), O.DT_BF16)
        assert_gemm_close(y, ref, torch.bfloat16, f"compile any-M {m}")


def test_two_streams_keep_separate_workspaces(cuda, hk):
    """K-split calls (small-M kernel, workspace from the C++ op's per-stream
    pool) issued on two streams at once give the single-stream results."""
    g = torch.Generator(device=cuda).manual_seed(11)
    K, N = 8192, 1024
    b = (torch.randn(K, N, generator=g, device=cuda) * 0.02).to(torch.float8_e5m2)
    bp = hk.prepack_b_for_scaled_mm(b)
    s = torch.tensor(2.0, device=cuda)
    xs = [torch.randn(m, K, generator=g, device=cuda).half() for m in (16, 24, 8, 32)]
    for x in xs:  # every call takes the K split across workgroups
        assert hk._lib.lib().feather_scaled_mm_workspace_size(x.shape[0], N, K, *hk.any_m_config(x.shape[0], N, K)) > 0
    want = [hk.scaled_mm_hip_any_m(x, bp, s, None, torch.float16) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    got = [None] * len(xs)
    for rep in range(3):
        for i, x in enumerate(xs):
            with torch.cuda.stream(streams[i % 2]):
                got[i] = hk.scaled_mm_hip_any_m(x, bp, s, None, torch.float16)
        torch.cuda.synchronize()
        for i in range(len(xs)):
            assert torch.equal(got[i], want[i]), f"rep {rep} call {i}"


def test_graph_capture_replays_match_eager(cuda, hk, quant):
    """scaled_mm (small-M kernel with and without its K split, split-K tiles,
    bf16 activations) and quantize captured in a HIP graph: every replay, with
    eager work in between, equals the eager result (the split paths' arrival
    counters must come back to zero on every replay)."""
    g = torch.Generator(device=cuda).manual_seed(3)
    w = (torch.randn(512, 1024, generator=g, device=cuda) * 0.02).half()
    qt = quant.make_feather_quantized_weight(w, None, torch.float16)
    bp, scale = quant.get_feather_plain_tensors(qt)
    bias = (torch.randn(512, generator=g, device=cuda) * 0.01).half()
    for m, cfg in ((16, (1, 1, 2, 1, 2)), (48, (1, 1, 2, 1, 2)), (512, (2, 4, 4, 8, 4)), (40, None)):
        a = torch.randn(m, 1024, generator=g, device=cuda).half()
        if cfg is None:  # any-M entry with bf16 activations (small-M kernel, K split across workgroups)
            a = a.bfloat16()
            fn = lambda: hk.scaled_mm_hip_any_m(a, bp, scale, bias, torch.float16)  # noqa: E731
        else:
            fn = lambda: hk.scaled_mm_hip_configured(a, bp, scale, bias, torch.float16, *cfg)  # noqa: E731
        eager = fn()
        out = torch.empty_like(eager)
        fn()  # warm the op before capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out.copy_(fn())
        for rep in range(4):
            out.zero_()
            graph.replay()
            junk = torch.randn(1 << 16, device=cuda).sum()  # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {rep} m={m}"
            assert torch.isfinite(junk)


@pytest.mark.parametrize("M", [1, 15, 17, 63, 65, 100, 257, 1000])
def test_any_m_equals_padded(cuda, hk, M):
    """Unpadded call == reference-style pad + configured call + slice. Bit-exact
    when both run the same kernel with the same K order; the padded M can route
    to a different K split of the split-K tiles (fp32 reassociation), then both
    must pass the parity gate against the oracle."""
    g = torch.Generator(device=cuda).manual_seed(M)
    K, N = 512, 768
    a = torch.randn(M, K, generator=g, device=cuda).half()
    b = torch.randn(K, N, generator=g, device=cuda).to(torch.float8_e5m2)
    bp = hk.prepack_b_for_scaled_mm(b)
    s = torch.tensor(0.5, device=cuda)
    bias = torch.randn(N, generator=g, device=cuda).half()
    y = hk.scaled_mm_hip_any_m(a, bp, s, bias, torch.float16)
    cfg = hk.any_m_config(M, N, K)
    bm = 16 * cfg[0] * cfg[3]
    mp = (M + bm - 1) // bm * bm
    ap = torch.nn.functional.pad(a, (0, 0, 0, mp - M))
    yp = hk.scaled_mm_hip_configured(ap, bp, s, bias, torch.float16, *cfg)[:M]
    torch.cuda.synchronize()
    if hk.kernel_id(M, N, K, cfg) == hk.kernel_id(mp, N, K, cfg) and hk.kernel_id(M, N, K, cfg) < 30:
        assert torch.equal(y, yp)
    ref = O.scaled_mm_ref(a.cpu().numpy(), bp.view(torch.uint8).cpu().numpy(), np.float32(0.5),
                          bias.cpu().numpy(), O.DT_F16)
    assert_gemm_close(y, ref, torch.float16, f"any-M {M}")
    assert_gemm_close(yp, ref, torch.float16, f"padded {M}")


def test_inductor_autotunes_every_compatible_config(cuda, hk, monkeypatch, tmp_path):
    """Inductor's custom-op autotuning (reference kernel/hip/hip_kernel.py:133) on this torch:
    compiling scaled_mm_hip benchmarks the compatible configs through the op's decomposition
    and the compiled result equals the oracle. Inductor's caches are off and its cache
    directory is fresh: a result cached by an earlier process on the same machine would
    skip the benchmarking."""
    import torch._inductor.config as inductor_config
    import torch._inductor.lowering as L

    monkeypatch.setenv("TORCHINDUCTOR_CACHE_DIR", str(tmp_path / "inductor"))
    monkeypatch.setattr(inductor_config, "force_disable_caches", True)

    assert torch.ops.feather_ops_internal.scaled_mm_autotuned.default in L.lowerings
    seen = set()
    real = hk._autotune_decomposition

    def spy(a, b, scale, bias, **kw):
        seen.add((kw["block_warps_m"], kw["block_warps_n"], kw["unroll_k"], kw["repeat_m"], kw["repeat_n"]))
        return real(a, b, scale, bias, **kw)

    monkeypatch.setattr(hk, "_autotune_decomposition", spy)
    torch._dynamo.reset()
    g = torch.Generator().manual_seed(8)
    a = torch.randn(256, 1024, generator=g).half().to(cuda)
    bp = hk.prepack_b_for_scaled_mm((torch.randn(1024, 768, generator=g) * 0.1).to(torch.float8_e5m2).to(cuda))
    s = torch.tensor(1.5, device=cuda)
    bias = (torch.randn(768, generator=g) * 0.01).bfloat16().to(cuda)

    @torch.compile(fullgraph=True)
    def f(a, bp, s, bias):
        return hk.scaled_mm_hip(a, bp, s, bias, torch.bfloat16)

    y = f(a, bp, s, bias)
    assert len(seen) >= 2, f"autotuning ran {len(seen)} configs"
    ref = O.scaled_mm_ref(a.cpu().numpy(), bp.view(torch.uint8).cpu().numpy(), np.float32(1.5),
                          bias.cpu().view(torch.int16).numpy().view(np.uint16), O.DT_BF16)
    assert_gemm_close(y, ref, torch.bfloat16, "inductor autotuned")
    torch._dynamo.reset()
