"""The one-pass quantize (feather_quantize_prepack_e5m2_ws: each workgroup keeps
its share of the weight in registers, the part beyond them read again, while
the workgroups agree on the amax through a grid barrier) against the two-pass entry, feather_quantize_prepack_e5m2,
and the oracle: codes and scale bit for bit, on the load path (fp32 arithmetic
on w * ckpt_scale) and the patch path (the weight's dtype), with ragged
shapes, special values, the barrier's timeout fallback forced from the host
(a poll limit of 0), graph replay, and the workspace shared with the K-split
GEMM."""

import numpy as np
import pytest
import torch

from gpu_util import lib, stream
from oracle import feather_oracle as O

pytestmark = pytest.mark.gpu

SENTINEL = -1  # 0xffffffff: above every partial maximum the kernels write


def _ws(cuda):
    n = lib().feather_quantize_workspace_size()
    return torch.zeros(n, dtype=torch.uint8, device=cuda)


def _run(w, ck, native, ws=None, one_pass=True):
    N, K = w.shape
    code = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}[w.dtype]
    out = torch.full((K // 16, N, 16), 0xAB, dtype=torch.uint8, device=w.device)
    scale = torch.full((), float("nan"), dtype=torch.float32, device=w.device)
    ckp = ck.data_ptr() if ck is not None else None
    if one_pass:
        st = lib().feather_quantize_prepack_e5m2_ws(w.data_ptr(), code, N, K, ckp, native, out.data_ptr(),
                                                    scale.data_ptr(), ws.data_ptr(), ws.numel(), stream(w.device))
    else:
        parts = torch.empty(256, dtype=torch.int32, device=w.device)
        st = lib().feather_quantize_prepack_e5m2(w.data_ptr(), code, N, K, ckp, native, out.data_ptr(),
                                                 scale.data_ptr(), parts.data_ptr(), stream(w.device))
        torch.cuda.synchronize()
    assert st == 0, lib().feather_status_string(st)
    return out, scale


def _same(a, b, what):
    """Codes and scale bit for bit. With a NaN scale every code is a NaN code
    (0x7f with the sign bit of the NaN product); IEEE 754 leaves the sign of a
    NaN produced by arithmetic (0 * inf) open and the two kernels' instruction
    sequences differ there, so only that sign bit is exempt."""
    (qa, sa), (qb, sb) = a, b
    torch.cuda.synchronize()
    assert sa.view(torch.int32).item() == sb.view(torch.int32).item(), f"{what}: scale {sa.item()} vs {sb.item()}"
    if torch.isnan(sb).item():
        assert ((qa & 0x7F) == 0x7F).all() and ((qb & 0x7F) == 0x7F).all(), f"{what}: NaN scale, non-NaN codes"
        return
    assert torch.equal(qa, qb), f"{what}: codes differ"


# on 256 CUs: up to (10240, 4096) every workgroup's share fits its registers,
# (11264, 4096) needs the LDS as well, (4100, 12304) (ragged in both) and
# (13824, 5120) read the rest of a share twice
SHAPES = [(1, 16), (5, 48), (64, 64), (63, 80), (1000, 272), (3072, 3072), (5120, 5120), (2000, 9232),
          (10240, 4096), (11264, 4096), (4100, 12304), (13824, 5120)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("native", [0, 1])
@pytest.mark.parametrize("N,K", SHAPES)
def test_one_pass_matches_two_pass(cuda, dtype, native, N, K):
    print("one-pass", dtype, native, N, K, flush=True)
    g = torch.Generator(device=cuda).manual_seed(N * 7 + K + native)
    w = (torch.randn(N, K, generator=g, device=cuda) * 0.03).to(dtype)
    ck = None if native else torch.tensor([0.37], device=cuda)
    ws = _ws(cuda)
    for rep in range(2):  # twice on one workspace: the counters came back to zero
        _same(_run(w, ck, native, ws), _run(w, ck, native, one_pass=False), f"{N}x{K} rep {rep}")
    assert (ws[:65536] == 0).all(), "the counter region must be left zero"


def test_one_pass_against_oracle(cuda):
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(3072, 1024, generator=g) * 0.05).half()
    out, scale = _run(w.to(cuda), None, 1, _ws(cuda))
    torch.cuda.synchronize()
    codes, s_ref = O.quantize_native(w.numpy(), O.DT_F16)
    assert np.float32(scale.item()) == s_ref
    assert np.array_equal(O.unprepack_transpose(out.cpu().numpy()), codes)
    wb = (torch.randn(640, 2048, generator=g) * 3.0).bfloat16()
    ck = torch.tensor([0.125], device=cuda)
    out, scale = _run(wb.to(cuda), ck, 0, _ws(cuda))
    torch.cuda.synchronize()
    codes, s_ref = O.quantize_load(wb.float().numpy(), O.DT_F32, ckpt_scale=np.float32(0.125))
    assert np.float32(scale.item()) == s_ref
    assert np.array_equal(O.unprepack_transpose(out.cpu().numpy()), codes)


def test_one_pass_path_taken(cuda):
    """A 64 x 64 weight: the two-pass amax writes one partial, the one-pass
    kernel one per workgroup (one per CU) into the scratch after the counters."""
    w = torch.randn(64, 64, device=cuda).half()
    ws = _ws(cuda)
    ws[65536:].view(torch.int32).fill_(SENTINEL)
    _run(w, None, 1, ws)
    torch.cuda.synchronize()
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    parts = ws[65536:].view(torch.int32)
    assert (parts[:cus] != SENTINEL).all() and (parts[cus:] == SENTINEL).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_one_pass_special_values(cuda, dtype):
    ws = _ws(cuda)
    z = torch.zeros(96, 128, dtype=dtype, device=cuda)
    for native in (0, 1):
        _same(_run(z, None, native, ws), _run(z, None, native, one_pass=False), "zeros")
    w = (torch.randn(96, 128, device=cuda) * 100).to(dtype)
    w[0, :5] = 0.0
    for ck in (float("inf"), float("-inf"), float("nan"), -2.5, 0.0, 1e-30):  # per-element path for inf / NaN
        c = torch.tensor([ck], device=cuda)
        _same(_run(w, c, 0, ws), _run(w, c, 0, one_pass=False), f"ckpt_scale {ck}")
    w[17, 33] = float("nan")
    for native in (0, 1):
        _same(_run(w, None, native, ws), _run(w, None, native, one_pass=False), "nan weight")
    w[17, 33] = float("inf")
    for native in (0, 1):
        _same(_run(w, None, native, ws), _run(w, None, native, one_pass=False), "inf weight")
    assert (ws[:65536] == 0).all()


@pytest.mark.parametrize("N,K", [(64, 64), (1000, 272), (3072, 3072), (4100, 12304)])
def test_one_pass_barrier_fallback(cuda, monkeypatch, N, K):
    """FEATHEROPS_QUANT_SPIN=0: no workgroup waits for the others; each takes
    the amax over the whole weight itself. Same results, counters left zero."""
    monkeypatch.setenv("FEATHEROPS_QUANT_SPIN", "0")
    g = torch.Generator(device=cuda).manual_seed(N + K)
    w = (torch.randn(N, K, generator=g, device=cuda) * 0.5).half()
    ws = _ws(cuda)
    for native in (0, 1):
        ck = None if native else torch.tensor([3.0], device=cuda)
        _same(_run(w, ck, native, ws), _run(w, ck, native, one_pass=False), f"fallback {N}x{K}")
    bad = torch.tensor([float("inf")], device=cuda)
    _same(_run(w, bad, 0, ws), _run(w, bad, 0, one_pass=False), "fallback, per-element")
    assert (ws[:65536] == 0).all()


def test_one_pass_graph_replay(cuda):
    """Captured once, replayed three times with eager work in between: each
    replay equals the eager call (the counters return to zero every time)."""
    w = (torch.randn(2048, 2048, device=cuda) * 0.1).bfloat16()
    ws = _ws(cuda)
    ref = _run(w, None, 1, ws)
    torch.cuda.synchronize()
    out = torch.empty_like(ref[0])
    scale = torch.empty_like(ref[1])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            st = lib().feather_quantize_prepack_e5m2_ws(w.data_ptr(), 1, 2048, 2048, None, 1, out.data_ptr(),
                                                        scale.data_ptr(), ws.data_ptr(), ws.numel(), s.cuda_stream)
    assert st == 0
    for rep in range(3):
        out.fill_(0)
        scale.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        _same((out, scale), ref, f"replay {rep}")
        _run(w, None, 1, ws)  # eager call on the same workspace between replays
        torch.cuda.synchronize()
    assert (ws[:65536] == 0).all()


def test_workspace_shared_with_split_k_gemm(cuda):
    """One zero-filled workspace serves the quantize and the K-split small-M
    GEMM in turn on one stream: each result equals the same call on a fresh
    workspace of its own (the split-K sum is deterministic)."""
    M, N, K = 8, 2048, 12288
    cfg = (1, 1, 2, 1, 2)
    gemm_ws = lib().feather_scaled_mm_workspace_size(M, N, K, *cfg)
    assert gemm_ws > 65536, "the GEMM splits K"
    need = max(gemm_ws, lib().feather_quantize_workspace_size())
    g = torch.Generator(device=cuda).manual_seed(9)
    wt = (torch.randn(N, K, generator=g, device=cuda) * 0.02).half()
    a = torch.randn(M, K, generator=g, device=cuda).half()

    def gemm(q, ws):
        c = torch.full((M, N), float("nan"), dtype=torch.float16, device=cuda)
        ok = lib().feather_launch_scaled_mm_ws(a.data_ptr(), q[0].data_ptr(), q[1].data_ptr(), None, c.data_ptr(),
                                               M, N, K, 1, 0, *cfg, 1, 0, ws.data_ptr(), ws.numel(), stream(cuda))
        assert ok
        torch.cuda.synchronize()
        return c

    q_ref = _run(wt, None, 1, one_pass=False)
    c_ref = gemm(q_ref, torch.zeros(need, dtype=torch.uint8, device=cuda))
    ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
    for rep in range(2):
        q = _run(wt, None, 1, ws)
        _same(q, q_ref, f"quantize after GEMM, rep {rep}")
        assert torch.equal(gemm(q, ws), c_ref), f"GEMM after quantize, rep {rep}"
    assert (ws[:65536] == 0).all()
