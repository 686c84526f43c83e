"""The allocation-free GEMM entry (feather_launch_scaled_mm_noalloc): through the C ABI its
output equals feather_launch_scaled_mm_ex's with a caller workspace, bit for bit, on calls in
a row that share the static scratch array (each sequence's second call is smaller); shapes
whose K split needs no scratch and the rejection paths are covered too."""

import subprocess
import sys

import numpy as np
import pytest
import torch

from conftest import REPO
from gpu_util import lib, stream, to_dev_codes, weight_like

FEATHER_OK, FEATHER_ERR_UNSUPPORTED, FEATHER_ERR_SCRATCH = 0, 2, 4


def _operands(M, N, K, seed, cuda, a_dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g).to(a_dtype).to(cuda)
    packed, s = weight_like(N, K, g)
    bias = (torch.randn(N, generator=g) * 0.01).half().to(cuda)
    return a, to_dev_codes(packed, cuda), torch.tensor([s], device=cuda), bias


def _run_ex(a, bd, sd, bias, M, N, K, cfg, a_code):
    nbytes = lib().feather_scaled_mm_workspace_size(M, N, K, *cfg)
    ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=a.device)
    c = torch.full((M, N), float("nan"), dtype=torch.float16, device=a.device)
    ok = lib().feather_launch_scaled_mm_ex(a.data_ptr(), a_code, bd.data_ptr(), sd.data_ptr(), bias.data_ptr(),
                                           c.data_ptr(), M, N, K, 1, 1, *cfg, 1, 0, ws.data_ptr(), nbytes,
                                           stream(a.device))
    assert ok
    torch.cuda.synchronize()
    return c, nbytes


def _run_noalloc(a, bd, sd, bias, M, N, K, cfg, a_code):
    c = torch.full((M, N), float("nan"), dtype=torch.float16, device=a.device)
    st = lib().feather_launch_scaled_mm_noalloc(a.data_ptr(), a_code, bd.data_ptr(), sd.data_ptr(), bias.data_ptr(),
                                                c.data_ptr(), M, N, K, 1, 1, *cfg, 1, 0, stream(a.device))
    assert st == FEATHER_OK, lib().feather_status_string(st)
    torch.cuda.synchronize()
    return c


SEQUENCES = [
    # small-M kernel with a K split across workgroups, then a smaller one
    [(16, 5120, 13824, (1, 1, 2, 1, 2)), (8, 2048, 12288, (1, 1, 2, 1, 2))],
    # split-K LDS tiles (64 x 64 and 32 x 128), then smaller
    [(64, 4096, 4096, (2, 2, 4, 4, 4)), (48, 1024, 1024, (2, 2, 4, 4, 4))],
    [(256, 3072, 3072, (2, 2, 4, 4, 4)), (128, 1024, 1024, (2, 2, 4, 4, 4))],
    # no split needed (large tiles), then a split-K shape
    [(512, 2048, 1024, (2, 4, 4, 8, 4)), (16, 2048, 12288, (1, 1, 2, 1, 2))],
]


@pytest.mark.gpu
@pytest.mark.parametrize("seq", range(len(SEQUENCES)))
def test_noalloc_matches_workspace_entry(cuda, seq):
    for i, (M, N, K, cfg) in enumerate(SEQUENCES[seq]):
        print("noalloc", seq, i, M, N, K, cfg, flush=True)
        a, bd, sd, bias = _operands(M, N, K, 100 * seq + i, cuda)
        ref, nbytes = _run_ex(a, bd, sd, bias, M, N, K, cfg, 0)
        assert nbytes <= 16 << 20
        got = _run_noalloc(a, bd, sd, bias, M, N, K, cfg, 0)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"{M}x{N}x{K}"
        # again on the same scratch: the counters were left at zero
        assert torch.equal(_run_noalloc(a, bd, sd, bias, M, N, K, cfg, 0).view(torch.int16), ref.view(torch.int16))


@pytest.mark.gpu
def test_noalloc_bf16_activations_and_refusals(cuda):
    M, N, K = 16, 4096, 8192
    a, bd, sd, bias = _operands(M, N, K, 7, cuda, torch.bfloat16)
    cfg = (1, 1, 2, 1, 2)
    ref, _ = _run_ex(a, bd, sd, bias, M, N, K, cfg, 1)
    assert torch.equal(_run_noalloc(a, bd, sd, bias, M, N, K, cfg, 1).view(torch.int16), ref.view(torch.int16))
    L = lib()
    # unknown tuple: nothing launched
    assert L.feather_launch_scaled_mm_noalloc(a.data_ptr(), 1, bd.data_ptr(), sd.data_ptr(), bias.data_ptr(),
                                              a.data_ptr(), M, N, K, 1, 1, 3, 3, 3, 3, 3, 1, 0,
                                              stream(cuda)) == FEATHER_ERR_UNSUPPORTED


def test_noalloc_rejects_a_split_larger_than_the_array():
    """With a workgroup target far above the default the K split needs more than 16 MiB:
    refused with FEATHER_ERR_SCRATCH before any HIP call (runs without a GPU, in a fresh process
    because the target is read once)."""
    code = ("import __graft_entry__; __graft_entry__.load_package();"
            "from featherops_amd.kernel.hip import _lib; L = _lib.lib();"
            "need = L.feather_scaled_mm_workspace_size(64, 8192, 8192, 2, 2, 4, 4, 4);"
            "st = L.feather_launch_scaled_mm_noalloc(None, 0, None, None, None, None, 64, 8192, 8192, 1, 1,"
            " 2, 2, 4, 4, 4, 1, 0, None);"
            "print(need, st, L.feather_status_string(st).decode())")
    env = dict(__import__("os").environ, FEATHEROPS_SMALLM_GROUPS="4096")
    out = subprocess.run([sys.executable, "-c", code], cwd=REPO, env=env, capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr
    need, st, msg = out.stdout.split(maxsplit=2)
    assert int(need) > 16 << 20 and int(st) == FEATHER_ERR_SCRATCH and "scratch" in msg


@pytest.mark.gpu
def test_noalloc_under_graph_capture(cuda):
    """The entry's use case: calls captured in a HIP graph (no allocation during capture) and
    replayed, with eager work between replays; every replay equals the eager workspace entry."""
    shapes = [(16, 5120, 13824, (1, 1, 2, 1, 2)), (64, 4096, 4096, (2, 2, 4, 4, 4))]
    ops = []
    for i, (M, N, K, cfg) in enumerate(shapes):
        a, bd, sd, bias = _operands(M, N, K, 300 + i, cuda)
        ref, _ = _run_ex(a, bd, sd, bias, M, N, K, cfg, 0)
        _run_noalloc(a, bd, sd, bias, M, N, K, cfg, 0)  # set-up call (symbol address) before capture
        out = torch.empty(M, N, dtype=torch.float16, device=cuda)
        ops.append((a, bd, sd, bias, out, ref, M, N, K, cfg))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        s = torch.cuda.current_stream().cuda_stream
        for a, bd, sd, bias, out, _, M, N, K, cfg in ops:
            st = lib().feather_launch_scaled_mm_noalloc(a.data_ptr(), 0, bd.data_ptr(), sd.data_ptr(), bias.data_ptr(),
                                                        out.data_ptr(), M, N, K, 1, 1, *cfg, 1, 0, s)
            assert st == FEATHER_OK
    for rep in range(4):
        for op in ops:
            op[4].zero_()
        graph.replay()
        junk = torch.randn(1 << 16, device=cuda).sum()  # eager work between replays
        torch.cuda.synchronize()
        for op in ops:
            assert torch.equal(op[4].view(torch.int16), op[5].view(torch.int16)), f"replay {rep} {op[6:9]}"
        assert torch.isfinite(junk)
