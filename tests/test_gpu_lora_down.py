"""GPU parity of the LoRA down-projection kernel (feather_lora_down, T = x . D^T) against the
oracle's lora_down_ref, through the C ABI and the torch op, and against torch's F.linear (what
the reference's comfy_feather/lora.py:27 computes) within the GEMM gate."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gpu_util import assert_gemm_close, assert_gemm_close_dev, lib, stream
from oracle import feather_oracle as O

pytestmark = pytest.mark.gpu


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    return t.numpy() if t.dtype == torch.float16 else t.view(torch.int16).numpy().view(np.uint16)


def _capi(x, d, split=True):
    """feather_lora_down through the C ABI; split=False passes no workspace (unsplit K)."""
    M, K = x.shape
    R = d.shape[0]
    nbytes = lib().feather_lora_down_workspace_size(M, K, R) if split else 0
    ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=x.device)
    t = torch.full((M, R), float("nan"), dtype=x.dtype, device=x.device)
    st = lib().feather_lora_down(x.data_ptr(), 0 if x.dtype == torch.float16 else 1, d.data_ptr(), t.data_ptr(),
                                 M, K, R, ws.data_ptr() if nbytes else None, nbytes, stream(x.device))
    assert st == 0, lib().feather_status_string(st)
    torch.cuda.synchronize()
    if nbytes:
        assert (ws[:65536] == 0).all(), "arrival counters must be left at zero"
    return t


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K,R", [(1, 8, 32), (17, 24, 64), (300, 1040, 96), (256, 3072, 128), (40, 520, 160),
                                   (129, 2048, 256), (8200, 64, 32), (4096, 3072, 64),
                                   (1, 4160, 32), (1, 520, 32), (70, 4160, 128)])
def test_lora_down_vs_oracle(cuda, hk, dtype, M, K, R):
    g = torch.Generator().manual_seed(M + K + R)
    x = torch.randn(M, K, generator=g).to(dtype)
    d = (torch.randn(R, K, generator=g) * 0.05).to(dtype)
    od = O.DT_F16 if dtype == torch.float16 else O.DT_BF16
    print("lora_down", M, K, R, dtype, flush=True)
    t = _capi(x.to(cuda), d.to(cuda))
    ref = O.lora_down_ref(_np(x), _np(d), od)
    assert_gemm_close(t, ref, dtype, f"T {M}x{K}x{R}")
    # deterministic: the same bits again
    assert torch.equal(t.view(torch.int16), _capi(x.to(cuda), d.to(cuda)).view(torch.int16))
    # without a workspace (no K split across workgroups): the same gate
    assert_gemm_close(_capi(x.to(cuda), d.to(cuda), split=False), ref, dtype, f"T unsplit {M}x{K}x{R}")
    # the torch op and the library's Python entry agree with the C ABI
    t2 = torch.ops.feather_ops.lora_down.default(x.to(cuda), d.to(cuda))
    assert torch.equal(t.view(torch.int16), t2.view(torch.int16))


def test_lora_down_special_values_and_refusals(cuda, hk):
    M, K, R = 64, 256, 32
    x = torch.zeros(M, K, dtype=torch.float16)
    x[0, 0] = float("inf")
    x[1, 3] = float("nan")
    x[2, :] = 60000.0
    d = torch.zeros(R, K, dtype=torch.float16)
    d[:, 0] = 1.0
    d[5, :] = 1.0
    t = _capi(x.to(cuda), d.to(cuda))
    ref = O.lora_down_ref(x.numpy(), d.numpy(), O.DT_F16)
    assert_gemm_close(t, ref, torch.float16, "special")
    L = lib()
    xd, dd = x.to(cuda), d.to(cuda)
    tt = torch.empty(M, R, dtype=torch.float16, device=cuda)
    s = stream(cuda)
    args = (None, 0, s)
    assert L.feather_lora_down(xd.data_ptr(), 0, dd.data_ptr(), tt.data_ptr(), M, K, 48, *args) == 2  # R % 32
    assert L.feather_lora_down(xd.data_ptr(), 0, dd.data_ptr(), tt.data_ptr(), M, 250, R, *args) == 2  # K % 8
    assert L.feather_lora_down(xd.data_ptr(), 5, dd.data_ptr(), tt.data_ptr(), M, K, R, *args) == 1  # dtype
    assert L.feather_lora_down(xd.data_ptr() + 2, 0, dd.data_ptr(), tt.data_ptr(), M, K, R, *args) == 1  # alignment
    with pytest.raises(RuntimeError):
        torch.ops.feather_ops.lora_down.default(xd, dd[:, :250].contiguous())


@pytest.mark.parametrize("M,K,R", [(4096, 12288, 64), (32768, 5120, 128)])
def test_lora_down_full_size_vs_torch_linear(cuda, hk, M, K, R):
    """Image-/video-DiT sizes: the whole T against a float64 evaluation on the device and
    against torch's F.linear (hipBLASLt, fp32 accumulation) within the same gate."""
    gd = torch.Generator(device=cuda).manual_seed(M + R)
    x = torch.randn(M, K, generator=gd, device=cuda).bfloat16()
    d = (torch.randn(R, K, generator=gd, device=cuda) * 0.02).bfloat16()
    t = torch.ops.feather_ops.lora_down.default(x, d)
    ref = (x.double() @ d.double().t()).float().bfloat16()
    assert_gemm_close_dev(t, ref, torch.bfloat16, f"T {M}x{K}x{R} vs float64")
    assert_gemm_close_dev(t, F.linear(x, d), torch.bfloat16, f"T {M}x{K}x{R} vs F.linear")


def test_lora_down_workspace_shared_across_shapes(cuda, hk):
    """One zeroed workspace serves K-split calls of different shapes in sequence (fewer tiles
    before more), each against the oracle: the counters come back to zero every call."""
    seq = [(64, 3072, 32), (4096, 3072, 64), (1000, 1024, 128), (4096, 12288, 96), (64, 3072, 32), (2000, 4096, 256)]
    need = max(lib().feather_lora_down_workspace_size(M, K, R) for M, K, R in seq)
    ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
    for i, (M, K, R) in enumerate(seq):
        assert lib().feather_lora_down_workspace_size(M, K, R) > 0, "every shape here splits K"
        g = torch.Generator().manual_seed(50 + i)
        x = torch.randn(M, K, generator=g).bfloat16()
        d = (torch.randn(R, K, generator=g) * 0.05).bfloat16()
        xd, dd = x.to(cuda), d.to(cuda)
        t = torch.empty(M, R, dtype=torch.bfloat16, device=cuda)
        st = lib().feather_lora_down(xd.data_ptr(), 1, dd.data_ptr(), t.data_ptr(), M, K, R, ws.data_ptr(), need,
                                     stream(cuda))
        assert st == 0
        torch.cuda.synchronize()
        assert_gemm_close(t, O.lora_down_ref(_np(x), _np(d), O.DT_BF16), torch.bfloat16, f"ws {M}x{K}x{R}")
    assert (ws[:65536] == 0).all()


def test_lora_down_graph_replays_match_eager(cuda, hk):
    """The down-projection (with its K split across workgroups) captured in a HIP graph:
    every replay, with eager work in between, equals the eager result."""
    g = torch.Generator(device=cuda).manual_seed(12)
    x = torch.randn(4096, 3072, generator=g, device=cuda).bfloat16()
    d = (torch.randn(64, 3072, generator=g, device=cuda) * 0.05).bfloat16()
    op = torch.ops.feather_ops.lora_down.default
    eager = op(x, d)
    out = torch.empty_like(eager)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out.copy_(op(x, d))
    for rep in range(4):
        out.zero_()
        graph.replay()
        junk = torch.randn(1 << 16, device=cuda).sum()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
        assert torch.isfinite(junk)


def test_lora_down_python_entry_falls_back_on_misaligned_x(cuda, hk, pkg):
    """comfy_feather.lora.lora_down takes torch's F.linear where the kernel's entry would refuse
    the operands (here: x at a storage offset of one element, off the 16-byte boundary) instead
    of raising; aligned x goes to the kernel and agrees with the oracle."""
    from featherops_amd.comfy_feather import lora

    M, K, R = 33, 256, 32
    g = torch.Generator().manual_seed(7)
    buf = torch.randn(M * K + 1, generator=g).half().to(cuda)
    d = (torch.randn(R, K, generator=g) * 0.05).half().to(cuda)
    x_off = buf[1:].view(M, K)
    assert x_off.data_ptr() % 16 != 0
    t_off = lora.lora_down(x_off, d)
    assert torch.equal(t_off, F.linear(x_off, d).contiguous())
    x_al = x_off.clone()
    t_al = lora.lora_down(x_al, d)
    assert_gemm_close(t_al, O.lora_down_ref(_np(x_al), _np(d), O.DT_F16), torch.float16, "aligned x")
