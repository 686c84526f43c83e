"""GPU bit-exactness of quantize/prepack, the layout kernels, dequantize and
the bf16 -> fp16 cast against the oracle and the golden fixtures."""

import hashlib

import importlib

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from gpu_util import lib, stream
from oracle import feather_oracle as O

pytestmark = pytest.mark.gpu

ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _bytes(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).cpu().numpy()


def test_config1_golden_all_paths(cuda, quant):
    q = np.load(GOLDEN / "quant_c1.npz")
    g = torch.Generator().manual_seed(0)
    w32 = torch.randn(1024, 1024, generator=g) * 0.02
    cases = {
        "load_f16": lambda: quant.make_feather_quantized_weight(w32.half().to(cuda), None, torch.float16),
        "load_f32": lambda: quant.make_feather_quantized_weight(w32.to(cuda), None, torch.float32),
        "native_f16": lambda: quant.quantize_feather_weight(w32.half().to(cuda)),
        "native_bf16": lambda: quant.quantize_feather_weight(w32.bfloat16().to(cuda)),
    }
    for name, fn in cases.items():
        qt = fn()
        qdata, scale = quant.get_feather_plain_tensors(qt)
        assert qdata.shape == (64, 1024, 16) and qdata.dtype == torch.float8_e5m2
        assert np.float32(scale.item()) == q[f"{name}_scale"][0], name
        assert hashlib.sha256(_bytes(qdata).tobytes()).digest() == q[f"{name}_sha256"].tobytes(), name


def test_exhaustive_fp16_bf16_encode(cuda, quant):
    z = np.load(GOLDEN / "e5m2_codes.npz")
    x16 = torch.from_numpy(ALL16.view(np.int16).copy()).view(torch.float16).to(cuda)
    q, s = quant.quantize_fp8e5m2_scaled(x16, scale=1.0)
    assert np.array_equal(_bytes(q), z["from_fp16"])
    # bf16: x * bf16(1/1) is rounded to bf16 first, which makes every NaN the
    # canonical positive NaN (as c10's float -> bfloat16 does); compare the rest
    xbf = torch.from_numpy(ALL16.view(np.int16).copy()).view(torch.bfloat16).to(cuda)
    q, s = quant.quantize_fp8e5m2_scaled(xbf, scale=1.0)
    nan = np.isnan(O.bf16_bits_to_f32(ALL16))
    got = _bytes(q)
    assert np.array_equal(got[~nan], z["from_bf16"][~nan])
    assert np.all((got[nan] & 0x7F) == 0x7F)


def test_fp32_boundaries_and_scales(cuda, quant):
    vals = np.unique(np.abs(O.E5M2_TABLE[np.isfinite(O.E5M2_TABLE)]))
    mids = (vals[1:] + vals[:-1]) / 2
    pts = np.concatenate([vals, mids, [61440.0, 65536.0]]).astype(np.float32)
    bits = (pts.view(np.uint32)[:, None].astype(np.int64) + np.arange(-8, 9)[None, :]).reshape(-1)
    x = np.concatenate([bits.astype(np.uint32).view(np.float32), -bits.astype(np.uint32).view(np.float32)])
    x = x[: len(x) // 16 * 16].reshape(16, -1)
    for scale in (1.0, 0.37, 3.0e-5):
        q, _ = quant.quantize_fp8e5m2_scaled(torch.from_numpy(x).to(cuda), scale=scale)
        ref, _ = O.quantize_native(x, O.DT_F32, scale=scale)
        assert np.array_equal(_bytes(q), ref), scale


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape,std", [((48, 64), 1.0), ((3072, 3072), 0.02), ((7, 1000), 5.0)])
def test_quantize_native_vs_oracle(cuda, quant, dtype, shape, std):
    g = torch.Generator().manual_seed(shape[0])
    x = (torch.randn(*shape, generator=g) * std).to(dtype)
    q, s = quant.quantize_fp8e5m2_scaled(x.to(cuda))
    if dtype == torch.bfloat16:
        xin, dt = x.view(torch.int16).numpy().view(np.uint16), O.DT_BF16
    else:
        xin, dt = x.numpy(), {torch.float16: O.DT_F16, torch.float32: O.DT_F32}[dtype]
    codes, s_ref = O.quantize_native(xin, dt)
    assert np.float32(s.item()) == s_ref
    assert q.shape == x.shape and np.array_equal(_bytes(q).reshape(shape), codes)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_load_path_with_checkpoint_scale(cuda, quant, dtype):
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(256, 512, generator=g) * 0.5).to(dtype)
    ck = torch.tensor(0.73)
    qt = quant.make_feather_quantized_weight(w.to(cuda), ck.to(cuda), torch.bfloat16)
    qdata, scale = quant.get_feather_plain_tensors(qt)
    w32 = w.float().numpy()
    codes, s_ref = O.quantize_load(w32, O.DT_F32, ckpt_scale=np.float32(0.73))
    assert np.float32(scale.item()) == s_ref
    assert np.array_equal(_bytes(qdata), O.prepack_transpose(codes))


@pytest.mark.parametrize("ck", [-0.73, 0.0, float("inf"), 1e-30, 1.0e38])
def test_load_path_checkpoint_scale_edge_values(cuda, quant, ck):
    """amax is max|w| times |ckpt_scale| once per workgroup for a finite scale and
    per element otherwise; both must equal amax(|float32(w) * ckpt_scale|)."""
    g = torch.Generator().manual_seed(5)
    w = (torch.randn(128, 256, generator=g) * 0.5).half()
    w[0, :7] = 0.0  # zeros make inf * 0 = NaN for an infinite scale
    qt = quant.make_feather_quantized_weight(w.to(cuda), torch.tensor(ck).to(cuda), torch.float16)
    qdata, scale = quant.get_feather_plain_tensors(qt)
    codes, s_ref = O.quantize_load(w.float().numpy(), O.DT_F32, ckpt_scale=np.float32(ck))
    s_gpu = np.float32(scale.item())
    if np.isnan(s_ref):
        assert np.isnan(s_gpu)
    else:
        assert s_gpu == s_ref
        assert np.array_equal(_bytes(qdata), O.prepack_transpose(codes))


def test_special_inputs(cuda, quant):
    z = torch.zeros(32, 64, dtype=torch.float16, device=cuda)
    q, s = quant.quantize_fp8e5m2_scaled(z)
    assert s.item() == 1.0 and (_bytes(q) == 0).all()
    w = torch.randn(32, 64, dtype=torch.float16)
    w[3, 4] = float("nan")
    q, s = quant.quantize_fp8e5m2_scaled(w.to(cuda))
    assert np.isnan(s.item())
    # a CPU weight is processed on the GPU and returned on the CPU, identical bits
    w = torch.randn(64, 128, dtype=torch.bfloat16)
    qc = quant.quantize_feather_weight(w)
    qg = quant.quantize_feather_weight(w.to(cuda))
    assert qc._qdata.device.type == "cpu"
    assert np.array_equal(_bytes(qc._qdata), _bytes(qg._qdata))
    with pytest.raises(ValueError):
        quant.FeatherFP8E5M2PackedLayout.quantize(torch.randn(16, 24, device=cuda))
    with pytest.raises(ValueError):
        quant.FeatherFP8E5M2PackedLayout.quantize(torch.randn(16, device=cuda))


@pytest.mark.parametrize("N,K", [(1, 16), (5, 48), (64, 64), (63, 4112), (1000, 272), (3072, 3072)])
def test_layout_kernels(cuda, quant, hk, N, K):
    rng = np.random.default_rng(N + K)
    w = rng.integers(0, 256, (N, K), dtype=np.uint8)
    wt = torch.from_numpy(w).view(torch.float8_e5m2).to(cuda)
    p = quant.prepack_transpose(wt)
    assert np.array_equal(_bytes(p), O.prepack_transpose(w))
    assert np.array_equal(_bytes(quant.unprepack_transpose(p)), w)
    b = np.ascontiguousarray(w.T)  # (K, N); N % 4 != 0 takes the byte path
    pb = hk.prepack_b_for_scaled_mm(torch.from_numpy(b).view(torch.float8_e5m2).to(cuda))
    assert np.array_equal(_bytes(pb), O.prepack_kn(b))


@pytest.mark.parametrize("dtype,code", [(torch.float16, O.DT_F16), (torch.bfloat16, O.DT_BF16),
                                        (torch.float32, O.DT_F32)])
@pytest.mark.parametrize("N,K", [(96, 160), (1, 16), (63, 272), (130, 4112), (640, 2048)])
def test_dequantize(cuda, quant, dtype, code, N, K):
    """Every code value, ragged row blocks (N % 64) and K blocks (K % 256) of the block-wise kernel."""
    rng = np.random.default_rng(3 + N + K)
    codes = rng.integers(0, 256, (N, K), dtype=np.uint8)
    codes.reshape(-1)[:256] = np.arange(256, dtype=np.uint8)[: codes.size]
    packed = torch.from_numpy(O.prepack_transpose(codes)).view(torch.float8_e5m2).to(cuda)
    params = quant.FeatherFP8E5M2PackedParams(scale=torch.tensor(0.0123, device=cuda), orig_dtype=dtype,
                                              orig_shape=(N, K))
    out = quant.FeatherFP8E5M2PackedLayout.dequantize(packed, params)
    ref = O.dequantize(codes, np.float32(0.0123), code)
    got = out.cpu()
    if dtype == torch.bfloat16:
        got_bits = got.view(torch.int16).numpy().view(np.uint16)
        fin = ~np.isnan(O.bf16_bits_to_f32(ref))
        assert np.array_equal(got_bits[fin], ref[fin])
    else:
        g = got.numpy()
        assert np.array_equal(np.isnan(g), np.isnan(ref))
        assert np.array_equal(g[~np.isnan(g)], ref[~np.isnan(ref)])
        # signed zeros too: code 0x80 is -0 and must dequantize to -0
        assert np.array_equal(np.signbit(g[~np.isnan(g)]), np.signbit(ref[~np.isnan(ref)]))
        assert np.signbit(g[codes == 0x80]).all() and (codes == 0x80).any() or codes.size < 129
    sd = quant.FeatherFP8E5M2PackedLayout.state_dict_tensors(packed, params)
    assert np.array_equal(_bytes(sd[""]), codes)


def test_bf16_to_fp16_exhaustive(cuda, pkg):
    from featherops_amd.kernel import convert

    z = np.load(GOLDEN / "bf16_rtz.npz")["fp16_bits"]
    x = torch.from_numpy(ALL16.view(np.int16).copy()).view(torch.bfloat16).to(cuda)
    y = convert.bf16_to_fp16(x).view(torch.int16).cpu().numpy().view(np.uint16)
    nan = np.isnan(z.view(np.float16))
    assert np.array_equal(y[~nan], z[~nan])
    assert np.isnan(y[nan].view(np.float16)).all()
    # reference test_convert.py: 1024^2 randn vs torch's cast, max diff < 1e-5
    xr = torch.randn(1024, 1024, dtype=torch.bfloat16, device=cuda)
    assert (convert.bf16_to_fp16(xr).float() - xr.to(torch.float16).float()).abs().max().item() < 1e-5
    # odd element counts through the C ABI (the tail path)
    for n in (1, 7, 9, 1023):
        xs = x[:n].contiguous()
        out = torch.empty(n, dtype=torch.float16, device=cuda)
        assert lib().feather_bf16_to_fp16(xs.data_ptr(), out.data_ptr(), n, stream(cuda)) == 0
        torch.cuda.synchronize()
        o = out.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(o[~nan[:n]], z[:n][~nan[:n]])


def test_bf16_to_fp16_rne_exhaustive(cuda, pkg):
    """Round-to-nearest cast (the any-M entry's stand-in for ops.py:88's
    x.to(float16)): all 65,536 bf16 patterns equal torch's CPU cast (NaN -> NaN),
    plus a large array (4 loads in flight per thread) and odd tails."""
    x_cpu = torch.from_numpy(ALL16.view(np.int16).copy()).view(torch.bfloat16)
    want = x_cpu.to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(want.view(np.float16))
    for n in (65536, 1, 7, 9, 1023):
        xs = x_cpu[:n].to(cuda)
        out = torch.empty(n, dtype=torch.float16, device=cuda)
        assert lib().feather_bf16_to_fp16_rne(xs.data_ptr(), out.data_ptr(), n, stream(cuda)) == 0
        torch.cuda.synchronize()
        o = out.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(o[~nan[:n]], want[:n][~nan[:n]]), n
        assert np.isnan(o[nan[:n]].view(np.float16)).all()
    xr = torch.randn(3, 1 << 20, dtype=torch.bfloat16, device=cuda) * 3000
    out = torch.empty(xr.shape, dtype=torch.float16, device=cuda)
    assert lib().feather_bf16_to_fp16_rne(xr.data_ptr(), out.data_ptr(), xr.numel(), stream(cuda)) == 0
    assert torch.equal(out, xr.to(torch.float16))
    # the Python entry (kernel.convert.bf16_to_fp16_rne), odd length and 2-D shape kept
    conv = importlib.import_module(f"{pkg.__name__}.kernel.convert")
    for shape in ((65536,), (3, 7), (1000, 999)):
        x = (torch.randn(shape, dtype=torch.float32) * 3e4).bfloat16().to(cuda)
        y = conv.bf16_to_fp16_rne(x)
        assert y.shape == x.shape and y.dtype == torch.float16
        assert torch.equal(y.view(torch.int16), x.to(torch.float16).view(torch.int16)), shape


def test_bf16_to_fp16_large_streaming_path(cuda):
    """Inputs of 64 Mi elements and more take the cast's nontemporal-access variant: RNE equals
    torch's cast, RTZ equals the same data cast in pieces below that size (the ordinary
    variant, itself pinned exhaustively above); the element count is odd (tail path)."""
    n = (64 << 20) + 7
    x = torch.randn(n, dtype=torch.bfloat16, device=cuda) * 3000
    out = torch.empty(n, dtype=torch.float16, device=cuda)
    assert lib().feather_bf16_to_fp16_rne(x.data_ptr(), out.data_ptr(), n, stream(cuda)) == 0
    assert torch.equal(out, x.to(torch.float16))
    assert lib().feather_bf16_to_fp16(x.data_ptr(), out.data_ptr(), n, stream(cuda)) == 0
    pieces = torch.empty_like(out)
    step = 1 << 24
    for o in range(0, n, step):
        m = min(step, n - o)
        assert lib().feather_bf16_to_fp16(x[o:].data_ptr(), pieces[o:].data_ptr(), m, stream(cuda)) == 0
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), pieces.view(torch.int16))


def test_config5_weight_on_device(cuda, quant):
    """Config 5 quantizes 5120x13824 weights on the device: sampled rows vs the oracle."""
    gd = torch.Generator(device=cuda).manual_seed(5)
    w = (torch.randn(13824, 5120, generator=gd, device=cuda) * 0.02).half()
    qt = quant.make_feather_quantized_weight(w, None, torch.float16)
    qdata, scale = quant.get_feather_plain_tensors(qt)
    amax = w.abs().max().float().item()
    assert np.float32(scale.item()) == np.float32(amax) / np.float32(57344.0)
    rows = torch.tensor([0, 1, 4095, 7777, 13823], device=cuda)
    codes_nk = quant.unprepack_transpose(qdata)[rows]
    ref = O.e5m2_encode(w[rows].float().cpu().numpy() * (np.float32(1.0) / np.float32(scale.item())))
    assert np.array_equal(_bytes(codes_nk), ref)


def test_capi_quantize_workspace_reused_across_shapes(cuda):
    """feather_quantize_prepack_e5m2 through the C ABI with one 1 KB workspace
    reused across weights of different sizes (different numbers of partial
    maxima): codes and scale bit-exact against the oracle each time."""
    ws = torch.full((256,), -1, dtype=torch.int32, device=cuda)  # garbage: no clearing needed
    for i, (N, K) in enumerate([(4096, 4096), (7, 48), (3072, 1024), (1, 16), (640, 2048)]):
        g = torch.Generator().manual_seed(40 + i)
        w = (torch.randn(N, K, generator=g) * 0.05).half()
        out = torch.empty(K // 16, N, 16, dtype=torch.uint8, device=cuda)
        scale = torch.empty((), dtype=torch.float32, device=cuda)
        wd = w.to(cuda)
        st = lib().feather_quantize_prepack_e5m2(wd.data_ptr(), 0, N, K, None, 1, out.data_ptr(), scale.data_ptr(),
                                                 ws.data_ptr(), stream(cuda))
        assert st == 0
        torch.cuda.synchronize()
        codes, s_ref = O.quantize_native(w.numpy(), O.DT_F16)
        assert np.float32(scale.item()) == s_ref, f"{N}x{K}"
        assert np.array_equal(O.unprepack_transpose(out.cpu().numpy()), codes), f"{N}x{K}"


@pytest.mark.parametrize("with_scale", [False, True])
def test_load_path_e5m2_checkpoint(cuda, quant, with_scale):
    """An e5m2 checkpoint is only prepacked (reference quant.py:120-126): the codes pass through
    unchanged, the scale is the checkpoint's weight_scale as fp32, or 1 when there is none."""
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(384, 512, generator=g) * 3.0).to(torch.float8_e5m2)
    codes = w.view(torch.uint8).numpy()
    ck = torch.tensor(0.0123, dtype=torch.bfloat16) if with_scale else None
    qt = quant.make_feather_quantized_weight(w.to(cuda), None if ck is None else ck.to(cuda), torch.bfloat16)
    qdata, scale = quant.get_feather_plain_tensors(qt)
    assert qdata.dtype == torch.float8_e5m2 and qdata.shape == (32, 384, 16) and qdata.device == cuda
    assert np.array_equal(_bytes(qdata), O.prepack_transpose(codes))
    assert scale.dtype == torch.float32 and scale.device == cuda
    assert scale.item() == (np.float32(ck.float().item()) if with_scale else 1.0)
    assert qt.params.orig_dtype == torch.bfloat16 and qt.params.orig_shape == (384, 512)
    # the layout's dequantize undoes it: code value times the scale, in orig_dtype
    deq = qt.dequantize()
    ref = O.dequantize(codes, np.float32(scale.item()), O.DT_BF16)
    assert np.array_equal(deq.view(torch.int16).cpu().numpy().view(np.uint16), ref)
