"""CPU tests of the host side: the C-ABI library loads and exports every
declared symbol, argument validation fails the way the reference's op does,
and config/autotune helpers keep the reference's semantics. No kernel runs."""

import re

import pytest
import torch

from conftest import REPO


def _declared_functions():
    text = (REPO / "include" / "featherops_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*([a-z_0-9]+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol(pkg):
    from featherops_amd.kernel.hip import _lib

    L = _lib.lib()
    names = _declared_functions()
    assert "launch_scaled_mm" in names and len(names) >= 10
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must cover the header exactly"
    assert L.feather_abi_version() == 1
    assert L.feather_status_string(1) == b"invalid argument"


def test_capi_rejects_without_launching(pkg):
    from featherops_amd.kernel.hip import _lib

    L = _lib.lib()
    # unknown config tuple -> false before any HIP call (reference hip_kernel.cu:631)
    assert not L.launch_scaled_mm(None, None, None, None, None, 256, 256, 256, 0, 0, 3, 3, 3, 3, 3, 1, 0, None)
    # N not a multiple of 16
    assert not L.launch_scaled_mm(None, None, None, None, None, 256, 250, 256, 0, 0, 1, 1, 2, 1, 2, 1, 0, None)
    # bad dtypes
    assert not L.launch_scaled_mm(None, None, None, None, None, 256, 256, 256, 0, 0, 1, 1, 2, 1, 2, 7, 0, None)
    assert not L.launch_scaled_mm(None, None, None, None, None, 256, 256, 256, 0, 0, 1, 1, 2, 1, 2, 1, 5, None)
    assert L.feather_prepack_transpose(None, None, 16, 16, None) == 1
    assert L.feather_quantize_prepack_e5m2(None, 0, 16, 16, None, 0, None, None, None, None) == 1
    assert L.feather_bf16_to_fp16(None, None, -1, None) == 1
    assert L.feather_bf16_to_fp16(None, None, 0, None) == 0
    assert L.feather_dequantize_e5m2(None, None, None, 0, 16, 16, None) == 1


def test_kernel_id_mapping(hk):
    assert hk.kernel_id(32768, 13824, 5120, (2, 4, 4, 8, 4)) == 20  # 256x256 LDS-DMA pipeline
    assert hk.kernel_id(32768, 13824, 5120, (4, 2, 4, 4, 8)) == 20  # the same tile and kernel
    assert hk.kernel_id(32768, 13824, 5136, (2, 4, 4, 8, 4)) == 1  # K % 64 != 0: register-staged tile
    assert hk.kernel_id(16, 4096, 4096, (1, 1, 2, 1, 2)) == 10  # small-M
    assert hk.kernel_id(40, 2048, 2048, (1, 8, 4, 8, 2)) == 10
    assert hk.kernel_id(40, 1024, 8192, (1, 8, 4, 8, 2)) == 10
    assert hk.kernel_id(24, 4096, 4096, (1, 8, 4, 8, 2)) == 10
    assert hk.kernel_id(16, 13824, 5120, (1, 8, 4, 8, 2)) == 10
    # split-K LDS tiles: M > 48; 32 < M <= 48 with N >= 3072 or a weight of at least 4096 x 4096;
    # 16 < M <= 32 with a larger one (32 x 128 tiles); larger M when the grid fits one round
    assert hk.kernel_id(64, 4096, 4096, (1, 8, 4, 8, 2)) == 30
    assert hk.kernel_id(40, 4096, 4096, (1, 8, 4, 8, 2)) == 30
    assert hk.kernel_id(33, 3072, 3072, (1, 8, 4, 8, 2)) == 30
    assert hk.kernel_id(24, 5120, 5120, (1, 8, 4, 8, 2)) == 34
    assert hk.kernel_id(24, 2800, 9984, (1, 8, 4, 8, 2)) == 34  # the small-M plan would split K
    assert hk.kernel_id(24, 3280, 6016, (1, 8, 4, 8, 2)) == 10  # unsplit, one round of strips
    assert hk.kernel_id(40, 13824, 5120, (1, 1, 2, 1, 2)) == 30
    assert hk.kernel_id(256, 3072, 3072, (2, 4, 4, 8, 4)) == 30
    # 64 x 128 split-K tiles where 64 x 64 ones would overfill the grid
    assert hk.kernel_id(512, 3072, 12288, (2, 2, 4, 4, 4)) == 31
    assert hk.kernel_id(128, 5120, 5120, (2, 2, 4, 4, 4)) == 31
    assert hk.kernel_id(768, 3072, 3072, (2, 2, 4, 4, 4)) == 24
    # M > 64 takes the split-K tiles when their grid fits one round of 256 workgroups
    assert hk.kernel_id(154, 10240, 4096, (2, 2, 4, 4, 4)) == 31  # 240 workgroups of 64 x 128
    assert hk.kernel_id(256, 10240, 4096, (2, 2, 4, 4, 4)) == 24  # 320: the 128 x 128 tuple tile
    assert hk.kernel_id(2048, 3072, 3072, (2, 2, 4, 4, 4)) == 24
    assert hk.kernel_id(256, 3072, 3088, (2, 2, 4, 4, 4)) == 4  # K % 64 != 0: register-staged tile
    assert hk.kernel_id(4096, 4096, 4096, (1, 8, 4, 8, 2)) == 23  # BlockM 128, BlockN 256
    assert hk.kernel_id(4096, 4096, 4096, (3, 3, 3, 3, 3)) == 0
    assert hk.kernel_id(4096, 4096, 4090, (2, 4, 4, 8, 4)) == 0  # K % 16 != 0
    assert hk.kernel_id(4096, 3072, 3072, (2, 4, 4, 8, 3)) == 25  # 256x192
    assert hk.kernel_id(4096, 3072, 3072, (2, 4, 4, 4, 6)) == 26  # 128x384
    assert hk.kernel_id(4096, 3072, 3088, (2, 4, 4, 4, 6)) == 4  # K % 64 != 0: register-staged 128x128
    assert hk.kernel_id(4096, 3072, 3080, (2, 4, 4, 8, 3)) == 0  # K % 16 != 0
    for cfg in hk._CONFIGS:
        assert hk.kernel_id(4096, 4096, 4096, cfg) in (5, 6, 20, 22, 23, 24, 25, 26)
        assert hk.kernel_id(1024, 1024, 1024, cfg) == 30


def test_pick_config(hk):
    """The any-M entry's shape-based tile pick (256 CUs assumed without a GPU)."""
    assert hk.any_m_config(32768, 13824, 5120) == (2, 4, 4, 8, 4)  # 256x256, 27 full waves
    assert hk.any_m_config(4096, 3072, 3072) == (2, 4, 4, 4, 6)  # 128x384: 256 tiles, one per CU
    assert hk.any_m_config(512, 9216, 3072) == (2, 4, 4, 4, 4)  # 128x256: 144 tiles in one wave
    assert hk.any_m_config(16, 4096, 4096) == (1, 1, 2, 1, 2)  # small-M kernel
    for shape in [(100, 3072, 3072), (1000, 5120, 13824), (65, 768, 512)]:
        assert tuple(hk.any_m_config(*shape)) in set(hk._CONFIGS)


def test_configs_keep_reference_entries(hk):
    ref = {(1, 1, 2, 1, 2), (1, 1, 4, 1, 2), (1, 2, 2, 1, 2), (1, 2, 4, 1, 2), (1, 4, 2, 1, 2), (1, 4, 4, 1, 2),
           (1, 8, 2, 1, 2), (1, 8, 4, 1, 2), (1, 1, 2, 2, 2), (1, 1, 4, 2, 2), (1, 1, 2, 4, 4), (1, 1, 4, 4, 4),
           (1, 2, 2, 2, 2), (1, 2, 4, 2, 2), (2, 1, 2, 2, 2), (2, 1, 4, 2, 2), (1, 4, 2, 4, 2), (1, 4, 4, 4, 2),
           (1, 8, 2, 8, 2), (1, 8, 4, 8, 2), (2, 2, 2, 4, 4), (2, 2, 4, 4, 4), (2, 4, 2, 4, 2), (2, 4, 4, 4, 2),
           (2, 4, 2, 4, 4), (2, 4, 4, 4, 4), (4, 2, 2, 2, 4), (4, 2, 4, 2, 4)}
    assert ref <= set(hk._CONFIGS)
    assert hk._CONFIGS == sorted(hk._CONFIGS, key=lambda x: (x[0], x[1], x[3], x[4], x[2]))


def test_config_compatible_rules(pkg):
    from featherops_amd.kernel.hip import utils

    assert utils._config_compatible((1, 1, 2, 1, 2), 16, 128, 128)
    assert not utils._config_compatible((1, 1, 2, 2, 2), 16, 128, 128)  # BlockM 32
    assert not utils._config_compatible((1, 1, 4, 1, 2), 16, 128, 96)  # ChunkK 64
    # large shapes need blocks >= 64 (utils.py:141-142)
    assert not utils._config_compatible((1, 1, 2, 1, 2), 4096, 4096, 4096)
    assert utils._config_compatible((2, 4, 4, 8, 4), 32768, 13824, 5120)
    a = torch.empty(16, 128, dtype=torch.float16)
    b = torch.empty(8, 128, 16, dtype=torch.uint8)
    assert utils.get_compatible_config(a, b, 1, [(1, 1, 2, 2, 2), (1, 1, 2, 1, 2)]) == (1, 1, 2, 1, 2)
    with pytest.raises(RuntimeError, match="No compatible config"):
        utils.get_compatible_config(a, b, 1, [(1, 1, 2, 2, 2)])


def _good_args(M=64, N=128, K=256, out=torch.float16):
    a = torch.empty(M, K, dtype=torch.float16)
    b = torch.empty(K // 16, N, 16, dtype=torch.float8_e5m2)
    c = torch.empty(M, N, dtype=out)
    return a, b, torch.ones((), dtype=torch.float32), torch.zeros(N, dtype=out), c


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: dict(a=a["a"].float()), "a must be float16"),
    (lambda a: dict(c=a["c"].float()), "c must be float16 or bfloat16"),
    (lambda a: dict(b=a["b"].view(torch.uint8)), "b_prepacked must be float8_e5m2"),
    (lambda a: dict(b_dtype=2), "b_dtype must be 0"),
    (lambda a: dict(a=a["a"][:, :128]), r"b_prepacked.shape\[0\] must equal K/16"),
    (lambda a: dict(a=torch.empty(64, 264, dtype=torch.float16)), "K must be divisible by 16"),
    (lambda a: dict(c=torch.empty(32, 128, dtype=torch.float16)), r"c.shape\[0\] must equal M"),
    (lambda a: dict(a=torch.empty(256, 64, dtype=torch.float16).t()), r"a.stride\(0\) must equal K"),
    (lambda a: dict(scale=torch.ones(2)), "scale must have one element"),
    (lambda a: dict(scale=torch.ones((), dtype=torch.float16)), "scale must be float32"),
    (lambda a: dict(bias=torch.zeros(128, dtype=torch.bfloat16)), "bias must have the same dtype as c"),
    (lambda a: dict(bias=torch.zeros(64, dtype=torch.float16)), "bias must have N elements"),
    (lambda a: dict(cfg=(1, 1, 2, 8, 2)), r"M \(64\) must be divisible by kBlockM \(128\)"),
    (lambda a: dict(cfg=(1, 8, 4, 1, 2)), r"N \(128\) must be divisible by kBlockN \(256\)"),
])
def test_validation_messages(hk, mutate, msg):
    a, b, s, bias, c = _good_args()
    args = dict(a=a, b=b, scale=s, bias=bias, c=c, cfg=(1, 1, 2, 1, 2), b_dtype=1)
    hk.validate_scaled_mm(args["a"], args["b"], args["scale"], args["bias"], args["c"], *args["cfg"],
                          args["b_dtype"], require_cuda=False)
    args.update(mutate(args))
    with pytest.raises(RuntimeError, match=msg):
        hk.validate_scaled_mm(args["a"], args["b"], args["scale"], args["bias"], args["c"], *args["cfg"],
                              args["b_dtype"], require_cuda=False)


def test_cpu_tensors_raise_loudly(hk):
    a, b, s, bias, c = _good_args()
    # the op has only a GPU kernel: CPU tensors hit torch's "no kernel for backend" error
    with pytest.raises((RuntimeError, NotImplementedError), match="CUDA"):
        torch.ops.feather_ops.scaled_mm.default(a, b, s, bias, c, 1, 1, 2, 1, 2, 1)


def test_native_op_registered_in_cpp(hk):
    """torch.ops.feather_ops.scaled_mm comes from the C++ op library with the
    reference's schema (hip_kernel.cu:746-767) and only a CUDA kernel."""
    from featherops_amd.kernel.hip import _lib

    assert _lib.OPS_LIB_PATH.exists()
    op = torch.ops.feather_ops.scaled_mm.default
    assert str(op._schema) == (
        "feather_ops::scaled_mm(Tensor a, Tensor b_prepacked, Tensor? scale, Tensor? bias, Tensor(a!) c, "
        "int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, int repeat_n, int b_dtype) -> ()")
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CUDA")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CPU")
    # registered from a shared library, not from Python
    assert "csrc/torch_op.cpp" in torch._C._dispatch_dump(op.name())
    anym = torch.ops.feather_ops.scaled_mm_any_m.default
    assert str(anym._schema) == ("feather_ops::scaled_mm_any_m(Tensor a, Tensor b_prepacked, Tensor? scale, "
                                 "Tensor? bias, ScalarType out_dtype) -> Tensor")
    assert torch._C._dispatch_has_kernel_for_dispatch_key(anym.name(), "CUDA")
    assert torch._C._dispatch_has_kernel_for_dispatch_key(anym.name(), "Meta")
    assert "csrc/torch_op.cpp" in torch._C._dispatch_dump(anym.name())
    cfg = torch.ops.feather_ops_internal.scaled_mm_configured.default
    assert str(cfg._schema) == (
        "feather_ops_internal::scaled_mm_configured(Tensor a, Tensor b_prepacked, Tensor? scale, Tensor? bias, "
        "ScalarType out_dtype, int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, int repeat_n) "
        "-> Tensor")
    assert torch._C._dispatch_has_kernel_for_dispatch_key(cfg.name(), "Meta")
    assert hk.scaled_mm_hip_configured is cfg
    q = torch.ops.feather_ops.quantize_prepack_e5m2.default
    assert str(q._schema) == ("feather_ops::quantize_prepack_e5m2(Tensor w, Tensor? ckpt_scale, bool native) "
                              "-> (Tensor, Tensor)")
    qs = torch.ops.feather_ops.quantize_prepack_e5m2_scaled.default
    assert str(qs._schema) == "feather_ops::quantize_prepack_e5m2_scaled(Tensor w, Tensor scale) -> Tensor"
    cv = torch.ops.feather_ops.bf16_to_fp16.default
    assert str(cv._schema) == "feather_ops::bf16_to_fp16(Tensor x, bool rne) -> Tensor"
    assert torch._C._dispatch_has_kernel_for_dispatch_key(cv.name(), "Meta")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key(cv.name(), "CPU")
    for op_ in (q, qs, cv):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op_.name(), "CUDA")
        assert "csrc/torch_op.cpp" in torch._C._dispatch_dump(op_.name())


def test_convert_entries_keep_reference_checks(pkg):
    """kernel/convert.py keeps the reference's assertions (bf16, contiguous, even
    length for the RTZ cast) and refuses host tensors before any launch."""
    import importlib

    conv = importlib.import_module(f"{pkg.__name__}.kernel.convert")
    with pytest.raises(AssertionError):
        conv.bf16_to_fp16(torch.zeros(4, dtype=torch.float16))
    with pytest.raises(AssertionError):
        conv.bf16_to_fp16(torch.zeros(4, 4, dtype=torch.bfloat16).t())
    with pytest.raises(AssertionError):
        conv.bf16_to_fp16(torch.zeros(3, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="GPU"):
        conv.bf16_to_fp16_rne(torch.zeros(3, dtype=torch.bfloat16))
    meta = torch.ops.feather_ops.bf16_to_fp16.default(torch.empty(5, 6, dtype=torch.bfloat16, device="meta"), True)
    assert meta.shape == (5, 6) and meta.dtype == torch.float16


def test_op_library_loads_first_in_fresh_process():
    """Importing the op module before anything else has loaded the C library
    (a fresh interpreter) registers the ops without blocking."""
    import subprocess
    import sys
    from pathlib import Path

    repo = Path(__file__).resolve().parents[1]
    code = ("import sys; sys.path.insert(0, %r); import __graft_entry__ as g; g.load_package(); "
            "import featherops_amd.kernel.hip.hip_kernel, torch; "
            "print(torch.ops.feather_ops.scaled_mm_any_m.default.name())") % str(repo)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "feather_ops::scaled_mm_any_m" in r.stdout


def test_any_m_fake_shapes(hk):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        a = torch.empty(37, 256, dtype=torch.bfloat16)
        b = torch.empty(16, 128, 16, dtype=torch.float8_e5m2)
        out = hk.scaled_mm_hip_any_m(a, b, None, None, torch.float16)
        assert out.shape == (37, 128) and out.dtype == torch.float16


def test_fake_impl_shapes_for_compile(hk):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        a = torch.empty(64, 256, dtype=torch.float16)
        b = torch.empty(16, 128, 16, dtype=torch.float8_e5m2)
        out = hk._configured_op(a, b, None, None, torch.bfloat16, 1, 1, 2, 1, 2)
        assert out.shape == (64, 128) and out.dtype == torch.bfloat16


def test_ops_m_padding_rule(pkg):
    from featherops_amd.comfy_feather import ops

    assert [ops._m_block(m) for m in (1, 64, 65, 128, 129, 256, 257)] == [16, 16, 32, 32, 64, 64, 128]


def test_small_m_plan_workspace(pkg):
    """Small-M plan (256-CU target without a GPU): a K split across
    workgroups, which needs a workspace, only where it balances the grid."""
    from featherops_amd.kernel.hip import _lib

    lib = _lib.lib()
    cfg = (1, 1, 2, 1, 2)
    assert lib.feather_scaled_mm_workspace_size(16, 4096, 4096, *cfg) == 0  # 256 strips: one per CU
    assert lib.feather_scaled_mm_workspace_size(16, 13824, 5120, *cfg) == 0  # 216 strips of 64 columns
    # 80 strips of 64 columns x 3 K ranges: the fixed 64 KB counter region + 3 fp32 partial tiles per strip
    assert lib.feather_scaled_mm_workspace_size(16, 5120, 13824, *cfg) == 65536 + 80 * 3 * 16 * 64 * 4
    assert lib.feather_scaled_mm_workspace_size(1, 3072, 12288, *cfg) == 0  # lean kernel: 192 strips of 16 columns
    # 128 strips of 16 columns x 2 K ranges
    assert lib.feather_scaled_mm_workspace_size(8, 2048, 12288, *cfg) == 65536 + 128 * 2 * 8 * 16 * 4


def test_packed_params_protocol(quant):
    """FeatherFP8E5M2PackedParams (reference comfy_feather/quant.py:22-49): to_device and clone
    return new params with their own scale tensor; copy_from updates in place, keeping the
    scale's storage."""
    P = quant.FeatherFP8E5M2PackedParams
    p = P(scale=torch.tensor(0.5), orig_dtype=torch.float16, orig_shape=(8, 16))
    assert p._tensor_fields() == ["scale"]
    c = p.clone()
    assert c.scale.data_ptr() != p.scale.data_ptr() and c.scale.item() == 0.5
    d = p.to_device("cpu")
    assert d.scale.item() == 0.5 and d.orig_dtype == torch.float16 and d.orig_shape == (8, 16)
    src = P(scale=torch.tensor(2.0), orig_dtype=torch.bfloat16, orig_shape=(4, 32))
    ptr = p.scale.data_ptr()
    p.copy_from(src)
    assert p.scale.data_ptr() == ptr and p.scale.item() == 2.0
    assert p.orig_dtype == torch.bfloat16 and p.orig_shape == (4, 32)


def test_capi_rejects_shapes_past_offset_limits(pkg):
    """K >= 2^22 or N >= 2^25 would overflow the LDS kernels' 32-bit per-lane copy offsets:
    refused before any launch (kernel id 0, launch returns false)."""
    from featherops_amd.kernel.hip import _lib

    L = _lib.lib()
    cfg = (2, 4, 4, 8, 4)
    assert L.feather_scaled_mm_kernel_id(256, 16, (1 << 22) - 16, *cfg) != 0
    assert L.feather_scaled_mm_kernel_id(256, 16, 1 << 22, *cfg) == 0
    assert L.feather_scaled_mm_kernel_id(256, (1 << 25) - 16, 16, *cfg) != 0
    assert L.feather_scaled_mm_kernel_id(256, 1 << 25, 16, *cfg) == 0
    assert not L.launch_scaled_mm(None, None, None, None, None, 256, 16, 1 << 22, 0, 0, *cfg, 1, 0, None)


def test_splitk_plan_without_counter_room_needs_no_workspace():
    """A split-K tile plan with more output tiles than the 16384 arrival counters runs
    unsplit: it asks for no workspace (run in a fresh process, the workgroup target is read
    once)."""
    import subprocess
    import sys

    code = ("import __graft_entry__; __graft_entry__.load_package();"
            "from featherops_amd.kernel.hip import _lib; L = _lib.lib();"
            "print(L.feather_scaled_mm_workspace_size(64, 16400 * 128, 2048, 2, 2, 4, 4, 4),"
            " L.feather_scaled_mm_workspace_size(64, 4096, 4096, 2, 2, 4, 4, 4))")
    env = dict(__import__("os").environ, FEATHEROPS_SMALLM_GROUPS="40000")
    out = subprocess.run([sys.executable, "-c", code], cwd=REPO, env=env, capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr
    big, small = map(int, out.stdout.split())
    assert big == 0 and small > 0


def test_lora_down_plan_leaves_no_split_empty(pkg):
    """The LoRA down-projection splits K across workgroups (split q owns stages
    [q * per, min((q + 1) * per, nst)) of 64 K): every split must own at least one
    stage, else its prologue copies would address past the ends of x and D. The
    split count is read back from the workspace size (counters + tiles x splits
    fp32 partial tiles of 64 rows x R ranks)."""
    from featherops_amd.kernel.hip import _lib

    L = _lib.lib()
    checked = 0
    for M, R in ((1, 32), (40, 128), (200, 64)):
        tiles = (M + 63) // 64
        for K in range(8, 20001, 8):
            ws = L.feather_lora_down_workspace_size(M, K, R)
            nst = (K + 63) // 64
            if ws == 0:
                assert nst < 4  # no split below two stages per split
                continue
            part = tiles * 64 * R * 4
            assert (ws - 65536) % part == 0
            ks = (ws - 65536) // part
            per = -(-nst // ks)
            assert 2 <= ks <= 16 and ks <= nst // 2
            assert (ks - 1) * per < nst, (M, K, R, ks, per, nst)
            checked += 1
    assert checked > 7000
