"""Drop-in Python surface of the scaled_mm hot path (reference kernel/hip/hip_kernel.py).

Public names and signatures are the reference's:
    scaled_mm_hip(a, b_prepacked, scale, bias, out_dtype)              (:136-167)
    scaled_mm_hip_configured(a, b_prepacked, scale, bias, out_dtype,
                             block_warps_m, block_warps_n, unroll_k,
                             repeat_m, repeat_n)                        (:12-58)
    prepack_b_for_scaled_mm(b)                                          (:170-171)
    _CONFIGS                                                            (:60-91)
plus the native op `torch.ops.feather_ops.scaled_mm` with the reference
schema (hip_kernel.cu:746-767) and its validation (hip_kernel.cu:648-730).

The native op is registered in C++ (csrc/torch_op.cpp, built into
lib/libfeather_torch_ops.so) and calls libfeatherops_amd.so's launch entry on
torch's current stream; the any-M op calls the library through ctypes. There
is no other compute path.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .utils import generate_autotune_configs, get_compatible_config, old_autotune

# ---------------------------------------------------------------------------
# validation (hip_kernel.cu:648-730), usable without a GPU for host-side tests
# ---------------------------------------------------------------------------


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


_OUT_DTYPES = (torch.float16, torch.bfloat16)


def _valid_fast(a, b_prepacked, scale, bias, c, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, b_dtype,
                block_divisible, allow_bf16_a) -> bool:
    """True when every check of validate_scaled_mm passes (device, dtypes,
    shapes, strides, alignment, divisibility); one expression, no messages.
    False sends the caller to the full checks, which name what failed."""
    if a.dim() != 2 or b_prepacked.dim() != 3 or c.dim() != 2:
        return False
    M, K = a.shape
    Kg, N, sixteen = b_prepacked.shape
    dev = a.device
    bm = 16 * block_warps_m * repeat_m
    bn = 16 * block_warps_n * repeat_n
    return (dev.type == "cuda" and b_prepacked.device == dev and c.device == dev
            and (a.dtype == torch.float16 or (allow_bf16_a and a.dtype == torch.bfloat16))
            and c.dtype in _OUT_DTYPES
            and ((b_dtype == 1 and b_prepacked.dtype == torch.float8_e5m2)
                 or (b_dtype == 0 and b_prepacked.dtype == torch.float8_e4m3fn))
            and K % 16 == 0 and Kg == K // 16 and sixteen == 16 and tuple(c.shape) == (M, N)
            and (M == 1 or a.stride(0) == K) and a.stride(1) == 1
            and (Kg == 1 or b_prepacked.stride(0) == N * 16) and b_prepacked.stride(1) == 16
            and b_prepacked.stride(2) == 1 and (M == 1 or c.stride(0) == N) and c.stride(1) == 1
            and (scale is None or (scale.device == dev and scale.dtype == torch.float32 and scale.numel() == 1))
            and (bias is None or (bias.device == dev and bias.dtype == c.dtype and bias.numel() == N))
            and a.data_ptr() % 16 == 0 and b_prepacked.data_ptr() % 16 == 0 and c.data_ptr() % 16 == 0
            and ((M % bm == 0 and N % bn == 0 and K % (16 * unroll_k) == 0) if block_divisible else N % 16 == 0)
            and 32 * block_warps_m * block_warps_n <= 1024)


def validate_scaled_mm(a, b_prepacked, scale, bias, c, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n,
                       b_dtype, require_cuda: bool = True, block_divisible: bool = True,
                       allow_bf16_a: bool = False) -> None:
    """Raise RuntimeError with the reference's message for any argument the
    kernel cannot take. `require_cuda=False` skips the device checks;
    `block_divisible=False` replaces the BlockM/BlockN/ChunkK divisibility
    rules by what the gfx950 kernels need (N % 16 == 0; K % 16 is always
    required) and `allow_bf16_a` accepts bf16 activations -- the any-M entry."""
    if require_cuda and _valid_fast(a, b_prepacked, scale, bias, c, block_warps_m, block_warps_n, unroll_k, repeat_m,
                                    repeat_n, b_dtype, block_divisible, allow_bf16_a):
        return
    if require_cuda:
        _check(a.is_cuda, "a must be a CUDA tensor")
        _check(b_prepacked.is_cuda, "b_prepacked must be a CUDA tensor")
        _check(c.is_cuda, "c must be a CUDA tensor")
        _check(b_prepacked.device == a.device, "b_prepacked must be on the same device as a")
        _check(c.device == a.device, "c must be on the same device as a")
    if allow_bf16_a:
        _check(a.dtype in (torch.float16, torch.bfloat16), "a must be float16 or bfloat16")
    else:
        _check(a.dtype == torch.float16, "a must be float16")
    _check(c.dtype in (torch.float16, torch.bfloat16), "c must be float16 or bfloat16")
    _check(b_dtype in (0, 1), "b_dtype must be 0 (fp8e4m3) or 1 (fp8e5m2)")
    if b_dtype == 0:
        _check(b_prepacked.dtype == torch.float8_e4m3fn, "b_prepacked must be float8_e4m3fn when b_dtype=0")
    else:
        _check(b_prepacked.dtype == torch.float8_e5m2, "b_prepacked must be float8_e5m2 when b_dtype=1")
    _check(a.dim() == 2, "a must be 2D")
    _check(b_prepacked.dim() == 3, "b_prepacked must be 3D (K/16, N, 16)")
    _check(c.dim() == 2, "c must be 2D")
    M, K = a.shape
    N = b_prepacked.shape[1]
    _check(K % 16 == 0, "K must be divisible by 16")
    _check(b_prepacked.shape[0] == K // 16, f"b_prepacked.shape[0] must equal K/16 ({K // 16})")
    _check(b_prepacked.shape[2] == 16, "b_prepacked.shape[2] must be 16")
    _check(c.shape[0] == M, "c.shape[0] must equal M")
    _check(c.shape[1] == N, "c.shape[1] must equal N")
    # (the stride of a dimension of size 1 is never used, so any value passes)
    _check(M == 1 or a.stride(0) == K, f"a.stride(0) must equal K ({K})")
    _check(a.stride(1) == 1, "a.stride(1) must be 1")
    _check(K // 16 == 1 or b_prepacked.stride(0) == N * 16, f"b_prepacked.stride(0) must equal N*16 ({N * 16})")
    _check(b_prepacked.stride(1) == 16, "b_prepacked.stride(1) must be 16")
    _check(b_prepacked.stride(2) == 1, "b_prepacked.stride(2) must be 1")
    _check(M == 1 or c.stride(0) == N, f"c.stride(0) must equal N ({N})")
    _check(c.stride(1) == 1, "c.stride(1) must be 1")
    if scale is not None:
        if require_cuda:
            _check(scale.is_cuda, "scale must be a CUDA tensor")
            _check(scale.device == a.device, "scale must be on the same device as a")
        _check(scale.dtype == torch.float32, "scale must be float32")
        _check(scale.numel() == 1, "scale must have one element")
    if bias is not None:
        if require_cuda:
            _check(bias.is_cuda, "bias must be a CUDA tensor")
            _check(bias.device == a.device, "bias must be on the same device as a")
        _check(bias.dtype == c.dtype, "bias must have the same dtype as c")
        _check(bias.numel() == N, "bias must have N elements")
    if require_cuda:
        for name, t in (("a", a), ("b_prepacked", b_prepacked), ("c", c)):
            _check(t.data_ptr() % 16 == 0, f"{name} data pointer must be 16-byte aligned")
    block_m = 16 * block_warps_m * repeat_m
    block_n = 16 * block_warps_n * repeat_n
    chunk_k = 16 * unroll_k
    if block_divisible:
        _check(M % block_m == 0, f"M ({M}) must be divisible by kBlockM ({block_m})")
        _check(N % block_n == 0, f"N ({N}) must be divisible by kBlockN ({block_n})")
        _check(K % chunk_k == 0, f"K ({K}) must be divisible by kChunkK ({chunk_k})")
    else:
        _check(N % 16 == 0, f"N ({N}) must be divisible by 16")
    _check(32 * block_warps_m * block_warps_n <= 1024, "Block size exceeds HIP thread-per-block limit")


# torch op feather_ops::scaled_mm with the reference schema (hip_kernel.cu:746-767),
# registered in C++ by lib/libfeather_torch_ops.so (csrc/torch_op.cpp): the same
# checks and messages as validate_scaled_mm, then feather_launch_scaled_mm_ws on
# torch's current stream with a per-(device, stream) workspace.
_lib.load_torch_ops()


def kernel_id(M: int, N: int, K: int, cfg) -> int:
    """gfx950 kernel a config runs for this shape (0 = unsupported)."""
    return int(_lib.lib().feather_scaled_mm_kernel_id(M, N, K, *cfg))


# ---------------------------------------------------------------------------
# torch.library custom ops (hip_kernel.py:12-133)
# ---------------------------------------------------------------------------


# feather_ops_internal::scaled_mm_configured (hip_kernel.py:12-58) is registered
# in C++ with the native op (csrc/torch_op.cpp), with a Meta kernel for fake
# tensors: (a, b_prepacked, scale, bias, out_dtype, block_warps_m, block_warps_n,
# unroll_k, repeat_m, repeat_n) -> C of out_dtype.
_configured_op = torch.ops.feather_ops_internal.scaled_mm_configured.default
scaled_mm_hip_configured = _configured_op

# Reference configurations (hip_kernel.py:60-89), then five gfx950 tiles:
# (2,4,4,8,4) -> 256x256 (2x4 waves), (4,2,4,4,8) -> 256x256 (4x2 waves),
# (4,2,4,4,4) -> 256x128, (2,4,4,8,3) -> 256x192 and (2,4,4,4,6) -> 128x384
# output tiles (the last two give M=4096, N=3072 exactly 256 tiles, one per CU).
_CONFIGS = [
    (1, 1, 2, 1, 2), (1, 1, 4, 1, 2), (1, 2, 2, 1, 2), (1, 2, 4, 1, 2), (1, 4, 2, 1, 2), (1, 4, 4, 1, 2),
    (1, 8, 2, 1, 2), (1, 8, 4, 1, 2), (1, 1, 2, 2, 2), (1, 1, 4, 2, 2), (1, 1, 2, 4, 4), (1, 1, 4, 4, 4),
    (1, 2, 2, 2, 2), (1, 2, 4, 2, 2), (2, 1, 2, 2, 2), (2, 1, 4, 2, 2), (1, 4, 2, 4, 2), (1, 4, 4, 4, 2),
    (1, 8, 2, 8, 2), (1, 8, 4, 8, 2), (2, 2, 2, 4, 4), (2, 2, 4, 4, 4), (2, 4, 2, 4, 2), (2, 4, 4, 4, 2),
    (2, 4, 2, 4, 4), (2, 4, 4, 4, 4), (4, 2, 2, 2, 4), (4, 2, 4, 2, 4),
    (2, 4, 4, 8, 4), (4, 2, 4, 4, 8), (4, 2, 4, 4, 4), (2, 4, 4, 8, 3), (2, 4, 4, 4, 6),
]
_CONFIGS = sorted(_CONFIGS, key=lambda x: (x[0], x[1], x[3], x[4], x[2]))


@torch.library.custom_op("feather_ops_internal::scaled_mm_autotuned", mutates_args=())
def _autotuned_op(
    a: torch.Tensor,
    b_prepacked: torch.Tensor,
    scale: torch.Tensor,
    bias: torch.Tensor,
    out_dtype: torch.dtype,
    has_scale: bool,
    has_bias: bool,
    block_warps_m: int = 0,
    block_warps_n: int = 0,
    unroll_k: int = 0,
    repeat_m: int = 0,
    repeat_n: int = 0,
) -> torch.Tensor:
    if min(block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n) <= 0:
        block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n = get_compatible_config(a, b_prepacked, 1, _CONFIGS)
    return _configured_op(a, b_prepacked, scale if has_scale else None, bias if has_bias else None, out_dtype,
                          block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n)


@_autotuned_op.register_fake
def _(a, b_prepacked, scale, bias, out_dtype, has_scale, has_bias, block_warps_m=0, block_warps_n=0, unroll_k=0,
      repeat_m=0, repeat_n=0):
    return torch.empty((a.shape[0], b_prepacked.shape[1]), device=a.device, dtype=out_dtype)


def _autotune_decomposition(a, b_prepacked, scale, bias, **kw):
    """What one Inductor autotuning choice of _autotuned_op runs: the configured op with that
    choice's tuple. Inductor passes the op's non-tensor arguments by keyword: by name (the
    lowering wrapper below names them), or as arg_<position> where a torch version's lowering
    renames positional scalars itself; both spellings are read."""
    out_dtype = kw["out_dtype"] if "out_dtype" in kw else kw["arg_4"]
    has_scale = kw["has_scale"] if "has_scale" in kw else kw["arg_5"]
    has_bias = kw["has_bias"] if "has_bias" in kw else kw["arg_6"]
    cfg = (kw["block_warps_m"], kw["block_warps_n"], kw["unroll_k"], kw["repeat_m"], kw["repeat_n"])
    return _configured_op(a, b_prepacked, scale if has_scale else None, bias if has_bias else None, out_dtype, *cfg)


# Inductor's custom-op autotuning (reference hip_kernel.py:133): under torch.compile with
# max-autotune, every compatible config is benchmarked and the fastest one is compiled in.
from torch._inductor.kernel.custom_op import register_custom_op_autotuning  # noqa: E402

register_custom_op_autotuning(
    _autotuned_op,
    config_generator=lambda fake_tensors: generate_autotune_configs(fake_tensors, _CONFIGS, 1,
                                                                    decomposition=_autotune_decomposition))


def _contiguous_inputs_first(op) -> None:
    """Wrap the autotuning lowering of `op`: its tensor inputs reach it as contiguous, realized
    buffers (the op needs contiguous operands anyway, and torch 2.10's autotuning cannot take an
    unrealized view such as x.to(fp16).view(-1, K) fused into the graph), and its non-tensor
    arguments by their schema names (torch 2.10's lowering would rename positional ones to
    arg_<i>, which neither the op nor its decompositions accept)."""
    from torch._inductor import ir
    from torch._inductor.lowering import lowerings

    inner = lowerings[op]
    names = [a.name for a in op._schema.arguments]

    def lowering(*args, **kwargs):
        tensors = []
        named = dict(kwargs)
        for i, arg in enumerate(args):
            if isinstance(arg, ir.TensorBox):
                arg = ir.ExternKernel.require_contiguous(arg)
                tensors.append(arg if isinstance(arg, ir.TensorBox) else ir.TensorBox(arg))
            else:
                named[names[i]] = arg
        return inner(*tensors, **named)

    lowerings[op] = lowering


_contiguous_inputs_first(torch.ops.feather_ops_internal.scaled_mm_autotuned.default)


def scaled_mm_hip(
    a: torch.Tensor,
    b_prepacked: torch.Tensor,
    scale: torch.Tensor | None,
    bias: torch.Tensor | None,
    out_dtype: torch.dtype,
) -> torch.Tensor:
    """Autotuned entry (hip_kernel.py:136-167)."""
    if torch.compiler.is_compiling():
        return _autotuned_op(a, b_prepacked, scale if scale is not None else a, bias if bias is not None else a,
                             out_dtype, scale is not None, bias is not None)

    def run_fn(cfg):
        return _configured_op(a, b_prepacked, scale, bias, out_dtype, *cfg)

    M, K = a.shape[0], a.shape[1]
    N = b_prepacked.shape[1]
    best_cfg = old_autotune(M, N, K, _CONFIGS, run_fn, "mixed", b_prepacked.dtype, out_dtype,
                            kernel_id=lambda cfg: kernel_id(M, N, K, cfg))
    return _configured_op(a, b_prepacked, scale, bias, out_dtype, *best_cfg)


# ---------------------------------------------------------------------------
# any-M entry (no M padding): the gfx950 kernels mask rows past M
# ---------------------------------------------------------------------------

# The any-M entry's configuration: the library's shape-based pick
# (feather_scaled_mm_pick_config: the output tile whose waves x tile cost is
# smallest on this device), cached per shape and device. The op itself asks
# the library for the same pick on every call.
_PICKED: dict = {}


def any_m_config(M: int, N: int, K: int, device: torch.device | None = None) -> tuple:
    dev = device.index if device is not None and device.index is not None else (
        torch.cuda.current_device() if torch.cuda.is_available() else -1)
    key = (dev, M, N, K)
    cfg = _PICKED.get(key)
    if cfg is None:
        out = (ctypes.c_int * 5)()
        if dev >= 0:
            with torch.cuda.device(dev):
                status = _lib.lib().feather_scaled_mm_pick_config(M, N, K, out)
        else:
            status = _lib.lib().feather_scaled_mm_pick_config(M, N, K, out)
        _lib.check(status, "feather_scaled_mm_pick_config")
        cfg = tuple(out)
        _PICKED[key] = cfg
    return cfg


# torch.ops.feather_ops.scaled_mm_any_m, registered in C++ with the native op
# (csrc/torch_op.cpp): checks as validate_scaled_mm(block_divisible=False,
# allow_bf16_a=True), the any_m_config tile, a Meta kernel for fake tensors.
_any_m_op = torch.ops.feather_ops.scaled_mm_any_m.default


def scaled_mm_hip_any_m(a, b_prepacked, scale, bias, out_dtype) -> torch.Tensor:
    """scaled_mm for any row count M, without padding A or slicing C (the
    kernels mask rows past M). Rows are independent, so the result equals
    padding M to a block multiple, calling scaled_mm_hip and slicing. `a` may
    also be bf16: it is then rounded to fp16 (round to nearest even) inside the
    GEMM, the same values as calling it with a.to(torch.float16)."""
    return torch.ops.feather_ops.scaled_mm_any_m.default(a, b_prepacked, scale, bias, out_dtype)


def scaled_mm_hip_any_m_lora(a, b_prepacked, scale, bias, out_dtype, lora_t, lora_u) -> torch.Tensor:
    """scaled_mm_hip_any_m(...) + lora_t @ lora_u.T: the unmerged-LoRA term
    (reference comfy_feather/lora.py:4-35) with the strengths folded into
    lora_t (M, R); lora_u is (N, R); both contiguous fp16 or bf16, R % 32 == 0.
    On the large tiles the term joins the fp32 accumulator before the output
    rounding (no second pass over C); other routes add it to C afterwards."""
    return torch.ops.feather_ops.scaled_mm_any_m_lora.default(a, b_prepacked, scale, bias, out_dtype, lora_t, lora_u)


def prepack_b_for_scaled_mm(b: torch.Tensor) -> torch.Tensor:
    """(K, N) -> (K/16, N, 16) (hip_kernel.py:170-171), on the GPU.

    Any 1-byte dtype works (fp8 weights are the use); a CPU tensor is moved to
    the current GPU, repacked there and returned on its own device."""
    if b.dim() != 2 or b.element_size() != 1:
        raise ValueError(f"prepack_b_for_scaled_mm expects a 2-D 1-byte tensor, got {tuple(b.shape)} {b.dtype}")
    K, N = b.shape
    if K % 16 != 0:
        raise ValueError(f"K ({K}) must be divisible by 16")
    src = b if b.is_cuda else b.to("cuda")
    src = src.contiguous()
    out = torch.empty((K // 16, N, 16), dtype=b.dtype, device=src.device)
    with torch.cuda.device(src.device):
        _lib.check(_lib.lib().feather_prepack_b(src.data_ptr(), out.data_ptr(), K, N, _lib.stream_ptr(src.device)),
                   "prepack_b_for_scaled_mm")
    return out if b.is_cuda else out.to(b.device)
