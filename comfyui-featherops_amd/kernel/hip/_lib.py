"""ctypes binding of libfeatherops_amd.so (declared in include/featherops_amd.h).

The library is the only compute path: if it is missing, every entry point
raises instead of falling back to anything else.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parents[2] / "lib" / "libfeatherops_amd.so"
# torch op library: feather_ops::scaled_mm registered in C++ over the same C ABI
OPS_LIB_PATH = LIB_PATH.with_name("libfeather_torch_ops.so")

FEATHER_OK = 0
DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
B_E4M3FN, B_E5M2 = 0, 1

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p

# name -> (restype, argtypes); every symbol the header declares
SIGNATURES: dict[str, tuple] = {
    "launch_scaled_mm": (ctypes.c_bool, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _int, _int,
                                         _int, _int, _int, _int, _vp]),
    "feather_launch_scaled_mm_ws": (ctypes.c_bool, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _int,
                                                    _int, _int, _int, _int, _int, _vp, ctypes.c_size_t, _vp]),
    "feather_launch_scaled_mm_ex": (ctypes.c_bool, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int,
                                                    _int, _int, _int, _int, _int, _int, _vp, ctypes.c_size_t, _vp]),
    "feather_launch_scaled_mm_noalloc": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int,
                                                _int, _int, _int, _int, _int, _int, _vp]),
    "feather_launch_scaled_mm_lora": (ctypes.c_bool, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp, _vp,
                                                      _i64, _int, _int, _int, _int, _int, _int, _int, _int, _vp]),
    "feather_lora_down": (_int, [_vp, _int, _vp, _vp, _i64, _i64, _i64, _vp, ctypes.c_size_t, _vp]),
    "feather_lora_down_workspace_size": (ctypes.c_size_t, [_i64, _i64, _i64]),
    "feather_scaled_mm_pick_config": (_int, [_i64, _i64, _i64, ctypes.POINTER(ctypes.c_int)]),
    "feather_scaled_mm_workspace_size": (ctypes.c_size_t, [_i64, _i64, _i64, _int, _int, _int, _int, _int]),
    "feather_scaled_mm_kernel_id": (_int, [_i64, _i64, _i64, _int, _int, _int, _int, _int]),
    "feather_quantize_prepack_e5m2": (_int, [_vp, _int, _i64, _i64, _vp, _int, _vp, _vp, _vp, _vp]),
    "feather_quantize_prepack_e5m2_ws": (_int, [_vp, _int, _i64, _i64, _vp, _int, _vp, _vp, _vp, ctypes.c_size_t,
                                                 _vp]),
    "feather_quantize_workspace_size": (ctypes.c_size_t, []),
    "feather_quantize_prepack_e5m2_scaled": (_int, [_vp, _int, _i64, _i64, _vp, _vp, _vp]),
    "feather_prepack_transpose": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "feather_unprepack_transpose": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "feather_prepack_b": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "feather_bf16_to_fp16": (_int, [_vp, _vp, _i64, _vp]),
    "feather_bf16_to_fp16_rne": (_int, [_vp, _vp, _i64, _vp]),
    "feather_dequantize_e5m2": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp]),
    "feather_status_string": (ctypes.c_char_p, [_int]),
    "feather_abi_version": (_int, []),
}

_lock = threading.RLock()  # load_torch_ops loads the C library while holding it
_handle: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load the library once and attach the C signatures."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"FeatherOps HIP library not found at {LIB_PATH}; build it with "
                    "`python comfyui-featherops_amd/build.py` (there is no non-HIP fallback)"
                )
            h = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _handle = h
    return _handle


_ops_loaded = False


def load_torch_ops() -> None:
    """Register torch.ops.feather_ops.scaled_mm from the C++ op library (once)."""
    global _ops_loaded
    if _ops_loaded:
        return
    with _lock:
        if not _ops_loaded:
            if not OPS_LIB_PATH.exists():
                raise RuntimeError(
                    f"FeatherOps torch op library not found at {OPS_LIB_PATH}; build it with "
                    "`python comfyui-featherops_amd/build.py` (there is no non-HIP fallback)"
                )
            lib()  # the op library resolves the launch entry from libfeatherops_amd.so
            torch.ops.load_library(str(OPS_LIB_PATH))
            _ops_loaded = True


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on `device` (torch's direct
    accessor: ~0.1 us against ~2 us for building a Stream object)."""
    if _RAW_STREAM is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(device).cuda_stream


def check(status: int, what: str) -> None:
    if status != FEATHER_OK:
        msg = lib().feather_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def require_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("FeatherOps HIP kernels need GPU (ROCm) tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("all tensors must be on the same device")
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev
