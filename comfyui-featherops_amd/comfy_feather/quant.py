"""fp8 e5m2 weight quantization and the (K/16, N, 16) prepack, on the GPU.

Drop-in for the reference's comfy_feather/quant.py: same function and class
names, arguments, return values and errors. The arithmetic runs in
libfeatherops_amd.so:
  * quantize + prepack is one fused pass (amax kernel, then a streaming
    quantize kernel writing the prepacked bytes), bit-exact with the
    reference's torch sequence (quant.py:52-74 followed by quant.py:11-13);
  * prepack / unprepack / dequantize are HIP kernels.
CPU tensors are processed on the current GPU and the result is returned on
the input's device; with no GPU the functions raise.

ComfyUI's `comfy.quant_ops` (QuantizedTensor, register_layout_class) is used
when it is importable; otherwise a minimal local QuantizedTensor with the
attributes this path reads (`_qdata`, `_layout_cls`, `_params`, `params`,
`dequantize()`) stands in, so the module also works outside ComfyUI.
Stochastic rounding (seed > 0) is ComfyUI's own routine and needs ComfyUI.

Difference: with inplace_ops=True the reference also scales the caller's
tensor in place (quant.py:65-66) as a memory saving; here the input is left
untouched (the fused kernel never materialises the scaled copy).
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from ..kernel.hip import _lib

# the quantize ops (torch.ops.feather_ops.quantize_prepack_e5m2[_scaled]) live in the C++ op library
_lib.load_torch_ops()

try:  # ComfyUI host process
    import comfy.float as _comfy_float
    from comfy.quant_ops import QuantizedLayout, QuantizedTensor, register_layout_class

    HAVE_COMFY = True
except ImportError:  # standalone use
    HAVE_COMFY = False
    _comfy_float = None
    _LAYOUTS: dict = {}

    class QuantizedLayout:  # noqa: D101 - stand-in for comfy.quant_ops.QuantizedLayout
        pass

    class QuantizedTensor:
        """Minimal stand-in for comfy.quant_ops.QuantizedTensor."""

        def __init__(self, qdata: torch.Tensor, layout_cls: str, params) -> None:
            self._qdata = qdata
            self._layout_cls = layout_cls
            self._params = params

        @property
        def params(self):
            return self._params

        @property
        def shape(self):
            return self._params.orig_shape

        @property
        def dtype(self):
            return self._params.orig_dtype

        @property
        def device(self):
            return self._qdata.device

        def dequantize(self) -> torch.Tensor:
            return _LAYOUTS[self._layout_cls].dequantize(self._qdata, self._params)

        def to(self, device=None, **kwargs):
            return QuantizedTensor(self._qdata.to(device=device), self._layout_cls, self._params.to_device(device))

    def register_layout_class(name: str, cls) -> None:
        _LAYOUTS[name] = cls


FEATHER_FP8E5M2_LAYOUT = "FeatherFP8E5M2PackedLayout"
_E5M2_DTYPE_CODES = _lib.DTYPE_CODES


def _gpu(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_cuda else t.to("cuda")


def _home(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return t if t.device == like.device else t.to(like.device)


def _as_bytes(t: torch.Tensor) -> torch.Tensor:
    if t.element_size() != 1:
        raise ValueError(f"expected a 1-byte (fp8) tensor, got {t.dtype}")
    return t


# (N, K) -> (K/16, N, 16)
def prepack_transpose(x):
    """quant.py:11-13, as a HIP chunk transpose."""
    N, K = x.shape
    if K % 16 != 0:
        raise RuntimeError(f"shape '[{N}, {K // 16}, 16]' is invalid for input of size {N * K}")
    src = _gpu(_as_bytes(x)).contiguous()
    out = torch.empty((K // 16, N, 16), dtype=x.dtype, device=src.device)
    with torch.cuda.device(src.device):
        _lib.check(_lib.lib().feather_prepack_transpose(src.data_ptr(), out.data_ptr(), N, K,
                                                        _lib.stream_ptr(src.device)), "prepack_transpose")
    return _home(out, x)


# (K/16, N, 16) -> (N, K)
def unprepack_transpose(x):
    """quant.py:17-19, as a HIP chunk transpose."""
    k, N, _ = x.shape
    src = _gpu(_as_bytes(x)).contiguous()
    out = torch.empty((N, k * 16), dtype=x.dtype, device=src.device)
    with torch.cuda.device(src.device):
        _lib.check(_lib.lib().feather_unprepack_transpose(src.data_ptr(), out.data_ptr(), N, k * 16,
                                                          _lib.stream_ptr(src.device)), "unprepack_transpose")
    return _home(out, x)


@dataclass(frozen=True)
class FeatherFP8E5M2PackedParams:
    """quant.py:22-49."""

    scale: torch.Tensor
    orig_dtype: torch.dtype
    orig_shape: tuple[int, ...]

    # the one tensor-valued field; the rest is plain metadata
    _TENSORS = ("scale",)

    def _tensor_fields(self):
        return list(self._TENSORS)

    def to_device(self, device):
        return replace(self, scale=self.scale.to(device=device))

    def clone(self):
        return replace(self, scale=self.scale.clone())

    def copy_from(self, src, non_blocking=False):
        """In-place update: the scale tensor keeps its storage, the metadata is taken from src."""
        self.scale.copy_(src.scale, non_blocking=non_blocking)
        for name in ("orig_dtype", "orig_shape"):
            object.__setattr__(self, name, getattr(src, name))


def _dtype_code(dtype: torch.dtype) -> int:
    code = _E5M2_DTYPE_CODES.get(dtype)
    if code is None:
        raise TypeError(f"FeatherOps quantization supports float16, bfloat16 and float32 inputs, got {dtype}")
    return code


def _quantize_2d(w2d: torch.Tensor, native: bool, ckpt_scale: torch.Tensor | None,
                 given_scale: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, K) GPU tensor -> ((K/16, N, 16) e5m2, fp32 scale) via the fused kernel
    (torch.ops.feather_ops.quantize_prepack_e5m2[_scaled], registered in C++)."""
    _dtype_code(w2d.dtype)
    if given_scale is not None:
        return torch.ops.feather_ops.quantize_prepack_e5m2_scaled.default(w2d, given_scale), given_scale
    return torch.ops.feather_ops.quantize_prepack_e5m2.default(w2d, ckpt_scale, native)


def _scale_arg(scale, device) -> torch.Tensor | None:
    if scale is None or (isinstance(scale, str) and scale == "recalculate"):
        return None
    if not isinstance(scale, torch.Tensor):
        return torch.tensor(scale, device=device, dtype=torch.float32)
    return scale.to(device=device, dtype=torch.float32)


def quantize_fp8e5m2_scaled(x, scale="recalculate", seed=None, inplace_ops=False):
    """quant.py:52-74: returns (x quantized to e5m2 in x's shape, fp32 scale).

    scale "recalculate"/None: s = amax|x| / 57344 (1 if 0; fp16 inputs clamp
    1/s to +-65504); otherwise the given scale. Values are x * dtype(1/s) in
    x's dtype, cast to e5m2 with round-to-nearest-even (inf at |v| >= 61440)."""
    given = _scale_arg(scale, x.device)
    if seed is not None and seed > 0:
        if not HAVE_COMFY:
            raise NotImplementedError("stochastic rounding (seed > 0) uses ComfyUI's comfy.float routine")
        return _stochastic_quantize(x, given, seed)
    flat = _gpu(x).reshape(1, -1)
    n = flat.shape[1]
    pad = (-n) % 16
    if pad:  # zeros change neither amax nor the other codes
        flat = torch.nn.functional.pad(flat, (0, pad))
    if n == 0:
        s = given if given is not None else torch.ones((), dtype=torch.float32, device=x.device)
        return torch.empty(x.shape, dtype=torch.float8_e5m2, device=x.device), s.float()
    q, s = _quantize_2d(flat, native=True, ckpt_scale=None, given_scale=given)
    q = q.reshape(-1)[:n].reshape(x.shape)
    if given is not None:
        return _home(q, x), given.float()
    return _home(q, x), _home(s, x).float()


def _stochastic_quantize(x, given, seed):
    """Reference behaviour for seed > 0 (quant.py:53-71), delegated to ComfyUI."""
    if given is None:
        s = torch.amax(x.abs()).to(dtype=torch.float32) / torch.finfo(torch.float8_e5m2).max
        s = torch.where(s == 0, torch.ones_like(s), s)
        if x.dtype not in {torch.float32, torch.bfloat16}:
            info = torch.finfo(x.dtype)
            s = 1.0 / torch.clamp(1.0 / s, min=info.min, max=info.max)
    else:
        s = given
    xs = x * (1.0 / s).to(dtype=x.dtype)
    return _comfy_float.stochastic_rounding(xs, dtype=torch.float8_e5m2, seed=seed), s.float()


class FeatherFP8E5M2PackedLayout(QuantizedLayout):
    """quant.py:77-113."""

    Params = FeatherFP8E5M2PackedParams

    @classmethod
    def quantize(cls, tensor, scale="recalculate", stochastic_rounding=0, inplace_ops=False):
        if tensor.ndim != 2:
            raise ValueError(f"Feather FP8 packed weights require a 2D tensor, got {tensor.ndim}D")
        if tensor.shape[1] % 16 != 0:
            raise ValueError(f"Feather FP8 packed weights require K divisible by 16, got {tensor.shape}")
        orig_dtype = tensor.dtype
        orig_shape = tuple(tensor.shape)
        if stochastic_rounding is not None and stochastic_rounding > 0:
            qdata, scale = quantize_fp8e5m2_scaled(tensor, scale=scale, seed=stochastic_rounding,
                                                   inplace_ops=inplace_ops)
            qdata = prepack_transpose(qdata)
        else:
            given = _scale_arg(scale, tensor.device)
            qdata, scale = _quantize_2d(_gpu(tensor), native=True, ckpt_scale=None, given_scale=given)
            qdata, scale = _home(qdata, tensor), _home(scale, tensor).float()
        params = cls.Params(scale=scale, orig_dtype=orig_dtype, orig_shape=orig_shape)
        return qdata, params

    @classmethod
    def dequantize(cls, qdata, params):
        k, N, _ = qdata.shape
        K = k * 16
        out_dtype = params.orig_dtype
        src = _gpu(qdata).contiguous()
        dev = src.device
        kernel_dtype = out_dtype if out_dtype in _E5M2_DTYPE_CODES else torch.float32
        out = torch.empty((N, K), dtype=kernel_dtype, device=dev)
        s = params.scale.reshape(1).to(device=dev, dtype=torch.float32).contiguous()
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().feather_dequantize_e5m2(src.data_ptr(), s.data_ptr(), out.data_ptr(),
                                                          _E5M2_DTYPE_CODES[kernel_dtype], N, K,
                                                          _lib.stream_ptr(dev)), "dequantize")
        if kernel_dtype != out_dtype:
            out = out.to(out_dtype)
        return _home(out, qdata)

    @classmethod
    def get_plain_tensors(cls, qtensor):
        return qtensor._qdata, qtensor._params.scale

    @classmethod
    def state_dict_tensors(cls, qdata, params):
        return {
            "": unprepack_transpose(qdata),
            "_scale": params.scale,
        }


def make_feather_quantized_weight(weight, scale, orig_dtype):
    """quant.py:116-136: load path. An e5m2 weight is only prepacked; any other
    weight is quantized from float32(weight) * scale (fused in the kernel)."""
    if weight.ndim != 2:
        raise ValueError(f"Feather FP8 packed weights require a 2D tensor, got {weight.ndim}D")
    ckpt = None if scale is None else scale.to(device=weight.device, dtype=torch.float32)
    if weight.dtype == torch.float8_e5m2:
        qdata = prepack_transpose(weight)
        out_scale = ckpt if ckpt is not None else torch.ones((), device=weight.device, dtype=torch.float32)
    else:
        if weight.shape[1] % 16 != 0:
            raise RuntimeError(f"K ({weight.shape[1]}) must be divisible by 16")
        w = weight if weight.dtype in _E5M2_DTYPE_CODES else weight.to(torch.float32)
        qdata, out_scale = _quantize_2d(_gpu(w), native=False, ckpt_scale=ckpt, given_scale=None)
        qdata, out_scale = _home(qdata, weight), _home(out_scale, weight)
    params = FeatherFP8E5M2PackedLayout.Params(scale=out_scale, orig_dtype=orig_dtype,
                                               orig_shape=tuple(weight.shape))
    return QuantizedTensor(qdata, FEATHER_FP8E5M2_LAYOUT, params)


def quantize_feather_weight(weight, seed=None, inplace_ops=False):
    """quant.py:139-146: patch path (quantize in the weight's own dtype)."""
    qdata, params = FeatherFP8E5M2PackedLayout.quantize(weight, scale="recalculate", stochastic_rounding=seed,
                                                        inplace_ops=inplace_ops)
    return QuantizedTensor(qdata, FEATHER_FP8E5M2_LAYOUT, params)


def is_feather_quantized_weight(weight):
    return isinstance(weight, QuantizedTensor) and weight._layout_cls == FEATHER_FP8E5M2_LAYOUT


def get_feather_plain_tensors(weight):
    if not is_feather_quantized_weight(weight):
        raise TypeError(f"Expected {FEATHER_FP8E5M2_LAYOUT}, got {type(weight).__name__}")
    return FeatherFP8E5M2PackedLayout.get_plain_tensors(weight)


register_layout_class(FEATHER_FP8E5M2_LAYOUT, FeatherFP8E5M2PackedLayout)
