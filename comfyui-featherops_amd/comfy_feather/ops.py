"""Linear replacement that runs the fp16 x e5m2 kernel (reference comfy_feather/ops.py).

`feather_ops(out_dtype, excluded_names)` returns an operations class for
ComfyUI's `custom_operations` hook whose `Linear`:
  * at state-dict load quantizes the weight to prepacked e5m2 on the GPU
    (make_feather_quantized_weight) unless the layer is excluded, 1-wide, or
    has in_features % 16 != 0 (ops.py:31-64);
  * in forward casts x to fp16, runs the scaled_mm kernel with the weight
    scale and bias, casts back to the input dtype and applies basic LoRA
    patches (ops.py:85-146). The reference pads the flattened M to a multiple
    of 16/32/64/128 (a copy) and slices the result (another copy) because its
    kernel has no row masking; the gfx950 kernels mask rows past M, so by
    default M is passed as is (`pad_m=True` on the class restores the
    reference's padding + autotuned scaled_mm_hip call).

Inside ComfyUI it subclasses comfy.ops.manual_cast. Without ComfyUI, a
minimal base (plain nn.Linear; weight/bias used as stored) stands in so the
layer can be used and tested on its own.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from ..kernel.hip.hip_kernel import scaled_mm_hip, scaled_mm_hip_any_m, scaled_mm_hip_any_m_lora
from .lora import apply_lora_patches, lora_factors
from .quant import (
    HAVE_COMFY,
    get_feather_plain_tensors,
    is_feather_quantized_weight,
    make_feather_quantized_weight,
    quantize_feather_weight,
)

if HAVE_COMFY:
    from comfy.ops import cast_bias_weight, manual_cast, run_every_op, uncast_bias_weight
else:

    class manual_cast:  # noqa: N801 - mirrors comfy.ops.manual_cast
        class Linear(nn.Linear):
            comfy_cast_weights = True

            def __init__(self, *args, **kwargs):
                kwargs.pop("dtype", None)
                kwargs.pop("device", None)
                super().__init__(*args, **kwargs)
                self.weight_function = []
                self.bias_function = []

    def run_every_op() -> None:
        return None

    def cast_bias_weight(s, input=None, dtype=None, device=None, bias_dtype=None, offloadable=False, **kwargs):
        weight = s.weight
        bias = s.bias
        if input is not None and isinstance(weight, torch.Tensor) and weight.device != input.device:
            weight = weight.to(input.device)
        if bias is not None and input is not None:
            bias = bias.to(device=input.device, dtype=bias_dtype or bias.dtype)
        return weight, bias, None

    def uncast_bias_weight(s, weight, bias, offload_stream) -> None:
        return None


def _set_weight(module: nn.Module, weight) -> None:
    """Store `weight` as the module's weight (a Parameter when it is a tensor)."""
    if isinstance(weight, torch.Tensor):
        module.weight = nn.Parameter(weight, requires_grad=False)
    else:  # stand-in QuantizedTensor outside ComfyUI
        module._parameters.pop("weight", None)
        object.__setattr__(module, "weight", weight)


def _m_block(m: int) -> int:
    """ops.py:126-133: M padding granularity."""
    if m > 256:
        return 128
    if m > 128:
        return 64
    if m > 64:
        return 32
    return 16


def feather_ops(out_dtype=torch.bfloat16, excluded_names=()):
    excluded_names = tuple(excluded_names)

    class FeatherOps(manual_cast):
        _excluded_names = excluded_names
        _out_dtype = out_dtype

        class Linear(manual_cast.Linear):
            pad_m = False
            fuse_lora = True

            def __init__(self, *args, **kwargs):
                super().__init__(*args, **kwargs)
                self.excluded_names = FeatherOps._excluded_names
                self.out_dtype = FeatherOps._out_dtype
                self.is_quantized = False

            def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs):
                weight = state_dict.pop(prefix + "weight", None)
                bias = state_dict.pop(prefix + "bias", None)
                weight_scale = state_dict.pop(prefix + "weight_scale", None)
                if weight_scale is None:
                    weight_scale = state_dict.pop(prefix + "scale_weight", None)

                if weight is not None:
                    excluded = any(x in prefix for x in self.excluded_names)
                    dim1 = self.in_features == 1 or self.out_features == 1 or weight.ndim == 1
                    if excluded or dim1 or self.in_features % 16 != 0:
                        if self.in_features % 16 != 0:
                            print(f"Warning: Not prepacked {prefix + 'weight'} {tuple(weight.shape)}")
                        self.is_quantized = False
                        _set_weight(self, weight)
                    else:
                        self.is_quantized = True
                        _set_weight(self, make_feather_quantized_weight(weight, weight_scale, self.out_dtype))
                else:
                    missing_keys.append(prefix + "weight")

                if bias is not None:
                    self.bias = nn.Parameter(bias.to(self.out_dtype), requires_grad=False)
                else:
                    self.bias = None

            def convert_weight(self, weight, inplace=False, **kwargs):
                if not self.is_quantized:
                    return weight
                if not is_feather_quantized_weight(weight):
                    raise TypeError(f"Expected Feather quantized weight, got {type(weight).__name__}")
                return weight.dequantize()

            def set_weight(self, weight, inplace_update=False, seed=None, return_weight=False, **kwargs):
                if not self.is_quantized:
                    weight = weight.to(self.weight.dtype)
                else:
                    weight = quantize_feather_weight(weight, seed=seed, inplace_ops=True)
                if return_weight:
                    return weight
                assert inplace_update is False
                _set_weight(self, weight)

            def _forward_padded(self, x, lora=None):
                dtype_orig = x.dtype
                x = x.contiguous()
                if self.pad_m or x.dtype != torch.bfloat16:
                    # (bf16 activations go to the any-M entry as they are: the
                    # kernel rounds them to fp16 itself, the same values as this cast)
                    x = x.to(torch.float16)
                # no low-VRAM weight patches on the prepacked weight while casting
                saved_weight_function = self.weight_function
                self.weight_function = []
                bias_dtype = self.bias.dtype if self.bias is not None else None
                weight, bias, offload_stream = cast_bias_weight(self, x, dtype=getattr(self.weight, "dtype", None),
                                                                bias_dtype=bias_dtype, offloadable=True)
                weight, scale = get_feather_plain_tensors(weight)
                scale = scale.to(device=x.device, dtype=torch.float32)
                if self.pad_m:
                    y = scaled_mm_hip(x, weight, scale, bias, out_dtype=self.out_dtype)
                elif lora is not None:
                    y = scaled_mm_hip_any_m_lora(x, weight, scale, bias, self.out_dtype, *lora)
                else:
                    y = scaled_mm_hip_any_m(x, weight, scale, bias, self.out_dtype)
                uncast_bias_weight(self, weight, bias, offload_stream)
                self.weight_function = saved_weight_function
                return y.to(dtype_orig)

            def forward(self, input: torch.Tensor) -> torch.Tensor:
                x = input
                del input
                run_every_op()
                if not self.is_quantized:
                    weight, bias, offload_stream = cast_bias_weight(self, x, offloadable=True)
                    y = F.linear(x, weight, bias)
                    uncast_bias_weight(self, weight, bias, offload_stream)
                    return y

                shape = x.shape
                x = x.reshape(-1, shape[-1])
                m = x.shape[0]
                if m == 0:
                    return x.new_empty(*shape[:-1], self.out_features)
                if self.pad_m:
                    block = _m_block(m)
                    m_padded = (m + block - 1) // block * block
                    x_padded = F.pad(x, (0, 0, 0, m_padded - m)) if m_padded != m else x
                    y = self._forward_padded(x_padded)[:m]
                    y = apply_lora_patches(x, y, self.weight_function)
                else:
                    # basic LoRA patches go into the GEMM's epilogue (one pass over C)
                    if self.fuse_lora:
                        cache = self.__dict__.setdefault("_lora_factor_cache", {})
                        lora = lora_factors(x, self.weight_function, cache)
                    else:
                        lora = None
                    y = self._forward_padded(x, lora)
                    if lora is None:
                        y = apply_lora_patches(x, y, self.weight_function)
                return y.view(*shape[:-1], y.shape[-1])

    return FeatherOps
