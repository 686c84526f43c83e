"""Unmerged LoRA side path (reference comfy_feather/lora.py:4-35).

For each basic LoRA patch attached to a quantized Linear, adds
(x @ A^T) @ B^T * strength_patch * strength_model (* alpha / rank) to y. Only
the "basic LoRA" patch shape is accepted, as in the reference.

Two forms:
  * apply_lora_patches(x, y, weight_functions): the reference's separate pass,
    y += F.linear(F.linear(x, down), up) * s per patch;
  * lora_factors(x, weight_functions): the factors of the same term for the
    GEMM's fused epilogue -- T = F.linear(x, [down_i * s_i]_i) (M, R), computed
    by the library's down-projection kernel (lora_down), and
    U = [up_i]_i (N, R), stacked over the patches along the rank and
    zero-padded to a multiple of 32, in x's dtype. The GEMM then adds T . U^T
    to its fp32 accumulator before rounding, so C is written once.
"""

import torch
import torch.nn.functional as F

from ..kernel.hip import _lib


def _basic_patches(weight_functions):
    """(down, up, scale) of every basic LoRA patch; NotImplementedError for any
    other patch shape (the reference's rule)."""
    out = []
    for patch_fn in weight_functions:
        if not (hasattr(patch_fn, "patches") and hasattr(patch_fn, "key")):
            raise NotImplementedError("FeatherOps currently only supports basic LoRA")
        for patch in patch_fn.patches.get(patch_fn.key, []):
            strength_patch, adapter, strength_model = patch[0], patch[1], patch[2]
            weights = getattr(adapter, "weights", None)
            if weights is None:
                raise NotImplementedError("FeatherOps currently only supports basic LoRA")
            up, down, alpha = weights[0], weights[1], weights[2]
            scale = strength_patch * strength_model
            if alpha is not None:
                scale *= alpha / down.shape[0]
            out.append((down, up, scale))
    return out


def apply_lora_patches(x, y, weight_functions):
    for down, up, scale in _basic_patches(weight_functions):
        down = down.to(device=x.device, dtype=x.dtype)
        up = up.to(device=x.device, dtype=x.dtype)
        y += F.linear(F.linear(x, down), up) * scale
    return y


def _stacked_factors(x: torch.Tensor, patches):
    """[down_i * s_i]_i (R, K) and [up_i]_i (N, R) in x's dtype on x's device,
    the rank zero-padded to a multiple of 32."""
    downs, ups = [], []
    for down, up, scale in patches:
        downs.append((down.to(device=x.device, dtype=torch.float32) * scale).to(x.dtype))
        ups.append(up.to(device=x.device, dtype=x.dtype))
    rank = sum(d.shape[0] for d in downs)
    pad = (-rank) % 32
    if pad:
        downs.append(x.new_zeros(pad, downs[0].shape[1]))
        ups.append(x.new_zeros(ups[0].shape[0], pad))
    d = torch.cat(downs, dim=0) if len(downs) > 1 else downs[0].contiguous()
    u = torch.cat(ups, dim=1) if len(ups) > 1 else ups[0].contiguous()
    return d, u


def lora_factors(x: torch.Tensor, weight_functions, cache: dict | None = None):
    """(T, U) for the fused epilogue, or None when there is no patch or x is not
    fp16/bf16 (then the separate pass keeps the reference's fp32 arithmetic).

    T comes from one F.linear of x with every patch's down matrix, scaled by its
    strength and stacked along the rank, zero rows padding the rank to a
    multiple of 32; U stacks the up matrices to match (zero columns).

    `cache` (a dict the caller keeps, e.g. one per layer) holds the stacked
    matrices between calls. An entry is reused only while the patch list holds
    the same tensor objects, unmodified in place (version counters), with the
    same strengths, and x has the same dtype and device; the entry keeps the
    tensors themselves, so their ids cannot be recycled while it lives."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        return None
    patches = _basic_patches(weight_functions)
    if not patches:
        return None
    if cache is None:
        d, u = _stacked_factors(x, patches)
    else:
        key = (x.dtype, x.device, tuple((id(dn), dn._version, id(up), up._version, float(sc))
                                        for dn, up, sc in patches))
        hit = cache.get("entry")
        if hit is not None and hit[0] == key:
            d, u = hit[2], hit[3]
        else:
            d, u = _stacked_factors(x, patches)
            cache["entry"] = (key, [(dn, up) for dn, up, _ in patches], d, u)
    return lora_down(x, d), u


def lora_down(x: torch.Tensor, d: torch.Tensor) -> torch.Tensor:
    """T = F.linear(x, d) on the library's skinny-GEMM kernel (torch.ops.feather_ops.lora_down:
    fp32 accumulation, rounded to x's dtype); torch's F.linear wherever the kernel's entry would
    refuse the operands: x not on the GPU, K not a multiple of 8 (16-byte row loads), ranks not a
    multiple of 32 or above 65536, K >= 2^24, or a storage offset that leaves x or d off a
    16-byte boundary."""
    x2 = x.reshape(-1, x.shape[-1])
    K, R = x2.shape[1], d.shape[0]
    if x2.is_cuda and K % 8 == 0 and R % 32 == 0 and R <= 65536 and K < (1 << 24):
        x2 = x2.contiguous()
        dc = d.contiguous()
        if x2.data_ptr() % 16 == 0 and dc.data_ptr() % 16 == 0:
            _lib.load_torch_ops()
            t = torch.ops.feather_ops.lora_down.default(x2, dc)
            return t.reshape(*x.shape[:-1], R)
    return F.linear(x, d).contiguous()
