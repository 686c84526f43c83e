"""Unmerged LoRA side path (reference comfy_feather/lora.py:4-35).

For each basic LoRA patch attached to a quantized Linear, adds
(x @ A^T) @ B^T * strength_patch * strength_model (* alpha / rank) to y. Only
the "basic LoRA" patch shape is accepted, as in the reference.

Two forms:
  * apply_lora_patches(x, y, weight_functions): the reference's separate pass,
    y += F.linear(F.linear(x, down), up) * s per patch;
  * lora_factors(x, weight_functions): the factors of the same term for the
    GEMM's fused epilogue -- T = [F.linear(x, down_i) * s_i]_i (M, R) and
    U = [up_i]_i (N, R), concatenated over the patches along the rank and
    zero-padded to a multiple of 32, in x's dtype. The GEMM then adds T . U^T
    to its fp32 accumulator before rounding, so C is written once.
"""

import torch
import torch.nn.functional as F


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


def lora_factors(x: torch.Tensor, weight_functions):
    """(T, U) for the fused epilogue, or None when there is no patch or x is not
    fp16/bf16 (then the separate pass keeps the reference's fp32 arithmetic)."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        return None
    patches = _basic_patches(weight_functions)
    if not patches:
        return None
    ts, us = [], []
    for down, up, scale in patches:
        down = down.to(device=x.device, dtype=x.dtype)
        up = up.to(device=x.device, dtype=x.dtype)
        ts.append((F.linear(x, down).float() * scale).to(x.dtype))
        us.append(up)
    rank = sum(t.shape[1] for t in ts)
    pad = (-rank) % 32
    if pad:
        ts.append(x.new_zeros(x.shape[0], pad))
        us.append(x.new_zeros(us[0].shape[0], pad))
    t = torch.cat(ts, dim=1) if len(ts) > 1 else ts[0].contiguous()
    u = torch.cat(us, dim=1) if len(us) > 1 else us[0].contiguous()
    return t, u
