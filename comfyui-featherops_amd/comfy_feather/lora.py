"""Unmerged LoRA side path (reference comfy_feather/lora.py:4-35).

For each basic LoRA patch attached to a quantized Linear, adds
(x @ A^T) @ B^T * strength_patch * strength_model (* alpha / rank) to y. Only
the "basic LoRA" patch shape is accepted, as in the reference.
"""

import torch.nn.functional as F


def apply_lora_patches(x, y, weight_functions):
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
            down = down.to(device=x.device, dtype=x.dtype)
            up = up.to(device=x.device, dtype=x.dtype)
            y += F.linear(F.linear(x, down), up) * scale
    return y
