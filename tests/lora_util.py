"""Stand-ins for ComfyUI's weight-function patch objects (the shape
comfy_feather/lora.py reads: patch_fn.patches[patch_fn.key] is a list of
(strength_patch, adapter, strength_model, ...) with adapter.weights =
(up, down, alpha, ...)), shared by the CPU and GPU LoRA tests."""

from types import SimpleNamespace

import torch


def make_patches(N, K, ranks, gen, device="cpu", dtype=torch.float32, alpha=True):
    """One weight function holding a basic LoRA patch per rank; returns
    (weight_functions, [(down, up, scale)]) with the effective scale of each."""
    patches, expect = [], []
    for i, r in enumerate(ranks):
        down = (torch.randn(r, K, generator=gen) * 0.05).to(dtype).to(device)
        up = (torch.randn(N, r, generator=gen) * 0.05).to(dtype).to(device)
        a = float(r) * 0.5 if alpha else None
        sp, sm = 0.8 + 0.1 * i, 1.25
        patches.append((sp, SimpleNamespace(weights=(up, down, a, None)), sm, None, None))
        expect.append((down, up, sp * sm * (a / r if a is not None else 1.0)))
    return [SimpleNamespace(patches={"w": patches}, key="w")], expect
