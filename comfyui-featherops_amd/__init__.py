"""FeatherOps for MI355X (gfx950): the fp16 x fp8-e5m2 `scaled_mm` hot path.

ComfyUI imports this directory as a custom-node package. The callers of the
hot path are `kernel.hip.hip_kernel` (scaled_mm_hip and friends),
`comfy_feather.quant` (quantize / prepack) and `comfy_feather.ops`
(`feather_ops`, the Linear replacement); all of them run hand-written HIP
kernels from `lib/libfeatherops_amd.so` (built by `build.py`).

The reference's model-loader node (comfy_feather/loader.py) is not part of
this package, so no node classes are registered.
"""

NODE_CLASS_MAPPINGS: dict = {}
NODE_DISPLAY_NAME_MAPPINGS: dict = {}
