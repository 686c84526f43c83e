"""ComfyUI-facing layer of the hot path: quantized weights and the Linear replacement."""
