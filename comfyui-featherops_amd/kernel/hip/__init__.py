"""HIP kernels for gfx950 and their torch bindings."""
