"""Config compatibility and autotuning helpers for the scaled_mm op.

Mirrors the public helpers of the reference's kernel/hip/utils.py:132-223
(`_config_compatible`, `generate_autotune_configs`, `get_compatible_config`,
`old_autotune`) with the same names, arguments and errors. Differences by
design:
  * timing uses HIP events on the current stream (no Triton);
  * several reference configurations run the same gfx950 kernel, so
    `old_autotune` times each distinct kernel once.
The reference's extension-building helpers are replaced by build.py.
"""

from __future__ import annotations

import os
import threading
from collections.abc import Callable

import torch

Config = tuple[int, int, int, int, int]


def _config_compatible(cfg: Config, M: int, N: int, K: int) -> bool:
    """Divisibility rule of utils.py:132-142: BlockM = 16*wm*rm, BlockN =
    16*wn*rn, ChunkK = 16*u must divide M, N, K; large shapes need blocks >= 64."""
    warps_m, warps_n, unroll_k, repeat_m, repeat_n = cfg
    block_m = 16 * warps_m * repeat_m
    block_n = 16 * warps_n * repeat_n
    chunk_k = 16 * unroll_k
    if M % block_m != 0 or N % block_n != 0 or K % chunk_k != 0:
        return False
    is_large = K >= 3072 and min(M, N) >= 3072 and max(M, N) >= 4096
    return not (is_large and (block_m < 64 or block_n < 64))


def _size_hint(value) -> int:
    try:
        return int(value)
    except TypeError:
        from torch.fx.experimental.symbolic_shapes import hint_int

        return hint_int(value)


def generate_autotune_configs(fake_tensors: dict, configs: list[Config], b_dim: int,
                              decomposition: Callable | None = None) -> list:
    """Inductor config generator (utils.py:152-175). `decomposition`, when given, is the
    function each config runs (else Inductor runs the op's own implementation)."""
    from torch._inductor.kernel.custom_op import CustomOpConfig

    a = fake_tensors["a"]
    b_prepacked = fake_tensors["b_prepacked"]
    M = _size_hint(a.shape[0])
    N = _size_hint(b_prepacked.shape[b_dim])
    K = _size_hint(a.shape[1])
    compatible = [cfg for cfg in configs if _config_compatible(cfg, M, N, K)]
    if not compatible:
        raise RuntimeError(f"No compatible config for M={M} N={N} K={K}.")
    return [
        CustomOpConfig(decomposition, block_warps_m=c[0], block_warps_n=c[1], unroll_k=c[2], repeat_m=c[3],
                       repeat_n=c[4])
        for c in compatible
    ]


def get_compatible_config(a: torch.Tensor, b_prepacked: torch.Tensor, b_dim: int, configs: list[Config]) -> Config:
    """First compatible config in list order (utils.py:178-185)."""
    M = _size_hint(a.shape[0])
    N = _size_hint(b_prepacked.shape[b_dim])
    K = _size_hint(a.shape[1])
    for cfg in configs:
        if _config_compatible(cfg, M, N, K):
            return cfg
    raise RuntimeError(f"No compatible config for M={M} N={N} K={K}.")


def do_bench(fn: Callable[[], object], warmup_ms: float = 25.0, rep_ms: float = 100.0) -> float:
    """Median milliseconds of `fn` timed with HIP events on the current stream."""
    fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(5):
        fn()
    end.record()
    end.synchronize()
    est = max(start.elapsed_time(end) / 5, 1e-3)
    n_warm = max(1, int(warmup_ms / est))
    n_rep = max(1, int(rep_ms / est))
    for _ in range(n_warm):
        fn()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_rep)]
    for s, e in evs:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    times = sorted(s.elapsed_time(e) for s, e in evs)
    return times[len(times) // 2]


_AUTOTUNE_CACHE: dict = {}
_AUTOTUNE_LOCK = threading.Lock()


def old_autotune(M: int, N: int, K: int, configs: list[Config], run_fn: Callable[[Config], object],
                 *extra_keys: object, kernel_id: Callable[[Config], int] | None = None) -> Config:
    """Eager per-shape autotune with a module-level cache (utils.py:188-223).

    `kernel_id(cfg)` names the kernel a config runs; configs sharing a kernel
    are timed once (the first in list order represents them)."""
    key = (M, N, K, *extra_keys)
    cached = _AUTOTUNE_CACHE.get(key)
    if cached is not None:
        return cached
    candidates = [c for c in configs if _config_compatible(c, M, N, K)]
    if not candidates:
        raise RuntimeError(f"No compatible config for M={M} N={N} K={K}.")
    if kernel_id is not None:
        seen: set[int] = set()
        unique = []
        for c in candidates:
            kid = kernel_id(c)
            if kid not in seen:
                seen.add(kid)
                unique.append(c)
        candidates = unique
    warmup_ms = max(1, int(os.environ.get("AUTOTUNE_WARMUP_MS", "25")))
    rep_ms = max(1, int(os.environ.get("AUTOTUNE_REP_MS", "100")))
    best_cfg = candidates[0]
    best_ms = None
    if len(candidates) > 1:
        for cfg in candidates:
            ms = do_bench(lambda cfg=cfg: run_fn(cfg), warmup_ms, rep_ms)
            if best_ms is None or ms < best_ms:
                best_ms, best_cfg = ms, cfg
    with _AUTOTUNE_LOCK:
        _AUTOTUNE_CACHE[key] = best_cfg
    if best_ms is not None:
        print(f"autotune key={key} cfg={best_cfg} time={best_ms:.3f} ms")
    return best_cfg
