"""Shared pieces of the plugin-root benchmark scripts: importing the plugin folder
(whose name is not a Python identifier) as `featherops_amd`, and timing a
callable with HIP events on torch's current stream (no Triton).
"""

from __future__ import annotations

import importlib.util
import statistics
import sys
from pathlib import Path

import torch

PLUGIN_ROOT = Path(__file__).resolve().parent


def load_plugin():
    """Import the plugin folder as the package `featherops_amd` (once)."""
    if "featherops_amd" in sys.modules:
        return sys.modules["featherops_amd"]
    spec = importlib.util.spec_from_file_location("featherops_amd", PLUGIN_ROOT / "__init__.py",
                                                  submodule_search_locations=[str(PLUGIN_ROOT)])
    pkg = importlib.util.module_from_spec(spec)
    sys.modules["featherops_amd"] = pkg
    spec.loader.exec_module(pkg)
    return pkg


def time_calls(fn, warmup_ms: float, rep_ms: float) -> list[float]:
    """Per-call milliseconds of fn: ~warmup_ms of untimed calls, then ~rep_ms of
    calls each bracketed by its own pair of HIP events."""
    fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(5):
        fn()
    e.record()
    e.synchronize()
    est = max(s.elapsed_time(e) / 5, 1e-3)
    for _ in range(max(1, int(warmup_ms / est))):
        fn()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(max(1, int(rep_ms / est)))]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in evs]


def quantiles(times: list[float], qs=(0.5, 0.2, 0.8)) -> list[float]:
    """The given quantiles of the per-call times (the reference's scripts report
    the median with the 0.2 / 0.8 quantiles)."""
    if len(times) == 1:
        return [times[0]] * len(qs)
    cuts = statistics.quantiles(times, n=100, method="inclusive")
    return [statistics.median(times) if q == 0.5 else cuts[int(round(q * 100)) - 1] for q in qs]


def parse_ints(text: str) -> list[int]:
    return [int(p) for p in text.replace(";", ",").split(",") if p.strip()]
