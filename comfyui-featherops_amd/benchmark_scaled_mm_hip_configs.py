#!/usr/bin/env python3
"""Per-config sweep of scaled_mm_hip_configured over one or more shapes.

Same command line and report as the reference's benchmark_scaled_mm_hip_configs.py:
--shapes "M,N,K;M,N,K", --configs "wm,wn,u,rm,rn;..." (default: every entry of
_CONFIGS whose block sizes divide the shape, plus the library's shape-based pick
and the any-M entry), --rep / --warmup in ms per config, --no-scale, --no-bias;
one line per config with avg_ms, std_ms and avg_TFLOPS. Timing uses HIP events
on torch's current stream (no Triton). Extra: --out fp16|bf16 and the kernel id
each config runs (several reference tuples share a gfx950 kernel).

Run from this folder (the plugin root), as the reference's script is run from its
repository root: python benchmark_scaled_mm_hip_configs.py --shapes 4096,3072,3072
"""

from __future__ import annotations

import argparse
import statistics
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
from _bench_common import load_plugin, time_calls  # noqa: E402

load_plugin()
from featherops_amd.kernel.hip.hip_kernel import (  # noqa: E402
    _CONFIGS, any_m_config, kernel_id, prepack_b_for_scaled_mm, scaled_mm_hip_any_m, scaled_mm_hip_configured)
from featherops_amd.kernel.hip.utils import _config_compatible  # noqa: E402


def _parse_tuples(text: str, width: int, what: str) -> list[tuple[int, ...]]:
    out = []
    for chunk in text.split(";"):
        chunk = chunk.strip()
        if not chunk:
            continue
        parts = [p.strip() for p in chunk.split(",")]
        if len(parts) != width:
            raise ValueError(f"Invalid {what} '{chunk}', expected {width} comma-separated ints")
        out.append(tuple(int(p) for p in parts))
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", type=str, default="8192,8192,8192",
                    help="Semicolon-separated M,N,K tuples, e.g. '32,3072,3072;8192,12288,3072'")
    ap.add_argument("--configs", type=str, default="", help="Semicolon-separated configs, empty for all")
    ap.add_argument("--rep", type=int, default=1000, help="Repetition time (in ms) per config")
    ap.add_argument("--warmup", type=int, default=100, help="Warmup time (in ms) per config")
    ap.add_argument("--no-scale", action="store_true")
    ap.add_argument("--no-bias", action="store_true")
    ap.add_argument("--out", choices=["fp16", "bf16"], default="fp16")
    args = ap.parse_args()

    shapes = _parse_tuples(args.shapes, 3, "shape")
    configs = _parse_tuples(args.configs, 5, "config") if args.configs else list(_CONFIGS)
    out_dtype = torch.float16 if args.out == "fp16" else torch.bfloat16
    dev = "cuda"
    for m, n, k in shapes:
        print(f"\nShape M={m} N={n} K={k}")
        a = torch.randn(m, k, device=dev, dtype=torch.float32).to(torch.float16)
        b = torch.randn(k, n, device=dev, dtype=torch.float32).to(torch.float8_e5m2)
        scale = None if args.no_scale else torch.tensor(2.34, device=dev, dtype=torch.float32)
        bias = None if args.no_bias else torch.randn(n, device=dev, dtype=torch.float32).to(out_dtype)
        bp = prepack_b_for_scaled_mm(b)
        runs = []
        for cfg in configs:
            if not args.configs and not _config_compatible(cfg, m, n, k):
                continue
            runs.append((f"cfg=({','.join(map(str, cfg))})", kernel_id(m, n, k, cfg),
                         lambda cfg=cfg: scaled_mm_hip_configured(a, bp, scale, bias, out_dtype, *cfg)))
        if not args.configs:
            pick = any_m_config(m, n, k)
            runs.append((f"any_m pick=({','.join(map(str, pick))})", kernel_id(m, n, k, pick),
                         lambda: scaled_mm_hip_any_m(a, bp, scale, bias, out_dtype)))
        for label, kid, fn in runs:
            t = time_calls(fn, args.warmup, args.rep)
            avg = statistics.mean(t)
            std = statistics.pstdev(t) if len(t) > 1 else 0.0
            print(f"  {label} kernel={kid} avg_ms={avg:.3f} std_ms={std:.3f} "
                  f"avg_TFLOPS={2 * m * n * k / avg * 1e-9:.3f}")


if __name__ == "__main__":
    main()
