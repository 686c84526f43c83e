#!/usr/bin/env python3
"""A fixed scaled_mm_hip_configured workload for running under a profiler.

The counterpart of the reference's profile_scaled_mm_hip.py, with the same
command line: -N (square size, default 8192), --iters (default 10), --config
(default 1,8,4,8,2), --no-scale, --no-bias. Three untimed warm-up calls, then
--iters calls, fp16 out. For example, from this folder (the plugin root):
    rocprofv3 --kernel-trace --stats -d prof -- python3 profile_scaled_mm_hip.py
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
from _bench_common import load_plugin  # noqa: E402

load_plugin()
from featherops_amd.kernel.hip.hip_kernel import (  # noqa: E402
    kernel_id, prepack_b_for_scaled_mm, scaled_mm_hip_configured)


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--no-scale", action="store_true")
    parser.add_argument("--no-bias", action="store_true")
    parser.add_argument("-N", type=int, default=8192, help="Matrix size (N x N)")
    parser.add_argument("--iters", type=int, default=10, help="Number of iterations to profile")
    parser.add_argument("--config", type=str, default="1,8,4,8,2", help="Specific config to use, e.g. 1,8,4,8,2")
    args = parser.parse_args()

    device = "cuda"
    m = n = k = args.N
    print(f"Allocating tensors (N={args.N})...")
    a = torch.randn((m, k), device=device, dtype=torch.float32).to(torch.float16)
    b = torch.randn((k, n), device=device, dtype=torch.float32).to(torch.float8_e5m2)
    b_prepacked = prepack_b_for_scaled_mm(b)
    scale = None if args.no_scale else torch.tensor(2.34, device=device, dtype=torch.float32)
    bias = None if args.no_bias else torch.randn(n, device=device, dtype=torch.float16)
    cfg = tuple(int(x.strip()) for x in args.config.split(","))
    print(f"Config {cfg} runs kernel {kernel_id(m, n, k, cfg)}")

    def run_fn():
        return scaled_mm_hip_configured(a, b_prepacked, scale, bias, torch.float16, *cfg)

    print("Warming up...")
    for _ in range(3):
        run_fn()
    torch.cuda.synchronize()
    print(f"Profiling {args.iters} iterations...")
    for _ in range(args.iters):
        run_fn()
    torch.cuda.synchronize()
    print("Done")


if __name__ == "__main__":
    main()
