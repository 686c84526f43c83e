#!/usr/bin/env python3
"""GB/s of the bf16 -> fp16 casts over N x N tensors, beside torch.

The counterpart of the reference's benchmark_convert.py: x (N, N) bf16 from randn,
N = 1024 ... 16384, 4 N^2 bytes per call (2 read, 2 written); the median with the
0.2 / 0.8 quantiles of per-call HIP-event times. Providers:
  * torch: x.to(torch.float16) (round to nearest even, inf past the fp16 range);
  * hip: kernel.convert.bf16_to_fp16 (the reference's round-toward-zero cast,
    saturating at +-65504);
  * hip_rne: the library's round-to-nearest-even cast (the values of
    x.to(torch.float16)), which the any-M entry runs before the large GEMM tiles
    for bf16 activations.
The reference's compiled-torch provider is left out (Inductor's Triton backend).

Run from this folder (the plugin root): python benchmark_convert.py
"""

from __future__ import annotations

import argparse
import gc
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
from _bench_common import load_plugin, parse_ints, quantiles, time_calls  # noqa: E402

load_plugin()
from featherops_amd.kernel.convert import bf16_to_fp16, bf16_to_fp16_rne  # noqa: E402


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--sizes", type=str, default="1024,2048,4096,8192,16384", help="N values, comma-separated")
    ap.add_argument("--rep", type=float, default=1000, help="timed milliseconds per point")
    ap.add_argument("--warmup", type=float, default=100, help="untimed milliseconds per point")
    args = ap.parse_args()
    providers = {"torch": lambda x: x.to(torch.float16), "hip": bf16_to_fp16, "hip_rne": bf16_to_fp16_rne}
    rows = []
    for n in parse_ints(args.sizes):
        gc.collect()
        torch.cuda.empty_cache()
        x = torch.randn((n, n), device="cuda", dtype=torch.bfloat16)
        row = [n]
        for name, f in providers.items():
            print("N", n, "provider", name, "begin", flush=True)
            med, lo, hi = quantiles(time_calls(lambda: f(x), args.warmup, args.rep))
            gbs = 4 * n * n / med * 1e-6
            print("N", n, "provider", name, "end", gbs, flush=True)
            row.append(gbs)
        rows.append(row)
    print("convert_bf16_to_fp16 (GB/s, median per call):")
    print(f"{'N':>8}" + "".join(f"{p:>12}" for p in providers))
    for r in rows:
        print(f"{r[0]:>8}" + "".join(f"{v:>12.1f}" for v in r[1:]))


if __name__ == "__main__":
    with torch.inference_mode():
        main()
