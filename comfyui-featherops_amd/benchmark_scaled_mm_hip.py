#!/usr/bin/env python3
"""TFLOPS of scaled_mm_hip over square N x N x N GEMMs, beside torch.

The counterpart of the reference's benchmark_scaled_mm_hip.py: A (N, N) fp16 from
randn, B (N, N) e5m2 from randn (prepacked once, outside the timing), scale 2.34,
fp16 bias, fp16 out; N = 128 ... 8192; 2 N^3 flop per call; the median with the
0.2 / 0.8 quantiles of per-call HIP-event times. Providers:
  * torch: the same product in eager torch on the device -- the weight decoded
    to fp16 and multiplied with torch's fp16 matmul, then the scale in fp32, the
    cast and the bias (the steps of the reference's kernel/naive.py);
  * hip: scaled_mm_hip (this plugin's kernels, the tile picked by shape).
The reference's third provider, naive.py under torch.compile, is left out: its
kernels would come from Inductor's Triton backend.

Run from this folder (the plugin root): python benchmark_scaled_mm_hip.py
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
from featherops_amd.kernel.hip.hip_kernel import prepack_b_for_scaled_mm, scaled_mm_hip  # noqa: E402


def torch_scaled_mm(a, b, scale, bias, out_dtype):
    c = a @ b.to(torch.float16)
    if scale is not None:
        c = c.float() * scale.float()
    c = c.to(out_dtype)
    if bias is not None:
        c = c + bias.to(out_dtype)
    return c


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--sizes", type=str, default="128,256,512,1024,2048,4096,8192", help="N values, comma-separated")
    ap.add_argument("--rep", type=float, default=1000, help="timed milliseconds per point")
    ap.add_argument("--warmup", type=float, default=100, help="untimed milliseconds per point")
    args = ap.parse_args()
    providers = ["torch", "hip"]
    rows = []
    dev = "cuda"
    for n in parse_ints(args.sizes):
        gc.collect()
        torch.cuda.empty_cache()
        a = torch.randn((n, n), device=dev, dtype=torch.float32).to(torch.float16)
        b = torch.randn((n, n), device=dev, dtype=torch.float32).to(torch.float8_e5m2)
        scale = torch.tensor(2.34, device=dev, dtype=torch.float32)
        bias = torch.randn(n, device=dev, dtype=torch.float16)
        bp = prepack_b_for_scaled_mm(b)
        fns = {"torch": lambda: torch_scaled_mm(a, b, scale, bias, torch.float16),
               "hip": lambda: scaled_mm_hip(a, bp, scale, bias, torch.float16)}
        row = [n]
        for p in providers:
            print("N", n, "provider", p, "begin", flush=True)
            med, lo, hi = quantiles(time_calls(fns[p], args.warmup, args.rep))
            tf = lambda ms: 2 * n**3 / ms * 1e-9
            print("N", n, "provider", p, "end", tf(med), flush=True)
            row.append(tf(med))
        rows.append(row)
    print("scaled_mm_hip (TFLOPS, median per call):")
    print(f"{'N':>8}" + "".join(f"{p:>12}" for p in providers))
    for r in rows:
        print(f"{r[0]:>8}" + "".join(f"{v:>12.3f}" for v in r[1:]))


if __name__ == "__main__":
    with torch.inference_mode():
        main()
