#!/usr/bin/env python3
"""Headline benchmark: fp16 x fp8-e5m2 scaled_mm on one MI355X.

One step = one launch of the scaled_mm hot path (torch.ops.feather_ops.scaled_mm,
i.e. launch_scaled_mm of libfeatherops_amd.so) on the BASELINE headline shape
M=32768, K=5120, N=13824 (config 4, video-DiT FFN up-projection), fp16 out,
per-tensor scale and bias, inputs resident in HBM. The weight is a synthetic
~N(0, 0.02) fp16 matrix quantized and prepacked on the device by the
quantize kernel; A ~ N(0, 1).

Also measured in the same run (extra keys of the JSON line):
  small_m     config 2 (M=16, K=N=4096): GB/s, rotating over enough distinct
              weights (> 256 MB) that the Infinity Cache cannot serve them
  quantize    quantize+prepack of a 13824x5120 fp16 weight (config 5's op)
  cpu_baseline  the oracle's restatement of kernel/naive.py on the host cores,
              on a bounded sample of the headline rows

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E
METRIC = "TFLOPS & % fp16-MFMA peak, fp16×e5m2 GEMM M32768 K5120 N13824; GB/s at M=16"
HEADLINE_CFG = (2, 4, 4, 8, 4)
TRAFFIC_FILE = REPO / "profiles" / "scaled_mm_lds256_headline_pmc.txt"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemm_bytes(M: int, N: int, K: int) -> int:
    """Algorithmic bytes of one call (reference cpp bench formula): A fp16 + B fp8 + C fp16."""
    return 2 * M * K + N * K + 2 * M * N


def _quantized_weight(N, K, seed, dev, quant):
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
    qt = quant.make_feather_quantized_weight(w, None, torch.float16)
    return quant.get_feather_plain_tensors(qt)


def time_launches(fn, n: int):
    """Average ms per call of n back-to-back calls, bracketed by HIP events on the current stream."""
    import torch

    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for i in range(n):
        fn(i)
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / n


def read_traffic():
    """HBM bytes per headline launch from the committed rocprofv3 PMC summary, if present."""
    if not TRAFFIC_FILE.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", TRAFFIC_FILE.read_text(), flags=re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(budget_s: float = 12.0):
    """Oracle restatement of kernel/naive.py (decode B, fp16-rounded matmul, scale, cast, bias)
    on the host, over a growing number of headline rows until ~budget_s of work is timed."""
    import numpy as np
    import torch

    from oracle import feather_oracle as O

    threads = None
    try:
        from threadpoolctl import threadpool_info

        threads = max((i.get("num_threads") or 0) for i in threadpool_info()) or None
    except Exception:
        pass
    threads = threads or os.cpu_count()
    M, N, K = 32768, 13824, 5120
    g = torch.Generator().manual_seed(0)
    w = torch.randn(N, K, generator=g) * 0.02
    s = np.float32(w.abs().max().item()) / np.float32(57344.0)
    codes = (w * float(np.float32(1.0) / s)).to(torch.float8_e5m2).view(torch.uint8)
    packed = codes.view(N, K // 16, 16).permute(1, 0, 2).contiguous().numpy()
    bias = (torch.randn(N, generator=g) * 0.01).half().numpy()
    rows = 64
    total_t, total_rows = 0.0, 0
    while True:
        a = torch.randn(rows, K, generator=g).half().numpy()
        t0 = time.perf_counter()
        O.scaled_mm_naive(a, packed, s, bias, O.DT_F16)
        dt = time.perf_counter() - t0
        total_t, total_rows = total_t + dt, total_rows + rows
        if total_t >= budget_s or rows >= 4096:
            break
        rows *= 2
    tflops = 2.0 * total_rows * N * K / total_t / 1e12
    return {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
            "sample": f"oracle scaled_mm_naive (kernel/naive.py restated in numpy, fp32 BLAS matmul rounded to "
                      f"fp16) on {total_rows} of the {M} headline rows, K={K}, N={N}, {total_t:.1f} s",
            "full_job_seconds_extrapolated": round(total_t * M / total_rows, 1)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only-headline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported on this single-GPU build "
              "(see the sharding notes in DESIGN.md)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    import importlib

    hk = importlib.import_module("featherops_amd.kernel.hip.hip_kernel")
    quant = importlib.import_module("featherops_amd.comfy_feather.quant")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # ---------------- headline GEMM ----------------
    M, N, K = 32768, 13824, 5120
    log(f"bench: headline M={M} N={N} K={K} cfg={HEADLINE_CFG}")
    bp, scale = _quantized_weight(N, K, 1, dev, quant)
    g = torch.Generator(device=dev).manual_seed(2)
    a = torch.randn(M, K, generator=g, device=dev).half()
    bias = (torch.randn(N, generator=g, device=dev) * 0.01).half()
    c = torch.empty(M, N, dtype=torch.float16, device=dev)
    op = torch.ops.feather_ops.scaled_mm.default

    def step(_i):
        op(a, bp, scale, bias, c, *HEADLINE_CFG, 1)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    ms = time_launches(step, args.steps)
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    assert torch.isfinite(c).all().item(), "non-finite output in the headline GEMM"
    log(f"bench: headline {ms:.3f} ms/step, {tflops:.1f} TFLOP/s ({100 * tflops / PEAK_FP16_TFLOPS:.1f}% of peak)")
    traffic = read_traffic()
    result = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (A ~ N(0,1) fp16; W ~ N(0,0.02) fp16 quantized+prepacked on device to e5m2)",
        "config": {"workload": "scaled_mm fp16 x e5m2, M32768 K5120 N13824, fp16 out, scale+bias "
                               "(BASELINE config 4 headline)",
                   "M": M, "N": N, "K": K, "out_dtype": "fp16", "kernel_config": list(HEADLINE_CFG)},
        "pct_fp16_mfma_peak": round(100 * tflops / PEAK_FP16_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_FP16_TFLOPS, 4), "traffic": traffic,
                     "algorithmic_bytes": gemm_bytes(M, N, K)},
    }
    if not args.only_headline:
        # context: the vendor fp16 x fp16 GEMM (torch.matmul -> hipBLASLt) on the same shape
        b16 = torch.randn(K, N, generator=g, device=dev).half()
        for _ in range(2):
            torch.matmul(a, b16)
        ms_ref = time_launches(lambda _i: torch.matmul(a, b16), max(3, args.steps // 2))
        result["context_fp16xfp16_torch_matmul"] = {"ms": round(ms_ref, 4),
                                                    "TFLOP_per_s": round(flops / (ms_ref * 1e-3) / 1e12, 2)}
        log(f"bench: torch fp16 matmul (hipBLASLt) same shape {ms_ref:.3f} ms")
        del b16
    del a, c

    if not args.only_headline:
        # ---------------- small M (config 2), weight rotation past the 256 MB MALL ----------------
        Ms, Ns, Ks = 16, 4096, 4096
        nrot = 24  # 24 x 16.8 MB = 403 MB of distinct weights
        log(f"bench: small-M M={Ms} N={Ns} K={Ks}, rotating {nrot} weights")
        ws = [_quantized_weight(Ns, Ks, 100 + r, dev, quant) for r in range(nrot)]
        a16 = torch.randn(Ms, Ks, generator=g, device=dev).half()
        b16 = (torch.randn(Ns, generator=g, device=dev) * 0.01).half()
        c16 = torch.empty(Ms, Ns, dtype=torch.float16, device=dev)

        def step16(i):
            w, s = ws[i % nrot]
            op(a16, w, s, b16, c16, 1, 1, 2, 1, 2, 1)

        for i in range(2 * nrot):
            step16(i)
        torch.cuda.synchronize()
        # a ~3-5 us kernel is shorter than one Python dispatch, so the calls are
        # captured once in a HIP graph (one launch per rotated weight) and the
        # graph is replayed: the timed region then holds device work only
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(nrot):
                step16(i)
        graph.replay()
        torch.cuda.synchronize()
        reps = 20
        ms16 = time_launches(lambda _i: graph.replay(), reps) / nrot
        eager_ms16 = time_launches(step16, 4 * nrot)
        gbps = gemm_bytes(Ms, Ns, Ks) / (ms16 * 1e-3) / 1e9
        log(f"bench: small-M {ms16 * 1e3:.2f} us/call (graph replay), {gbps:.0f} GB/s; eager {eager_ms16 * 1e3:.2f} us")
        result["small_m"] = {"M": Ms, "N": Ns, "K": Ks, "us_per_call": round(ms16 * 1e3, 3),
                             "GB_per_s": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / PEAK_HBM_GBPS, 2),
                             "weights_rotated": nrot, "calls": reps * nrot, "timing": "HIP graph replay",
                             "eager_us_per_call": round(eager_ms16 * 1e3, 3)}
        del ws

        # ---------------- quantize + prepack (config 5's on-device op) ----------------
        Nq, Kq = 13824, 5120
        wq = (torch.randn(Nq, Kq, generator=g, device=dev) * 0.02).half()

        def stepq(_i):
            quant.make_feather_quantized_weight(wq, None, torch.float16)

        stepq(0)
        msq = time_launches(stepq, 10)
        qbytes = Nq * Kq * (2 + 2 + 1)  # amax read + quantize read + e5m2 write
        result["quantize"] = {"N": Nq, "K": Kq, "ms_per_weight": round(msq, 4),
                              "GB_per_s": round(qbytes / (msq * 1e-3) / 1e9, 1),
                              "bytes_model": "2 B read (amax) + 2 B read + 1 B write per element"}
        log(f"bench: quantize {msq:.3f} ms per 13824x5120 weight")

    if not args.no_cpu:
        log("bench: CPU baseline (oracle naive restatement) ...")
        result["cpu_baseline"] = cpu_baseline()
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
