"""Benchmark of the FP8 W8A8 DiT linear on one MI355X.

One step is one pass of the quantized-linear hot path over one batch of the
c2 workload (DiT QKV projection at a 480p streaming chunk):

    X [8192, 5120] bf16  --per-token dynamic e4m3fn act quant-->  codes + scales
    codes x W [15360, 5120] e4m3fn (per-channel scales, quantized offline)
      + bias bf16  --scaled MFMA GEMM, fused dequant + bias-->  Y [8192, 15360] bf16

Inputs are synthetic (seed 0, 1% outlier channels x15) and resident in HBM
before the timed region; four activation buffers rotate so the act-quant
reads exceed the 256 MB Infinity Cache.  `value` is 2*M*N*K / step time.
Each kernel is also timed alone with HIP events on the stream it runs on
(torch's current stream) over the timed steps: the GEMM gives `roofline`
(MFMA-bound, FP8 dense peak 5.0 PFLOP/s) and the act-quant its HBM GB/s
(3*M*K + 4*M bytes per call against 8 TB/s).  `cpu_baseline` times the
reference's own torch expressions (oracle/torch_path.py) on the host cores
over one full c2 batch, repeated for about 12 s of CPU work.  `traffic` is
read from profiles/gemm_fp8_c2_traffic.json (rocprof FETCH_SIZE/WRITE_SIZE
of this same command, scaled by a known-size copy).

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP8_PEAK_TFLOPS = 5000.0   # MI355X dense FP8 MFMA
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
M, K, N = 8192, 5120, 15360
TRAFFIC_FILE = ROOT / "profiles" / "gemm_fp8_c2_traffic.json"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(torch, device, rotations: int):
    gen = torch.Generator().manual_seed(0)
    xs = []
    for r in range(rotations):
        x = torch.randn(M, K, generator=gen)
        idx = torch.randperm(K, generator=gen)[: K // 100]
        x[:, idx] *= 15.0
        xs.append(x.to(torch.bfloat16).to(device))
    w = (torch.randn(N, K, generator=gen) * 0.02).to(torch.bfloat16)
    bias = (torch.randn(N, generator=gen) * 0.01).to(torch.bfloat16)
    return xs, w, bias


def cpu_baseline(torch, w_cpu, bias_cpu, x_cpu, budget_s: float = 12.0) -> dict:
    """Reference torch path on the host (oracle/torch_path.py): per-token e4m3
    quant of the activations, then dequant-then-matmul against the offline
    quantized weights with bias, on the full c2 batch, repeated until about
    `budget_s` seconds of CPU work (at least 3 runs); the median is reported."""
    from oracle import torch_path as TP

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    q_w, s_w = TP.quantize_rows_e4m3(w_cpu)
    rows = x_cpu.shape[0]
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        TP.w8a8_fp8_linear_step(x_cpu, q_w, s_w, bias_cpu)
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    return {
        "value": round(2.0 * rows * N * K / t / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"all {rows} tokens of one c2 batch (per-token e4m3 quant + dequant-then-matmul + bias, "
                  f"torch CPU fp32), median of {len(times)} runs: {t:.2f} s per batch",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 512 MiB device copy (known bytes) for scaling rocprof "
                         "FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2

    import torch
    import __graft_entry__

    __graft_entry__.load_package()
    from taomate_h3_amd import ops

    dev = torch.device("cuda:0")
    rotations = 4
    xs, w, bias = make_inputs(torch, dev, rotations)
    x_cpu = xs[0].cpu()
    w_dev, bias_dev = w.to(dev), bias.to(dev)
    q_w, s_w = ops.quant_rows(w_dev, ops.FMT_E4M3FN)       # offline weight quantization
    s_w = s_w.reshape(-1)
    q_a = torch.empty(M, K, device=dev, dtype=torch.float8_e4m3fn)
    s_a = torch.empty(M, 1, device=dev, dtype=torch.float32)
    out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()

    def step(i: int, ev=None):
        x = xs[i % rotations]
        if ev is not None:
            ev[0].record()
        ops.quant_rows(x, ops.FMT_E4M3FN, codes=q_a, scales=s_a)
        if ev is not None:
            ev[1].record()
        ops.scaled_mm(q_a, q_w, s_a.reshape(-1), s_w, bias=bias_dev, out=out)
        if ev is not None:
            ev[2].record()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # Timed region: exactly K steps between two synchronisations.
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # Per-kernel durations with HIP events on the launch stream.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    q_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    g_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps

    flops = 2.0 * M * N * K
    ms_per_step = elapsed / args.steps * 1e3
    value = flops / (elapsed / args.steps) / 1e12
    gemm_tflops = flops / (g_ms * 1e-3) / 1e12
    q_bytes = 3 * M * K + 4 * M
    q_gbs = q_bytes / (q_ms * 1e-3) / 1e9

    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except (ValueError, OSError):
            traffic = None

    result = {
        "metric": "FP8 W8A8 linear TFLOP/s + % FP8 MFMA peak; act-quant HBM GB/s (1 GPU)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3fn (fp32 accumulate, bf16 out)",
        "data": "synthetic (seed 0; N(0,1) activations with 1% channels x15; N(0,0.02) weights)",
        "config": {
            "workload": "c2: DiT QKV projection, 480p streaming chunk (BASELINE configs[1])",
            "M_tokens": M, "K": K, "N": N,
            "act_quant": "per-token dynamic e4m3fn",
            "weight_quant": "per-output-channel e4m3fn (offline)",
            "bias": True, "out": "bf16",
            "activation_buffers_rotated": rotations,
        },
        "pct_fp8_peak": round(100.0 * value / FP8_PEAK_TFLOPS, 2),
        "roofline": {
            "kernel": "h3q gemm_kernel (scaled e4m3 GEMM + dequant + bias epilogue)",
            "bound": "mfma",
            "achieved": round(gemm_tflops, 2),
            "peak": FP8_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / FP8_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "avg_launch_us": round(g_ms * 1e3, 2),
        },
        "act_quant": {
            "kernel": "h3q quant_rows_vec_kernel (per-token e4m3fn)",
            "bound": "hbm",
            "achieved": round(q_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(q_gbs / HBM_PEAK_GBS, 4),
            "avg_launch_us": round(q_ms * 1e3, 2),
            "algorithmic_bytes": q_bytes,
        },
    }
    if args.calibrate_copy:
        src = torch.empty(256 << 20, device=dev, dtype=torch.bfloat16).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = int(src.numel() * src.element_size())
        del src, dst
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, w, bias, x_cpu)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
