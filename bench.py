"""Benchmark of the FP8 W8A8 DiT linear on one MI355X.

One step is one pass of the quantized-linear hot path over one batch of the
c2 workload (DiT QKV projection at a 480p streaming chunk):

    X [8192, 5120] bf16  --per-token dynamic e4m3fn act quant-->  codes + scales
    codes x W [15360, 5120] e4m3fn (per-channel scales, quantized offline into
      the tiled weight layout) + bias bf16  --scaled MFMA GEMM, fused dequant
      + bias-->  Y [8192, 15360] bf16

Inputs are synthetic (seed 0, 1% outlier channels x15) and resident in HBM
before the timed region; four activation buffers rotate so the act-quant
reads exceed the 256 MB Infinity Cache.  ``value`` is 2*M*N*K / step time,
with each step replayed from a HIP graph captured for its input buffer (the
same two kernels and arguments as an eager step, without per-launch host
work); the eager step time is reported beside it as ``eager_ms_per_step``.

Each kernel is also timed with HIP events on the stream it runs on (torch's
current stream): the GEMM over the timed steps gives ``roofline`` (MFMA-bound,
FP8 dense peak 5.0 PFLOP/s); the act-quant, timed back to back over the
rotating inputs, gives ``act_quant`` (HBM-bound: 3*M*K + 4*M bytes per call
against 8 TB/s; its time inside the step, right after the previous GEMM's
252 MB of output, is reported beside it).  ``traffic`` is read from
profiles/gemm_fp8_c2_traffic.json (rocprofv3 FETCH_SIZE / WRITE_SIZE of this
same command, scaled by a copy of known size) when it belongs to the GEMM
kernel measured here.

The other BASELINE.json configurations are timed as secondary objects (not the
headline): ``c3`` FFN up / down at 768p with the rank-128 LoRA epilogue, ``c4``
skinny M in {16, 64, 128} (weight-streaming, HBM roofline; launches replayed
from a HIP graph, weights rotated past the Infinity Cache) and ``c5`` the int8
W8A8 GEMM at 1080p; ``f1`` the fused RMSNorm/AdaLN + int8 act-quant producer
against the unfused pair.  ``cpu_baseline`` times the reference's own torch
expressions (oracle/torch_path.py) on the host cores over one full c2 batch.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-extra] [--no-cpu-baseline]
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
INT8_PEAK_TOPS = 5000.0    # MI355X dense INT8 MFMA
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
M, K, N = 8192, 5120, 15360
TRAFFIC_FILE = ROOT / "profiles" / "gemm_fp8_c2_traffic.json"
GEMM_KERNEL_TAG = "gemm_w4_kernel<0, true, true, true, false, false>"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gpu_randn(torch, shape, gen, device, scale=1.0):
    return (torch.randn(shape, generator=gen, device=device) * scale).to(torch.bfloat16)


def make_inputs(torch, device, rotations: int):
    gen = torch.Generator(device=device).manual_seed(0)
    xs = []
    for _ in range(rotations):
        x = torch.randn(M, K, generator=gen, device=device)
        idx = torch.randperm(K, generator=gen, device=device)[: K // 100]
        x[:, idx] *= 15.0
        xs.append(x.to(torch.bfloat16))
    w = gpu_randn(torch, (N, K), gen, device, 0.02)
    bias = gpu_randn(torch, (N,), gen, device, 0.01)
    return xs, w, bias


def time_events(torch, fn, iters: int) -> float:
    """Average ms of fn() over iters launches, HIP events on the current stream."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(iters):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def time_in_step(torch, quant, gemm, iters: int):
    """Average ms of quant() and of gemm() inside steps (quant, then gemm),
    HIP events on the current stream around each, like the headline step."""
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(iters)]
    for i in range(iters):
        evs[i][0].record()
        quant(i)
        evs[i][1].record()
        gemm(i)
        evs[i][2].record()
    torch.cuda.synchronize()
    return (sum(e[0].elapsed_time(e[1]) for e in evs) / iters, sum(e[1].elapsed_time(e[2]) for e in evs) / iters)


def settle_clock(torch, replay, block: int = 8, tol: float = 0.01, cap: int = 1024) -> dict:
    """Untimed replays of the captured step, in blocks, until the GPU's clock
    has settled: the sync gaps before the timed region (the eager pass, the
    capture) let it drop, and it takes ~10-20 ms of load to come back, so the
    first timed steps would otherwise run slower than every later one.  Stops
    when a block's median device time is within ``tol`` of the previous
    block's (or after ``cap`` replays); returns the count and the medians."""
    medians, done = [], 0
    while done < cap:
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(block + 1)]
        ev[0].record()
        for i in range(block):
            replay(done + i)
            ev[i + 1].record()
        torch.cuda.synchronize()
        done += block
        t = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(block))[block // 2] * 1e3
        medians.append(round(t, 1))
        if len(medians) > 1 and t >= medians[-2] * (1.0 - tol):
            break
    return {"replays": done, "block_median_us": medians}


def _c3_lora_module(torch, qw, sw, la, lb):
    """A column-parallel FP8 W8A8 base (tiled e4m3 weight + per-channel scales,
    no bias) under the reference's LoRA wrapper, swapped by
    fuse_h3_lora_wrappers_ for the fused wrapper: the module the c3 object times."""
    from taomate_h3_amd import ops
    from taomate_h3_amd.distributed import linear
    from taomate_h3_amd.inference import lora

    class Base(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.tp_size, self.tp_rank, self.bias = 1, 0, None
            self.weight = torch.nn.Parameter(qw, requires_grad=False)
            self.register_buffer("_fp8_w8a8_weight_scale", sw, persistent=False)
            ops.mark_module_weight_tiled(self)  # as the loaders record a tiled weight

        def forward(self, x):
            return linear._module_linear(self, x, None)

    # The attributes of the wrapper the reference's apply_h3_lora_checkpoint
    # installs (H3/inference/lora_checkpoint.py:172-205): what
    # fuse_h3_lora_wrappers_ reads when it swaps it for this package's.
    installed = torch.nn.Module()
    installed.base, installed.kind, installed.scale = Base(), "column", 1.0
    installed.fused_row_reduce_enabled = False
    installed._taomate_h3_inference_lora = True
    installed.register_buffer("lora_a", la, persistent=False)
    installed.register_buffer("lora_b", lb, persistent=False)
    root = torch.nn.Module()
    root.proj = installed.eval()
    receipt = lora.fuse_h3_lora_wrappers_(root)
    if receipt["replaced_count"] != 1 or receipt["fused_epilogue_ready_count"] != 1:
        raise RuntimeError(f"c3: the LoRA wrapper was not swapped for the fused one: {receipt}")
    return root.proj


def bench_c3(torch, ops, dev) -> dict:
    """FFN at 768p, M=24576, up N=13824 K=5120 and down
    N=5120 K=13824, e4m3 per-token x per-channel (activation codes in the
    tiled layout), rank-128 LoRA (scale 1.0) added in the GEMM epilogue.
    Times act-quant + LoRA down + scaled GEMM inside steps (as the headline
    step), and the GEMM back to back, where the MFMA clock settles lower.
    Then the same linear through the module path a model runs: the
    reference's LoRA wrapper swapped by fuse_h3_lora_wrappers_, whose forward
    (LoRA down, tiled act-quant, GEMM with the LoRA epilogue) is timed whole
    and checked bit for bit against the kernel-level step."""
    gen = torch.Generator(device=dev).manual_seed(0)
    m, out = 24576, {}
    for name, n, k in (("up", 13824, 5120), ("down", 5120, 13824)):
        x = gpu_randn(torch, (m, k), gen, dev)
        qw, sw = ops.quant_rows_tiled(gpu_randn(torch, (n, k), gen, dev, 0.02), ops.FMT_E4M3FN)
        la, lb = gpu_randn(torch, (128, k), gen, dev, 0.01), gpu_randn(torch, (n, 128), gen, dev, 0.01)
        q_a = torch.empty(m, k, device=dev, dtype=torch.float8_e4m3fn)
        s_a = torch.empty(m, 1, device=dev, dtype=torch.float32)
        t = torch.empty(m, 128, device=dev, dtype=torch.bfloat16)
        y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)

        def quant(_i):
            ops.quant_rows_tiled(x, ops.FMT_E4M3FN, codes=q_a, scales=s_a)
            ops.lora_down(x, la, out=t)

        def gemm(_i):
            ops.scaled_mm(q_a, qw, s_a.reshape(-1), sw.reshape(-1), lora_t=t, lora_b=lb, lora_scale=1.0, out=y,
                          a_tiled=True, b_tiled=True, m=m)

        for _ in range(30):  # steady clocks before timing (the headline step is warmed up likewise)
            quant(0)
            gemm(0)
        torch.cuda.synchronize()
        q_ms, g_ms = time_in_step(torch, quant, gemm, 8)
        b2b_ms = time_events(torch, gemm, 8)
        module = _c3_lora_module(torch, qw, sw, la, lb)
        same = bool(torch.equal(module(x), y))
        for _ in range(3):  # the module path's own buffers come from torch's allocator: warm its cache
            module(x)
        w_ms = time_events(torch, lambda _i: module(x), 8)
        fl = 2.0 * m * n * k
        out[name] = {"M": m, "N": n, "K": k, "gemm_us": round(g_ms * 1e3, 1),
                     "gemm_back_to_back_us": round(b2b_ms * 1e3, 1),
                     "gemm_fp8_tflops": round(fl / (g_ms * 1e-3) / 1e12, 1),
                     "pct_fp8_peak": round(100 * fl / (g_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 1),
                     "act_quant_plus_lora_down_us": round(q_ms * 1e3, 1),
                     "step_tflops": round(fl / ((g_ms + q_ms) * 1e-3) / 1e12, 1),
                     "lora_gflop": round(2.0 * m * 128 * (k + n) / 1e9, 1),
                     "fused_wrapper_forward_us": round(w_ms * 1e3, 1),
                     "fused_wrapper_matches_kernel_step": same}
        del x, qw, sw, la, lb, q_a, s_a, t, y, module
    return out


def bench_c4(torch, ops, dev) -> dict:
    """skinny M in {16, 64, 128}, K = N = 5120, tiled
    e4m3 weights, activations quantized into the tiled layout.  Bytes per call
    N*K + 4N + M*K + 4M + 2MN against 8 TB/s; twelve weight copies (315 MB)
    rotate past the Infinity Cache; 48 launches captured in a HIP graph."""
    gen = torch.Generator(device=dev).manual_seed(0)
    n = k = 5120
    copies = 12
    ws = []
    for _ in range(copies):
        qw, sw = ops.quant_rows_tiled(gpu_randn(torch, (n, k), gen, dev, 0.02), ops.FMT_E4M3FN)
        ws.append((qw, sw.reshape(-1)))
    res = {}
    for m in (16, 64, 128):
        x = gpu_randn(torch, (m, k), gen, dev)
        q_a, s_a = ops.quant_rows_tiled(x, ops.FMT_E4M3FN)
        s_a = s_a.reshape(-1)
        y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        per = 48

        def launches():
            for i in range(per):
                qw, sw = ws[i % copies]
                ops.scaled_mm(q_a, qw, s_a, sw, out=y, a_tiled=True, b_tiled=True, m=m)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            launches()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            launches()
        graph.replay()
        torch.cuda.synchronize()
        ms = time_events(torch, lambda _i: graph.replay(), 5) / per
        byts = n * k + 4 * n + m * k + 4 * m + 2 * m * n
        gbs = byts / (ms * 1e-3) / 1e9
        res[f"M{m}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3),
                        "bytes": byts}
    return res


def bench_f1(torch, ops, dev) -> dict:
    """Next row (f)1: the QKV-input producer (RMSNorm + AdaLN modulate) with the
    per-token int8 act-quant of the W8A8 linear fused in, against the same two
    steps unfused (modulated bf16 rows written, then re-read by the
    quantizer).  At the c2 activation shape and at the real H3 QKV input
    (1088x1920 phase 0, M=6224, K=5376); four rotating inputs, four table rows.
    Bytes: fused 2MK in + MK + 4M out; unfused adds 4MK.  Then the fc2-input
    producer (SwiGLU + e4m3 act-quant) the same way."""
    res = {}
    for name, m, k in (("c2_shape", 8192, 5120), ("h3_qkv_1088p", 6224, 5376)):
        gen = torch.Generator(device=dev).manual_seed(0)
        xs = [gpu_randn(torch, (m, k), gen, dev) for _ in range(4)]
        w = (1.0 + 0.1 * torch.randn(k, device=dev, generator=gen)).to(torch.bfloat16)
        sc = gpu_randn(torch, (4, k), gen, dev, 0.1)
        sh = gpu_randn(torch, (4, k), gen, dev, 0.1)
        idx = torch.randint(0, 4, (m,), device=dev, generator=gen)
        codes = torch.empty(m, k, device=dev, dtype=torch.int8)
        scales = torch.empty(m, 1, device=dev, dtype=torch.float32)
        y = torch.empty(m, k, device=dev, dtype=torch.bfloat16)

        def fused(i):
            ops.norm_modulate_quant(xs[i % 4], w, sc, sh, idx, 1e-6, fmt=ops.FMT_INT8, rounding=ops.ROUND_RCP_MUL,
                                    codes=codes, scales=scales)

        def unfused(i):
            ops.norm_modulate_quant(xs[i % 4], w, sc, sh, idx, 1e-6, out=y)
            ops.quant_rows(y, ops.FMT_INT8, ops.ROUND_RCP_MUL, codes=codes, scales=scales)

        for fn in (fused, unfused):
            for i in range(4):
                fn(i)
        torch.cuda.synchronize()
        tf = time_events(torch, fused, 40) * 1e3
        tu = time_events(torch, unfused, 40) * 1e3
        byts = 3 * m * k + 4 * m
        res[name] = {"M": m, "K": k, "fused_us": round(tf, 1), "unfused_us": round(tu, 1),
                     "fused_GB/s": round(byts / tf / 1e3, 1), "frac_hbm": round(byts / tf / 1e3 / HBM_PEAK_GBS, 3),
                     "saved_bytes": 4 * m * k}
        del xs, codes, y
    # The fc2-input producer: SwiGLU of [M, 2F] with the per-token e4m3
    # quantizer folded in, at c3's FFN width (F = 13824).  Bytes: fused 4MF in
    # + MF + 4M out; unfused adds 4MF (bf16 rows written, then re-read).
    m, f = 8192, 13824
    gen = torch.Generator(device=dev).manual_seed(0)
    xs = [gpu_randn(torch, (m, 2 * f), gen, dev, 2.0) for _ in range(4)]
    codes = torch.empty(m, f, device=dev, dtype=torch.float8_e4m3fn)
    scales = torch.empty(m, 1, device=dev, dtype=torch.float32)
    y = torch.empty(m, f, device=dev, dtype=torch.bfloat16)

    def sw_fused(i):
        ops.swiglu_quant(xs[i % 4], fmt=ops.FMT_E4M3FN, codes=codes, scales=scales)

    def sw_unfused(i):
        ops.swiglu_quant(xs[i % 4], out=y)
        ops.quant_rows(y, ops.FMT_E4M3FN, ops.ROUND_DIV, codes=codes, scales=scales)

    for fn in (sw_fused, sw_unfused):
        for i in range(4):
            fn(i)
    torch.cuda.synchronize()
    tf = time_events(torch, sw_fused, 20) * 1e3
    tu = time_events(torch, sw_unfused, 20) * 1e3
    byts = 5 * m * f + 4 * m
    res["swiglu_c3_width"] = {"M": m, "F": f, "fused_us": round(tf, 1), "unfused_us": round(tu, 1),
                              "fused_GB/s": round(byts / tf / 1e3, 1),
                              "frac_hbm": round(byts / tf / 1e3 / HBM_PEAK_GBS, 3), "saved_bytes": 4 * m * f}
    del xs, codes, y
    return res


def bench_a6(torch, ops, dev) -> dict:
    """Row a6/a7: per-tensor e4m3fn activation quantization at the c2
    activation shape (M=8192, K=5120), four rotating inputs.  Dynamic: two
    launches (partial maxima, then fold + quantize), the input read twice;
    static (a calibrated scale): one launch.  Algorithmic bytes: 2MK in + MK
    out (+4)."""
    gen = torch.Generator(device=dev).manual_seed(0)
    m, k = M, K
    xs = [gpu_randn(torch, (m, k), gen, dev) for _ in range(4)]
    codes = torch.empty(m, k, device=dev, dtype=torch.float8_e4m3fn)
    scale = torch.empty((), device=dev, dtype=torch.float32)
    ws = torch.empty(int(ops._lib.lib().h3q_quant_tensor_workspace_floats(m, k)), device=dev, dtype=torch.float32)
    static = torch.tensor(0.05, device=dev, dtype=torch.float32)

    def dynamic(i):
        ops.quant_tensor_e4m3(xs[i % 4], codes=codes, scale=scale, workspace=ws)

    def calibrated(i):
        ops.quant_tensor_e4m3(xs[i % 4], static, codes=codes, scale=scale)

    for fn in (dynamic, calibrated):
        for i in range(4):
            fn(i)
    torch.cuda.synchronize()
    td = time_events(torch, dynamic, 40) * 1e3
    ts = time_events(torch, calibrated, 40) * 1e3
    byts = 3 * m * k + 4
    del xs, codes
    return {"M": m, "K": k, "dynamic_us": round(td, 1), "dynamic_GB/s": round(byts / td / 1e3, 1),
            "dynamic_frac_hbm": round(byts / td / 1e3 / HBM_PEAK_GBS, 3), "static_us": round(ts, 1),
            "static_GB/s": round(byts / ts / 1e3, 1), "static_frac_hbm": round(byts / ts / 1e3 / HBM_PEAK_GBS, 3),
            "algorithmic_bytes": byts}


def bench_h3_lora(torch, ops, dev) -> dict:
    """The H3 QKV projection with a rank-128 LoRA at a production shape
    (1088x1920 phase 1: M=3200 tokens, K=5376, N=10752; e4m3 tiled weights and
    activations): the LoRA down-projection split over K (the path ops.lora_down
    takes) against the unsplit kernel, then the scaled GEMM with the LoRA
    epilogue; act-quant + down-projection + GEMM timed inside steps."""
    from taomate_h3_amd import _lib
    gen = torch.Generator(device=dev).manual_seed(0)
    m, k, n = 3200, 5376, 10752
    x = gpu_randn(torch, (m, k), gen, dev)
    qw, sw = ops.quant_rows_tiled(gpu_randn(torch, (n, k), gen, dev, 0.02), ops.FMT_E4M3FN)
    la, lb = gpu_randn(torch, (128, k), gen, dev, 0.01), gpu_randn(torch, (n, 128), gen, dev, 0.01)
    q_a = torch.empty(m, k, device=dev, dtype=torch.float8_e4m3fn)
    s_a = torch.empty(m, 1, device=dev, dtype=torch.float32)
    t = torch.empty(m, 128, device=dev, dtype=torch.bfloat16)
    y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)

    def down_unsplit(_i):
        _lib.call("h3q_lora_down", x.data_ptr(), k, la.data_ptr(), k, t.data_ptr(), 128, m, k, 128,
                  torch.cuda.current_stream().cuda_stream)

    def quant(_i):
        ops.quant_rows_tiled(x, ops.FMT_E4M3FN, codes=q_a, scales=s_a)
        ops.lora_down(x, la, out=t)

    def gemm(_i):
        ops.scaled_mm(q_a, qw, s_a.reshape(-1), sw.reshape(-1), lora_t=t, lora_b=lb, lora_scale=1.0, out=y,
                      a_tiled=True, b_tiled=True, m=m)

    for _ in range(60):  # steady clocks before timing (~13 ms of steps)
        quant(0)
        gemm(0)
    torch.cuda.synchronize()
    split_ms = time_events(torch, lambda i: ops.lora_down(x, la, out=t), 16)
    unsplit_ms = time_events(torch, down_unsplit, 16)
    q_ms, g_ms = time_in_step(torch, quant, gemm, 8)
    fl = 2.0 * m * n * k
    return {"M": m, "N": n, "K": k, "rank": 128, "lora_down_split_us": round(split_ms * 1e3, 1),
            "lora_down_unsplit_us": round(unsplit_ms * 1e3, 1), "gemm_lora_us": round(g_ms * 1e3, 1),
            "gemm_fp8_tflops": round(fl / (g_ms * 1e-3) / 1e12, 1),
            "act_quant_plus_lora_down_us": round(q_ms * 1e3, 1)}


def bench_f4(torch, ops, dev) -> dict:
    """Next row (f)4: per-(batch, head) FP8 quantization of one attention
    operand, [1, 8192, 56, 128] bf16 (the FL transformer's 56 heads of 128 at
    one GPU), four rotating inputs.  Algorithmic bytes: 2 in + 1 out per
    element (the kernel reads the input twice: per-head maxima, then
    quantization).  Beside it, the same expression in eager torch on the GPU
    (what the reference runs without Triton: amax, divide, clamp, cast)."""
    gen = torch.Generator(device=dev).manual_seed(0)
    shape = (1, 8192, 56, 128)
    xs = [gpu_randn(torch, shape, gen, dev) for _ in range(4)]
    n = xs[0].numel()
    codes = torch.empty(shape, device=dev, dtype=torch.float8_e4m3fn)
    scales = torch.empty(shape[0], shape[2], device=dev, dtype=torch.float32)
    ws = torch.empty(int(ops._lib.lib().h3q_quant_per_head_workspace_floats(*shape)), device=dev,
                     dtype=torch.float32)

    def native(i):
        ops.quant_per_head_e4m3(xs[i % 4], codes=codes, scales=scales, workspace=ws)

    def eager(i):
        v = xs[i % 4]
        sc = torch.clamp(v.float().abs().amax(dim=(1, 3)) / 448.0, min=1.0e-12)
        torch.clamp(v / sc[:, None, :, None], -448.0, 448.0).to(torch.float8_e4m3fn)

    for fn in (native, eager):
        for i in range(4):
            fn(i)
    torch.cuda.synchronize()
    t_native = time_events(torch, native, 40) * 1e3
    t_eager = time_events(torch, eager, 5) * 1e3
    byts = 3 * n + 4 * shape[0] * shape[2]
    del xs, codes
    return {"shape": list(shape), "us": round(t_native, 1), "GB/s": round(byts / t_native / 1e3, 1),
            "frac_hbm": round(byts / t_native / 1e3 / HBM_PEAK_GBS, 3), "algorithmic_bytes": byts,
            "torch_eager_us": round(t_eager, 1)}


def bench_c5(torch, ops, dev) -> dict:
    """int8 W8A8 at 1080p, M=40960, K=N=5120: per-token
    int8 act quant (vLLM formula) + int32-exact GEMM with fused dequant.  The
    GEMM is timed inside steps (act-quant, then GEMM) and back to back; the
    act-quant back to back (its HBM figure)."""
    gen = torch.Generator(device=dev).manual_seed(0)
    m, n, k = 40960, 5120, 5120
    x = torch.randn(m, k, generator=gen, device=dev)
    idx = torch.randperm(k, generator=gen, device=dev)[: k // 100]
    chi = torch.distributions.Chi2(torch.full((idx.numel(),), 3.0, device=dev)).sample((m,))
    x[:, idx] = torch.randn(m, idx.numel(), generator=gen, device=dev) / torch.sqrt(chi / 3.0)
    x = x.to(torch.bfloat16)
    qw, sw = ops.quant_rows_tiled(gpu_randn(torch, (n, k), gen, dev, 0.02), ops.FMT_INT8)
    q_a = torch.empty(m, k, device=dev, dtype=torch.int8)
    s_a = torch.empty(m, 1, device=dev, dtype=torch.float32)
    y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)

    def quant(_i):
        ops.quant_rows_tiled(x, ops.FMT_INT8, ops.ROUND_RCP_MUL, codes=q_a, scales=s_a)

    def gemm(_i):
        ops.scaled_mm(q_a, qw, s_a.reshape(-1), sw.reshape(-1), out=y, a_tiled=True, b_tiled=True, m=m)

    for _ in range(30):  # steady clocks before timing (the MFMA clock settles over ~10-30 ms)
        quant(0)
        gemm(0)
    torch.cuda.synchronize()
    _, g_ms = time_in_step(torch, quant, gemm, 8)
    q_ms = time_events(torch, quant, 8)
    b2b_ms = time_events(torch, gemm, 8)
    ops_ = 2.0 * m * n * k
    q_bytes = 3 * m * k + 4 * m
    return {"M": m, "N": n, "K": k, "gemm_us": round(g_ms * 1e3, 1), "gemm_back_to_back_us": round(b2b_ms * 1e3, 1),
            "gemm_int8_tops": round(ops_ / (g_ms * 1e-3) / 1e12, 1),
            "pct_int8_peak": round(100 * ops_ / (g_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 1),
            "act_quant_us": round(q_ms * 1e3, 1), "act_quant_GB/s": round(q_bytes / (q_ms * 1e-3) / 1e9, 1),
            "step_tops": round(ops_ / ((g_ms + q_ms) * 1e-3) / 1e12, 1)}


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


def _ceilings_lib():
    import ctypes

    path = ROOT / "taomate-h3_amd" / "libh3q_ceilings.so"
    if not path.exists():
        raise RuntimeError(f"{path.name} is not built: run `python taomate-h3_amd/build.py`")
    lib = ctypes.CDLL(str(path))
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    for name, args in (("h3q_ceil_read", [P, I64, P, I, P]), ("h3q_ceil_copy", [P, P, I64, I, P]),
                       ("h3q_ceil_transform", [P, I64, I64, P, I, P]), ("h3q_ceil_mfma", [I, P, I, P, I, P])):
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = I, args
    return lib


def bench_ceilings(torch, ops, dev) -> dict:
    """Attainable ceilings on this GPU, beside the nominal peaks
    (taomate-h3_amd/csrc/ceilings.hip, a separate measurement library):
    * ``hbm_read`` / ``hbm_copy``: stream read of 1 GiB, copy of 512 MiB
      (read + write bytes), best of three grid sizes;
    * ``transform``: the per-token quantizer's traffic with no arithmetic
      (bf16 rows in, one byte per element out, one wavefront per row, a
      persistent grid), at the c2, c5 and c3-down activation shapes, rotating
      inputs past the Infinity Cache, best and worst of three grids -- the
      ceiling of ``act_quant``;
    * ``mfma_e4m3`` / ``mfma_int8``: the four-wave GEMM's MFMA stream with no
      memory traffic (one workgroup of four waves per CU, 4 x 4 accumulators
      of the 32 x 32 MFMA per wave, two fragment sets of bench codes:
      N(0,1) activations and N(0,0.02) weights quantized per row), at the
      clock the GPU sustains under it -- the ceiling of ``roofline``."""
    import ctypes

    lib = _ceilings_lib()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def call(name, *args):
        rc = getattr(lib, name)(*args, stream)
        if rc != 0:
            raise RuntimeError(f"{name} failed ({rc})")

    def p(t):
        return ctypes.c_void_p(t.data_ptr())

    def best(fn, grids, iters=10):
        times = {}
        for g in grids:
            for i in range(3):
                fn(g, i)
            torch.cuda.synchronize()
            times[g] = time_events(torch, lambda i, g=g: fn(g, i), iters)
        return times

    res = {"cus": cus}
    buf = torch.empty(1 << 30, device=dev, dtype=torch.uint8)
    sink = torch.zeros(64 * cus, device=dev, dtype=torch.int32)
    grids = (4 * cus, 8 * cus, 16 * cus)
    t = best(lambda g, _i: call("h3q_ceil_read", p(buf), buf.numel(), p(sink), g), grids)
    res["hbm_read"] = {"GB/s": round(buf.numel() / (min(t.values()) * 1e-3) / 1e9, 1), "bytes": buf.numel(),
                       "us_by_grid": {str(g): round(v * 1e3, 1) for g, v in t.items()}}
    half = buf.numel() // 2
    src, dst = buf[:half], buf[half:]
    t = best(lambda g, _i: call("h3q_ceil_copy", p(src), p(dst), half, g), grids)
    res["hbm_copy"] = {"GB/s": round(2 * half / (min(t.values()) * 1e-3) / 1e9, 1), "bytes_moved": 2 * half,
                       "us_by_grid": {str(g): round(v * 1e3, 1) for g, v in t.items()}}
    del buf, src, dst
    gen = torch.Generator(device=dev).manual_seed(0)
    res["transform"] = {}
    for name, m, k, rot in (("c2", 8192, 5120, 4), ("c5", 40960, 5120, 1), ("c3_down", 24576, 13824, 1)):
        xs = [gpu_randn(torch, (m, k), gen, dev) for _ in range(rot)]
        out = torch.empty(m, k, device=dev, dtype=torch.uint8)
        t = best(lambda g, i, xs=xs, out=out, m=m, k=k: call("h3q_ceil_transform", p(xs[i % len(xs)]), m, k, p(out),
                                                               g), (cus, 4 * cus, 8 * cus), iters=4 * rot)
        byts = 3 * m * k
        res["transform"][name] = {"M": m, "K": k, "best_us": round(min(t.values()) * 1e3, 2),
                                  "worst_us": round(max(t.values()) * 1e3, 2),
                                  "GB/s": round(byts / (min(t.values()) * 1e-3) / 1e9, 1), "bytes": byts}
        del xs, out
    # MFMA stream on bench codes: fragments q < 4 of each set from activation
    # codes, q >= 4 from weight codes.
    xq, _ = ops.quant_rows(gpu_randn(torch, (128, 1024), gen, dev), ops.FMT_E4M3FN)
    wq, _ = ops.quant_rows(gpu_randn(torch, (128, 1024), gen, dev, 0.02), ops.FMT_E4M3FN)
    frags = torch.cat([xq.view(torch.uint8).reshape(-1, 8, 2048)[:, :4], wq.view(torch.uint8).reshape(-1, 8, 2048)[:, :4]],
                      dim=1).contiguous()            # [8 (wave, set), 8 fragments, 2048]
    xi, _ = ops.quant_rows(gpu_randn(torch, (128, 1024), gen, dev), ops.FMT_INT8, ops.ROUND_RCP_MUL)
    wi, _ = ops.quant_rows(gpu_randn(torch, (128, 1024), gen, dev, 0.02), ops.FMT_INT8)
    frags_i8 = torch.cat([xi.view(torch.uint8).reshape(-1, 8, 2048)[:, :4],
                          wi.view(torch.uint8).reshape(-1, 8, 2048)[:, :4]], dim=1).contiguous()
    if frags.numel() != 128 * 1024 or frags_i8.numel() != 128 * 1024:
        raise RuntimeError("ceilings: the MFMA stream needs 128 KiB of fragment codes")
    msink = torch.empty(cus * 256, device=dev, dtype=torch.float32)
    iters = 2000
    for name, codes, int8 in (("mfma_e4m3", frags, 0), ("mfma_int8", frags_i8, 1)):
        def run(_g, _i, codes=codes, int8=int8):
            call("h3q_ceil_mfma", int8, p(codes), iters, p(msink), cus)

        for _ in range(20):   # about 20 ms of MFMA work: the clock settles under it
            run(0, 0)
        torch.cuda.synchronize()
        ms = time_events(torch, lambda i: run(0, i), 10)
        flops = cus * 4 * iters * 16 * 131072.0
        res[name] = {"TFLOP/s" if not int8 else "TOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
                     "us": round(ms * 1e3, 1), "workgroups": cus, "steps_per_wave": iters}
    return res


def cpu_baseline_per_config(torch, budget_s: float = 1.0) -> dict:
    """The reference's formulas on the host (oracle/torch_path.py) for each
    BASELINE.json config, on a bounded row sample (synthetic inputs of the config's
    shape and distribution): act-quant (3MK + 4M bytes), the quantized GEMM
    (2MNK; FP8 dequant-then-matmul, which dequantizes the weight every call as
    that path does, int8 torch._int_mm then the epilogue), LoRA (c3) and the
    end-to-end time scaled to the config's full M.  Median of at least 3 runs
    per piece, about budget_s seconds each (about 20 s in all on 8 cores)."""
    from oracle import torch_path as TP
    import torch.nn.functional as F

    gen = torch.Generator().manual_seed(0)

    def med(fn):
        times, t_start = [], time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 15):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return sorted(times)[len(times) // 2]

    out = {}
    cases = (("c1", 256, 1024, 1024, 256, "e4m3", 8, 20.0, False, True),
             ("c3_up", 24576, 5120, 13824, 512, "e4m3", 0, 0.0, True, False),
             ("c3_down", 24576, 13824, 5120, 256, "e4m3", 0, 0.0, True, False),
             ("c4_M16", 16, 5120, 5120, 16, "e4m3", 0, 0.0, False, False),
             ("c4_M64", 64, 5120, 5120, 64, "e4m3", 0, 0.0, False, False),
             ("c4_M128", 128, 5120, 5120, 128, "e4m3", 0, 0.0, False, False),
             ("c5", 40960, 5120, 5120, 512, "int8", 51, 0.0, False, False))
    for name, m, k, n, rows, fmt, outl, oscale, lora, bias in cases:
        x = torch.randn(rows, k, generator=gen)
        if outl:
            idx = torch.randperm(k, generator=gen)[:outl]
            if fmt == "int8":   # heavy-tailed Student-t(3) channels
                chi = torch.distributions.Chi2(torch.full((outl,), 3.0)).sample((rows,))
                x[:, idx] = torch.randn(rows, outl, generator=gen) / torch.sqrt(chi / 3.0)
            else:
                x[:, idx] *= oscale
        x = x.to(torch.bfloat16)
        w = (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16)
        b = (torch.randn(n, generator=gen) * 0.01).to(torch.bfloat16) if bias else None
        if fmt == "int8":
            q_w, s_w = TP.quantize_weight_int8(w)
            quant = lambda: TP.quantize_act_int8_vllm(x)  # noqa: E731
            q_a, s_a = quant()
            gemm = lambda: TP.int8_linear(q_a, s_a, q_w, s_w)  # noqa: E731
        else:
            q_w, s_w = TP.quantize_rows_e4m3(w)
            quant = lambda: TP.quantize_rows_e4m3(x)  # noqa: E731
            q_a, s_a = quant()
            gemm = lambda: TP.fp8_linear(q_a, s_a, q_w, s_w, b)  # noqa: E731
        t_q, t_g = med(quant), med(gemm)
        rec = {"M": m, "K": k, "N": n, "rows_timed": rows,
               "act_quant_GB/s": round((3 * rows * k + 4 * rows) / t_q / 1e9, 3),
               "gemm_TFLOP/s" if fmt != "int8" else "gemm_TOP/s": round(2.0 * rows * n * k / t_g / 1e12, 4)}
        t_all = t_q + t_g
        if lora:
            la = (torch.randn(128, k, generator=gen) * 0.01).to(torch.bfloat16)
            lb = (torch.randn(n, 128, generator=gen) * 0.01).to(torch.bfloat16)
            base = gemm()
            t_l = med(lambda: TP.lora_update(x, base, la, lb, 1.0))
            rec["lora_GFLOP/s"] = round(2.0 * rows * 128 * (k + n) / t_l / 1e9, 2)
            t_all += t_l
        rec["end_to_end_ms_full_M"] = round(t_all * m / rows * 1e3, 3)
        out[name] = rec
    return out


# Secondary measurements, in the order they run.
EXTRAS = {"c3": bench_c3, "c4": bench_c4, "c5": bench_c5, "f1": bench_f1, "f4": bench_f4, "a6": bench_a6,
          "h3_qkv_lora": bench_h3_lora, "ceilings": bench_ceilings}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Default warm-up of 40 steps (about 20 ms): after an idle spell the
    # MFMA clock takes about 10 ms to settle at its loaded value.
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the c3 / c4 / c5 secondary measurements")
    ap.add_argument("--extra", default=",".join(EXTRAS),
                    help="comma-separated secondary measurements to run (default: all of %s)" % ",".join(EXTRAS))
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 512 MiB device copy (known bytes) for scaling rocprof "
                         "FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    extras = [] if args.no_extra else [e for e in args.extra.split(",") if e]
    unknown = [e for e in extras if e not in EXTRAS]
    if unknown:
        print(f"bench.py: unknown --extra names {unknown} (known: {list(EXTRAS)})", file=sys.stderr)
        return 2

    import torch
    import __graft_entry__

    __graft_entry__.load_package()
    from taomate_h3_amd import ops

    dev = torch.device("cuda:0")
    rotations = 4
    xs, w, bias = make_inputs(torch, dev, rotations)
    q_w, s_w = ops.quant_rows_tiled(w, ops.FMT_E4M3FN)      # offline weight quantize + pack
    s_w = s_w.reshape(-1)
    # Activation codes in the tiled layout (M is a multiple of 16), the
    # operand layout the four-wave GEMM reads fastest.
    q_a = torch.empty(M, K, device=dev, dtype=torch.float8_e4m3fn)
    s_a = torch.empty(M, 1, device=dev, dtype=torch.float32)
    out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()

    def quant(i: int):
        ops.quant_rows_tiled(xs[i % rotations], ops.FMT_E4M3FN, codes=q_a, scales=s_a)

    def gemm(_i: int):
        ops.scaled_mm(q_a, q_w, s_a.reshape(-1), s_w, bias=bias, out=out, a_tiled=True, b_tiled=True, m=M)

    def quant_row_major(i: int):
        ops.quant_rows(xs[i % rotations], ops.FMT_E4M3FN, codes=q_rm, scales=s_a)

    q_rm = torch.empty(M, K, device=dev, dtype=torch.float8_e4m3fn)

    def step(i: int, ev=None):
        if ev is not None:
            ev[0].record()
        quant(i)
        if ev is not None:
            ev[1].record()
        gemm(i)
        if ev is not None:
            ev[2].record()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # One HIP graph per rotating input, each holding one step (act-quant and
    # GEMM, the same two kernels with the same arguments), as a serving loop
    # replays a captured step without per-launch host work.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(rotations):
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs = []
    for i in range(rotations):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(i)
        graphs.append(g)
    for i in range(args.warmup):
        graphs[i % rotations].replay()
    torch.cuda.synchronize()
    settle = settle_clock(torch, lambda i: graphs[i % rotations].replay())

    # Timed region: exactly K steps (graph replays) between two synchronisations.
    # An event after each replay, on the replay stream, gives every step's
    # device duration (the first from the event before the loop).
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    marks[0].record()
    for i in range(args.steps):
        graphs[i % rotations].replay()
        marks[i + 1].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    replay_us = [marks[i].elapsed_time(marks[i + 1]) * 1e3 for i in range(args.steps)]

    # Eager launches, for reference (on the clock the timed region left):
    # exactly K steps between two synchronisations.
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    eager_elapsed = time.perf_counter() - t0

    # Per-kernel durations with HIP events on the launch stream.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    q_step_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    g_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    q_ms = time_events(torch, quant, 4 * rotations)        # act-quant back to back, rotating inputs
    q_rm_ms = time_events(torch, quant_row_major, 4 * rotations)

    flops = 2.0 * M * N * K
    ms_per_step = elapsed / args.steps * 1e3
    value = flops / (elapsed / args.steps) / 1e12
    gemm_tflops = flops / (g_ms * 1e-3) / 1e12
    q_bytes = 3 * M * K + 4 * M
    q_gbs = q_bytes / (q_ms * 1e-3) / 1e9

    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            rec = json.loads(TRAFFIC_FILE.read_text())
            if GEMM_KERNEL_TAG in rec.get("kernel", ""):
                traffic = rec.get("hbm_bytes_per_launch")
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
            "workload": "c2: DiT QKV projection, 480p streaming chunk (BASELINE.json configs[1])",
            "M_tokens": M, "K": K, "N": N,
            "act_quant": "per-token dynamic e4m3fn, codes in the tiled layout",
            "weight_quant": "per-output-channel e4m3fn (offline, tiled layout)",
            "bias": True, "out": "bf16",
            "activation_buffers_rotated": rotations,
            "launch": "one HIP graph per step (act-quant + GEMM), replayed",
        },
        "eager_ms_per_step": round(eager_elapsed / args.steps * 1e3, 4),
        # untimed replays after the W warm-up steps, until the step time stopped falling
        "settle": settle,
        # device time of each timed step (events between the replays, in order):
        # a falling sequence is the clock still settling, a flat one a fixed cost
        "step_replay_us": {
            "min": round(min(replay_us), 1),
            "median": round(sorted(replay_us)[len(replay_us) // 2], 1),
            "max": round(max(replay_us), 1),
            "sum_ms": round(sum(replay_us) / 1e3, 4),
            "in_order": [round(v, 1) for v in replay_us],
            # the last quarter of the timed steps: the clock nearest to settled
            "last_quarter_median": round(sorted(replay_us[-max(1, len(replay_us) // 4):])[
                max(1, len(replay_us) // 4) // 2], 1),
        },
        "pct_fp8_peak": round(100.0 * value / FP8_PEAK_TFLOPS, 2),
        "roofline": {
            "kernel": "h3q gemm_w4_kernel (four-wave persistent scaled e4m3 GEMM + dequant + bias epilogue)",
            "bound": "mfma",
            "achieved": round(gemm_tflops, 2),
            "peak": FP8_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / FP8_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "avg_launch_us": round(g_ms * 1e3, 2),
            "algorithmic_flops": flops,
        },
        "act_quant": {
            "kernel": "h3q quant_rows_tiled_img_kernel (per-token e4m3fn, tiled codes)",
            "bound": "hbm",
            "achieved": round(q_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(q_gbs / HBM_PEAK_GBS, 4),
            "avg_launch_us": round(q_ms * 1e3, 2),
            "in_step_us": round(q_step_ms * 1e3, 2),
            "algorithmic_bytes": q_bytes,
            "row_major_kernel": "h3q quant_rows_vec_kernel",
            "row_major_us": round(q_rm_ms * 1e3, 2),
            "row_major_frac": round(q_bytes / (q_rm_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
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
    x_cpu, w_cpu, bias_cpu = xs[0].cpu(), w.cpu(), bias.cpu()
    del xs, w, q_w, q_a, q_rm, out
    torch.cuda.empty_cache()
    if extras:
        log("secondary configs: " + ", ".join(extras))
    for name in extras:
        result[name] = EXTRAS[name](torch, ops, dev)
        torch.cuda.empty_cache()
    ceil = result.get("ceilings")
    if ceil:
        # attainable beside nominal: the GEMM against the MFMA stream this GPU
        # sustains, the act-quant against the plain transform of its traffic
        att = ceil["mfma_e4m3"]["TFLOP/s"]
        result["roofline"]["attainable"] = att
        result["roofline"]["frac_attainable"] = round(result["roofline"]["achieved"] / att, 4)
        tr = ceil["transform"]["c2"]["GB/s"]
        result["act_quant"]["attainable"] = tr
        result["act_quant"]["frac_attainable"] = round(result["act_quant"]["achieved"] / tr, 4)
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(torch, w_cpu, bias_cpu, x_cpu)
        result["cpu_baseline"]["per_config"] = cpu_baseline_per_config(torch)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
