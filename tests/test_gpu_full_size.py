"""The BASELINE.json configurations at their own sizes, on the kernels the bench times.

Every GEMM here runs at full size on the GPU; the CPU oracle checks a
stratified set of output rows: at least one row of every 256-row tile-row,
plus the tile boundaries (rows 255 and 256) and the last row, across all N
columns.  With more tiles than workgroups, each workgroup walks several
tiles, so these rows also cover the hand-over from one tile to the next.

* int8: int32 accumulators and bf16 outputs bit-exact against the oracle's
  s_a * (s_w * float(acc)) epilogue.
* e4m3: against the oracle's model of the FP8 matrix instruction, within the
  per-element bound of ``_assert_fp8_close`` (almost all outputs bit-identical).
* LoRA (c3): against the reference's three rounding points
  (H3/inference/lora_checkpoint.py:196-205): per element within one bf16
  ulp of each of the three rounded quantities plus the FP8 accumulator
  bound, 99% within one ulp of the output, and 2^-7 relative error.

References: H3/inference/w8a8.py:178-186 (per-token int8 + CUTLASS GEMM),
FL/distributed/linear.py:92-100 (FP8 GEMM), H3/inference/lora_checkpoint.py:196-205.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import activations, bf16_ulp, bits16, bits8, from_tiled, weights
from test_gpu_gemm import _assert_fp8_close

pytestmark = pytest.mark.gpu


def stratified_rows(m: int, seed: int = 0, per_tile: int = 1) -> np.ndarray:
    """One (or more) seeded row of every 256-row tile-row, plus rows 0, 255,
    256 and m - 1."""
    rng = np.random.default_rng(seed)
    rows = {0, min(255, m - 1), min(256, m - 1), m - 1}
    for t in range((m + 255) // 256):
        lo, hi = 256 * t, min(256 * t + 256, m)
        rows.update(int(r) for r in rng.integers(lo, hi, size=per_tile))
    return np.array(sorted(rows))


def _bias(n: int, seed: int) -> torch.Tensor:
    return (torch.randn(n, generator=torch.Generator().manual_seed(seed)) * 0.01).to(torch.bfloat16)


def _quant_weights(ops, w, device, fmt):
    f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
    return ops.quant_rows_tiled(w.to(device), f, ops.ROUND_DIV)


@pytest.mark.parametrize("a_tiled", [False, True])
def test_c2_qkv_tiled_weights_stratified(ops, oracle, device, a_tiled):
    """c2 (M=8192, K=5120, N=15360, e4m3, bias): the bench's instance (tiled
    weights), with row-major and with tiled activations; 1920 tiles over the
    persistent grid, so every workgroup runs several tiles."""
    m, k, n = 8192, 5120, 15360
    print(f"c2 tiled weights a_tiled={a_tiled}", flush=True)
    x = activations(m, k, seed=0, outlier_channels=k // 100, outlier_scale=15.0)
    w = weights(n, k, seed=1)
    bias = _bias(n, 2)
    qw, sw = _quant_weights(ops, w, device, "e4m3")
    xg = x.to(device)
    if a_tiled:
        qa, sa = ops.quant_rows_tiled(xg, ops.FMT_E4M3FN, ops.ROUND_DIV)
    else:
        qa, sa = ops.quant_rows(xg, ops.FMT_E4M3FN)
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), bias=bias.to(device), a_tiled=a_tiled,
                        b_tiled=True, m=m, n=n)
    torch.cuda.synchronize()
    rows = stratified_rows(m)
    rqa, rsa = oracle.quant_rows(bits16(x[torch.from_numpy(rows)]), "e4m3")
    rqw, rsw = oracle.quant_rows(bits16(w), "e4m3")
    np.testing.assert_array_equal(sw.cpu().numpy().ravel(), rsw)
    _assert_fp8_close(oracle, bits16(out)[rows], rqa, rsa, rqw, rsw, bits16(bias))


def test_c2_row_major_and_tiled_layouts_agree(ops, device):
    """The four operand-layout combinations of the c2 GEMM give the same bits."""
    m, k, n = 8192, 5120, 15360
    x = activations(m, k, seed=3, outlier_channels=k // 100, outlier_scale=15.0).to(device)
    w = weights(n, k, seed=4).to(device)
    bias = _bias(n, 5).to(device)
    qa, sa = ops.quant_rows(x, ops.FMT_E4M3FN)
    qat, _ = ops.quant_rows_tiled(x, ops.FMT_E4M3FN, ops.ROUND_DIV)
    qw, sw = ops.quant_rows(w, ops.FMT_E4M3FN)
    qwt, _ = ops.quant_rows_tiled(w, ops.FMT_E4M3FN, ops.ROUND_DIV)
    outs = []
    for a, at in ((qa, False), (qat, True)):
        for b, bt in ((qw, False), (qwt, True)):
            outs.append(ops.scaled_mm(a, b, sa.reshape(-1), sw.reshape(-1), bias=bias, a_tiled=at, b_tiled=bt,
                                      m=m, n=n))
    torch.cuda.synchronize()
    ref = bits16(outs[0])
    for o in outs[1:]:
        np.testing.assert_array_equal(bits16(o), ref)


@pytest.mark.parametrize("a_tiled", [False, True])
@pytest.mark.parametrize("which", ["up", "down"])
def test_c3_ffn_lora_stratified(ops, oracle, device, which, a_tiled):
    """c3 (768p FFN, M=24576): up N=13824 K=5120 and down N=5120 K=13824,
    e4m3 tiled weights, rank-128 bf16 LoRA with alpha=128 (scale 1.0) in the
    GEMM epilogue; row-major activation codes, and the tiled ones the bench
    times."""
    m = 24576
    n, k = (13824, 5120) if which == "up" else (5120, 13824)
    rank = 128
    print(f"c3 {which}: {m}x{n}x{k} LoRA rank {rank} a_tiled={a_tiled}", flush=True)
    x = activations(m, k, seed=7, outlier_channels=0)
    w = weights(n, k, seed=8)
    gen = torch.Generator().manual_seed(9)
    la = (torch.randn(rank, k, generator=gen) * 0.01).to(torch.bfloat16)
    lb = (torch.randn(n, rank, generator=gen) * 0.01).to(torch.bfloat16)
    xg = x.to(device)
    qw, sw = _quant_weights(ops, w, device, "e4m3")
    quant = ops.quant_rows_tiled if a_tiled else ops.quant_rows
    qa, sa = quant(xg, ops.FMT_E4M3FN)
    t = ops.lora_down(xg, la.to(device))
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), lora_t=t, lora_b=lb.to(device), lora_scale=1.0,
                        a_tiled=a_tiled, b_tiled=True, m=m, n=n)
    torch.cuda.synchronize()
    rows = stratified_rows(m, seed=1)
    xr = bits16(x[torch.from_numpy(rows)])
    # t = bf16(x @ A^T): the GPU's binary32 sum over K and the oracle's binary64
    # one round to bf16 within one ulp of each other (plus the binary32 sum error).
    t_exact = oracle.lora_down_reference(xr, bits16(la))
    t_gpu = oracle.bf16_to_f32(bits16(t)[rows]).astype(np.float64)
    t_abs = np.abs(oracle.bf16_to_f32(xr).astype(np.float64)) @ np.abs(oracle.bf16_to_f32(bits16(la))).T
    assert np.all(np.abs(t_gpu - t_exact) <= bf16_ulp(np.abs(t_exact)) + k * 2.0 ** -24 * t_abs)
    # The epilogue is then checked from the GPU's t, with the reference's
    # rounding points (H3/inference/lora_checkpoint.py:196-205):
    #   u = bf16(t @ B^T); out = bf16(base + bf16(u * 1.0)).
    rqa, rsa = oracle.quant_rows(xr, "e4m3")
    rqw, rsw = oracle.quant_rows(bits16(w), "e4m3")
    model, rbound = oracle.gemm_e4m3_mfma(rqa, rqw)
    base_f = oracle.bf16_to_f32(oracle.epilogue(model, rsa, rsw)).astype(np.float64)
    lbf = oracle.bf16_to_f32(bits16(lb)).astype(np.float64)
    upd = oracle.bf16_to_f32(oracle.f32_to_bf16_fast((t_gpu @ lbf.T).astype(np.float32))).astype(np.float64)
    ref = oracle.bf16_to_f32(oracle.f32_to_bf16_fast((base_f + upd).astype(np.float32))).astype(np.float64)
    got = oracle.bf16_to_f32(bits16(out)[rows]).astype(np.float64)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 2.0 ** -7, rel
    # The reference rounds the base output, the update and the sum to bf16
    # (three roundings); the fused epilogue rounds the binary32 sum once.  Per
    # element the two differ by at most an ulp of each rounded quantity, plus
    # what separates the GPU's accumulators from the oracle's models: the FP8
    # instruction's binary32 combination rounding (rbound, times the two
    # scales), the epilogue's scale products (2^-22 relative) and the binary32
    # sum over the rank (rank * 2^-24 of sum |t||b|).
    scale = np.abs(rsa.astype(np.float64)).reshape(-1, 1) * np.abs(rsw.astype(np.float64)).reshape(1, -1)
    upd_abs = np.abs(t_gpu) @ np.abs(lbf).T
    bound = (bf16_ulp(base_f) + bf16_ulp(upd) + bf16_ulp(np.maximum(np.abs(ref), np.abs(got))) + rbound * scale
             + 2.0 ** -22 * np.abs(base_f) + rank * 2.0 ** -24 * upd_abs)
    err = np.abs(got - ref)
    assert np.all(err <= bound), (err / bound).max()
    assert np.mean(err <= bf16_ulp(np.abs(ref))) >= 0.99


@pytest.mark.parametrize("a_tiled", [False, True])
def test_c5_int8_full_size_bit_exact(ops, oracle, device, a_tiled):
    """c5 (1080p, M=40960, K=N=5120, int8 with Student-t outlier channels):
    per-token vLLM-form activation codes (row-major, and tiled as the bench
    times them), per-channel weight codes (tiled), bf16 outputs bit-exact on
    the stratified rows; int32 accumulators bit-exact on the same rows."""
    m, k, n = 40960, 5120, 5120
    print(f"c5 int8 full size a_tiled={a_tiled}", flush=True)
    x = activations(m, k, seed=11, outlier_channels=k // 100, student_t=True)
    w = weights(n, k, seed=12)
    xg = x.to(device)
    qw, sw = _quant_weights(ops, w, device, "int8")
    quant = ops.quant_rows_tiled if a_tiled else ops.quant_rows
    qa, sa = quant(xg, ops.FMT_INT8, ops.ROUND_RCP_MUL)
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), a_tiled=a_tiled, b_tiled=True, m=m, n=n)
    torch.cuda.synchronize()
    rows = stratified_rows(m, seed=2)
    rqa, rsa = oracle.quant_rows(bits16(x[torch.from_numpy(rows)]), "int8", "rcp")
    codes = from_tiled(bits8(qa), m, k) if a_tiled else bits8(qa)
    np.testing.assert_array_equal(codes[rows], rqa.view(np.uint8))
    if a_tiled:
        qa = ops.quant_rows(xg, ops.FMT_INT8, ops.ROUND_RCP_MUL)[0]  # row-major rows for the i32 entry point
    rqw, rsw = oracle.quant_rows(bits16(w), "int8", "div")
    acc = oracle.gemm_i8_i32(rqa, rqw)
    np.testing.assert_array_equal(bits16(out)[rows], oracle.epilogue(acc, rsa, rsw))
    # raw accumulators of the same rows through the integer entry point
    qw_rows, _ = ops.quant_rows(w.to(device), ops.FMT_INT8, ops.ROUND_DIV)
    acc_gpu = ops.gemm_i8_i32(qa[torch.from_numpy(rows).to(device)].contiguous(), qw_rows)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc_gpu.cpu().numpy(), acc)


@pytest.mark.parametrize("fmt", ["int8", "e4m3"])
@pytest.mark.parametrize("per_tensor", [False, True])
def test_more_tiles_than_workgroups(ops, oracle, device, fmt, per_tensor):
    """m=4608, n=4096, k=1024 with tiled weights and bias: 288 output tiles,
    more than the persistent grid, so 32 workgroups run a second tile.
    int8: every row bit-exact.  e4m3: whole tile-rows 0, 8 and 17 and the
    boundaries against the instruction model.  Per-row and per-tensor scales."""
    m, n, k = 4608, 4096, 1024
    f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
    ar = ops.ROUND_DIV if fmt == "e4m3" else ops.ROUND_RCP_MUL
    x = activations(m, k, seed=13, outlier_channels=10, outlier_scale=15.0)
    w = weights(n, k, seed=14)
    bias = _bias(n, 15)
    qw, sw = _quant_weights(ops, w, device, fmt)
    qa, sa = ops.quant_rows(x.to(device), f, ar)
    if per_tensor:
        sa = sa.reshape(-1)[:1].clone()
        sw = sw.reshape(-1)[:1].clone()
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), bias=bias.to(device), b_tiled=True, n=n)
    torch.cuda.synchronize()
    rqa, rsa = oracle.quant_rows(bits16(x), fmt, "div" if fmt == "e4m3" else "rcp")
    rqw, rsw = oracle.quant_rows(bits16(w), fmt, "div")
    if per_tensor:
        rsa, rsw = rsa[:1], rsw[:1]
    if fmt == "int8":
        ref = oracle.epilogue(oracle.gemm_i8_i32(rqa, rqw), rsa, rsw, bits16(bias))
        np.testing.assert_array_equal(bits16(out), ref)
    else:
        rows = np.unique(np.concatenate([np.arange(0, 256), np.arange(2048, 2304), np.arange(4352, 4608),
                                         [255, 256, 511, 512, 4607]]))
        _assert_fp8_close(oracle, bits16(out)[rows], rqa[rows], rsa if per_tensor else rsa[rows], rqw, rsw,
                          bits16(bias))


def test_ragged_large_m_tiled_activations(ops, oracle, device):
    """A ragged M (not a multiple of 16 or 256) with tiled activations and
    tiled weights through the four-wave GEMM, int8: every output bit-exact."""
    m, n, k = 1000, 3000, 1024
    x = activations(m, k, seed=17, outlier_channels=5)
    w = weights(n - 8, k, seed=18)            # n = 2992: a partial last tile column
    n = n - 8
    qw, sw = _quant_weights(ops, w, device, "int8")
    qa, sa = ops.quant_rows_tiled(x.to(device), ops.FMT_INT8, ops.ROUND_RCP_MUL)
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), a_tiled=True, b_tiled=True, m=m, n=n)
    torch.cuda.synchronize()
    rqa, rsa = oracle.quant_rows(bits16(x), "int8", "rcp")
    rqw, rsw = oracle.quant_rows(bits16(w), "int8", "div")
    np.testing.assert_array_equal(bits16(out), oracle.epilogue(oracle.gemm_i8_i32(rqa, rqw), rsa, rsw))


@pytest.mark.parametrize("fmt", ["int8", "e4m3"])
def test_split_tail_ragged_half_tiles(ops, oracle, device, fmt):
    """300 tile-rows of one tile-column (m = 299 * 256 + 100, n = 200, k = 256,
    bias, tiled weights): on a 256-workgroup grid the last round holds 44
    tiles, so they run as 128-row halves, the ragged last tile-row among them
    (its second half is empty).  int8: every output bit-exact.  e4m3: the
    first tile-row and the last 1380 rows against the instruction model."""
    m, n, k = 299 * 256 + 100, 200, 256
    f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
    ar = ops.ROUND_DIV if fmt == "e4m3" else ops.ROUND_RCP_MUL
    print(f"split tail {fmt}: {m}x{n}x{k}", flush=True)
    x = activations(m, k, seed=21, outlier_channels=3, outlier_scale=15.0)
    w = weights(n, k, seed=22)
    bias = _bias(n, 23)
    qw, sw = _quant_weights(ops, w, device, fmt)
    qa, sa = ops.quant_rows(x.to(device), f, ar)
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), bias=bias.to(device), b_tiled=True, n=n)
    torch.cuda.synchronize()
    rqw, rsw = oracle.quant_rows(bits16(w), fmt, "div")
    if fmt == "int8":
        rqa, rsa = oracle.quant_rows(bits16(x), "int8", "rcp")
        ref = oracle.epilogue(oracle.gemm_i8_i32(rqa, rqw), rsa, rsw, bits16(bias))
        np.testing.assert_array_equal(bits16(out), ref)
    else:
        rows = np.concatenate([np.arange(0, 256), np.arange(m - 1380, m)])
        rqa, rsa = oracle.quant_rows(bits16(x[torch.from_numpy(rows)]), "e4m3")
        _assert_fp8_close(oracle, bits16(out)[rows], rqa, rsa, rqw, rsw, bits16(bias))


@pytest.mark.parametrize("fmt,rank,b_tiled,a_tiled", [("e4m3", 128, True, False), ("e4m3", 72, False, False),
                                                    ("int8", 128, True, False), ("e4m3", 128, True, True),
                                                    ("int8", 64, False, True)])
def test_lora_epilogue_four_wave_vs_per_tile_kernel(ops, device, fmt, rank, b_tiled, a_tiled):
    """The LoRA epilogue of the persistent four-wave GEMM against the per-tile
    kernel's (reached through an output row stride that the four-wave GEMM
    does not take).  The per-tile kernel sums t . lora_b into a fresh
    accumulator L and rounds fma(scale, L, y) once; the four-wave GEMM adds
    t . lora_b onto y / scale in the accumulators and multiplies by the scale.
    Both are binary32 to within a few units in the last place of the
    operands, so every output is within one bf16 ulp of the other (plus
    2^-20 of |y| + scale |t| . |lora_b| where the two nearly cancel) and
    almost all are equal.
    m = 18 * 256 + 100, n = 4088: 304 tiles, a ragged last tile-row and
    tile-column, the last round as half tiles; bias; scale 0.75 (not a power
    of two); rank 128 and ranks (72, 64) that leave rank groups partly or
    wholly empty; the four-wave GEMM also with tiled activations (the
    per-tile kernel reads them row-major)."""
    m, n, k = 18 * 256 + 100, 4088, 512
    f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
    ar = ops.ROUND_DIV if fmt == "e4m3" else ops.ROUND_RCP_MUL
    print(f"LoRA four-wave vs per-tile {fmt} rank {rank} b_tiled={b_tiled} a_tiled={a_tiled}", flush=True)
    x = activations(m, k, seed=31, outlier_channels=5, outlier_scale=15.0).to(device)
    w = weights(n, k, seed=32).to(device)
    gen = torch.Generator().manual_seed(33)
    la = (torch.randn(rank, k, generator=gen) * 0.01).to(torch.bfloat16).to(device)
    lb = (torch.randn(n, rank, generator=gen) * 0.01).to(torch.bfloat16).to(device)
    bias = _bias(n, 34).to(device)
    qa, sa = ops.quant_rows(x, f, ar)
    qw, sw = ops.quant_rows_tiled(w, f, ops.ROUND_DIV) if b_tiled else ops.quant_rows(w, f, ops.ROUND_DIV)
    t = ops.lora_down(x, la)
    kw = dict(bias=bias, lora_t=t, lora_b=lb, lora_scale=0.75, b_tiled=b_tiled, n=n)
    if a_tiled:
        qat, _ = ops.quant_rows_tiled(x, f, ar)
        four_wave = ops.scaled_mm(qat, qw, sa.reshape(-1), sw.reshape(-1), a_tiled=True, m=m, **kw)
    else:
        four_wave = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), **kw)
    wide = torch.empty(m, n + 4, device=device, dtype=torch.bfloat16)
    per_tile = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), out=wide[:, :n], **kw)
    torch.cuda.synchronize()
    base = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), bias=bias, b_tiled=b_tiled, n=n)
    torch.cuda.synchronize()
    got = four_wave.float().cpu().numpy().astype(np.float64)
    ref = per_tile.contiguous().float().cpu().numpy().astype(np.float64)
    # Where y and scale * (t . lora_b) nearly cancel, the two binary32
    # summation orders differ by a few units of 2^-24 of the operands, which
    # can exceed a bf16 ulp of the small result: bound by 2^-20 of them.
    upd = 0.75 * (np.abs(t.float().cpu().numpy().astype(np.float64)) @
                  np.abs(lb.float().cpu().numpy().astype(np.float64)).T)
    ops_mag = np.abs(base.float().cpu().numpy().astype(np.float64)) + upd
    bound = bf16_ulp(np.maximum(np.abs(got), np.abs(ref))) + 2.0 ** -20 * ops_mag
    bad = np.argwhere(np.abs(got - ref) > bound)
    assert bad.size == 0, (f"{len(bad)} outputs differ by more than the bound, first at (row, col) "
                           f"{[tuple(b) for b in bad[:6]]}: {[(got[tuple(b)], ref[tuple(b)]) for b in bad[:6]]}")
    same = float(np.mean(bits16(four_wave) == bits16(per_tile.contiguous())))
    print(f"bit-identical to the per-tile kernel: {same:.5f}", flush=True)
    assert same >= 0.99, same


@pytest.mark.parametrize("name,m,n,k", [("qkv_480p_phase3", 592, 10752, 5376),
                                        ("fc1_1088p_phase3", 2640, 14336, 5376)])
def test_h3_production_shapes_int8(ops, oracle, device, name, m, n, k):
    """The production W8A8 path at real H3 shapes (TP-local QKV N = 10752 and
    fc1 N = 14336, K = 5376 = 42 k-steps of 128; M per Ulysses rank from
    H3/streaming/geometry.py:173-200, a multiple of 16 but not of 256):
    per-token int8 activations (vLLM form) in the tiled layout, tiled int8
    weights, no bias, as quant_activations_for feeds the four-wave GEMM.
    Codes and bf16 outputs bit-exact on every 256-row tile-row's sampled rows,
    the ragged last tile-row whole."""
    print(f"H3 {name}: {m}x{n}x{k} int8", flush=True)
    x = activations(m, k, seed=41, outlier_channels=k // 100, outlier_scale=15.0)
    w = weights(n, k, seed=42)
    xg = x.to(device)
    qw, sw = _quant_weights(ops, w, device, "int8")
    ops.mark_tiled(qw)  # as the module path records a packed weight
    qa, sa, a_tiled = ops.quant_activations_for(xg, ops.FMT_INT8, ops.ROUND_RCP_MUL, qw)
    assert a_tiled
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), a_tiled=True, b_tiled=True, m=m, n=n)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([stratified_rows(m, seed=5), np.arange(m // 256 * 256, m)]))
    rqa, rsa = oracle.quant_rows(bits16(x[torch.from_numpy(rows)]), "int8", "rcp")
    rqw, rsw = oracle.quant_rows(bits16(w), "int8", "div")
    np.testing.assert_array_equal(sw.cpu().numpy().ravel(), rsw)
    np.testing.assert_array_equal(sa.cpu().numpy().ravel()[rows], rsa)
    ref = oracle.epilogue(oracle.gemm_i8_i32(rqa, rqw), rsa, rsw)
    np.testing.assert_array_equal(bits16(out)[rows], ref)


def test_h3_production_shape_fp8_lora(ops, oracle, device):
    """FL2VA's FP8 path with a rank-128 LoRA at a real shape: QKV at 768p
    phase 0 (M = 3200, N = 10752, K = 5376), per-token x per-channel e4m3,
    tiled activations and weights, the fused LoRA epilogue (scale 1.0), against
    the reference's three rounding points (H3/inference/lora_checkpoint.py:196-205)
    on the stratified rows plus the ragged last tile-row."""
    m, n, k, rank = 3200, 10752, 5376, 128
    print(f"H3 FP8 + LoRA {m}x{n}x{k}", flush=True)
    x = activations(m, k, seed=43, outlier_channels=k // 100, outlier_scale=15.0)
    w = weights(n, k, seed=44)
    gen = torch.Generator().manual_seed(45)
    la = (torch.randn(rank, k, generator=gen) * 0.01).to(torch.bfloat16)
    lb = (torch.randn(n, rank, generator=gen) * 0.01).to(torch.bfloat16)
    xg = x.to(device)
    qw, sw = _quant_weights(ops, w, device, "e4m3")
    ops.mark_tiled(qw)
    qa, sa, a_tiled = ops.quant_activations_for(xg, ops.FMT_E4M3FN, ops.ROUND_DIV, qw, lora=True)
    assert a_tiled
    t = ops.lora_down(xg, la.to(device))
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), lora_t=t, lora_b=lb.to(device), lora_scale=1.0,
                        a_tiled=True, b_tiled=True, m=m, n=n)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([stratified_rows(m, seed=6), np.arange(m // 256 * 256, m)]))
    xr = bits16(x[torch.from_numpy(rows)])
    rqa, rsa = oracle.quant_rows(xr, "e4m3")
    rqw, rsw = oracle.quant_rows(bits16(w), "e4m3")
    model, rbound = oracle.gemm_e4m3_mfma(rqa, rqw)
    base_f = oracle.bf16_to_f32(oracle.epilogue(model, rsa, rsw)).astype(np.float64)
    t_gpu = oracle.bf16_to_f32(bits16(t)[rows]).astype(np.float64)
    lbf = oracle.bf16_to_f32(bits16(lb)).astype(np.float64)
    upd = oracle.bf16_to_f32(oracle.f32_to_bf16_fast((t_gpu @ lbf.T).astype(np.float32))).astype(np.float64)
    ref = oracle.bf16_to_f32(oracle.f32_to_bf16_fast((base_f + upd).astype(np.float32))).astype(np.float64)
    got = oracle.bf16_to_f32(bits16(out)[rows]).astype(np.float64)
    scale = np.abs(rsa.astype(np.float64)).reshape(-1, 1) * np.abs(rsw.astype(np.float64)).reshape(1, -1)
    upd_abs = np.abs(t_gpu) @ np.abs(lbf).T
    bound = (bf16_ulp(base_f) + bf16_ulp(upd) + bf16_ulp(np.maximum(np.abs(ref), np.abs(got))) + rbound * scale
             + 2.0 ** -22 * np.abs(base_f) + rank * 2.0 ** -24 * upd_abs + 2.0 ** -20 * (np.abs(base_f) + upd_abs))
    err = np.abs(got - ref)
    assert np.all(err <= bound), (err / bound).max()
    assert np.mean(err <= bf16_ulp(np.abs(ref))) >= 0.99
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2.0 ** -7
