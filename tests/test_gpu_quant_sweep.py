"""Seeded sweep of the per-token quantizers over ragged shapes: row-major
codes (any K, strided rows) and tiled codes (K a multiple of 128, any row
count), every format, bit-exact codes and scales against the oracle
(H3/inference/w8a8.py:57-63,178; FL/inference/fp8.py:107-113).

K ranges over every vector-count instance of the row kernels and the general
path (odd K); row counts over the grid's one-row-per-wave and several-rows-
per-wave regimes and the tiled kernel's ragged last block."""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from _util import activations, bits8, bits16

pytestmark = pytest.mark.gpu

FMTS = [("e4m3", "div"), ("int8", "div"), ("int8", "rcp")]


def _fmt(ops, fmt, rounding):
    return (ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8,
            ops.ROUND_DIV if rounding == "div" else ops.ROUND_RCP_MUL)


def _row_cases(count: int = 24, seed: int = 71):
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        k = rng.choice([rng.randint(1, 600), 8 * rng.randint(1, 2048), 16 * rng.randint(1, 1024)])
        m = rng.choice([rng.randint(1, 40), rng.randint(41, 3000)])
        if m * k <= 8e6:
            out.append((m, k, rng.choice([0, 0, 8, 24]), *rng.choice(FMTS)))
    return out


@pytest.mark.parametrize("m,k,pad,fmt,rounding", _row_cases())
def test_rows_sweep_bit_exact(ops, oracle, device, m, k, pad, fmt, rounding):
    print(f"rows sweep {fmt}/{rounding} m={m} k={k} ldx=k+{pad}", flush=True)
    wide = activations(m, k + pad, seed=m * 7 + k, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    x = wide[:, pad:]
    f, r = _fmt(ops, fmt, rounding)
    q, s = ops.quant_rows(wide.to(device)[:, pad:], f, r)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rows(bits16(x), fmt, rounding)
    np.testing.assert_array_equal(s.cpu().numpy().ravel().view(np.uint32), rs.view(np.uint32))
    np.testing.assert_array_equal(bits8(q), rq.view(np.uint8))


def _tiled_cases(count: int = 16, seed: int = 72):
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        k = 128 * rng.randint(1, 128)
        m = rng.choice([rng.randint(1, 48), rng.randint(49, 2100)])
        if m * k <= 8e6:
            out.append((m, k, *rng.choice(FMTS)))
    return out


@pytest.mark.parametrize("m,k,fmt,rounding", _tiled_cases())
def test_tiled_sweep_bit_exact(ops, oracle, device, m, k, fmt, rounding):
    from _util import from_tiled

    print(f"tiled sweep {fmt}/{rounding} m={m} k={k}", flush=True)
    x = activations(m, k, seed=m * 5 + k, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    f, r = _fmt(ops, fmt, rounding)
    q, s = ops.quant_rows_tiled(x.to(device), f, r)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rows(bits16(x), fmt, rounding)
    np.testing.assert_array_equal(s.cpu().numpy().ravel().view(np.uint32), rs.view(np.uint32))
    np.testing.assert_array_equal(from_tiled(bits8(q), q.shape[0], k)[:m], rq.view(np.uint8))
