"""GPU parity of the per-(batch, head) FP8 quantizer (h3q_quant_per_head_e4m3,
FL/inference/fused_kernels.py:823-877) against the CPU oracle: codes and
scales bit-exact.

Also pins the oracle's scale formula on the reference's own kind of device:
torch's evaluation of ``t / 448.0`` and ``t / 127.0`` on the GPU (a multiply
by the binary32 reciprocal) over every bf16 value, and the reference's eager
torch expressions (oracle/torch_path.py) evaluated on the GPU against the
oracle's weight, row, per-tensor and per-head quantizers.

Shapes cover the vector path (head_dim % 8 == 0) with one to eight
positions per lane and one to eight column groups, the 4096-head limit, many
batches, element positions (head_dim % 8 != 0), misaligned inputs and codes,
a full attention operand (1 x 8192 tokens x 56 heads x 128), ragged token
counts, zero heads and the module mirror."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import bits8, bits16

pytestmark = pytest.mark.gpu


def _head_inputs(b, s, h, d, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(b, s, h, d, generator=gen) * torch.exp2(torch.randint(-6, 7, (b, 1, h, 1), generator=gen).float())
    if d > 3:
        x[:, :, 0, 3] *= 40.0
    return x.to(torch.bfloat16)


def _check(ops, oracle, x_cpu, x_dev=None):
    b, s, h, d = x_cpu.shape
    print(f"per_head shape={tuple(x_cpu.shape)}", flush=True)
    codes, scales = ops.quant_per_head_e4m3(x_cpu.to("cuda:0") if x_dev is None else x_dev)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_per_head_e4m3(bits16(x_cpu))
    assert codes.dtype == torch.float8_e4m3fn and tuple(codes.shape) == (b, s, h, d)
    assert tuple(scales.shape) == (b, h)
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    np.testing.assert_array_equal(bits8(codes), rq)


@pytest.mark.parametrize("shape", [
    (2, 37, 5, 64),      # 40 positions per row: one per lane, lanes 40..63 idle
    (1, 300, 40, 128),   # 640 positions: two column groups of 5 per lane
    (3, 1, 7, 96),       # one token; 12-position heads
    (1, 50, 3, 1024),    # 384 positions: one group of 6 per lane
    (1, 10, 2, 4096),    # 1024 positions: two groups of 8
    (1, 129, 64, 128),   # 1024 positions, ragged chunks
    (1, 20, 130, 8),     # one position per head
    (300, 5, 2, 16),     # many batches
    (1, 3, 4096, 8),     # the head limit: 8 column groups, one chunk
    (2, 33, 3, 20),      # head_dim % 8 != 0: element positions
    (1, 7, 1, 1),
])
def test_per_head_matches_oracle(ops, oracle, device, shape):
    x = _head_inputs(*shape, seed=sum(shape))
    if shape[2] > 1:
        x[-1, :, 1, :] = 0.0  # an all-zero head: scale 1e-12
    _check(ops, oracle, x)


def test_per_head_full_attention_operand(ops, oracle, device):
    """One attention operand at its real size: 8192 tokens x 56 heads x 128
    (the FL transformer's heads at one GPU; two column groups of 7)."""
    _check(ops, oracle, _head_inputs(1, 8192, 56, 128, seed=5))


def test_per_head_misaligned_input_or_codes(ops, oracle, device):
    """A misaligned input or code buffer keeps the 8-element positions (and
    the workspace size) with element-wise accesses."""
    x = _head_inputs(1, 64, 4, 32, seed=6)
    flat = torch.empty(x.numel() + 1, dtype=torch.bfloat16, device=device)
    flat[1:].copy_(x.reshape(-1).to(device))
    view = flat[1:].view(x.shape)
    assert view.is_contiguous() and view.data_ptr() % 16 != 0
    _check(ops, oracle, x, view)
    raw = torch.empty(x.numel() + 3, dtype=torch.uint8, device=device)
    codes = raw[3:].view(torch.float8_e4m3fn).view(x.shape)
    assert codes.is_contiguous() and codes.data_ptr() % 8 != 0
    c, s = ops.quant_per_head_e4m3(x.to(device), codes=codes)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_per_head_e4m3(bits16(x))
    np.testing.assert_array_equal(bits8(c), rq)
    np.testing.assert_array_equal(s.cpu().numpy(), rs)


def test_per_head_repeated_calls_and_empty_batch(ops, oracle, device):
    """Back-to-back calls of different shapes (fresh workspaces), explicit
    outputs, and an empty batch (no-op, empty outputs)."""
    for shape in [(1, 600, 8, 128), (2, 17, 8, 128), (1, 600, 8, 128)]:
        _check(ops, oracle, _head_inputs(*shape, seed=shape[1]))
    x = _head_inputs(2, 40, 6, 64, seed=9).to(device)
    codes = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=device)
    scales = torch.empty(2, 6, dtype=torch.float32, device=device)
    c2, s2 = ops.quant_per_head_e4m3(x, codes=codes, scales=scales)
    assert c2 is codes and s2 is scales
    torch.cuda.synchronize()
    rq, rs = oracle.quant_per_head_e4m3(bits16(x))
    np.testing.assert_array_equal(bits8(codes), rq)
    e_codes, e_scales = ops.quant_per_head_e4m3(torch.empty(0, 5, 3, 64, dtype=torch.bfloat16, device=device))
    assert e_codes.shape == (0, 5, 3, 64) and e_scales.shape == (0, 3)
    with pytest.raises(RuntimeError, match="empty"):
        ops.quant_per_head_e4m3(torch.empty(1, 0, 3, 64, dtype=torch.bfloat16, device=device))


def test_module_mirror_per_head(ops, oracle, device):
    from taomate_h3_amd.inference import fused_kernels as fk

    x = _head_inputs(1, 129, 6, 128, seed=11)
    q, s = fk.quantize_fp8_e4m3_per_head(x.to(device))
    torch.cuda.synchronize()
    rq, rs = oracle.quant_per_head_e4m3(bits16(x))
    np.testing.assert_array_equal(bits8(q), rq)
    np.testing.assert_array_equal(s.cpu().numpy(), rs)
    with pytest.raises(TypeError, match="bfloat16"):
        fk.quantize_fp8_e4m3_per_head(x.float().to(device))
    with pytest.raises(ValueError, match="head_dim"):
        ops.quant_per_head_e4m3(x.reshape(129, 6, 128).to(device))


# ------------------------------------------- the reference's expressions on the GPU

def test_device_scalar_division_is_a_reciprocal_multiply(oracle, device):
    """torch on the GPU evaluates tensor / python_scalar as t * RN(1/c): the
    form the oracle's scales restate (torch on the CPU divides)."""
    from oracle import torch_path as TP

    vals = oracle.bf16_to_f32(np.arange(0x7F80, dtype=np.uint16))
    t = torch.from_numpy(vals)
    for c in (127.0, 448.0):
        got = (t.to(device) / c).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), TP.scalar_div(t, c).numpy().view(np.uint32))


def test_reference_expressions_on_the_gpu_match_the_oracle(oracle, device):
    """The reference's eager quantizers (H3/inference/w8a8.py:57-63,
    FL/inference/fused_kernels.py:771-796 and 823-834) evaluated by torch on
    the GPU equal the oracle bit for bit (the per-tensor one in its
    bf16-divisor form)."""
    from oracle import torch_path as TP
    from _util import activations, weights

    w = weights(96, 1024, seed=3)
    w[5] = 0.0
    q, s = TP.quantize_weight_int8(w.to(device))
    rq, rs = oracle.quant_rows(bits16(w), "int8", "div")
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(s.cpu().numpy().ravel(), rs)

    x = activations(64, 2048, seed=4, outlier_channels=9)
    q, s = TP.quantize_rows_e4m3(x.to(device))
    rq, rs = oracle.quant_rows(bits16(x), "e4m3", "div")
    np.testing.assert_array_equal(bits8(q), rq)
    np.testing.assert_array_equal(s.cpu().numpy().ravel(), rs)

    # a 0-dim fp32 scale: torch on the GPU divides by the scale cast to bf16
    q, s = TP.quantize_tensor_e4m3(x.to(device))
    rq, rs = oracle.quant_tensor_e4m3(bits16(x), bf16_divisor=True)
    np.testing.assert_array_equal(bits8(q), rq)
    assert np.float32(s.item()) == rs

    h = _head_inputs(2, 77, 5, 128, seed=12)
    q, s = TP.quantize_fp8_e4m3_per_head(h.to(device))
    rq, rs = oracle.quant_per_head_e4m3(bits16(h))
    np.testing.assert_array_equal(bits8(q), rq)
    np.testing.assert_array_equal(s.cpu().numpy(), rs)


@pytest.mark.parametrize("shape", [(1, 300, 40, 128), (2, 33, 3, 20)])
def test_heads_with_infinities_and_nans(ops, oracle, device, shape):
    """A head holding an infinity gets an infinite scale (its finite elements
    -> +-0, the infinite ones -> NaN), a head holding a NaN a NaN scale (every
    code NaN); the other heads are untouched.  Against the oracle and against
    the reference's eager expression evaluated by torch on this GPU
    (FL/inference/fused_kernels.py:826-834); NaN codes are compared as NaN."""
    from oracle import torch_path as TP

    b, s, h, d = shape
    x = _head_inputs(b, s, h, d, seed=b * s + h)
    x[0, 5, 1, 2] = float("inf")
    x[b - 1, s - 1, 1, d - 1] = float("-inf")
    x[0, 7, 2, 0] = float("nan")
    print(f"per_head inf/nan shape={shape}", flush=True)
    xd = x.to(device)
    codes, scales = ops.quant_per_head_e4m3(xd)
    tq, ts = TP.quantize_fp8_e4m3_per_head(xd)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_per_head_e4m3(bits16(x))
    got_s = scales.cpu().numpy()
    for want_s in (ts.cpu().numpy(), rs):
        np.testing.assert_array_equal(np.isnan(got_s), np.isnan(want_s))
        np.testing.assert_array_equal(got_s[~np.isnan(want_s)], want_s[~np.isnan(want_s)])
    assert np.isinf(got_s[0, 1]) and np.isnan(got_s[0, 2])
    got = bits8(codes)
    for want in (bits8(tq), rq.view(np.uint8)):
        nan_q = (want & 0x7F) == 0x7F
        np.testing.assert_array_equal((got & 0x7F) == 0x7F, nan_q)
        np.testing.assert_array_equal(np.where(nan_q, 0, got), np.where(nan_q, 0, want))
