"""The measurement kernels behind bench.py's ``ceilings`` object
(taomate-h3_amd/csrc/ceilings.hip) do the traffic they claim: the transform
writes the high byte of every bf16 input element, the copy copies, and the
MFMA stream runs to completion with a finite result."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.fixture(scope="module")
def ceil(device):
    import bench

    return bench._ceilings_lib()


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


@pytest.mark.parametrize("shape", [(37, 5120), (16, 13824), (5, 1000)])
def test_transform_writes_high_bytes(ceil, device, shape):
    m, k = shape
    x = torch.randn(m, k, device=device).to(torch.bfloat16)
    out = torch.full((m, k), 7, device=device, dtype=torch.uint8)
    assert ceil.h3q_ceil_transform(_p(x), m, k, _p(out), 64, _stream(device)) == 0
    torch.cuda.synchronize()
    expect = (x.view(torch.int16).to(torch.int32) >> 8 & 0xFF).to(torch.uint8)
    assert torch.equal(out, expect)


def test_copy_and_read(ceil, device):
    n = (3 << 20) + 48
    src = torch.randint(0, 255, (n,), device=device, dtype=torch.uint8)
    dst = torch.zeros_like(src)
    assert ceil.h3q_ceil_copy(_p(src), _p(dst), n, 256, _stream(device)) == 0
    sink = torch.zeros(1024, device=device, dtype=torch.int32)
    assert ceil.h3q_ceil_read(_p(src), n, _p(sink), 256, _stream(device)) == 0
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    assert ceil.h3q_ceil_copy(_p(src), _p(dst), 15, 256, _stream(device)) != 0  # not whole 16-byte vectors


@pytest.mark.parametrize("int8", [0, 1])
def test_mfma_stream_runs(ceil, device, int8):
    codes = torch.randint(0, 120, (128 * 1024,), device=device, dtype=torch.uint8)
    sink = torch.full((4 * 256,), float("nan"), device=device)
    assert ceil.h3q_ceil_mfma(int8, _p(codes), 4, _p(sink), 4, _stream(device)) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(sink).all()
    assert ceil.h3q_ceil_mfma(int8, _p(codes), 3, _p(sink), 4, _stream(device)) != 0  # odd step count
