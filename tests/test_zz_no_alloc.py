"""The allocation-free per-tensor quantizer against the workspace entry point.

``h3q_quant_tensor_e4m3_noalloc`` keeps its partial maxima in the library's
static device scratch instead of a caller workspace.  Through the C ABI, on
consecutive calls (each later one smaller than the one before, so the
scratch still holds a larger call's partials), its codes and scale must equal
``h3q_quant_tensor_e4m3``'s bit for bit, and it must not allocate device
memory."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from _util import activations, bits8

pytestmark = pytest.mark.gpu


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _device_memory(device):
    return (torch.cuda.memory_allocated(device), torch.cuda.memory_reserved(device),
            torch.cuda.mem_get_info(device)[0])


def _run(lib, name, x, static=None):
    rows, cols = x.shape
    codes = torch.empty((rows, cols), device=x.device, dtype=torch.float8_e4m3fn)
    scale = torch.empty((), device=x.device, dtype=torch.float32)
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    if name == "h3q_quant_tensor_e4m3":
        n = int(lib.h3q_quant_tensor_workspace_floats(rows, cols))
        ws = torch.empty(n, device=x.device, dtype=torch.float32)
        rc = lib.h3q_quant_tensor_e4m3(_p(x), rows, cols, x.stride(0), _p(static), _p(ws), _p(codes), cols,
                                       _p(scale), stream)
    else:
        torch.cuda.synchronize()
        before = _device_memory(x.device)
        rc = lib.h3q_quant_tensor_e4m3_noalloc(_p(x), rows, cols, x.stride(0), _p(static), _p(codes), cols,
                                               _p(scale), stream)
        torch.cuda.synchronize()
        # torch's allocator counters, and the device's free memory, which a
        # hipMalloc inside the library would lower
        assert _device_memory(x.device) == before
    assert rc == 0, lib.h3q_last_error()
    torch.cuda.synchronize()
    return bits8(codes), scale.cpu().numpy()


@pytest.mark.parametrize("static", [False, True])
def test_noalloc_matches_workspace_entry_point_on_consecutive_calls(device, static):
    from taomate_h3_amd import _lib

    lib = _lib.lib()
    # 8192 rows use all 1024 partial slots, then fewer and fewer; 33 x 1001 takes
    # the element-wise path (k not a multiple of 8).
    shapes = [(8192, 5120), (640, 5120), (33, 1001), (5, 256)]
    for seed, (m, k) in enumerate(shapes):
        print(f"noalloc per-tensor {m}x{k} static={static}", flush=True)
        x = activations(m, k, seed=100 + seed, outlier_channels=max(1, k // 100), outlier_scale=15.0).to(device)
        st = torch.full((), 0.0123, device=device, dtype=torch.float32) if static else None
        ref_codes, ref_scale = _run(lib, "h3q_quant_tensor_e4m3", x, st)
        codes, scale = _run(lib, "h3q_quant_tensor_e4m3_noalloc", x, st)
        np.testing.assert_array_equal(codes, ref_codes)
        np.testing.assert_array_equal(scale.view(np.uint32), ref_scale.view(np.uint32))


def test_noalloc_rejects_bad_requests(device):
    from taomate_h3_amd import _lib

    lib = _lib.lib()
    p = ctypes.c_void_p(256)
    assert lib.h3q_quant_tensor_e4m3_noalloc(p, 0, 16, 16, None, p, 16, p, None) == 1
    assert b"empty tensor" in lib.h3q_last_error()
    assert lib.h3q_quant_tensor_e4m3_noalloc(p, 4, 16, 8, None, p, 16, p, None) == 1
    assert b"leading dimension" in lib.h3q_last_error()
