"""The act-quant + GEMM step captured in a HIP graph (as bench.py and a
serving loop replay it): every replay, with eager work and synchronizations
between replays and the captured input overwritten in place, gives the eager
step's codes, scales and bf16 output bit for bit."""

from __future__ import annotations

import torch

import pytest

from _util import activations, bits16

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(ops, device):
    m, k, n = 512, 1024, 768
    gen = torch.Generator().manual_seed(21)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    bias = torch.randn(n, generator=gen).to(torch.bfloat16).to(device)
    q_w, s_w = ops.quant_rows_tiled(w, ops.FMT_E4M3FN)
    s_w = s_w.reshape(-1)
    x = activations(m, k, seed=22).to(device)
    q_a = torch.empty(m, k, device=device, dtype=torch.float8_e4m3fn)
    s_a = torch.empty(m, 1, device=device, dtype=torch.float32)
    out = torch.empty(m, n, device=device, dtype=torch.bfloat16)

    def step():
        ops.quant_rows(x, ops.FMT_E4M3FN, codes=q_a, scales=s_a)
        ops.scaled_mm(q_a, q_w, s_a.reshape(-1), s_w, bias=bias, out=out, b_tiled=True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()

    for replay in range(4):
        print(f"graph replay {replay}", flush=True)
        x.copy_(activations(m, k, seed=100 + replay).to(device))
        # eager reference on separate buffers, then the replay on the captured ones
        rq, rs = ops.quant_rows(x, ops.FMT_E4M3FN)
        ref = ops.scaled_mm(rq, q_w, rs.reshape(-1), s_w, bias=bias, b_tiled=True)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(q_a.view(torch.uint8), rq.view(torch.uint8))
        assert torch.equal(s_a.reshape(-1), rs.reshape(-1))
        assert (bits16(out) == bits16(ref)).all()


@pytest.mark.parametrize("rows,half", [(1024, 1024), (1030, 13824)])
def test_swiglu_table_form_in_a_graph(ops, device, rows, half):
    """The SwiGLU + e4m3 producer at table-form sizes (>= 1024 rows): an eager
    call builds the device's silu table, a captured call then replays with new
    inputs and gives the eager codes, scales and bf16 rows bit for bit."""
    gen = torch.Generator().manual_seed(rows + half)
    x = (torch.randn(rows, 2 * half, generator=gen) * 3.0).to(torch.bfloat16).to(device)
    out = torch.empty(rows, half, device=device, dtype=torch.bfloat16)
    codes = torch.empty(rows, half, device=device, dtype=torch.float8_e4m3fn)
    scales = torch.empty(rows, 1, device=device, dtype=torch.float32)

    def step():
        ops.swiglu_quant(x, fmt=ops.FMT_E4M3FN, out=out, codes=codes, scales=scales)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for replay in range(3):
        print(f"swiglu graph replay {replay} ({rows} x {half})", flush=True)
        x.copy_((torch.randn(rows, 2 * half, generator=gen) * 3.0).to(torch.bfloat16).to(device))
        r_out, r_codes, r_scales = ops.swiglu_quant(x, fmt=ops.FMT_E4M3FN, out=True)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert (bits16(out) == bits16(r_out)).all()
        assert torch.equal(codes.view(torch.uint8), r_codes.view(torch.uint8))
        assert torch.equal(scales.reshape(-1), r_scales.reshape(-1))


_FIRST_CALL_DURING_CAPTURE = r'''
import sys
sys.path.insert(0, sys.argv[1])
import torch
import __graft_entry__
__graft_entry__.load_package()
from taomate_h3_amd import ops
dev = torch.device("cuda:0")
gen = torch.Generator().manual_seed(5)
x = (torch.randn(1024, 2048, generator=gen) * 3.0).to(torch.bfloat16).to(dev)
a = torch.zeros(4, device=dev)
out = torch.empty(1024, 1024, device=dev, dtype=torch.bfloat16)
codes = torch.empty(1024, 1024, device=dev, dtype=torch.float8_e4m3fn)
scales = torch.empty(1024, 1, device=dev, dtype=torch.float32)
plain = torch.cuda.Stream()
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):            # torch's default: global capture mode
    a.add_(1.0)                      # captured on torch's capture stream
    with torch.cuda.stream(plain):   # this process's first table-form call, on a stream not being captured
        ops.swiglu_quant(x, fmt=ops.FMT_E4M3FN, out=out, codes=codes, scales=scales)
torch.cuda.synchronize()
g.replay()
torch.cuda.synchronize()
ref_out, ref_codes, ref_scales = ops.swiglu_quant(x, fmt=ops.FMT_E4M3FN, out=True)
torch.cuda.synchronize()
assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
assert torch.equal(codes.view(torch.uint8), ref_codes.view(torch.uint8))
assert torch.equal(scales, ref_scales)
assert a.tolist() == [1.0] * 4
print("ok")
'''


_FIRST_CALL_CAPTURED = r'''
import sys
sys.path.insert(0, sys.argv[1])
import torch
import __graft_entry__
__graft_entry__.load_package()
from taomate_h3_amd import ops
dev = torch.device("cuda:0")
gen = torch.Generator().manual_seed(6)
x = (torch.randn(1024, 2048, generator=gen) * 3.0).to(torch.bfloat16).to(dev)
out = torch.empty(1024, 1024, device=dev, dtype=torch.bfloat16)
codes = torch.empty(1024, 1024, device=dev, dtype=torch.float8_e4m3fn)
scales = torch.empty(1024, 1, device=dev, dtype=torch.float32)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):            # this process's first call, captured: the direct form
    ops.swiglu_quant(x, fmt=ops.FMT_E4M3FN, out=out, codes=codes, scales=scales)
torch.cuda.synchronize()
for i in range(3):
    x.copy_((torch.randn(1024, 2048, generator=gen) * 3.0).to(torch.bfloat16).to(dev))
    ref_out, ref_codes, ref_scales = ops.swiglu_quant(x, fmt=ops.FMT_E4M3FN, out=True)  # eager: the table form
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
    assert torch.equal(codes.view(torch.uint8), ref_codes.view(torch.uint8))
    assert torch.equal(scales, ref_scales)
print("ok")
'''


def test_swiglu_first_call_captured_runs_the_direct_form(device):
    """A process whose first table-form-sized call is captured into a graph
    (its stream capturing, no table yet) captures the direct form; its
    replays equal the eager calls that follow, which build the table and take
    the table form: the two forms give the same bits.  A fresh process."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True, text=True,
                         timeout=240)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stdout + res.stderr


def test_swiglu_table_first_built_while_another_stream_captures(device):
    """The silu table is built on a process's first table-form call, with a
    wait for it; that call may come on a plain stream while another stream
    of the thread is being captured in global mode (where a plain wait is
    refused), and must then build the table without disturbing the capture.
    A fresh process, so that this is its first call."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_DURING_CAPTURE, root], capture_output=True, text=True,
                         timeout=240)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stdout + res.stderr
