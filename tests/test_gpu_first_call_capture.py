"""First calls inside a HIP graph capture.

The library's one-time set-up (the prefill kernel's dynamic-LDS attribute,
the GEMV occupancy tables) runs in wush_init, which `import my_int4` calls;
the reference sets its attribute lazily on the first call and warns that
attribute calls are illegal during capture (csrc/gemm_cutlass_int4.cu:62-67).
A fresh process captures the very first fp16-tile prefill GEMM and the very
first K-split GEMV call, replays the graph twice, and compares every replay
with eager calls made afterwards (bit for bit).
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import torch
from my_int4 import _C

dev = torch.device("cuda:0")
g = torch.Generator(device=dev).manual_seed(0)
x = torch.randn(512, 4096, generator=g, device=dev).to(torch.bfloat16)
w = (torch.randn(32768, 4096, generator=g, device=dev) * 0.02).to(torch.bfloat16)
x8 = torch.randn(8, 8192, generator=g, device=dev).to(torch.bfloat16)
w8 = (torch.randn(33000, 8192, generator=g, device=dev) * 0.02).to(torch.bfloat16)
xq, xs = _C.quant_int4(x)
wq, ws = _C.quant_int4(w)
xq8, xs8 = _C.quant_int4(x8)
wq8, ws8 = _C.quant_int4(w8)
torch.cuda.synchronize()

s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(s):
    with torch.cuda.graph(graph):
        y_pre = _C.w4a4_gemm_s4(xq, xs, wq, ws)          # first call: 256x256 fp16-MFMA tiles
        y_dec = _C.w4a4_gemv_multi(xq8, xs8, wq8, ws8)   # first call: K-split GEMV (M=8, N > 32768)
torch.cuda.synchronize()
outs = []
for _ in range(2):
    graph.replay()
    torch.cuda.synchronize()
    outs.append((y_pre.clone(), y_dec.clone()))
e_pre = _C.w4a4_gemm_s4(xq, xs, wq, ws)
e_dec = _C.w4a4_gemv_multi(xq8, xs8, wq8, ws8)
torch.cuda.synchronize()
for a, b in outs:
    assert torch.equal(a.view(torch.int16), e_pre.view(torch.int16)), "prefill replay differs from eager"
    assert torch.equal(b.view(torch.int16), e_dec.view(torch.int16)), "GEMV replay differs from eager"
assert torch.isfinite(e_pre.float()).all() and torch.isfinite(e_dec.float()).all()
print("first-call capture OK", flush=True)
"""


def test_first_calls_inside_graph_capture():
    env = dict(os.environ)
    env["PYTHONPATH"] = ROOT + os.pathsep + env.get("PYTHONPATH", "")
    print("[first-call capture] fresh process: prefill 512x32768x4096, GEMV 8x33000x8192", flush=True)
    out = subprocess.run([sys.executable, "-c", SCRIPT], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=240)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-4000:]
    assert "first-call capture OK" in out.stdout
