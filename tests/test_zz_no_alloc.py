"""gllm_hip_matvec_dev_noalloc (the matvec entry point that allocates
nothing) against gllm_hip_matvec_dev through the C ABI: bit-identical
outputs on two calls in a row, the second with a smaller input, for every
path that uses the activation scratch (row kernels at batch 4 / 8, the
matrix-core batch path, the prequantised batch-1 path of wide rows), a
refusal past the 4 MiB maximum, and replays of a graph that captures the
call without any call before it on that stream."""
import ctypes as C

import numpy as np
import pytest

from conftest import normal, quant_matrix
from oracle import oracle as ref

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _call(L, name, w, x, p, out, stride, stream=None):
    return getattr(L, name)(w.handle, C.c_void_p(x.data_ptr()), p, C.c_void_p(out.data_ptr()),
                            stride, C.c_void_p(stream) if stream else None)


CASES = [
    # (type, rows, cols, first p, second p)
    (ref.Q4_K, 1024, 4096, 40, 8),    # matrix cores, then the row kernels at batch 8
    (ref.Q4_K, 512, 14336, 1, 1),     # batch 1 with 14336 columns: prequantised path
    (ref.Q6_K, 768, 4096, 8, 3),
    (ref.Q8_0, 640, 2048, 5, 2),
    (ref.Q4_K, 4096, 1024, 64, 4),
]


@pytest.mark.parametrize("qtype,rows,cols,p1,p2", CASES)
def test_noalloc_matches_matvec_dev(hip, qtype, rows, cols, p1, p2):
    import torch
    L = hip._lib.load()
    data, _ = quant_matrix(qtype, rows, cols, 900 + rows + p1)
    w = hip.Weight.from_host(data, {ref.Q4_K: hip.TYPE_Q4_K, ref.Q6_K: hip.TYPE_Q6_K,
                                    ref.Q8_0: hip.TYPE_Q8_0}[qtype], rows, cols)
    for i, p in enumerate((p1, p2)):
        print(f"noalloc type {qtype} {rows}x{cols} call {i} p={p}", flush=True)
        x = torch.from_numpy(normal(910 + i + p, (p, cols))).cuda()
        a = torch.full((p, rows), -1.0, device="cuda")
        b = torch.full((p, rows), -2.0, device="cuda")
        assert _call(L, "gllm_hip_matvec_dev", w, x, p, a, rows) == 0, hip._lib.last_error()
        assert _call(L, "gllm_hip_matvec_dev_noalloc", w, x, p, b, rows) == 0, \
            hip._lib.last_error()
        torch.cuda.synchronize()
        assert np.array_equal(bits(b.cpu().numpy()), bits(a.cpu().numpy())), (i, p)


def test_noalloc_refuses_beyond_its_maximum(hip):
    import torch
    L = hip._lib.load()
    rows, cols, p = 256, 14336, 300  # act_bytes ~ 5.6 MiB > 4 MiB
    data, _ = quant_matrix(ref.Q4_K, rows, cols, 920)
    w = hip.Weight.from_host(data, hip.TYPE_Q4_K, rows, cols)
    assert hip.act_bytes(cols, p) > 4 << 20
    x = torch.zeros((p, cols), dtype=torch.float32, device="cuda")
    out = torch.full((p, rows), 7.0, device="cuda")
    rc = _call(L, "gllm_hip_matvec_dev_noalloc", w, x, p, out, rows)
    assert rc == hip.EINVAL and "maximum" in hip._lib.last_error()
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 7.0).all()


def test_noalloc_captured_on_a_fresh_stream(hip):
    """The call needs no earlier call on its stream before capture (it takes
    no scratch from the stream's pool): capture it on a new stream, replay
    the graph three times with eager work in between, compare each replay
    with the eager gllm_hip_matvec_dev result."""
    import torch
    L = hip._lib.load()
    rows, cols, p = 2048, 4096, 16
    data, _ = quant_matrix(ref.Q4_K, rows, cols, 930)
    w = hip.Weight.from_host(data, hip.TYPE_Q4_K, rows, cols)
    x = torch.from_numpy(normal(931, (p, cols))).cuda()
    want = torch.empty((p, rows), device="cuda")
    assert _call(L, "gllm_hip_matvec_dev", w, x, p, want, rows) == 0
    torch.cuda.synchronize()
    out = torch.zeros((p, rows), device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    print("capture noalloc on a fresh stream", flush=True)
    with torch.cuda.graph(g, stream=s):
        assert _call(L, "gllm_hip_matvec_dev_noalloc", w, x, p, out, rows, s.cuda_stream) == 0
    other = torch.from_numpy(normal(932, (4, cols))).cuda()
    junk = torch.empty((4, rows), device="cuda")
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out.cpu().numpy()), bits(want.cpu().numpy())), i
        # an eager call in between overwrites the shared scratch
        assert _call(L, "gllm_hip_matvec_dev_noalloc", w, other, 4, junk, rows) == 0
        torch.cuda.synchronize()


_FIRST_CALL_CAPTURED = r"""
import sys, ctypes as C
import numpy as np, torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
import gopherllm_amd as g
from conftest import normal, quant_matrix
from oracle import oracle as ref
L = g.load()
assert g.available(), g._lib.last_error()
rows, cols, p = 1024, 4096, 4
data, _ = quant_matrix(ref.Q4_K, rows, cols, 940)
w = g.Weight.from_host(data, g.TYPE_Q4_K, rows, cols)
x = torch.from_numpy(normal(941, (p, cols))).cuda()
out = torch.zeros((p, rows), device="cuda")
s = torch.cuda.Stream()
gr = torch.cuda.CUDAGraph()
with torch.cuda.graph(gr, stream=s):  # the process's first noalloc call
    rc = L.gllm_hip_matvec_dev_noalloc(w.handle, C.c_void_p(x.data_ptr()), p,
                                       C.c_void_p(out.data_ptr()), rows, C.c_void_p(s.cuda_stream))
assert rc == 0, g._lib.last_error()
want = ref.matvec_batch(ref.Q4_K, data, normal(941, (p, cols)), rows, cols)
for i in range(3):
    out.zero_()
    gr.replay()
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), i
print("first noalloc call captured: ok", flush=True)
"""


def test_noalloc_first_call_inside_a_capture():
    """In a fresh process, the very first allocation-free call is made inside
    a stream capture: the device scratch address was looked up by the
    device's load-time check (before the weight existed), so the capture
    holds no lookup, and three replays equal the oracle."""
    import os
    import subprocess
    import sys
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("child process: first noalloc call under capture", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "first noalloc call captured: ok" in r.stdout
