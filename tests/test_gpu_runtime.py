"""Runtime contract of the C ABI on the device: several host threads at once
(several Runners in one process, kernels_amd64.go:71-80), several streams on
one thread, scratch that stays valid for captured graphs, the load-time
known-answer check (the reference's q8kSelfCheck, q8k_dot_arm64.go:146-228),
and failing calls that write nothing (the Metal seam's contract,
model.go:700-725)."""
import os
import subprocess
import sys
import threading

import numpy as np
import pytest

from conftest import normal, quant_matrix
from oracle import oracle as ref

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_four_host_threads_share_handles(hip):
    """4 host threads call gllm_hip_matvec (Q4_K and Q6_K weights) and
    gllm_hip_attend_group on shared handles at the same time; every result
    equals the oracle.  The first mismatch stops the run."""
    rows, cols = 2048, 1024
    d4, _ = quant_matrix(ref.Q4_K, rows, cols, 61)
    d6, _ = quant_matrix(ref.Q6_K, rows, cols, 62)
    w4 = hip.Weight.from_host(d4, hip.TYPE_Q4_K, rows, cols)
    w6 = hip.Weight.from_host(d6, hip.TYPE_Q6_K, rows, cols)
    hd, kvd, ctx = 128, 512, 96
    kv = hip.KVCacheF16(1, kvd, kvd, ctx)
    k, v = normal(63, (ctx, kvd)), normal(64, (ctx, kvd))
    for p in range(ctx):
        kv.store_kv(0, p, k[p], v[p])
    k16, v16 = ref.f32_to_f16(k), ref.f32_to_f16(v)
    n_threads, iters = 4, 12
    xs = [normal(70 + t, cols) for t in range(n_threads)]
    qs = [normal(80 + t, 4 * hd) for t in range(n_threads)]
    want4 = [ref.matvec(ref.Q4_K, d4, x, rows, cols) for x in xs]
    want6 = [ref.matvec(ref.Q6_K, d6, x, rows, cols) for x in xs]
    wanta = [ref.attend_group_f16(q, k16.ravel()[(t % 4) * hd:], v16.ravel()[(t % 4) * hd:], 4,
                                  kvd, kvd, hd, hd, 0, ctx - 1 - t, np.float32(0.088))
             for t, q in enumerate(qs)]
    errors = []
    stop = threading.Event()

    def work(t):
        try:
            for i in range(iters):
                if stop.is_set():
                    return
                if not np.array_equal(bits(w4.matvec_into(xs[t])), bits(want4[t])):
                    raise AssertionError(f"thread {t} iter {i}: Q4_K matvec differs")
                if not np.array_equal(bits(w6.matvec_into(xs[t])), bits(want6[t])):
                    raise AssertionError(f"thread {t} iter {i}: Q6_K matvec differs")
                got = kv.attend_head_group(0, t % 4, qs[t], 4, hd, hd, 0, ctx - 1 - t,
                                           np.float32(0.088))
                if not np.array_equal(bits(got), bits(wanta[t])):
                    raise AssertionError(f"thread {t} iter {i}: attention differs")
        except Exception as e:  # first failure stops every thread
            errors.append(e)
            stop.set()

    print("4 host threads x 12 iterations", flush=True)
    ths = [threading.Thread(target=work, args=(t,)) for t in range(n_threads)]
    for th in ths:
        th.start()
    for th in ths:
        th.join(timeout=90)
    assert not any(th.is_alive() for th in ths), "a thread did not finish"
    assert not errors, errors[0]


def test_two_streams_on_one_thread(hip):
    """Two batched matvecs enqueued back to back on two streams of one host
    thread (no synchronisation between them) each use their own scratch: both
    results equal the oracle."""
    import torch
    p = 8
    da, _ = quant_matrix(ref.Q4_K, 1024, 2048, 65)
    db, _ = quant_matrix(ref.Q6_K, 768, 4096, 66)
    wa = hip.Weight.from_host(da, hip.TYPE_Q4_K, 1024, 2048)
    wb = hip.Weight.from_host(db, hip.TYPE_Q6_K, 768, 4096)
    xa, xb = normal(67, (p, 2048)), normal(68, (p, 4096))
    dxa, dxb = torch.from_numpy(xa).cuda(), torch.from_numpy(xb).cuda()
    oa = torch.empty((p, 1024), dtype=torch.float32, device="cuda")
    ob = torch.empty((p, 768), dtype=torch.float32, device="cuda")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    print("two streams, one thread", flush=True)
    for _ in range(3):
        wa.matvec_dev(dxa, oa, stream=s1.cuda_stream)
        wb.matvec_dev(dxb, ob, stream=s2.cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(bits(oa.cpu().numpy()), bits(ref.matvec_batch(ref.Q4_K, da, xa, 1024, 2048)))
    assert np.array_equal(bits(ob.cpu().numpy()), bits(ref.matvec_batch(ref.Q6_K, db, xb, 768, 4096)))


def test_captured_graph_survives_scratch_growth(hip):
    """A batched matvec captured into a graph keeps its scratch: a later,
    larger call on the same stream grows the scratch slot (a new buffer; the
    captured one stays allocated), and every replay, with eager work and
    synchronisation in between, still equals the eager result.  A call that
    would have to grow the slot inside a capture fails with GLLM_EUNSUP
    instead of allocating."""
    import torch
    rows, cols = 512, 1024
    d, _ = quant_matrix(ref.Q4_K, rows, cols, 69)
    w = hip.Weight.from_host(d, hip.TYPE_Q4_K, rows, cols)
    x4, x64 = normal(70, (4, cols)), normal(71, (64, cols))
    dx4, dx64 = torch.from_numpy(x4).cuda(), torch.from_numpy(x64).cuda()
    o4 = torch.empty((4, rows), dtype=torch.float32, device="cuda")
    o64 = torch.empty((64, rows), dtype=torch.float32, device="cuda")
    want4 = ref.matvec_batch(ref.Q4_K, d, x4, rows, cols)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        w.matvec_dev(dx4, o4)  # sizes the slot outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("capture batch-4 matvec", flush=True)
    with torch.cuda.graph(g, stream=s):
        w.matvec_dev(dx4, o4)
    with torch.cuda.stream(s):
        w.matvec_dev(dx64, o64)  # grows the slot this stream's calls use
    torch.cuda.synchronize()
    for i in range(3):
        o4.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(o4.cpu().numpy()), bits(want4)), i
        with torch.cuda.stream(s):
            w.matvec_dev(dx64, o64)
        torch.cuda.synchronize()
    assert np.array_equal(bits(o64.cpu().numpy()),
                          bits(ref.matvec_batch(ref.Q4_K, d, x64, rows, cols)))
    # growth inside a capture is refused, and nothing is enqueued
    s2 = torch.cuda.Stream()
    x128 = torch.from_numpy(normal(72, (128, cols))).cuda()
    o128 = torch.empty((128, rows), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    print("capture that would grow scratch", flush=True)
    with pytest.raises(hip.GllmError) as ei:
        with torch.cuda.graph(g2, stream=s2):
            w.matvec_dev(x128, o128)
    assert ei.value.code == hip.EUNSUP
    torch.cuda.synchronize()


def test_self_check_passed_on_this_device(hip):
    """gllm_hip_available() runs the load-time known-answer check; it passes
    on a working MI355X."""
    assert hip.available(), hip._lib.last_error()


def test_self_check_failure_refuses_weights():
    """With a mistake planted in the host-side known answer
    (GLLM_SELF_CHECK_PLANT=1), the check fails: gllm_hip_available() is 0 and
    every weight constructor fails with GLLM_EUNSUP, so the caller falls
    back to its CPU kernels.  Runs in a child process (the check runs once
    per process and device)."""
    code = (
        "import ctypes, numpy as np, sys\n"
        f"sys.path.insert(0, {ROOT!r})\n"
        "from gopherllm_amd import _lib\n"
        "L = _lib.load()\n"
        "a = L.gllm_hip_available()\n"
        "msg = _lib.last_error()\n"
        "raw = np.zeros(144 * 4, np.uint8)\n"
        "h = L.gllm_hip_weight_new(raw.ctypes.data_as(ctypes.c_void_p), raw.nbytes, 12, 1, 1024)\n"
        "print('RESULT', a, bool(h), msg, '|', _lib.last_error(), flush=True)\n"
    )
    env = dict(os.environ, GLLM_SELF_CHECK_PLANT="1")
    print("child process with a planted known-answer mistake", flush=True)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=120)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out
    line = [ln for ln in out.splitlines() if ln.startswith("RESULT")][0]
    assert line.startswith("RESULT 0 False"), line
    assert "known answer" in line and "known-answer check" in line, line


def test_failing_calls_write_nothing(hip):
    """A call that fails (bad shape, bad range, bad token) returns an error
    and leaves every output buffer as it was."""
    import torch
    rows, cols = 256, 1024
    d, _ = quant_matrix(ref.Q4_K, rows, cols, 73)
    w = hip.Weight.from_host(d, hip.TYPE_Q4_K, rows, cols)
    sentinel = np.float32(-12345.5)
    L = hip._lib.load()
    vp = __import__("ctypes").c_void_p
    # the C ABI itself checks shapes (the Python wrappers would stop these
    # calls earlier): out stride below rows, and a fused group of two widths
    xs = torch.zeros(cols, dtype=torch.float32, device="cuda")
    o1 = torch.full((rows,), float(sentinel), device="cuda")
    o2 = torch.full((rows,), float(sentinel), device="cuda")
    torch.cuda.synchronize()
    rc = L.gllm_hip_matvec_dev(w.handle, vp(xs.data_ptr()), 1, vp(o1.data_ptr()), rows - 1, None)
    assert rc == hip.EINVAL
    d2, _ = quant_matrix(ref.Q4_K, rows, 512, 74)
    w2 = hip.Weight.from_host(d2, hip.TYPE_Q4_K, rows, 512)
    hs = (vp * 2)(w.handle, w2.handle)
    ps = (vp * 2)(o1.data_ptr(), o2.data_ptr())
    st = (__import__("ctypes").c_int * 2)(rows, rows)
    rc = L.gllm_hip_matvec_multi_dev(2, hs, vp(xs.data_ptr()), 1, ps, st, None)
    assert rc == hip.EINVAL
    torch.cuda.synchronize()
    assert (o1.cpu().numpy() == sentinel).all() and (o2.cpu().numpy() == sentinel).all()
    host_out = np.full(rows, sentinel, np.float32)
    rc = L.gllm_hip_matvec(w.handle, None, host_out.ctypes.data_as(vp))
    assert rc == hip.EINVAL and (host_out == sentinel).all()
    # attention past the cache
    kv = hip.KVCacheF16(1, 512, 512, 16)
    q = torch.zeros(16 * 128, dtype=torch.float32, device="cuda")
    ao = torch.full((16 * 128,), float(sentinel), device="cuda")
    with pytest.raises(hip.GllmError):
        kv.attend_dev(0, q, 16, 4, 128, 0, 16, 0.1, ao)
    torch.cuda.synchronize()
    assert (ao.cpu().numpy() == sentinel).all()
    # a token id past the vocabulary leaves the model's state alone
    from conftest import tiny_llama
    from gopherllm_amd.decoder import LlamaDecoder
    m = tiny_llama(seed=9, n_layers=1, dim=256, hidden=512, n_heads=4, n_kv_heads=1, head_dim=64,
                   vocab=400)
    dec = LlamaDecoder.from_host_model(m, 32)
    cpu = ref.Llama(m, 32)
    t = dec.prefill([1, 2, 3])
    assert t == cpu.prefill([1, 2, 3])[0]
    with pytest.raises(hip.GllmError):
        dec.decode(400, 3)
    assert dec.decode(t, 3) == cpu.decode(t, 3)[0]


def test_stream_scratch_freed_on_growth_and_release(hip):
    """Scratch that grows frees the buffer it replaces (after the stream
    drains) unless a capture handed it out, and gllm_hip_stream_release frees
    a stream's remaining scratch.  20 rounds, each on a new stream, grow the
    batch from 64 to 512 activation rows of 4096 columns and release the
    stream: without the freeing, every round would strand about 12 MB (the
    replaced buffers and the final set), 240 MB in all.  Results stay equal
    to the oracle, and a graph captured on a stream still replays correctly
    after that stream's scratch was grown and released (its buffer stays)."""
    import torch
    rows, cols = 256, 4096
    d, _ = quant_matrix(ref.Q4_K, rows, cols, 73)
    w = hip.Weight.from_host(d, hip.TYPE_Q4_K, rows, cols)
    ps = (64, 128, 256, 512)
    xs = {p: normal(74 + p, (p, cols)) for p in ps}
    want = {p: ref.matvec_batch(ref.Q4_K, d, x, rows, cols) for p, x in xs.items()}
    dx = {p: torch.from_numpy(x).cuda() for p, x in xs.items()}
    out = {p: torch.empty((p, rows), dtype=torch.float32, device="cuda") for p in ps}
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    print("20 streams, batches 64 -> 512 rows, released", flush=True)
    for r in range(20):
        s = torch.cuda.Stream()
        for p in ps:
            with torch.cuda.stream(s):
                w.matvec_dev(dx[p], out[p])
            s.synchronize()
            if r % 5 == 0:
                assert np.array_equal(bits(out[p].cpu().numpy()), bits(want[p])), (r, p)
        hip.stream_release(s.cuda_stream)
    torch.cuda.synchronize()
    assert free0 - torch.cuda.mem_get_info()[0] < 100 << 20
    s2 = torch.cuda.Stream()
    with torch.cuda.stream(s2):
        w.matvec_dev(dx[64], out[64])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("capture, grow, release, replay", flush=True)
    with torch.cuda.graph(g, stream=s2):
        w.matvec_dev(dx[64], out[64])
    with torch.cuda.stream(s2):
        w.matvec_dev(dx[512], out[512])  # grows the captured slot: kept
    s2.synchronize()
    hip.stream_release(s2.cuda_stream)
    for i in range(3):
        out[64].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out[64].cpu().numpy()), bits(want[64])), i
