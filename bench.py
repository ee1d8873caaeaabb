#!/usr/bin/env python3
"""Headline benchmark: Q4_K x Q8_K GEMV on one MI355X.

Workload (gate/up shape): W is 14336 x 4096 drawn
N(0, 0.02) on the device and encoded to Q4_K by the device RTN encoder
(QuantizeRowQ4K); x is N(0, 1).  One step is one MatvecQ4KInto (simd.go:261):
Q8K quantisation of x plus the row kernels over all 14336 rows; at this shape
the row kernel quantises x itself, so a step is one kernel launch.  Weight
copies rotate so the working set (>= 300 MB) exceeds the 256 MB Infinity
Cache, i.e. every step streams its weights from HBM.  Steps are replayed from
a HIP graph (captured through torch.cuda.CUDAGraph on the launch stream) so
host launch overhead is not measured.

value      = algorithmic bytes per step / time per step, bytes =
             rows*(cols/256)*144 + 4*cols + 4*rows (whole MatvecQ4KInto)
roofline   = the same bytes / the row kernel's average launch duration (HIP
             events on the launch stream around graph replays of back-to-back
             launches, so the inter-kernel gap is included), against the
             8 TB/s HBM3E peak; traffic from profiles/ (rocprofv3 PMC)
cpu_baseline = the oracle's AVX2 port of kernels_amd64.s (bit-identical
             results) on this host's cores, same bytes formula, rotating the
             same weight copies.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K×Q8_K GEMV GB/s (% HBM peak); decode tok/s on 8B-shape Q4_K synth"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
ROWS, COLS = 14336, 4096
PMC_FILE = os.path.join(ROOT, "profiles", "gemv_q4k_14336x4096_pmc.json")
CEILING_FILE = os.path.join(ROOT, "profiles", "read_ceiling_14336x4096.json")


def alg_bytes(rows, cols, p=1):
    return rows * (cols // 256) * 144 + p * (4 * cols + 4 * rows)


def make_weights(g, torch, rows, cols, copies, seed):
    """copies of a Q4_K matrix, generated and encoded on the device."""
    tmp = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
    raw = torch.empty(rows * (cols // 256) * 144, dtype=torch.uint8, device="cuda")
    ws = []
    for c in range(copies):
        g.fill_normal_dev(tmp, seed + c, 0.02)
        g.quantize_rows_dev(g.TYPE_Q4_K, tmp, raw)
        ws.append(g.Weight.from_device(raw, g.TYPE_Q4_K, rows, cols))
    torch.cuda.synchronize()
    del tmp, raw
    return ws


def timed_graph(torch, body, reps=1):
    """Capture body() into a HIP graph on a side stream and return it.  The
    eager warm-up runs on the same stream the capture uses, so any per-stream
    scratch the library sizes on first use exists before the capture."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()  # eager warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        body()
    graph.replay()
    torch.cuda.synchronize()
    return graph


def cpu_identity():
    """Host CPU model, L3 size and usable cores, for the cpu_baseline record."""
    model, l3 = "unknown", None
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        base = "/sys/devices/system/cpu/cpu0/cache"
        for ent in sorted(os.listdir(base)):
            if open(os.path.join(base, ent, "level")).read().strip() == "3":
                l3 = open(os.path.join(base, ent, "size")).read().strip()
    except OSError:
        pass
    return {"cpu": model, "l3": l3, "cores_usable": len(os.sched_getaffinity(0))}


def run(args):
    import numpy as np
    import torch

    import gopherllm_amd as g

    g.load()
    if not torch.cuda.is_available() or not g.available():
        raise SystemExit("bench.py needs an MI355X (gfx950) device: " + g._lib.last_error())
    rows, cols = ROWS, COLS
    wbytes = rows * (cols // 256) * 144
    copies = args.copies or max(2, math.ceil(300e6 / wbytes))
    weights = make_weights(g, torch, rows, cols, copies, seed=1000)
    x = torch.empty(cols, dtype=torch.float32, device="cuda")
    g.fill_normal_dev(x, 7, 1.0)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")

    # correctness guard: the benchmarked device entry point equals the
    # blocking host entry point on the same inputs
    xh = x.cpu().numpy()
    want = weights[0].matvec_into(xh)
    weights[0].matvec_dev(x.view(1, -1), out.view(1, -1))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))

    def launches(ws):
        def body():
            for w in ws:
                w.matvec_dev(x.view(1, -1), out.view(1, -1))
        return body

    # At this shape the row kernel quantises x itself: one step (one whole
    # MatvecQ4KInto) is one launch of the dominant kernel.  A graph holds one
    # rotation over the weight copies; a second graph holds the remainder, so
    # exactly --warmup and --steps steps run.
    rot = timed_graph(torch, launches(weights))
    rem_graphs = {}

    def run_steps(n):
        for _ in range(n // copies):
            rot.replay()
        r = n % copies
        if r:
            if r not in rem_graphs:
                rem_graphs[r] = timed_graph(torch, launches(weights[:r]))
            rem_graphs[r].replay()

    steps, warm = args.steps, args.warmup
    if args.steps % copies:
        rem_graphs[args.steps % copies] = timed_graph(torch, launches(weights[:args.steps % copies]))
    run_steps(warm)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    run_steps(steps)
    e1.record()
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / steps
    # one launch per step: the kernel's average launch duration over the
    # timed region (HIP events on the launch stream; includes the dispatch
    # gap between back-to-back launches)
    kernel_us = ms_per_step * 1e3

    # replayed graphs still produce the eager result
    rot.replay()
    torch.cuda.synchronize()
    last = weights[-1].matvec_into(xh)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), last.view(np.uint32))

    nbytes = alg_bytes(rows, cols)
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    achieved = nbytes / (kernel_us * 1e-6) / 1e9
    ceiling_us = None
    if os.path.exists(CEILING_FILE):
        ceiling_us = json.load(open(CEILING_FILE))["best"]["us"]
    traffic, trace_us = None, None
    if os.path.exists(PMC_FILE):
        pmc = json.load(open(PMC_FILE))
        traffic = pmc.get("traffic_bytes_per_launch")
        trace_us = pmc.get("kernel_mean_ns", 0) / 1e3 or None
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: W ~ N(0,0.02) encoded Q4_K on device (QuantizeRowQ4K), x ~ N(0,1)",
        "config": {
            "workload": "Q4_K x Q8_K GEMV 14336x4096 batch 1 (configs[1] gate/up; one step = "
                        "MatvecQ4KInto: Q8K quantise + row kernels)",
            "rows": rows, "cols": cols, "weight_copies": copies,
            "rotating_bytes": copies * wbytes, "hip_graph": True,
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "gemv_q4k_ws_kernel (wave-specialised loader / compute waves, Q8K "
                      "quantisation fused, one launch per step)",
            "kernel_avg_us": round(kernel_us, 3),
            "kernel_timing": "HIP events on the launch stream around the timed region: "
                             f"{steps} back-to-back launches replayed from HIP graphs "
                             "(dispatch gaps included); launches per step = 1",
            "bytes_per_launch": nbytes,
            # the kernel alone, from the committed rocprofv3 trace of this
            # shape (profiles/gemv_q4k_14336x4096.md), beside the live step figure
            "trace_kernel_us": round(trace_us, 3) if trace_us else None,
            "trace_frac": round(nbytes / (trace_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if trace_us else None,
            # the fastest launch that only reads the weight bytes, timed the
            # same way (bench.py --read-ceiling, profiles/read_ceiling_14336x4096.md)
            "read_ceiling_us": ceiling_us,
            "frac_of_read_ceiling": round(ceiling_us / kernel_us, 4) if ceiling_us else None,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(weights, xh, rows, cols, args.cpu_seconds, torch)
    return line


def cpu_baseline(weights, xh, rows, cols, seconds, torch):
    """The oracle's AVX2 port of kernels_amd64.s on this host, all cores, over
    the same rotating weight copies (downloaded from the device)."""
    import numpy as np

    from oracle import oracle as ref

    host = []
    for w in weights:
        buf = torch.empty(rows * (cols // 256) * 144, dtype=torch.uint8, device="cuda")
        w.download_dev(buf)
        torch.cuda.synchronize()
        host.append(buf.cpu().numpy())
    cores = len(os.sched_getaffinity(0))
    kind = "port"
    fast = ref.matvec_batch_fast(ref.Q4_K, host[0], xh, rows, cols, threads=cores)
    if fast is None:
        raise SystemExit("host lacks AVX2/FMA/F16C for the CPU baseline")
    n, t0 = 0, time.perf_counter()
    while True:
        ref.matvec_batch_fast(ref.Q4_K, host[n % len(host)], xh, rows, cols, threads=cores)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    gbs = alg_bytes(rows, cols) * n / el / 1e9
    rec = {"value": round(gbs, 2), "unit": "GB/s", "cores": cores, "kind": kind,
           "sample": f"{n} MatvecQ4KInto calls (14336x4096 Q4_K, AVX2 port of kernels_amd64.s, "
                     f"{len(host)} rotating weight copies) in {el:.1f} s"}
    rec.update(cpu_identity())
    return rec


def decode_bench(args):
    """synthetic Llama-3-8B-shape decoder (Q4_K layers, Q6_K
    head), 512-token prompt, 128 greedy tokens.  Prefill and decode are
    timed separately on a second run (the first warms buffers up); every
    decode step returns its token to the host, as the reference's runner
    loop consumes it (runtime.go:1129-1170)."""
    import numpy as np
    import torch

    from gopherllm_amd import synth

    cfg = dict(synth.LLAMA3_8B)
    P, N = 512, 128
    t0 = time.perf_counter()
    d = synth.build_decoder(cfg, max_len=P + N, seed=1)
    build_s = time.perf_counter() - t0
    prompt = np.random.default_rng(2024).integers(0, cfg["vocab"], P)
    warm = d.generate(prompt, N)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = d.prefill(prompt)
    t1 = time.perf_counter()
    toks = [tok]
    for i in range(1, N):
        tok = d.decode(tok, P + i - 1)
        toks.append(tok)
    t2 = time.perf_counter()
    assert np.array_equal(np.array(toks, np.uint32), warm), "decode is not deterministic"
    layer_bytes = sum(r * (c // 256) * 144 for r, c in synth.layer_shapes(cfg).values())
    head_bytes = cfg["vocab"] * (cfg["dim"] // 256) * 210
    kv_per_pos = cfg["n_layers"] * cfg["n_kv_heads"] * cfg["head_dim"] * 2 * 2
    mean_ctx = P + (N - 1) / 2.0
    tok_bytes = cfg["n_layers"] * layer_bytes + head_bytes + kv_per_pos * mean_ctx
    dec_s = (t2 - t1) / (N - 1)
    out = {
        "workload": "configs[4]: Llama-3-8B-shape synthetic decoder, Q4_K layers + Q6_K head, "
                    "prompt 512 uniform-random ids, 127 timed greedy decode steps",
        "tok_s": round(1.0 / dec_s, 2),
        "ms_per_token": round(dec_s * 1e3, 4),
        "prefill_tok_s": round(P / (t1 - t0), 2),
        "bytes_per_token": int(tok_bytes),
        "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / tok_bytes, 1),
        "frac": round((tok_bytes / dec_s) / (HBM_PEAK_GBS * 1e9), 4),
        "model_build_s": round(build_s, 2),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = decode_cpu_baseline(d, prompt, toks, P, N, args.cpu_seconds)
    else:
        d.release()
    out["q4km"] = q4km_prefill(P, prompt)
    return out


def q4km_prefill(P, prompt):
    """Prefill of the same 512 ids on a Q4_K_M-style 8B-shape decoder (Q6_K
    attn_v / ffn_down on every other layer: synth.q4km_type), the second of
    two runs, plus one greedy step as a smoke check of the mixed graph."""
    import torch

    from gopherllm_amd import synth

    cfg = dict(synth.LLAMA3_8B)
    d = synth.build_decoder(cfg, max_len=P + 8, seed=1, type_of=synth.q4km_type)
    d.prefill(prompt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = d.prefill(prompt)
    t1 = time.perf_counter()
    tok = d.decode(tok, P)
    d.release()
    return {"workload": "Llama-3-8B-shape synthetic decoder, Q4_K layers with Q6_K attn_v and "
                        "ffn_down on even layers, Q6_K head; prompt 512 ids (the decode record's)",
            "prefill_tok_s": round(P / (t1 - t0), 2)}


def decode_cpu_baseline(d, prompt, toks, P, N, seconds):
    """The oracle's decoder (row dots through the AVX2 port of
    kernels_amd64.s) at the positions the GPU decode was timed at.  Its KV
    cache for positions 0..P-1 is the device's (bit-identical to the
    oracle's own prefill, which the GPU tests check), so the CPU starts at
    position P without a 512-token CPU prefill; each CPU step must return
    the GPU's token."""
    import numpy as np

    from gopherllm_amd import synth
    from oracle import oracle as ref

    m = synth.host_model(d)
    kv = d.kv_cache()
    ks = [kv.read(l, 0, P) for l in range(d.config["n_layers"])]
    d.release()
    cpu = ref.Llama(m, P + N, fast=True)
    for l, (k16, v16) in enumerate(ks):
        cpu.set_kv(l, 0, k16, v16)
    del ks
    cores = len(os.sched_getaffinity(0))
    steps, c0 = 0, time.perf_counter()
    tok = int(toks[0])
    while steps < N - 1 and (steps < 4 or time.perf_counter() - c0 < seconds):
        tok = cpu.decode(tok, P + steps)[0]
        if tok != int(toks[steps + 1]):
            raise SystemExit(f"CPU decode step at position {P + steps} returned {tok}, "
                             f"GPU {int(toks[steps + 1])}")
        steps += 1
    el = time.perf_counter() - c0
    rec = {"value": round(steps / el, 3), "unit": "tok/s", "cores": cores, "kind": "port",
           "sample": f"{steps} greedy decode steps at positions {P}..{P + steps - 1} after the "
                     f"{P}-token prompt (oracle decoder, AVX2 port of kernels_amd64.s, same "
                     f"weights, KV rows 0..{P - 1} from the device), each step's token equal to "
                     f"the GPU's, in {el:.1f} s"}
    rec.update(cpu_identity())
    cpu.close()
    return rec


def suite(args):
    """One JSON line per measured workload of the other configs:
    configs[1] GEMVs (Q4_K / Q6_K / Q8_0, gate/up and down shapes, batch 1
    and 8; Q5_K / Q4_0 / Q4_1 / MXFP4 / Q2_K / Q3_K at the gate/up shape),
    configs[2] batched prefill (p = 512 activation rows), configs[3]
    decode attention (ctx 4096 and 32768, exact and split-K).  Weights rotate
    over >= 300 MB; every timing is a HIP-graph replay on the launch stream."""
    import torch

    import gopherllm_amd as g

    g.load()
    qnames = {g.TYPE_Q4_K: "Q4_K", g.TYPE_Q6_K: "Q6_K", g.TYPE_Q8_0: "Q8_0"}
    only = set(args.only.split(",")) if args.only else {"gemv", "formats", "groups", "prefill",
                                                        "attention"}

    def graph_time(body, reps):
        graph = timed_graph(torch, body, 1)
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3  # us per replay

    def weights_for(qtype, rows, cols, min_bytes=300e6):
        wb = rows * g.row_bytes(qtype, cols)
        copies = max(2, math.ceil(min_bytes / wb))
        tmp = torch.empty((rows, cols), dtype=torch.float32, device="cuda")
        raw = torch.empty(wb, dtype=torch.uint8, device="cuda")
        ws = []
        for c in range(copies):
            g.fill_normal_dev(tmp, 2000 + c, 0.02)
            g.quantize_rows_dev(qtype, tmp, raw)
            ws.append(g.Weight.from_device(raw, qtype, rows, cols))
        torch.cuda.synchronize()
        return ws, wb

    gemv_cases = [(g.TYPE_Q4_K, 4096, 4096)]  # configs[0]
    gemv_cases += [(q, r, c) for q in (g.TYPE_Q4_K, g.TYPE_Q6_K, g.TYPE_Q8_0)
                   for r, c in ((14336, 4096), (4096, 14336))]  # configs[1]
    for qtype, rows, cols in gemv_cases if "gemv" in only else ():
        ws, wb = weights_for(qtype, rows, cols)
        for p in (1, 8):
            x = torch.empty((p, cols), dtype=torch.float32, device="cuda")
            g.fill_normal_dev(x, 7, 1.0)
            out = torch.empty((p, rows), dtype=torch.float32, device="cuda")

            def body():
                for w in ws:
                    w.matvec_dev(x, out)

            us = graph_time(body, 20) / len(ws)
            nbytes = wb + p * (4 * cols + 4 * rows)
            cfg = "configs[0] gemv" if rows == cols else "configs[1] gemv"
            print(json.dumps({"suite": cfg, "type": qnames[qtype], "rows": rows,
                              "cols": cols, "batch": p, "us": round(us, 3),
                              "GB_s": round(nbytes / us / 1e3, 1),
                              "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)
        del ws

    # formats beyond Q4_K / Q6_K / Q8_0: random codes with valid f16 scales
    # (the block layouts of gguf.go:241-297), gate/up shape at batch 1 and 8,
    # down shape at batch 1
    fmt_layout = {g.TYPE_Q5_K: ("Q5_K", 176, 256, [(0, 2), (2, 4)], None),
                  g.TYPE_Q4_0: ("Q4_0", 18, 32, [(0, 2)], None),
                  g.TYPE_Q4_1: ("Q4_1", 20, 32, [(0, 2), (2, 4)], None),
                  g.TYPE_MXFP4: ("MXFP4", 17, 32, [], 16),
                  g.TYPE_Q2_K: ("Q2_K", 84, 256, [(80, 82), (82, 84)], None),
                  g.TYPE_Q3_K: ("Q3_K", 110, 256, [(108, 110)], None)}
    fmt_cases = [(q, shape) for shape in ((14336, 4096), (4096, 14336)) for q in fmt_layout]
    for qtype, (rows, cols) in fmt_cases if "formats" in only else ():
        import numpy as np
        name, bb, be, halfs, ebyte = fmt_layout[qtype]
        rng = np.random.default_rng(qtype)
        nb = rows * cols // be
        blk = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
        for lo, hi in halfs:
            blk[:, lo:hi] = rng.uniform(0.002, 0.02, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
        if ebyte is not None:
            blk[:, ebyte] = rng.integers(118, 130, nb)
        raw = blk.reshape(-1)
        wb = raw.size
        ws = [g.Weight.from_host(raw, qtype, rows, cols) for _ in range(max(2, math.ceil(300e6 / wb)))]
        for p in ((1, 8) if cols == 4096 else (1,)):
            x = torch.empty((p, cols), dtype=torch.float32, device="cuda")
            g.fill_normal_dev(x, 7, 1.0)
            out = torch.empty((p, rows), dtype=torch.float32, device="cuda")

            def body():
                for w in ws:
                    w.matvec_dev(x, out)

            us = graph_time(body, 20) / len(ws)
            nbytes = wb + p * (4 * cols + 4 * rows)
            print(json.dumps({"suite": "formats gemv", "type": name, "rows": rows, "cols": cols,
                              "batch": p, "us": round(us, 3), "GB_s": round(nbytes / us / 1e3, 1),
                              "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)
        del ws

    def random_weights(qtype, rows, cols, min_bytes):
        """Copies of one weight of a format without a device encoder: random
        code bytes, f16 scales in 0.002..0.02 (and MXFP4 exponents near 1)."""
        import numpy as np
        name, bb, be, halfs, ebyte = fmt_layout[qtype]
        rng = np.random.default_rng(qtype + rows)
        nb = rows * cols // be
        blk = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
        for lo, hi in halfs:
            blk[:, lo:hi] = rng.uniform(0.002, 0.02, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
        if ebyte is not None:
            blk[:, ebyte] = rng.integers(118, 130, nb)
        raw = blk.reshape(-1)
        return [g.Weight.from_host(raw, qtype, rows, cols)
                for _ in range(max(2, math.ceil(min_bytes / raw.size)))], raw.size

    # same-type fused groups of the float-kernel formats (matvecSameType2/3Into):
    # the gate/up pair and the Q/K/V triple of the 8B shape, batch 1
    groups = ((g.TYPE_Q8_0, "Q8_0"), (g.TYPE_Q4_0, "Q4_0"), (g.TYPE_Q5_K, "Q5_K"))
    for qtype, name in groups if "groups" in only else ():
        for shapes in (((14336, 4096), (14336, 4096)), ((4096, 4096), (1024, 4096), (1024, 4096))):
            copies = []
            nbytes = 0
            for rows, cols in shapes:
                if qtype == g.TYPE_Q8_0:
                    ws, wb = weights_for(qtype, rows, cols, min_bytes=100e6)
                else:
                    ws, wb = random_weights(qtype, rows, cols, 100e6)
                copies.append(ws)
                nbytes += wb
            x = torch.empty((1, 4096), dtype=torch.float32, device="cuda")
            g.fill_normal_dev(x, 7, 1.0)
            outs = [torch.empty((1, r), dtype=torch.float32, device="cuda") for r, _ in shapes]
            nc = min(len(c) for c in copies)

            def body():
                for i in range(nc):
                    g.matvec_multi_dev([c[i] for c in copies], x, outs)

            us = graph_time(body, 20) / nc
            print(json.dumps({"suite": "same-type group (float kernels)", "type": name,
                              "rows": [r for r, _ in shapes], "cols": 4096, "us": round(us, 2),
                              "GB_s": round(nbytes / us / 1e3, 1),
                              "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)
            del copies

    pf_cases = [(g.TYPE_Q4_K, 4096, 4096), (g.TYPE_Q4_K, 14336, 4096), (g.TYPE_Q4_K, 4096, 14336),
                (g.TYPE_Q6_K, 4096, 4096), (g.TYPE_Q6_K, 14336, 4096), (g.TYPE_Q6_K, 4096, 14336),
                (g.TYPE_Q8_0, 14336, 4096), (g.TYPE_Q8_0, 4096, 14336)]
    for qtype, rows, cols in pf_cases if "prefill" in only else ():
        ws, wb = weights_for(qtype, rows, cols, min_bytes=0)
        P = 512
        x = torch.empty((P, cols), dtype=torch.float32, device="cuda")
        g.fill_normal_dev(x, 9, 1.0)
        out = torch.empty((P, rows), dtype=torch.float32, device="cuda")

        def body():  # four calls per graph: the replay's host cost stays off the clock
            for _ in range(4):
                ws[0].matvec_dev(x, out)

        us = graph_time(body, 5) / 4
        ops = 2.0 * P * rows * cols
        # the matrix-core kernels issue f16 MFMAs (Q6_K two per product: the
        # code's 4-bit and 2-bit fields), hence both peaks
        print(json.dumps({"suite": "configs[2] prefill", "type": qnames[qtype], "rows": rows,
                          "cols": cols, "tokens": P, "us": round(us, 1),
                          "us_per_weight_mb": round(us / (wb / 1e6), 3),
                          "TOPS": round(ops / us / 1e6, 2),
                          "frac_int8_mfma": round(ops / us / 1e6 / 5000.0, 4),
                          "frac_f16_mfma": round(ops / us / 1e6 / 2500.0, 4),
                          "timed": "Q8K quantisation of the 512 rows + the batched product"}), flush=True)
        del ws

    n_heads, n_kv, hd = 32, 8, 128
    for ctx in (4096, 32768) if "attention" in only else ():
        if args.ctx and ctx != args.ctx:
            continue
        kv = g.KVCacheF16(1, n_kv * hd, n_kv * hd, ctx)
        k = torch.empty(ctx * n_kv * hd, dtype=torch.float32, device="cuda")
        v = torch.empty_like(k)
        g.fill_normal_dev(k, 11, 1.0)
        g.fill_normal_dev(v, 12, 1.0)
        kd = n_kv * hd
        for pos in range(ctx):
            kv.store_kv_dev(0, pos, k[pos * kd:(pos + 1) * kd], v[pos * kd:(pos + 1) * kd])
        torch.cuda.synchronize()
        q = torch.empty(n_heads * hd, dtype=torch.float32, device="cuda")
        g.fill_normal_dev(q, 13, 1.0)
        out = torch.empty(n_heads * hd, dtype=torch.float32, device="cuda")
        nbytes = ctx * n_kv * hd * 2 * 2
        for mode, name in ((g.ATTN_SPLITK, "split-K"), (g.ATTN_EXACT, "exact")):
            def body():  # ten calls per graph: one short call would time the host's replay
                for _ in range(10):
                    kv.attend_dev(0, q, n_heads, n_kv, hd, 0, ctx - 1, 1.0 / math.sqrt(hd), out,
                                  mode=mode)

            us = graph_time(body, 5) / 10
            print(json.dumps({"suite": "configs[3] attention", "ctx": ctx, "mode": name,
                              "us": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1),
                              "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)
        kv.release()


def launch_floor(args):
    """Per-node cost of short launches replayed back to back from one HIP
    graph (HIP events on the launch stream, no profiler): an empty one-thread
    kernel, a 64 KB elementwise fill over 64 workgroups, a 16 KB copy, and the
    smallest Q4_K matvec (256 x 256, one workgroup, quantiser fused).  This
    is the fixed cost each launch of the decode step pays before its own
    work."""
    import torch

    import gopherllm_amd as g

    g.load()
    n = 500
    a = torch.zeros(16384, dtype=torch.float32, device="cuda")
    b = torch.zeros(4096, dtype=torch.float32, device="cuda")
    c = torch.zeros(4096, dtype=torch.float32, device="cuda")
    raw = torch.empty(256 * 144, dtype=torch.uint8, device="cuda")
    tmp = torch.empty((256, 256), dtype=torch.float32, device="cuda")
    g.fill_normal_dev(tmp, 5, 0.02)
    g.quantize_rows_dev(g.TYPE_Q4_K, tmp, raw)
    w = g.Weight.from_device(raw, g.TYPE_Q4_K, 256, 256)
    x = torch.empty((1, 256), dtype=torch.float32, device="cuda")
    g.fill_normal_dev(x, 6, 1.0)
    y = torch.empty((1, 256), dtype=torch.float32, device="cuda")
    bodies = {
        "empty kernel (1 thread)": lambda: torch.cuda._sleep(0),
        "fill 64 KB": lambda: a.fill_(1.0),
        "copy 16 KB": lambda: b.copy_(c),
        "Q4_K matvec 256x256": lambda: w.matvec_dev(x, y),
    }
    for name, fn in bodies.items():
        def body():
            for _ in range(n):
                fn()
        graph = timed_graph(torch, body)
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / (5 * n) * 1e3
        print(json.dumps({"launch_floor": name, "nodes_per_graph": n, "us_per_node": round(us, 3)}),
              flush=True)


def read_ceiling(args):
    """Ceiling of one streaming launch: the headline GEMV's 33,103,872 bytes
    read once with 16-byte loads and nothing else (libgllm_probe.so, built
    beside the product library).  Ten rotating copies (331 MB, past the
    256 MB memory-side cache) make every launch read HBM; each point is
    20 launches replayed from one HIP graph and timed with HIP events, as the
    headline line times the GEMV, over grid sizes, workgroup sizes, loads in
    flight per thread and two access patterns (grid-stride / one contiguous
    chunk per workgroup).  Prints one line per point and a summary line with
    the fastest."""
    import ctypes as C

    import torch

    import gopherllm_amd as g
    from gopherllm_amd import build as hipbuild

    if not os.path.exists(hipbuild.PROBE_LIB):
        raise SystemExit(f"{hipbuild.PROBE_LIB} is missing: run __graft_entry__.build() first")
    lib = C.CDLL(hipbuild.PROBE_LIB)
    fn = lib.gllm_probe_stream_read
    fn.restype = C.c_int
    fn.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    rows, cols = 14336, 4096
    nbytes = rows * g.row_bytes(g.TYPE_Q4_K, cols)  # the GEMV's weight bytes
    gemv_bytes = nbytes + 4 * cols + 4 * rows
    copies = 10
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    for i, b in enumerate(bufs):
        b.view(torch.int32).random_(generator=torch.Generator(device="cuda").manual_seed(i))
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    reps = 20
    best = None
    for pattern in (0, 1):
        for threads in (256, 512, 1024):
            for wgs in (256, 512, 1024, 2048):
                for depth in (2, 4, 8, 16):
                    def body():
                        s = torch.cuda.current_stream().cuda_stream
                        for r in range(reps):
                            rc = fn(bufs[r % copies].data_ptr(), nbytes, wgs, threads, depth, pattern,
                                    sink.data_ptr(), s)
                            if rc:
                                raise RuntimeError(f"probe launch failed ({rc})")
                    graph = timed_graph(torch, body)
                    for _ in range(3):
                        graph.replay()
                    torch.cuda.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(5):
                        graph.replay()
                    e1.record()
                    torch.cuda.synchronize()
                    us = e0.elapsed_time(e1) / (5 * reps) * 1e3
                    rec = {"read_ceiling": "point", "pattern": "grid-stride" if pattern == 0 else "chunk",
                           "threads": threads, "workgroups": wgs, "loads_in_flight": depth,
                           "us": round(us, 3), "GB_s": round(nbytes / us / 1e3, 1)}
                    print(json.dumps(rec), flush=True)
                    if best is None or us < best["us"]:
                        best = rec
    print(json.dumps({"read_ceiling": "best", "bytes": nbytes, **{k: v for k, v in best.items() if k != "read_ceiling"},
                      "frac_of_8TBs": round(nbytes / best["us"] / 8e6, 4),
                      "gemv_at_ceiling_us": round(gemv_bytes / (nbytes / best["us"]), 3)}), flush=True)


def kernel_bench(args):
    """llm-kernel-bench.v1 (kernel_bench.go:26-203) for layer 0 of the
    synthetic Llama-3-8B-shape model of configs[4] (Q4_K layers and
    embeddings, Q6_K output): the embedding row lookup, every layer matvec
    alone, the fused paths a generation step runs (attn_qkv_path =
    tryMatvecAttentionInto, ffn_gate_up_path = tryMatvec2Into,
    ffn_swiglu_down_path = gate/up + siluMulF32 + down, output_argmax_path
    and its repeat-penalty form) on deterministicBenchVector inputs
    ((i % 251) - 125) / 125.  Each row's `runs` calls are one HIP graph of
    back-to-back launches, replayed and timed with HIP events on the replay
    stream, so avg_ms is the device time per call without host launch cost.
    With the CPU leg, cpu_avg_ms is the oracle's AVX2 port of
    kernels_amd64.s (all host cores) on the same weights for the matvec
    rows."""
    import numpy as np
    import torch

    import gopherllm_amd as g
    from gopherllm_amd import synth

    g.load()
    cfg = dict(synth.LLAMA3_8B)
    dim, hid, vocab = cfg["dim"], cfg["hidden"], cfg["vocab"]
    qd = cfg["n_heads"] * cfg["head_dim"]
    shapes = synth.layer_shapes(cfg)
    sc = synth._Scratch(torch, vocab * dim, vocab * g.row_bytes(cfg["out_type"], dim))
    W = {k: sc.weight(cfg["layer_type"], r, c, synth.tensor_seed(1, 0, k))
         for k, (r, c) in shapes.items()}
    emb = sc.weight(cfg["emb_type"], vocab, dim, synth.tensor_seed(1, -1, "tok_embd"))
    out_w = sc.weight(cfg["out_type"], vocab, dim, synth.tensor_seed(1, -1, "output"))
    torch.cuda.synchronize()
    del sc

    def bench_vec(n):
        i = np.arange(n)
        return torch.from_numpy((((i % 251) - 125) / 125).astype(np.float32)).cuda().view(1, -1)

    x_dim, x_attn, x_hid = bench_vec(dim), bench_vec(qd), bench_vec(hid)
    bufs = {n: torch.empty((1, n), dtype=torch.float32, device="cuda") for n in (dim, hid, vocab)}
    o2 = torch.empty((1, hid), dtype=torch.float32, device="cuda")
    o3 = torch.empty((1, shapes["wv"][0]), dtype=torch.float32, device="cuda")
    ok = torch.empty((1, shapes["wk"][0]), dtype=torch.float32, device="cuda")
    ids = torch.zeros(1, dtype=torch.int32, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    recent = torch.tensor([0, 1, 1, vocab - 1], dtype=torch.int32, device="cuda")
    names = {g.TYPE_Q4_K: "Q4_K", g.TYPE_Q6_K: "Q6_K", g.TYPE_Q8_0: "Q8_0"}
    T = {k: names[w.type] for k, w in W.items()}
    ot = names[out_w.type]

    rows = [
        ("token_embd.row", names[emb.type], vocab, dim, lambda: emb.rows_dev(ids, bufs[dim]),
         (dim // 256) * 144 + 4 * dim, None),
        ("attn_q", T["wq"], qd, dim, lambda: W["wq"].matvec_dev(x_dim, bufs[dim]), None, ["wq"]),
        ("attn_k", T["wk"], shapes["wk"][0], dim, lambda: W["wk"].matvec_dev(x_dim, ok), None, ["wk"]),
        ("attn_v", T["wv"], shapes["wv"][0], dim, lambda: W["wv"].matvec_dev(x_dim, o3), None, ["wv"]),
        ("attn_qkv_path", "/".join(T[k] for k in ("wq", "wk", "wv")),
         qd + 2 * shapes["wk"][0], dim,
         lambda: g.matvec_multi_dev([W["wq"], W["wk"], W["wv"]], x_dim, [bufs[dim], ok, o3]),
         None, ["wq", "wk", "wv"]),
        ("attn_output", T["wo"], dim, qd, lambda: W["wo"].matvec_dev(x_attn, bufs[dim]), None, ["wo"]),
        ("ffn_gate", T["w1"], hid, dim, lambda: W["w1"].matvec_dev(x_dim, bufs[hid]), None, ["w1"]),
        ("ffn_up", T["w3"], hid, dim, lambda: W["w3"].matvec_dev(x_dim, o2), None, ["w3"]),
        ("ffn_gate_up_path", f"{T['w1']}/{T['w3']}", 2 * hid, dim,
         lambda: g.matvec_multi_dev([W["w1"], W["w3"]], x_dim, [bufs[hid], o2]), None, ["w1", "w3"]),
        ("ffn_down", T["w2"], dim, hid, lambda: W["w2"].matvec_dev(x_hid, bufs[dim]), None, ["w2"]),
        ("ffn_swiglu_down_path", f"{T['w1']}/{T['w3']}/SiLU/{T['w2']}", 2 * hid + dim, dim,
         lambda: g.swiglu_down_dev(W["w1"], W["w3"], W["w2"], x_dim, bufs[dim]), None,
         ["w1", "w3", "w2"]),
        ("output", ot, vocab, dim, lambda: out_w.matvec_dev(x_dim, bufs[vocab]), None, ["output"]),
        ("output_argmax_path", f"{ot}/argmax", vocab, dim, lambda: out_w.argmax_dev(x_dim, tok),
         None, ["output"]),
        ("output_argmax_penalized_path", f"{ot}/argmax/repeat-penalty", vocab, dim,
         lambda: out_w.argmax_dev(x_dim, tok, recent=recent, penalty=1.1), None, ["output"]),
    ]
    wmap = dict(W, output=out_w)

    def wbytes(keys):
        tot = 0
        for k in keys:
            w = wmap[k]
            tot += w.rows * g.row_bytes(w.type, w.cols) + 4 * w.rows
        return tot + 4 * wmap[keys[0]].cols

    host = {}
    cores = len(os.sched_getaffinity(0))
    if not args.no_cpu_baseline:
        from oracle import oracle as ref
        for k, w in wmap.items():
            buf = torch.empty(w.rows * g.row_bytes(w.type, w.cols), dtype=torch.uint8, device="cuda")
            w.download_dev(buf)
            torch.cuda.synchronize()
            host[k] = buf.cpu().numpy()
    runs = args.kernel_bench_runs
    kernels = []
    for name, dtype, r, c, fn, nbytes, keys in rows:
        def body(fn=fn):
            for _ in range(runs):
                fn()
        graph = timed_graph(torch, body)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        avg_ms = e0.elapsed_time(e1) / (reps * runs)
        nbytes = nbytes if nbytes is not None else wbytes(keys)
        # every call reads the same weight: up to the 256 MB Infinity Cache the
        # repeats can be served from it, so the rate is not an HBM rate there
        row = {"name": name, "dtype": dtype, "rows": r, "cols": c, "runs": runs,
               "avg_ms": round(avg_ms, 6), "total_ms": round(avg_ms * runs, 4),
               "alg_bytes": int(nbytes), "gb_s": round(nbytes / (avg_ms * 1e-3) / 1e9, 1),
               "frac_hbm": round(nbytes / (avg_ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
               "cache_resident": bool(nbytes <= 256 << 20)}
        if host and keys and name.startswith(("attn_", "ffn_gate", "ffn_up", "ffn_down", "output")) \
                and "argmax" not in name and "swiglu" not in name:
            xin = bench_vec(wmap[keys[0]].cols).cpu().numpy()[0]
            n, t0 = 0, time.perf_counter()
            while n < 3 or (time.perf_counter() - t0 < 1.0 and n < 200):
                for k in keys:
                    w = wmap[k]
                    ref.matvec_batch_fast(w.type, host[k], xin, w.rows, w.cols, threads=cores)
                n += 1
            row["cpu_avg_ms"] = round((time.perf_counter() - t0) / n * 1e3, 4)
        kernels.append(row)
        print(json.dumps(row), file=sys.stderr, flush=True)
    doc = {"type": "gopherllm.kernel_benchmark", "format": "llm-kernel-bench.v1",
           "note": "each row repeats one weight (the reference tool's method); rows with "
                   "cache_resident true fit the 256 MB Infinity Cache, so their gb_s / frac_hbm "
                   "are cache rates, not HBM rates (the headline bench line rotates 330 MB)",
           "runtime": "gopherllm_amd (HIP, MI355X)",
           "command": " ".join(["python", "bench.py"] + sys.argv[1:]),
           "model": {"path": None, "name": "synthetic Llama-3-8B shape (configs[4])",
                     "arch": "llama", "dim": dim, "hidden_dim": hid, "layers": cfg["n_layers"]},
           "layer": 0, "runs": runs, "kernels": kernels,
           "timing": "device time per call: each row's runs calls captured as one HIP graph, "
                     "5 replays timed with HIP events on the replay stream",
           "alg_bytes": "weight bytes + 4*(rows + cols) per matvec; token_embd.row: one Q4_K "
                        "row + the f32 output"}
    if host:
        doc["cpu"] = dict(cpu_identity(), cores=cores, kind="port",
                          note="cpu_avg_ms: oracle AVX2 port of kernels_amd64.s (int8 row "
                               "dots, bit-identical results) per call, all listed cores")
    text = json.dumps(doc, indent=2)
    print(text, flush=True)
    if args.kernel_bench_json:
        with open(args.kernel_bench_json, "w") as f:
            f.write(text + "\n")


def bandwidth(args):
    """HBM calibration with library-independent kernels (torch's device copy and
    sum), graph replays timed with HIP events: what one launch of the
    headline's size (33 MB) and a large one (512 MiB) reach on this part."""
    import torch

    for mb in (33.1, 512.0):
        n = int(mb * 1e6 / 4) if mb < 100 else int(mb * (1 << 20) / 4)
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        out = torch.empty(1, dtype=torch.float32, device="cuda")
        reps = 200 if mb < 100 else 20
        for name, fn, bytes_moved in (("copy (read + write)", lambda: dst.copy_(src), 2 * n * 4),
                                      ("sum (read)", lambda: torch.sum(src.view(1, -1), dim=1, out=out),
                                       n * 4)):
            def body(fn=fn):
                for _ in range(reps):
                    fn()
            graph = timed_graph(torch, body)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(3):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / (3 * reps) * 1e3
            print(json.dumps({"bandwidth": name, "bytes_per_launch": bytes_moved,
                              "us_per_launch": round(us, 3),
                              "tb_s": round(bytes_moved / (us * 1e-6) / 1e12, 3)}), flush=True)
        del src, dst


def summarize_decode_trace(path):
    """Per-token kernel breakdown of the last 40 decode steps in a rocprofv3
    kernel-trace CSV of a bench run (each step ends with argmax_final_kernel)."""
    import collections
    import csv

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    # decode steps end with the vocabulary head and argmax_final_kernel; take
    # the longest run of them less than 10 ms apart (the configs[4] decode,
    # not the Q4_K_M record's lone step), its last 40 steps
    ends = [i for i, r in enumerate(rows) if "argmax_final" in r["Kernel_Name"] and i > 0 and
            "gemv_q6k" in rows[i - 1]["Kernel_Name"]]
    runs, cur = [], []
    for i in ends:
        if cur and int(rows[i]["Start_Timestamp"]) - int(rows[cur[-1]]["Start_Timestamp"]) > 10_000_000:
            runs.append(cur)
            cur = []
        cur.append(i)
    runs.append(cur)
    ends = max(runs, key=len)[-41:]
    seg = rows[ends[0] + 1: ends[-1] + 1]
    steps = len(ends) - 1
    agg = collections.defaultdict(lambda: [0, 0.0])
    for r in seg:
        name = r["Kernel_Name"].replace("gllm::", "").split("(")[0][:60]
        if "gemv" in name:
            name += f" grid {r['Grid_Size_X']} wg {r['Workgroup_Size_X']}"
        agg[name][0] += 1
        agg[name][1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    wall = (int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) / 1e3 / steps
    busy = sum(v[1] for v in agg.values()) / steps
    print(f"steps {steps}: wall per step {wall:.1f} us, kernel-busy {busy:.1f} us")
    print("| us per token | calls per token | us per call | kernel |")
    print("|---|---|---|---|")
    for name, (c, t) in sorted(agg.items(), key=lambda x: -x[1][1]):
        print(f"| {t / steps:.1f} | {c / steps:.1f} | {t / c:.2f} | `{name}` |")


def summarize_pmc(dirs):
    """Median per (kernel, counter) over the dispatches in the rocprofv3
    counter_collection CSVs under `dirs` (one counter pass per directory),
    and the median kernel duration of any kernel_trace CSV there."""
    import collections
    import csv
    import glob
    import statistics

    vals = collections.defaultdict(list)
    durs = collections.defaultdict(list)
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            per = collections.defaultdict(float)
            for r in csv.DictReader(open(f)):
                k = r.get("Kernel_Name", "?").replace("gllm::", "")[:70]
                per[(r["Dispatch_Id"], k, r["Counter_Name"])] += float(r["Counter_Value"])
            for (_, k, c), v in per.items():
                vals[(k, c)].append(v)
        for f in glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                k = r["Kernel_Name"].replace("gllm::", "").split("(")[0][:48]
                k += f" grid {r['Grid_Size_X']}x{r.get('Grid_Size_Y', 1)} wg {r['Workgroup_Size_X']}"
                durs[k].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    for (k, c), v in sorted(vals.items()):
        print(f"{k:70s} {c:28s} n={len(v):5d} median={statistics.median(v):16.1f}")
    for k, v in sorted(durs.items(), key=lambda kv: -sum(kv[1]))[:40]:
        print(f"{k:80s} n={len(v):5d} mean={statistics.mean(v) / 1e3:9.2f} us "
              f"median={statistics.median(v) / 1e3:9.2f} us min={min(v) / 1e3:.2f} us")


def profile_run():
    """Eager launches for rocprofv3 counter passes (no graphs, no timing):
    20 row-kernel launches over the rotating copies, then 5 elementwise
    kernels that read and write 512 MiB each, which calibrate FETCH_SIZE /
    WRITE_SIZE against a known byte count."""
    import torch

    import gopherllm_amd as g

    g.load()
    rows, cols = ROWS, COLS
    wbytes = rows * (cols // 256) * 144
    copies = max(2, math.ceil(300e6 / wbytes))
    weights = make_weights(g, torch, rows, cols, copies, seed=1000)
    x = torch.empty(cols, dtype=torch.float32, device="cuda")
    g.fill_normal_dev(x, 7, 1.0)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    for i in range(20):
        weights[i % copies].matvec_dev(x.view(1, -1), out.view(1, -1))
    torch.cuda.synchronize()
    src = torch.ones(512 << 18, dtype=torch.float32, device="cuda")  # 512 MiB
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.add(src, 1.0, out=dst)  # one elementwise kernel: reads 512 MiB, writes 512 MiB
    torch.cuda.synchronize()
    print(json.dumps({"profile_run": "done", "gemv_launches": 20, "copy_bytes": src.numel() * 4}),
          flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--suite", action="store_true",
                    help="measure the other configs (GEMV types/shapes/batch 8, prefill, attention)")
    ap.add_argument("--only", default="",
                    help="suite parts to run: comma list of gemv, formats, groups, prefill, attention")
    ap.add_argument("--ctx", type=int, default=0, help="suite attention: only this context")
    ap.add_argument("--profile-run", action="store_true",
                    help="eager launches for rocprofv3 counter collection")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="fastest single launch that only reads the headline GEMV's bytes (probe sweep)")
    ap.add_argument("--launch-floor", action="store_true",
                    help="per-node cost of short launches replayed from one HIP graph")
    ap.add_argument("--summarize-pmc", nargs="+", default=None,
                    help="medians of rocprofv3 counter / kernel-trace CSVs under these directories")
    ap.add_argument("--summarize-decode-trace", default="",
                    help="print the per-token kernel breakdown of a rocprofv3 kernel-trace CSV")
    ap.add_argument("--bandwidth", action="store_true",
                    help="HBM calibration: torch copy / sum of 33 MB and 512 MiB, graph replays")
    ap.add_argument("--kernel-bench", action="store_true",
                    help="llm-kernel-bench.v1 per-path report for layer 0 of the 8B-shape model")
    ap.add_argument("--kernel-bench-runs", type=int, default=100)
    ap.add_argument("--kernel-bench-json", default="", help="also write the report to this file")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=0, help="weight copies to rotate (0: >= 300 MB)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the configs[4] full-model decode measurement")
    args = ap.parse_args()
    if args.profile_run:
        profile_run()
        return
    if args.read_ceiling:
        read_ceiling(args)
        return
    if args.launch_floor:
        launch_floor(args)
        return
    if args.kernel_bench:
        kernel_bench(args)
        return
    if args.bandwidth:
        bandwidth(args)
        return
    if args.summarize_decode_trace:
        summarize_decode_trace(args.summarize_decode_trace)
        return
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc)
        return
    if args.suite:
        suite(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path would shard by output rows, see DESIGN.md)", file=sys.stderr)
        raise SystemExit(2)
    line = run(args)
    if not args.no_decode:
        line["decode"] = decode_bench(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
