#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

Headline (the `value`): decode attention HBM throughput at 32k context, the
BASELINE's configs[1] -- 10 attention layers, each with its OWN 67 MB fp16 KV
cache (670 MB in all, so the 256 MB MALL cannot serve the stream), captured as
10 x (split, combine) in one hipGraph, the way the engine replays its decode
step.  A step is one replay; bytes per layer are the reference's own count,
seq x 2048 (K and V read once; bench_attn.cu:257-264).

Also measured and reported under "results": C3 (131k x 10 layers, 2.7 GB),
C4 (one 4096-token prefill chunk, int8 scores, near 1024, sink) and C5 (a
131072-token prompt in 32 chunks of 4096), the per-kernel durations from HIP
events recorded on the launch stream around every launch, and the CPU oracle
(float64, single thread) as the reported CPU baseline.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--skip-prefill] [--cpu-seconds S]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "lfm2-ampere_amd"))

HBM_PEAK_GBS = 8000.0                 # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0               # dense int8 MFMA
PEAK_FP16_TFLOPS = 2500.0             # dense fp16 MFMA
REF_3090TI_GBS_32K = 669.3            # reference, RTX 3090 Ti, docs/ARCHITECTURE.md:2401


DECODE_SOURCES = ("lfm2-ampere_amd/csrc/decode.hip", "lfm2-ampere_amd/csrc/lk_common.h",
                  "lfm2-ampere_amd/Makefile")


def decode_source_sha16():
    """sha256 (first 16 hex digits) over the sources the split kernel is built
    from; a committed counter profile records the value it was taken on."""
    import hashlib
    h = hashlib.sha256()
    for rel in DECODE_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def split_traffic_from_profile():
    """HBM bytes per C2 split launch from the committed rocprofv3 FETCH_SIZE +
    WRITE_SIZE summary (calibrated against a 1 GiB copy) -- a counter figure
    that needs its own profiler runs, so it is read from the profile, not
    measured here -- and only when that profile was taken on these very
    sources: returns (bytes or None, note)."""
    import re
    try:
        txt = open(os.path.join(ROOT, "profiles", "decode_attn_c2_c3.md")).read()
    except OSError:
        return None, "no profile"
    m = re.search(r"traffic_bytes_per_launch = (\d+)", txt)
    s = re.search(r"source_sha16 = ([0-9a-f]{16})", txt)
    if not m:
        return None, "no traffic figure in profiles/decode_attn_c2_c3.md"
    cur = decode_source_sha16()
    if not s or s.group(1) != cur:
        return None, f"profiles/decode_attn_c2_c3.md is stale (taken on sources {s.group(1) if s else '?'}, now {cur})"
    return int(m.group(1)), f"from profiles/decode_attn_c2_c3.md, taken on sources {cur} (these)"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def timed_reps(fn, stream, iters, reps=11):
    """ms per call of fn() on `stream`, the way the reference's bench_attn.cu
    times (tests/bench_attn.cu:125-142): `reps` repetitions, each one pair of
    HIP events around `iters` back-to-back calls (launch overhead amortised, so
    the figure tracks the kernel's own duration as rocprof reports it), the
    average per call of each repetition, then the median over repetitions.
    Returns {"median", "min", "max", "reps", "iters"} in ms."""
    import torch
    fn()
    stream.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in evs:
        a.record(stream)
        for _ in range(iters):
            fn()
        b.record(stream)
    stream.synchronize()
    ms = sorted(a.elapsed_time(b) / iters for a, b in evs)
    return {"median": ms[len(ms) // 2], "min": ms[0], "max": ms[-1], "reps": reps, "iters": iters}


def spread_us(t):
    """A timed_reps result in microseconds, for the results record."""
    return {"median_us": t["median"] * 1e3, "min_us": t["min"] * 1e3, "max_us": t["max"] * 1e3,
            "reps": t["reps"], "iters": t["iters"]}


def bench_decode(lk, lkc, cfg, steps, warmup, kernel_iters, seq=None):
    import torch
    qs, kcs, vcs, seq = lkc.decode_inputs(cfg, layers=10, seq=seq)
    layers = len(qs)
    d_pos = torch.tensor([seq - 1], dtype=torch.int32, device="cuda")
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    outs = [torch.empty(32, 64, device="cuda") for _ in range(layers)]
    graph = lk.DecodeGraph(qs, kcs, vcs, d_pos, part, outs)
    st = graph.stream
    torch.cuda.synchronize()
    for _ in range(warmup):
        graph.launch()
    st.synchronize()
    # one event between consecutive replays: the total over the K steps is the
    # headline; the per-step spread is reported beside it
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    evs[0].record(st)
    for i in range(steps):
        graph.launch()
        evs[i + 1].record(st)
    st.synchronize()
    torch.cuda.synchronize()
    ms_step = evs[0].elapsed_time(evs[-1]) / steps
    per_step = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    bytes_layer = seq * 2048.0
    us_layer = ms_step * 1e3 / layers
    gbs = bytes_layer * layers / (ms_step * 1e-3) / 1e9
    # per-kernel: the split kernel alone, rotating over the 10 layers' caches
    i = [0]

    def one_split():
        j = i[0] % layers
        i[0] += 1
        lk.attn_split(qs[j], kcs[j], vcs[j], d_pos, part, stream=st)

    one_split()
    split_t = timed_reps(one_split, st, kernel_iters)
    comb_t = timed_reps(lambda: lk.attn_combine(part, d_pos, outs[0], None, stream=st), st, kernel_iters)
    graph.close()
    split_us, comb_us = split_t["median"] * 1e3, comb_t["median"] * 1e3
    res = {
        "seq": seq, "layers": layers, "ms_per_step": ms_step, "us_per_layer": us_layer,
        "us_per_layer_step_spread": {"median": per_step[len(per_step) // 2] * 1e3 / layers,
                                     "min": per_step[0] * 1e3 / layers, "max": per_step[-1] * 1e3 / layers},
        "GBps": gbs, "layer_frac": gbs / HBM_PEAK_GBS,
        "split_us": split_us, "combine_us": comb_us,
        "split": spread_us(split_t), "combine": spread_us(comb_t),
        "split_GBps": bytes_layer / (split_us * 1e-6) / 1e9,
        "split_frac": bytes_layer / (split_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "bytes_per_layer": bytes_layer, "graph_nodes": 2 * layers,
    }
    del qs, kcs, vcs
    torch.cuda.empty_cache()
    return res


def bench_decode_step(lk, steps, warmup, layers=10, ctx=32768, with_wo=False):
    """The decode step graph (per layer: qk norm + RoPE + cache append, split,
    combine; then d_pos += 1; reference engine.cu:1328-1342,
    1750-1760) replayed `steps` times around a 32k context: the attention slice
    of a whole decode step, producers included.  with_wo: each layer also runs
    the attention output projection (x += W_o . yq8, 2048 x 2048 Q4_0,
    engine.cu:655-657) as a third node."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(91)
    Ls = []
    for _ in range(layers):
        Ls.append({"q_src": torch.randn(2048, device="cuda", generator=g),
                   "k_src": torch.randn(512, device="cuda", generator=g),
                   "v_src": torch.randn(512, device="cuda", generator=g),
                   "q": torch.empty(2048, device="cuda"), "k": torch.empty(512, device="cuda"),
                   "q_norm": torch.rand(64, device="cuda", generator=g) + 0.5,
                   "k_norm": torch.rand(64, device="cuda", generator=g) + 0.5,
                   "kc": torch.randn(ctx, 8, 64, device="cuda", generator=g).half(),
                   "vc": torch.randn(ctx, 8, 64, device="cuda", generator=g).half(),
                   "out": torch.empty(32, 64, device="cuda")})
        if with_wo:
            Ls[-1].update({"out": None, "yq8": torch.zeros(64 * 36, dtype=torch.uint8, device="cuda"),
                           "wo_qs": torch.randint(0, 256, (2048 * 64 * 16,), dtype=torch.uint8, device="cuda", generator=g),
                           "wo_d": (torch.rand(2048 * 64, device="cuda", generator=g) * 0.02 + 0.001).half().view(torch.int16),
                           "x": torch.zeros(2048, device="cuda")})
    start = ctx - steps - warmup
    d_pos = torch.tensor([start], dtype=torch.int32, device="cuda")
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    gr = lk.DecodeStepGraph(Ls, d_pos, part)
    st = gr.stream
    torch.cuda.synchronize()
    gr.run(warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    gr.run(steps)
    e1.record(st)
    st.synchronize()
    ms = e0.elapsed_time(e1) / steps
    assert int(d_pos.item()) == ctx
    nodes = gr.nodes()
    gr.close()
    del Ls
    torch.cuda.empty_cache()
    return {"layers": layers, "context": f"{start + warmup} .. {ctx - 1}", "steps": steps,
            "us_per_step": ms * 1e3, "us_per_layer": ms * 1e3 / layers, "graph_nodes": nodes}


def pf_ops(m, P):
    """Algorithmic ops of one causal chunk: per (query, key) pair 64 int8 MAC for
    Q.K and 64 fp16 MAC for P.V, 2 ops per MAC (test_prefill.cu:652)."""
    pairs = 32.0 * m * (P + (m + 1) / 2.0)
    return pairs * 64 * 2, pairs * 64 * 2, pairs


def bench_prefill_c4(lk, lkc, iters, reps=11):
    import torch
    qh, kc, vc, S = lkc.prefill_inputs("C4")
    m, P = S, 0
    ks = lk.kstride_for(S)
    st = torch.cuda.Stream()
    q8 = torch.empty(m, 2048, dtype=torch.int8, device="cuda")
    qsc = torch.empty(m, 32, device="cuda")
    qcs = torch.empty(m, 32, device="cuda")
    k8 = torch.empty(S * 512, dtype=torch.int8, device="cuda")
    ksc = torch.empty(8 * ks + 4, device="cuda")
    o = torch.empty(m, 2048, device="cuda")
    torch.cuda.synchronize()
    q_t = timed_reps(lambda: lk.pf_q8(qh, m, None, q8, qsc, qcs, stream=st), st, iters)
    k_t = timed_reps(lambda: lk.pf_k8(kc, 0, S, None, ks, k8, ksc, stream=st), st, iters)
    # int8 scoring as an engine without smoothing calls it: Q quantised inside
    # the attention kernel (q8 = NULL; bit-identical to lk_pf_q8 + lk_pf_attn8);
    # the precomputed-q8 form is timed beside it
    f8 = lambda: lk.pf_attn8(None, None, None, qh, m, P, k8, ksc, ks, kc, vc, 1024, 1, o, stream=st)
    f8p = lambda: lk.pf_attn8(q8, qsc, qcs, qh, m, P, k8, ksc, ks, kc, vc, 1024, 1, o, stream=st)
    f16 = lambda: lk.pf_attn(qh, m, P, kc, vc, o, stream=st)
    # the next GEMM's planar Q8_1: a separate pass over o, or fused (o not written)
    aqs = torch.empty(m, 2048, dtype=torch.int8, device="cuda")
    asc = torch.empty(m, 64, 2, device="cuda")
    fq = lambda: (f8(), lk.pf_quant_rows(o, m, 2048, 64, aqs, asc, stream=st))
    ff = lambda: lk.pf_attn8_q81(None, None, None, qh, m, P, k8, ksc, ks, kc, vc, 1024, 1, None, aqs, asc, stream=st)
    lk.pf_q8(qh, m, None, q8, qsc, qcs, stream=st)
    for _ in range(iters):                  # warm-up (clocks settle over the first ~100 us)
        f8()
    # the int8 and fp16 kernels alternate repetition by repetition, so that a
    # drift of the clocks during the run affects them alike
    t8, t16, t8p = [], [], []
    for _ in range(reps):
        t8.append(timed_reps(f8, st, iters, reps=1)["median"])
        t16.append(timed_reps(f16, st, iters, reps=1)["median"])
        t8p.append(timed_reps(f8p, st, iters, reps=1)["median"])
    t8.sort()
    t16.sort()
    t8p.sort()
    a8_t = {"median": t8[reps // 2], "min": t8[0], "max": t8[-1], "reps": reps, "iters": iters}
    a16_t = {"median": t16[reps // 2], "min": t16[0], "max": t16[-1], "reps": reps, "iters": iters}
    q_pass_t = timed_reps(fq, st, iters, reps)
    q_fused_t = timed_reps(ff, st, iters, reps)
    a8_ms, a16_ms = a8_t["median"], a16_t["median"]
    oi, of, pairs = pf_ops(m, P)
    peak_ms = (oi / (PEAK_INT8_TOPS * 1e12) + of / (PEAK_FP16_TFLOPS * 1e12)) * 1e3
    return {
        "m": m, "P": P, "near": 1024, "sink": 1, "pairs": pairs,
        "attn8_us": a8_ms * 1e3, "attn8_TOPS": (oi + of) / (a8_ms * 1e-3) / 1e12,
        "attn8_frac_of_mixed_peak": peak_ms / a8_ms, "attn8": spread_us(a8_t),
        "attn_fp16_us": a16_ms * 1e3, "attn_fp16_TOPS": (oi + of) / (a16_ms * 1e-3) / 1e12,
        "attn_fp16_frac_of_mixed_peak": peak_ms / a16_ms, "attn_fp16": spread_us(a16_t),
        "attn8_q8_precomputed_us": t8p[reps // 2] * 1e3,
        "q8_us": q_t["median"] * 1e3, "k8_us": k_t["median"] * 1e3,
        "attn8_then_quant_rows_us": q_pass_t["median"] * 1e3, "attn8_q81_fused_us": q_fused_t["median"] * 1e3,
        "attn8_q81_fused": spread_us(q_fused_t),
    }


C5_SAMPLE_CHUNKS = (65536, 126976)    # chunk starts whose sampled rows are checked
C5_SAMPLE_ROWS = 6


def bench_prefill_c5(lk, lkc, reps):
    """C5: a 131072-token prompt in 32 chunks of 4096, the int8 kernel and the
    fp16 kernel (every tile exact) alternating repetition by repetition; per
    repetition the attention total over the 32 chunks (Q quantised inside the
    int8 attention kernel; the int8 K pass of each chunk is timed apart).  Also returns the two kernels' outputs on sampled rows of two
    chunks, which the CPU leg checks against float64 attention."""
    import torch
    import numpy as np
    qh, kc, vc, S = lkc.prefill_inputs("C5")
    m = 4096
    ks = lk.kstride_for(S)
    st = torch.cuda.Stream()
    k8 = torch.empty(S * 512, dtype=torch.int8, device="cuda")
    ksc = torch.empty(8 * ks + 4, device="cuda")
    o = torch.empty(m, 2048, device="cuda")
    qchunks = [qh[p:p + m].contiguous() for p in range(0, S, m)]
    rows = np.linspace(0, m - 1, C5_SAMPLE_ROWS).astype(np.int64)
    samples = {}
    torch.cuda.synchronize()

    def prompt(int8, keep):
        ev = []
        for c, P in enumerate(range(0, S, m)):
            a, b, c2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            a.record(st)
            if int8:
                lk.pf_k8(kc, P, P + m, None, ks, k8, ksc, stream=st)
            b.record(st)
            if int8:        # Q quantised inside the attention kernel (no smoothing)
                lk.pf_attn8(None, None, None, qchunks[c], m, P, k8, ksc, ks, kc, vc, 1024, 1, o, stream=st)
            else:
                lk.pf_attn(qchunks[c], m, P, kc, vc, o, stream=st)
            c2.record(st)
            ev.append((a, b, c2))
            if keep and P in C5_SAMPLE_CHUNKS:
                st.synchronize()
                samples.setdefault(P, {"rows": rows})["o8" if int8 else "o16"] = o[rows].cpu().numpy()
        st.synchronize()
        return (sum(a.elapsed_time(b) for a, b, _ in ev), sum(b.elapsed_time(c2) for _, b, c2 in ev))

    prompt(True, True)                                  # warm-up, and the sampled outputs
    prompt(False, True)
    t8, t16, tq = [], [], []
    for _ in range(reps):
        q_ms, a_ms = prompt(True, False)
        tq.append(q_ms)
        t8.append(a_ms)
        t16.append(prompt(False, False)[1])
    t8.sort(); t16.sort(); tq.sort()
    oi = of = 0.0
    for P in range(0, S, m):
        a, b, _ = pf_ops(m, P)
        oi += a
        of += b
    peak_ms = (oi / (PEAK_INT8_TOPS * 1e12) + of / (PEAK_FP16_TFLOPS * 1e12)) * 1e3
    attn_ms, a16_ms = t8[len(t8) // 2], t16[len(t16) // 2]
    del qh, kc, vc, qchunks, k8
    torch.cuda.empty_cache()
    return {
        "chunks": S // m, "chunk": m, "reps": reps,
        "attn_ms": attn_ms, "attn_ms_min": t8[0], "attn_ms_max": t8[-1],
        "quant_ms": tq[len(tq) // 2],
        "attn8_TOPS": (oi + of) / (attn_ms * 1e-3) / 1e12,
        "attn8_frac_of_mixed_peak": peak_ms / attn_ms,
        "attn_fp16_ms": a16_ms, "attn_fp16_ms_min": t16[0], "attn_fp16_ms_max": t16[-1],
        "attn_fp16_TOPS": (oi + of) / (a16_ms * 1e-3) / 1e12,
        "attn_fp16_frac_of_mixed_peak": peak_ms / a16_ms,
    }, samples


def bench_decode_curve(lk, lkc, c2, c3, steps, warmup, kernel_iters, extra=(8192, 65536)):
    """Decode attention per layer over context length -- the reference's own
    curve is 8192, 32768, 65536 and 131040 (docs/ARCHITECTURE.md:2400-2403)
    with the fixed-cost model 23.3 us + bytes / 856 GB/s (:2411).  The 8k and
    65k points are measured here (10-layer graphs, C2's distributions); 32k and
    131k are C2 and C3.  The same model is fitted by least squares to the
    layer times and, separately, to the split kernel's own times."""
    pts = []
    for seq in extra:
        r = bench_decode(lk, lkc, "C2", steps, warmup, kernel_iters, seq=seq)
        pts.append(r)
    pts += [c2, c3]
    pts.sort(key=lambda r: r["seq"])

    def fit(key):
        xs = [r["seq"] * 2048.0 for r in pts]
        ys = [r[key] for r in pts]
        n = len(xs)
        mx, my = sum(xs) / n, sum(ys) / n
        sxx = sum((x - mx) ** 2 for x in xs)
        sxy = sum((x - mx) * (y - my) for x, y in zip(xs, ys))
        slope = sxy / sxx                              # us per byte
        a = my - slope * mx
        resid = max(abs(y - (a + slope * x)) for x, y in zip(xs, ys))
        return {"fixed_us": a, "GBps": 1e-3 / slope, "max_residual_us": resid}

    return {
        "points": [{"seq": r["seq"], "us_per_layer": r["us_per_layer"], "GBps": r["GBps"],
                    "split_us": r["split_us"], "combine_us": r["combine_us"],
                    "layer_frac": r["layer_frac"]} for r in pts],
        "fit_layer": fit("us_per_layer"),
        "fit_split": fit("split_us"),
        "reference_fit": {"fixed_us": 23.3, "GBps": 856.0, "hardware": "RTX 3090 Ti"},
    }


def bench_read_reference(lk, bytes_list=(67108864, 268435456), nbuf=10, iters=20):
    """The practical HBM read rate of this GPU, for scale: the library's plain
    streaming-read probe (lk_read_probe) over buffers of the decode layers'
    sizes (C2 67 MB, C3 268 MB), cycling over nbuf distinct buffers so that the
    256 MB last-level cache does not serve them.  The split kernel's rate is
    best read against this, the datasheet 8 TB/s not being reachable by reads."""
    import torch
    out = {}
    sink = torch.zeros(1, device="cuda")
    for nb in bytes_list:
        bufs = [torch.ones(nb // 4, device="cuda") for _ in range(nbuf)]
        for b in bufs[:2]:
            lk.read_probe(b, sink)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(iters):
            lk.read_probe(bufs[i % nbuf], sink)
        e1.record(); e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        out[f"{nb >> 20}MiB"] = {"us": us, "GBps": nb / (us * 1e-6) / 1e9}
        del bufs
        torch.cuda.empty_cache()
    return out


def bench_gemv(lk, nmat=128, iters=256, graph_timing=True):
    """The attention-output GEMV (reference k_gemv_q4_0 at engine.cu:655-657):
    2048 x 2048 Q4_0 weights x the combine's 64 Q8_1 blocks, residual added.
    Cycles over nmat distinct weight matrices (302 MB for 128, more than the
    256 MB last-level cache), so every launch reads its weights from HBM as a
    decode step does.  Algorithmic bytes per launch: 2048 x 64 x 18 (weights
    and scales) + 64 x 36 (activation) + 2048 x 8 (residual read and write)."""
    import torch
    rows, bpr = 2048, 64
    g = torch.Generator(device="cuda").manual_seed(7)
    qs = [torch.randint(0, 256, (rows * bpr * 16,), dtype=torch.uint8, device="cuda", generator=g) for _ in range(nmat)]
    d = [(torch.rand(rows * bpr, device="cuda", generator=g) * 0.02 + 0.001).half().view(torch.int16) for _ in range(nmat)]
    xq = torch.zeros(bpr * 36, dtype=torch.uint8, device="cuda")
    xq.view(bpr, 36)[:, 4:] = torch.randint(-127, 128, (bpr, 32), device="cuda", generator=g).to(torch.int8).view(torch.uint8)
    xq.view(bpr, 36)[:, 0:2] = torch.full((bpr, 1), 0.01, device="cuda").half().view(torch.uint8)
    y = torch.zeros(rows, device="cuda")
    st = torch.cuda.Stream()
    f = lambda i: lk.gemv_q4_0(qs[i % nmat], d[i % nmat], xq, rows, bpr, y, True, None, 1e-5, stream=st)
    for i in range(nmat):
        f(i)
    st.synchronize()
    ctr = [0]

    def one():
        f(ctr[0])
        ctr[0] += 1

    t = timed_reps(one, st, iters)
    us = t["median"] * 1e3
    nbytes = rows * bpr * 18 + bpr * 36 + rows * 8
    res = {"rows": rows, "bpr": bpr, "us": us, "GBps": nbytes / (us * 1e-6) / 1e9, "bytes": nbytes,
           "distinct_weight_matrices": nmat, "spread": spread_us(t)}
    if not graph_timing:          # profiler runs: counter collection makes the replays slow
        return res
    # the same launches captured in one hipGraph (nmat nodes, as a decode step
    # graph holds them), replayed: per-launch time without the eager launch path
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        for i in range(nmat):
            f(i)
    def replay():
        with torch.cuda.stream(st):
            graph.replay()

    for _ in range(3):
        replay()
    st.synchronize()
    tg = timed_reps(replay, st, 5)
    us_graph = tg["median"] * 1e3 / nmat
    res.update({"us_in_graph": us_graph, "GBps_in_graph": nbytes / (us_graph * 1e-6) / 1e9})
    return res


def bench_pf_gemm(lk, ntok=4096, N=2048, bpr=64, iters=20):
    """The attention-output GEMM of a prefill chunk (reference pf_gemm_dense at
    engine.cu:1128-1131): C4's 4096 tokens of planar Q8_1 x 2048 x 2048 Q4_0,
    residual added.  Work: 2 * N * 32 * bpr * ntok int8 ops (the nibble x int8
    products and sums)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(11)
    qs = torch.randint(0, 256, (N * bpr * 16,), dtype=torch.uint8, device="cuda", generator=g)
    d = (torch.rand(N * bpr, device="cuda", generator=g) * 0.02 + 0.001).half().view(torch.int16)
    aqs = torch.randint(-127, 128, (ntok, bpr * 32), device="cuda", generator=g).to(torch.int8)
    asc = torch.rand(ntok, bpr, 2, device="cuda", generator=g) * 0.02
    out = torch.zeros(ntok, N, device="cuda")
    st = torch.cuda.Stream()
    f = lambda: lk.pf_gemm_q4_0(qs, d, N, bpr, aqs, asc, ntok, out, N, True, stream=st)
    for _ in range(iters):
        f()
    t = timed_reps(f, st, iters)
    ms = t["median"]
    ops = 2.0 * N * 32 * bpr * ntok
    return {"ntok": ntok, "N": N, "K": 32 * bpr, "us": ms * 1e3, "TOPS": ops / (ms * 1e-3) / 1e12,
            "frac_of_int8_peak": ops / (ms * 1e-3) / (PEAK_INT8_TOPS * 1e12), "spread": spread_us(t)}


def bench_producers(lk, iters):
    """The attention-input producers (reference kernels.cu:871-915,
    prefill.cu:975-1016): the prefill pass over one 4096-token chunk (C4's
    shape) with and without the fused int8 K copy, against qknr + pf_k8 as two
    passes, and the decode kernel for one token.  HBM-bound; algorithmic bytes
    = Y read (m x 3072 fp32) + qh, K, V written (fp16) [+ int8 K and scales]."""
    import torch
    m, P = 4096, 0
    S = P + m
    ks = lk.kstride_for(S)
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    Y = torch.randn(m, 3072, device="cuda", generator=g) * 3.0
    qn = torch.rand(64, device="cuda", generator=g) + 0.5
    kn = torch.rand(64, device="cuda", generator=g) + 0.5
    qh = torch.empty(m, 2048, dtype=torch.float16, device="cuda")
    kc = torch.empty(S, 8, 64, dtype=torch.float16, device="cuda")
    vc = torch.empty_like(kc)
    k8 = torch.empty(S * 512, dtype=torch.int8, device="cuda")
    ksc = torch.empty(8 * ks + 4, device="cuda")
    st = torch.cuda.Stream()
    torch.cuda.synchronize()
    f0 = lambda: lk.pf_qknr(Y, qn, kn, m, P, qh, kc, vc, stream=st)
    f1 = lambda: lk.pf_qknr(Y, qn, kn, m, P, qh, kc, vc, k8, ksc, ks, stream=st)
    f2 = lambda: (lk.pf_qknr(Y, qn, kn, m, P, qh, kc, vc, stream=st),
                  lk.pf_k8(kc, P, S, None, ks, k8, ksc, stream=st))
    for f in (f0, f1, f2):
        for _ in range(iters):
            f()
    t0 = timed_reps(f0, st, iters)["median"]
    t1 = timed_reps(f1, st, iters)["median"]
    t2 = timed_reps(f2, st, iters)["median"]
    b0 = m * 3072 * 4 + m * 2048 * 2 + m * 512 * 2 * 2
    b1 = b0 + m * 512 + m * 8 * 4
    qf = torch.randn(2048, device="cuda", generator=g)
    kf = torch.randn(512, device="cuda", generator=g)
    vf = torch.randn(512, device="cuda", generator=g)
    d_pos = torch.tensor([S - 1], dtype=torch.int32, device="cuda")
    fd = lambda: lk.qk_norm_rope(qf, kf, vf, qn, kn, d_pos, kc, vc, stream=st)
    for _ in range(iters):
        fd()
    td = timed_reps(fd, st, iters)["median"]
    return {
        "m": m, "qknr_us": t0 * 1e3, "qknr_GBps": b0 / (t0 * 1e-3) / 1e9, "qknr_bytes": b0,
        "qknr_k8_fused_us": t1 * 1e3, "qknr_k8_fused_GBps": b1 / (t1 * 1e-3) / 1e9,
        "qknr_then_k8_us": t2 * 1e3, "decode_qk_norm_rope_us": td * 1e3,
    }


def bench_pf_driver(lk, n_tok=32768, chunks=(4096, 8192)):
    """The prefill chunk driver (engine.cu:1064-1124, 1255-1260) over an
    n_tok prompt for one attention layer, per chunk size (the engine's default
    is 8192, engine.cu:1315): producers + int8 K + Q quantiser + attention,
    synthetic projections."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(93)
    qn = torch.rand(64, device="cuda", generator=g) + 0.5
    kn = torch.rand(64, device="cuda", generator=g) + 0.5
    kc = torch.empty(n_tok, 8, 64, dtype=torch.float16, device="cuda")
    vc = torch.empty_like(kc)
    res = {}
    for mc in chunks:
        ctx = lk.PrefillCtx(1, mc, n_tok)
        Y = torch.randn(mc, 3072, device="cuda", generator=g) * 3.0
        o = torch.empty(mc, 2048, device="cuda")
        st = torch.cuda.Stream()

        def prompt():
            for p0 in range(0, n_tok, mc):
                ctx.chunk_attn(0, Y, qn, kn, mc, p0, kc, vc, o, stream=st)
                ctx.chunk_done(p0 + mc)
        prompt()                                      # warm-up
        st.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        prompt()
        e1.record(st)
        st.synchronize()
        ms = e0.elapsed_time(e1)
        res[f"chunk_{mc}"] = {"ms": ms, "tokens_per_s": n_tok / (ms * 1e-3)}
        ctx.close()
        del Y, o
    del kc, vc
    torch.cuda.empty_cache()
    return {"prompt_tokens": n_tok, "layers": 1, **res}


def cpu_baseline(seconds, prefill=True, c5_samples=None, c4_full_1t=False):
    """The reference's CPU path restated in the oracle (float64, single
    thread): decode attention (tests/test_attn.cu:46-74) on a full C2 layer and
    on C1, and prefill attention (tests/test_prefill.cu:263-282) on sampled
    query rows of C4 and of C5's last chunk, extrapolated by the number of
    (query, key) pairs to the whole chunk / prompt.  Beside them, the whole C4
    chunk (every row and head, no extrapolation) timed once with OpenMP over
    (row, head) on all the host threads OpenMP is given, the thread count
    stated; with c4_full_1t also the whole C4 chunk on one thread (about 80 s).

    With c5_samples (the GPU kernels' outputs on sampled rows of C5 chunks),
    the float64 attention of those rows is also the checker of the int8 and
    fp16 kernels' accuracy, the figure the reference reports for its int8
    scoring (tests/test_prefill.cu:862-866, src/engine.cu:245-248): rel-RMS =
    RMS(err) / RMS(ref) and max-rel = max|err| / max|ref| over the rows."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import lk_oracle as orc
    import lk_configs as lkc
    res = {}
    orc.set_threads(1)
    for cfg, budget in (("C2", seconds), ("C1", max(2.0, seconds / 5))):
        qs, kcs, vcs, seq = lkc.decode_inputs(cfg, layers=1)
        q = qs[0].cpu().numpy()
        kh = kcs[0].view(torch.int16).cpu().numpy().view(np.uint16)
        vh = vcs[0].view(torch.int16).cpu().numpy().view(np.uint16)
        n, t0 = 0, time.perf_counter()
        while True:
            orc.decode_ref(q, kh, vh, seq)
            n += 1
            if time.perf_counter() - t0 >= budget:
                break
        dt = (time.perf_counter() - t0) / n
        res[cfg] = {"us_per_layer": dt * 1e6, "GBps": seq * 2048.0 / dt / 1e9, "reps": n}
    if not prefill:
        return res
    h16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    for cfg, nrows in (("C4", 48), ("C5", 2)):
        qh, kc, vc, S = lkc.prefill_inputs(cfg)
        m = 4096
        P = 0 if cfg == "C4" else S - m
        rows = np.linspace(0, m - 1, nrows).astype(np.int32)
        Q, K, V = h16(qh[P:P + m]), h16(kc[:P + m]), h16(vc[:P + m])
        t0 = time.perf_counter()
        orc.pf_ref(Q, m, P, K, V, rows=rows)
        dt = time.perf_counter() - t0
        pairs_s = 32.0 * float(np.sum(P + rows.astype(np.float64) + 1))
        if cfg == "C4":
            pairs_full = pf_ops(m, 0)[2]
        else:
            pairs_full = sum(pf_ops(m, p)[2] for p in range(0, S, m))
        tf = dt * pairs_full / pairs_s
        ops = pairs_full * 256.0
        res[cfg] = {"s_extrapolated": tf, "TOPS": ops / tf / 1e12, "sample_rows": int(nrows),
                    "sample_s": dt, "sample_pairs": pairs_s,
                    "note": "float64 reference on sampled query rows (all 32 heads), "
                            "extrapolated by (query, key) pairs"}
        if cfg == "C5" and c5_samples:
            acc = {}
            for P0, smp in sorted(c5_samples.items()):
                r = np.asarray(smp["rows"], np.int32)
                ref = orc.pf_ref(h16(qh[P0:P0 + m]), m, P0, h16(kc[:P0 + m]), h16(vc[:P0 + m]), rows=r)[r]
                ent = {"rows": [int(x) for x in r]}
                for key, name in (("o8", "int8"), ("o16", "fp16")):
                    if key in smp:
                        e = smp[key].astype(np.float64) - ref
                        ent[name] = {"rel_rms": float(np.sqrt(np.mean(e * e)) / np.sqrt(np.mean(ref * ref))),
                                     "max_rel": float(np.max(np.abs(e)) / np.max(np.abs(ref)))}
                acc[f"P{P0}"] = ent
            res["C5_accuracy"] = acc
        if cfg == "C4":
            # OpenMP's default thread count is OMP_NUM_THREADS (the box's CPU share)
            omp_default = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
            runs = [("C4_full_1thread", 1)] if c4_full_1t else []
            runs.append(("C4_full_openmp", omp_default))
            for key, th in runs:
                nth = orc.set_threads(th)
                t0 = time.perf_counter()
                orc.pf_ref(Q, m, P, K, V)
                dt = time.perf_counter() - t0
                res[key] = {"s": dt, "TOPS": pairs_full * 256.0 / dt / 1e12, "threads": nth,
                            "note": "float64 reference over the whole C4 chunk (all 4096 rows, 32 heads)"}
            orc.set_threads(1)
        del qh, kc, vc
        torch.cuda.empty_cache()
    return res


def profile_prefill(lk, lkc, which, launches):
    """For rocprofv3 --pmc runs: `launches` int8 prefill attention launches on
    C4 (the 4096 chunk at P = 0) or on C5's last chunk (P = 126976); c5pair:
    that chunk in the paired launch (forced), to set the two launch forms
    side by side on the same tiles."""
    import torch
    if which == "c5pair":
        lk.pf_pair_override(1)
    if which == "c4":
        qh, kc, vc, S = lkc.prefill_inputs("C4")
        m, P, qc = S, 0, qh
    else:
        qh, kc, vc, S = lkc.prefill_inputs("C5")
        m, P = 4096, S - 4096
        qc = qh[P:].contiguous()
    ks = lk.kstride_for(P + m)
    k8 = torch.empty((P + m) * 512, dtype=torch.int8, device="cuda")
    ksc = torch.empty(8 * ks + 4, device="cuda")
    o = torch.empty(m, 2048, device="cuda")
    lk.pf_k8(kc, 0, P + m, None, ks, k8, ksc)
    for _ in range(launches):       # Q quantised inside the kernel, as bench_prefill_c4/c5 time it
        lk.pf_attn8(None, None, None, qc, m, P, k8, ksc, ks, kc, vc, 1024, 1, o)
    torch.cuda.synchronize()
    lk.pf_pair_override(0)
    oi, of, pairs = pf_ops(m, P)
    log(f"profile: {launches} prefill attention launches ({which}, m {m}, P {P}, "
        f"{pairs:.0f} (query, key) pairs, {oi + of:.4g} algorithmic ops each)")


def profile_decode_split(lk, lkc, launches):
    """For rocprofv3 --pmc runs: `launches` back-to-back lk_attn_split launches
    on C2 (rotating over 10 distinct 67 MB caches), then one 1 GiB device copy
    whose FETCH_SIZE / WRITE_SIZE calibrate the counters (it reads and writes
    exactly 2^30 bytes)."""
    import torch
    qs, kcs, vcs, seq = lkc.decode_inputs("C2", layers=10)
    d_pos = torch.tensor([seq - 1], dtype=torch.int32, device="cuda")
    part = torch.empty(lk.part_bytes() // 4, device="cuda")
    for i in range(launches):
        lk.attn_split(qs[i % 10], kcs[i % 10], vcs[i % 10], d_pos, part)
    torch.cuda.synchronize()
    src = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"profile: {launches} split launches (C2, seq {seq}, {seq * 2048} algorithmic bytes each), "
        f"then a {src.numel() * 4} byte copy")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernel-iters", type=int, default=100)
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-c4-1thread", action="store_true",
                    help="also time the whole C4 chunk's float64 reference on one thread (about 80 s)")
    ap.add_argument("--profile-split", type=int, default=0,
                    help="only run N C2 split launches + a 1 GiB copy (for rocprofv3 --pmc)")
    ap.add_argument("--profile-prefill", choices=["c4", "c5", "c5pair"], default=None,
                    help="only run --profile-launches int8 prefill attention launches (for rocprofv3 --pmc)")
    ap.add_argument("--profile-launches", type=int, default=3)
    ap.add_argument("--profile-gemv", action="store_true",
                    help="only run the attention-output GEMV bench (for rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this attention path is built and measured on a single "
              "MI355X (no multi-GPU path); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import lk_attn as lk
    import lk_configs as lkc
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    lk.load()
    cfgp = lk.config()
    if args.profile_split:
        profile_decode_split(lk, lkc, args.profile_split)
        return
    if args.profile_prefill:
        profile_prefill(lk, lkc, args.profile_prefill, args.profile_launches)
        return
    if args.profile_gemv:
        log(json.dumps(bench_gemv(lk, iters=32, graph_timing=False)))
        log(json.dumps(bench_pf_gemm(lk)))
        return

    log("decode C2 (32k x 10 layers, one hipGraph)")
    c2 = bench_decode(lk, lkc, "C2", args.steps, args.warmup, args.kernel_iters)
    log(json.dumps(c2))
    log("decode C3 (131k x 10 layers, one hipGraph)")
    c3 = bench_decode(lk, lkc, "C3", max(20, args.steps // 4), max(3, args.warmup // 4), args.kernel_iters // 2)
    log(json.dumps(c3))
    results = {"C2_decode_32k": c2, "C3_decode_131k": c3}
    log("decode curve over context length (C2 distributions, 10 layers, one hipGraph)")
    results["decode_curve"] = bench_decode_curve(lk, lkc, c2, c3, max(20, args.steps // 4), max(3, args.warmup // 4),
                                                 args.kernel_iters // 2)
    log(json.dumps(results["decode_curve"]))
    log("practical HBM read rate (plain streaming read of the decode layer sizes)")
    results["hbm_read_reference"] = bench_read_reference(lk)
    log(json.dumps(results["hbm_read_reference"]))
    log("attention-output GEMV (2048 x 2048 Q4_0 x Q8_1, residual add)")
    results["attn_out_gemv"] = bench_gemv(lk)
    log(json.dumps(results["attn_out_gemv"]))
    log("decode step graph (producer + attention, 10 layers, 32k context)")
    results["C2_decode_step_graph"] = bench_decode_step(lk, 50, 10)
    log(json.dumps(results["C2_decode_step_graph"]))
    log("decode step graph with the attention output projection (3 nodes per layer)")
    results["C2_decode_step_graph_wo"] = bench_decode_step(lk, 50, 10, with_wo=True)
    log(json.dumps(results["C2_decode_step_graph_wo"]))
    c5_samples = None
    if not args.skip_prefill:
        log("prefill C4 (4096 chunk, P=0)")
        results["C4_prefill_4k"] = bench_prefill_c4(lk, lkc, 20)
        log(json.dumps(results["C4_prefill_4k"]))
        log("prefill C5 (131072 prompt, 32 chunks)")
        results["C5_prefill_131k"], c5_samples = bench_prefill_c5(lk, lkc, 3)
        log(json.dumps(results["C5_prefill_131k"]))
        log("prefill attention-output GEMM (4096 tokens x 2048 x 2048 Q4_0)")
        results["pf_attn_out_gemm"] = bench_pf_gemm(lk)
        log(json.dumps(results["pf_attn_out_gemm"]))
        log("attention-input producers (qk norm + rope + cache write)")
        results["producers"] = bench_producers(lk, 20)
        log(json.dumps(results["producers"]))
        log("prefill chunk driver (32k prompt, one attention layer)")
        results["prefill_driver_32k"] = bench_pf_driver(lk)
        log(json.dumps(results["prefill_driver_32k"]))

    cpu = None
    if not args.skip_cpu:
        log("cpu baseline (float64 oracle, 1 thread; the whole C4 chunk also over all host threads)")
        cb = cpu_baseline(args.cpu_seconds, prefill=not args.skip_prefill, c5_samples=c5_samples,
                          c4_full_1t=args.cpu_c4_1thread)
        if "C5_accuracy" in cb:
            results["C5_prefill_131k"]["accuracy_vs_float64"] = cb.pop("C5_accuracy")
        results["cpu_float64"] = cb
        cpu = {"value": cb["C2"]["GBps"], "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"full C2 layer (32q/8kv/64, ctx 32768) float64 decode attention, "
                         f"{cb['C2']['reps']} repetitions, {cb['C2']['us_per_layer']:.0f} us/layer; "
                         f"host nproc {os.cpu_count()}; prefill CPU figures (sampled rows, "
                         f"extrapolated) under results.cpu_float64"}

    ach = c2["split_GBps"]
    traffic, traffic_note = split_traffic_from_profile()
    line = {
        "metric": "decode attn us/layer + HBM GB/s @32k/131k; prefill attn TOPS @4k/131k",
        "value": round(c2["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(c2["GBps"] / REF_3090TI_GBS_32K, 3),
        "dtype": "fp16",
        "data": "synthetic (seeded device generator, BASELINE configs C2-C5)",
        "config": {
            "workload": "C2: decode attention, ctx 32768, 32q/8kv/64, 10 layers with distinct "
                        "fp16 KV caches replayed as one hipGraph of 10 x (split, combine)",
            "seq": c2["seq"], "layers": c2["layers"], "us_per_layer": round(c2["us_per_layer"], 3),
            "split_cap": cfgp["split_cap"], "target_n": cfgp["target_n"], "split_min": cfgp["split_min"],
            "baseline": "reference on RTX 3090 Ti: 669.3 GB/s, 100.27 us/layer @32768",
        },
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_note,
                     "kernel": "lk_k_attn_split (C2, seq x 2048 B per launch)"},
        "cpu_baseline": cpu,
        "results": results,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
