#!/usr/bin/env python3
"""Benchmark of the quantized KV-cache path on one MI355X (BASELINE.json's metric).

Headline (`value`): the 101,600-context workload -- single-query decode attention at 101,600 context, preset F (K 5-bit
Hadamard-rotated, V 6-bit, 2,048-position q8 window; the reference's window rule puts 3,040 positions in the ring and
98,560 in the packed store), 16 layers x 4 kv heads x head_dim 256, 24 query heads.  One step = the 16 layers'
attention (16 attend calls, one per layer, as a decoder issues them, captured once as a HIP graph and replayed, as a
serving loop issues a decode step; every kernel of every call runs), inputs resident in HBM.  The same calls issued
one by one from Python are reported too (extra.cfg3.eager_*).
value = KV positions/s = 16 * 101,600 / step time.

Also measured (in "extra"): config 1 (q8, 4,096 positions), config 2 (append: 8 positions x 16 layers per step,
512 steps, us/step), config 4 (T = 8 verify at 38,000, q8), config 5 (4 paged sequences, preset F), and the fused
16-layer launch of config 3.  cpu_baseline: the oracle's restatement of the reference's split-K arithmetic
(kv_oracle.c) timed on the host cores over a bounded sample of config 3 (layer 0, all 4 kv heads).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4,5] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen38-megakernel_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HD, NKV, NH = 256, 4, 24
HBM_PEAK = 8.0e12
METRIC = "decode-attn KV positions/s & HBM GB/s (% of 8 TB/s) at 100k ctx; append µs/step"
BYTES = {8: 272, 4: 144, 5: 176, 6: 208, 7: 240}  # one row incl. its 8 fp16 scales


def kv_bytes(L, ws, kb, vb, ring):
    """Algorithmic bytes of one (layer, kv head) pass: packed rows below ws, q8 rows from ws on."""
    if not ring:
        ws = L
    return ws * (BYTES[kb] + BYTES[vb]) + (L - ws) * 2 * BYTES[8]


def gen_fill(torch, st, seq, L, nl, seed, outliers, chunk=4096):
    """Synthetic K/V ~ N(0,1) (fp16, generated on the GPU), K with 4 outlier channels per head x12, appended in chunks."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    scale = torch.ones(NKV, HD, device="cuda", dtype=torch.float16)
    if outliers:
        for h in range(NKV):
            ch = np.random.default_rng(1000 + h).choice(HD, 4, replace=False)
            scale[h, torch.from_numpy(ch).cuda()] = 12.0
    for p in range(0, L, chunk):
        c = min(chunk, L - p)
        k = torch.randn(c, nl, NKV, HD, device="cuda", dtype=torch.float16, generator=g) * scale
        v = torch.randn(c, nl, NKV, HD, device="cuda", dtype=torch.float16, generator=g)
        st.append(seq, 0, nl, p, c, k.data_ptr(), v.data_ptr(), 1)
    torch.cuda.synchronize()


def timed(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def graph_call_us(torch, fn, n, reps=5):
    """fn(stream) -- n library calls on that stream -- captured once as a HIP graph and replayed `reps` times:
    wall-clock µs per call (every kernel of every call runs; the graph removes the host's per-call cost)."""
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        fn(side.cuda_stream)  # warm on the capture stream
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            fn(torch.cuda.current_stream().cuda_stream)
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        graph.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / (reps * n) * 1e6


def profiled(torch, st, fn, steps):
    """`steps` calls of fn with the store's kernel timing on (after one untimed call); the event totals + wall time."""
    fn()
    torch.cuda.synchronize()
    st.profile(1)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / steps
    p = st.profile(0)
    p["step_s"] = t
    return p


def traffic_from_profiles(name):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary, if present."""
    p = os.path.join(ROOT, "profiles", name)
    try:
        with open(p) as f:
            d = json.load(f)
        return d.get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def rocprof_duration(name):
    """Mean launch duration (µs) of the dominant kernel in the committed rocprofv3 kernel trace, if present."""
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            return json.load(f).get("mean_us")
    except (OSError, ValueError):
        return None


def bench_cfg3(torch, qkv, steps, warmup, step_only=False):
    L, nl, win = 101600, 16, 2048
    st = qkv.KVStore("K*=5r,V*=6", win=win, n_layers=nl, ctx=L)
    gen_fill(torch, st, 0, L, nl, seed=3, outliers=True)
    ws = qkv.window_start(L, win)
    g = torch.Generator(device="cuda")
    g.manual_seed(33)
    q = torch.randn(nl, 1, 1, NH, HD, device="cuda", generator=g)
    out = torch.empty_like(q)
    qp, op = q.data_ptr(), out.data_ptr()
    lay = q[0].numel() * 4

    def step_layers():
        for l in range(nl):
            st.attend(l, 1, [0], [L], 1, qp + l * lay, op + l * lay)

    def step_fused():
        st.attend(0, nl, [0], [L], 1, qp, op)

    per_layer_bytes = NKV * kv_bytes(L, ws, 5, 6, True)
    # step times with profiling off; kernel durations from a second, profiled pass of the same calls (HIP events on the
    # launch stream around each attention / combine launch; warmup calls excluded)
    t_layers = timed(torch, step_layers, steps, warmup)
    prof = profiled(torch, st, step_layers, steps)
    calls = prof["calls"]
    attn_avg = prof["attn_ms"] / calls * 1e-3
    # the same 16 one-layer calls captured once as a HIP graph and replayed (how a serving loop issues a decode step's
    # launches; every kernel runs, the graph removes the host's launch cost and the gaps between launches)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        step_layers()  # warm (workspace sized, kernel attributes set)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for l in range(nl):
                st.attend(l, 1, [0], [L], 1, qp + l * lay, op + l * lay, stream=side.cuda_stream)
    t_graph = timed(torch, graph.replay, steps, warmup)
    if step_only:  # (the profiling run: only the headline's one-layer launches)
        return {"L": L, "ws": ws, "layers": nl, "step_s": t_graph, "positions_per_s": nl * L / t_graph,
                "gbps": nl * per_layer_bytes / t_graph / 1e9, "eager_step_s": t_layers, "attn_kernel_avg_s": attn_avg,
                "attn_kernel_bytes": per_layer_bytes, "attn_kernel_gbps": per_layer_bytes / attn_avg / 1e9,
                "combine_avg_s": prof["combine_ms"] / calls * 1e-3}
    t_fused = timed(torch, step_fused, steps, warmup)
    prof_f = profiled(torch, st, step_fused, steps)
    fused_attn_avg = prof_f["attn_ms"] / prof_f["calls"] * 1e-3
    # a decode slot per layer: store this step's K/V row (position L-1, rewritten every step so L stays fixed) and
    # attend -- as two calls (append, attend) and as one launch (mk_kv_append_attend)
    kn = torch.randn(nl, NKV, HD, device="cuda", dtype=torch.float16, generator=g)
    vn = torch.randn(nl, NKV, HD, device="cuda", dtype=torch.float16, generator=g)
    kp, vp, rl = kn.data_ptr(), vn.data_ptr(), NKV * HD * 2

    def slot_separate():
        for l in range(nl):
            st.append(0, l, 1, L - 1, 1, kp + l * rl, vp + l * rl, 1)
            st.attend(l, 1, [0], [L], 1, qp + l * lay, op + l * lay)

    def slot_fused():
        for l in range(nl):
            st.append_attend(l, 1, [0], [L], 1, kp + l * rl, vp + l * rl, 1, qp + l * lay, op + l * lay)

    t_slot_sep = timed(torch, slot_separate, steps, warmup)
    t_slot_fused = timed(torch, slot_fused, steps, warmup)
    # the slot with a stand-in for the layer's q/k/v projection before the attention (an fp16 GEMV of a 7,168 x 4,096
    # weight, 58.7 MB, one per layer), without and with mk_kv_prefetch of the layer's first tiles on a second stream
    # beside it; attention kernel times from the store's events
    wts = torch.randn(nl, 7168, 4096, device="cuda", dtype=torch.float16, generator=g)
    xin = torch.randn(4096, device="cuda", dtype=torch.float16, generator=g)
    side = torch.cuda.Stream()

    def slot_proj(prefetch):
        main = torch.cuda.current_stream()
        for l in range(nl):
            if prefetch:
                side.wait_stream(main)
                st.prefetch(l, 1, [0], [L], 1, 1, side.cuda_stream)
            torch.mv(wts[l], xin)
            if prefetch:
                main.wait_stream(side)
            st.attend(l, 1, [0], [L], 1, qp + l * lay, op + l * lay)

    proj = {}
    for pf in (False, True):
        t = timed(torch, lambda: slot_proj(pf), steps, warmup)
        pp = profiled(torch, st, lambda: slot_proj(pf), steps)
        proj["prefetch" if pf else "plain"] = {"step_s": t, "attn_kernel_avg_s": pp["attn_ms"] / pp["calls"] * 1e-3}
    del wts
    # speculative verify over the same store: T query tokens per call (T = 2, 4, 8 -> 12, 24, 48 query rows per kv head),
    # one-layer calls, us per layer
    spec = {}
    for T in (2, 4, 8):
        qs = torch.randn(nl, 1, T, NH, HD, device="cuda", generator=g)
        os_ = torch.empty_like(qs)
        lt = qs[0].numel() * 4

        def spec_step():
            for l in range(nl):
                st.attend(l, 1, [0], [L], T, qs.data_ptr() + l * lt, os_.data_ptr() + l * lt)

        spec[f"T{T}_us_per_layer"] = timed(torch, spec_step, steps, warmup) / nl * 1e6
        if T == 8:  # the other verify form on this packed store: one pass of the 8-wave kernel (k_verify)
            st.config("wide", 1)
            spec["T8_one_pass_us_per_layer"] = timed(torch, spec_step, steps, warmup) / nl * 1e6
            st.config("wide", 2)
    ok = bool(torch.isfinite(out).all().item())
    return {
        "L": L, "ws": ws, "ring_positions": L - ws, "layers": nl,
        # the headline step: the 16 one-layer calls replayed from one captured HIP graph (every kernel of every call
        # runs; the host's per-call launch cost is not in it), as config 2's us_per_step; eager_*: one library call
        # per layer from Python
        "step_s": t_graph, "positions_per_s": nl * L / t_graph, "gbps": nl * per_layer_bytes / t_graph / 1e9,
        "eager_step_s": t_layers, "eager_positions_per_s": nl * L / t_layers, "eager_gbps": nl * per_layer_bytes / t_layers / 1e9,
        "attn_kernel_avg_s": attn_avg, "attn_kernel_bytes": per_layer_bytes,
        "attn_kernel_gbps": per_layer_bytes / attn_avg / 1e9,
        "combine_avg_s": prof["combine_ms"] / calls * 1e-3, "profiled_step_s": prof["step_s"],
        "graph_step_s": t_graph, "graph_positions_per_s": nl * L / t_graph, "graph_gbps": nl * per_layer_bytes / t_graph / 1e9,
        "fused16_step_s": t_fused, "fused16_positions_per_s": nl * L / t_fused,
        "fused16_gbps": nl * per_layer_bytes / t_fused / 1e9, "fused16_attn_kernel_avg_s": fused_attn_avg,
        "fused16_attn_kernel_gbps": nl * per_layer_bytes / fused_attn_avg / 1e9,
        "slot_append_then_attend_step_s": t_slot_sep, "slot_append_attend_fused_step_s": t_slot_fused,
        "slot_after_projection": proj, "spec_verify": spec, "finite": ok,
    }


def bench_cfg1(torch, qkv, steps, warmup):
    L = 4096
    st = qkv.KVStore("", n_layers=1, ctx=L)
    gen_fill(torch, st, 0, L, 1, seed=0, outliers=False)
    q = torch.randn(1, 1, 1, NH, HD, device="cuda")
    out = torch.empty_like(q)
    fn = lambda: st.attend(0, 1, [0], [L], 1, q.data_ptr(), out.data_ptr())
    t = timed(torch, fn, steps * 5, warmup)
    prof = profiled(torch, st, fn, steps * 5)
    attn = prof["attn_ms"] / prof["calls"] * 1e-3
    comb = prof["combine_ms"] / prof["calls"] * 1e-3
    ncalls = 64
    tg = graph_call_us(torch, lambda stream: [st.attend(0, 1, [0], [L], 1, q.data_ptr(), out.data_ptr(), stream=stream)
                                              for _ in range(ncalls)], ncalls) * 1e-6
    b = NKV * L * 2 * BYTES[8]
    return {"L": L, "call_s": t, "positions_per_s": L / t, "gbps": b / t / 1e9,
            "graph_call_s": tg, "graph_positions_per_s": L / tg,
            "attn_kernel_avg_s": attn, "combine_avg_s": comb, "attn_kernel_gbps": b / attn / 1e9,
            "note": "call_s: one library call at a time from Python (the host's per-call cost included); graph_call_s: 64 "
                    "calls captured once as a HIP graph and replayed (the GPU's time per call, as a serving loop issues "
                    "them). 8.9 MB per call: resident in the 256 MB last-level cache across calls; the kernel times "
                    "come from a second pass with per-launch events, which lengthen short launches"}


def bench_cfg2(torch, qkv, nsteps=512):
    """512 append steps of 8 positions x 16 layers (one k_append launch each): eager (one library call per step, the
    host's launch rate included) and as one captured HIP graph of the 512 launches replayed (how a serving loop
    issues them; every kernel still runs)."""
    nl = 16
    st = qkv.KVStore("K*=5r,V*=6", win=2048, n_layers=nl, ctx=nsteps * 8)
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    k = torch.randn(nsteps, 8, nl, NKV, HD, device="cuda", dtype=torch.float16, generator=g)
    v = torch.randn(nsteps, 8, nl, NKV, HD, device="cuda", dtype=torch.float16, generator=g)
    for h in range(NKV):  # 4 outlier channels per kv head scaled x12 (the workload's K distribution)
        ch = torch.from_numpy(np.random.default_rng(1000 + h).choice(HD, 4, replace=False)).cuda()
        k[:, :, :, h, ch] *= 12.0
    kp, vp, stride = k.data_ptr(), v.data_ptr(), k[0].numel() * 2

    def run(stream=0):
        for s in range(nsteps):
            st.append(0, 0, nl, 8 * s, 8, kp + s * stride, vp + s * stride, 1, stream)

    run()  # warm
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run()
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / nsteps
    prof = profiled(torch, st, run, 1)

    graph_us = lambda fn: graph_call_us(torch, fn, nsteps)
    tg = graph_us(run) * 1e-6
    # the dispatch floor of one graph node (a one-element add), and the steps with cache-resident input rows
    one = torch.zeros(1, device="cuda")
    floor_us = graph_us(lambda stream: [one.add_(1) for _ in range(nsteps)])
    hot_us = graph_us(lambda stream: [st.append(0, 0, nl, 8 * s, 8, kp, vp, 1, stream) for s in range(nsteps)])
    return {"steps": nsteps, "us_per_step": tg * 1e6, "graph_us_per_step": tg * 1e6, "eager_us_per_step": t * 1e6,
            "kernel_us_per_step": prof["append_ms"] / nsteps * 1e3, "rows_per_step": 8 * nl * NKV * 2,
            "graph_node_floor_us": floor_us, "cache_resident_inputs_us_per_step": hot_us,
            "note": "us_per_step: the 512 steps captured once as a HIP graph and replayed (wall clock / 512); eager: one "
                    "library call per step from Python; kernel: per-launch events (which lengthen short launches)"}


def bench_cfg4(torch, qkv, steps, warmup):
    L, nl, T = 38000, 16, 8
    st = qkv.KVStore("", n_layers=nl, ctx=L)
    gen_fill(torch, st, 0, L, nl, seed=3, outliers=False)
    q = torch.randn(nl, 1, T, NH, HD, device="cuda")
    out = torch.empty_like(q)
    fn = lambda: st.attend(0, nl, [0], [L], T, q.data_ptr(), out.data_ptr())
    forms = {}
    for name, wide in (("k_verify", 1), ("two_batches", 0)):  # both verify forms, the same bits
        st.config("wide", wide)
        forms[name + "_us_per_layer"] = timed(torch, fn, steps, warmup) / nl * 1e6
    st.config("wide", 2)
    # the default form, timed after the others (the first timed calls of a run find the GPU's clocks still ramping)
    t = timed(torch, fn, steps, warmup)
    b = nl * NKV * L * 2 * BYTES[8]
    flops = nl * 2 * 2 * 48 * L * HD * NKV
    return {"L": L, "T": T, "layers": nl, "step_s": t, "us_per_layer": t / nl * 1e6, "gbps": b / t / 1e9,
            "tflops": flops / t / 1e12, "positions_per_s": nl * L / t, "forms": forms}


def bench_cfg5(torch, qkv, steps, warmup):
    lens, nl, page, win = [23000, 23000, 60000, 262144], 16, 256, 2048
    npg = [-(-L // page) for L in lens]
    st = qkv.KVStore("K*=5r,V*=6", win=win, n_layers=nl, n_seq=4, ctx=max(lens), page=page, n_pages=sum(npg))
    perm = np.random.default_rng(5).permutation(sum(npg))
    o = 0
    for s, L in enumerate(lens):
        st.set_pages(s, perm[o:o + npg[s]])
        o += npg[s]
        gen_fill(torch, st, s, L, nl, seed=50 + s, outliers=True)
    q = torch.randn(nl, 4, 1, NH, HD, device="cuda")
    out = torch.empty_like(q)
    t = timed(torch, lambda: st.attend(0, nl, [0, 1, 2, 3], lens, 1, q.data_ptr(), out.data_ptr()), steps, warmup)
    b = nl * NKV * sum(kv_bytes(L, qkv.window_start(L, win), 5, 6, True) for L in lens)
    return {"lens": lens, "layers": nl, "step_s": t, "gbps": b / t / 1e9, "positions_per_s": nl * sum(lens) / t,
            "bytes_per_step": b}


def bench_prefill(torch, qkv, steps, warmup):
    """Prefill of a 16,384-position prompt in one call (640-bucket pieces inside) over 4 preset-F layers: K/V store +
    causal attention.  FLOPs counted as the causal S and P V products (4 * 256 per visible (row, key) pair)."""
    P, nl, win = 16384, 4, 2048
    st = qkv.KVStore("K*=5r,V*=6", win=win, n_layers=nl, ctx=P)
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    k = torch.randn(P, nl, NKV, HD, device="cuda", dtype=torch.float16, generator=g)
    v = torch.randn(P, nl, NKV, HD, device="cuda", dtype=torch.float16, generator=g)
    q = torch.randn(nl, P, NH, HD, device="cuda", generator=g)
    out = torch.empty_like(q)

    def step():
        st.rewind(0, 0)
        st.prefill(0, 0, nl, 0, P, k.data_ptr(), v.data_ptr(), 1, q.data_ptr(), out.data_ptr())

    t = timed(torch, step, steps, warmup)
    pairs = NH * P * (P + 1) / 2  # visible (query row, key) pairs per layer
    flops = nl * 4 * HD * pairs
    return {"prompt": P, "layers": nl, "step_s": t, "tokens_per_s": P / t, "ms_per_layer": t / nl * 1e3,
            "attn_tflops": flops / t / 1e12, "finite": bool(torch.isfinite(out).all().item())}


def host_threads():
    """Host threads for the CPU baseline: every CPU this process may run on (its affinity mask), capped by the
    box's CPU share when OMP_NUM_THREADS states one (16 per GPU on the GPU boxes), and by the oracle's 64."""
    n = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, min(64, n))


def cpu_baseline(qkv, seconds=10.0):
    """The oracle (kv_oracle.c, the reference's split-K arithmetic restated in C) on host cores: layer 0 of config 3
    (101,600 positions, 4 kv heads, 24 query heads, T = 1) on dequantized operands, repeated for ~`seconds`."""
    from oracle import oracle as o
    if not os.path.exists(o.LIB):
        from oracle import build
        build.build()
    threads = host_threads()
    L, win = 101600, 2048
    ws = qkv.window_start(L, win)
    rng = np.random.default_rng(3)
    Kd = np.zeros((NKV, L, HD), np.float32)
    Vd = np.zeros((NKV, L, HD), np.float32)
    for g in range(NKV):
        k = rng.standard_normal((L, HD)).astype(np.float32)
        k[:, np.random.default_rng(1000 + g).choice(HD, 4, replace=False)] *= 12
        v = rng.standard_normal((L, HD)).astype(np.float32)
        for X, D, bits, rot in ((k, Kd, 5, 1), (v, Vd, 6, 0)):
            mq, ms, rq, rs = o.store_rows(X, rot, bits, ring=True, threads=threads)
            D[g, :ws] = o.dequant_rows(mq[:ws], ms[:ws], bits)
            D[g, ws:] = o.dequant_rows(rq[ws:], rs[ws:], 8)
    q = np.stack([np.stack([o.q_prep(x, 1) for x in rng.standard_normal((6, HD)).astype(np.float32)]) for _ in range(NKV)])
    n, t0 = 0, time.perf_counter()
    while True:
        o.attn_heads(q, Kd, Vd, 1, threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": L * n / el, "unit": "KV positions/s", "cores": threads, "kind": "port",
            "host_cpus": len(os.sched_getaffinity(0)), "cpu_share": os.environ.get("OMP_NUM_THREADS"),
            "sample": f"layer 0 of config 3 (101,600 positions, ws {ws}, 4 kv heads x 6 query rows, T=1) on dequantized "
                      f"fp16-valued operands, {n} repetitions in {el:.1f} s with {threads} threads (kv_oracle.c)"}


def cpu_extras(seconds=3.0):
    """The oracle on host cores for config 1 (q8 attention over 4,096 positions, 4 kv heads x 6 rows) and config 2
    (one append step: 16 layers x 4 kv heads x 8 positions x K/V rows, FWHT on K, K 5-bit + V 6-bit + q8 ring copies)."""
    from oracle import oracle as o
    threads = host_threads()
    rng = np.random.default_rng(0)
    L = 4096
    K = np.stack([o.dequant_rows(*o.store_rows(rng.standard_normal((L, HD)).astype(np.float32), 0, 8, ring=False)[:2], 8)
                  for _ in range(NKV)])
    V = np.stack([o.dequant_rows(*o.store_rows(rng.standard_normal((L, HD)).astype(np.float32), 0, 8, ring=False)[:2], 8)
                  for _ in range(NKV)])
    q = np.stack([np.stack([o.q_prep(x, 0) for x in rng.standard_normal((6, HD)).astype(np.float32)]) for _ in range(NKV)])
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        o.attn_heads(q, K, V, 1, threads)
        n += 1
    c1 = L * n / (time.perf_counter() - t0)
    rows = rng.standard_normal((16 * NKV * 8, HD)).astype(np.float32)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        o.store_rows(rows, 1, 5, ring=True, threads=threads)
        o.store_rows(rows, 0, 6, ring=True, threads=threads)
        n += 1
    us = (time.perf_counter() - t0) / n * 1e6
    return {"cfg1_attention": {"value": c1, "unit": "KV positions/s", "cores": threads, "kind": "port"},
            "cfg2_append": {"value": us, "unit": "us/step", "cores": threads, "kind": "port",
                            "sample": "512 K rows (FWHT, 5-bit) + 512 V rows (6-bit), each with its q8 ring copy"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="1,2,3,4,5,6")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--step-only", action="store_true",
                    help="config 3: only the headline step's one-layer calls (eager, event-timed, graph), for profiling")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (the byte-counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the KV path would shard by kv head / sequence / context; "
              "no multi-GPU path is built); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 5}))
        return
    import qkv
    cfgs = {int(c) for c in args.configs.split(",") if c}
    extra = {}
    if 3 in cfgs:
        extra["cfg3"] = bench_cfg3(torch, qkv, args.steps, args.warmup, args.step_only)
    if 1 in cfgs:
        extra["cfg1"] = bench_cfg1(torch, qkv, args.steps, args.warmup)
    if 2 in cfgs:
        extra["cfg2_append"] = bench_cfg2(torch, qkv)
    if 4 in cfgs:
        extra["cfg4"] = bench_cfg4(torch, qkv, args.steps, args.warmup)
    if 5 in cfgs:
        extra["cfg5"] = bench_cfg5(torch, qkv, args.steps, args.warmup)
    if 6 in cfgs:
        extra["prefill"] = bench_prefill(torch, qkv, min(args.steps, 3), min(args.warmup, 1))
    c3 = extra.get("cfg3")
    cpu = None if args.no_cpu or 3 not in cfgs else cpu_baseline(qkv, args.cpu_seconds)
    if cpu:
        cpu["other_configs"] = cpu_extras()
    roof = None
    if c3:
        ach = c3["attn_kernel_gbps"] * 1e9
        roof = {"bound": "hbm", "achieved": ach / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": ach / HBM_PEAK,
                "traffic": traffic_from_profiles("attn_cfg3_traffic.json"),
                "kernel": "k_attn<1,5,6> (one layer, 4 kv heads, 101,600 positions)",
                "algorithmic_bytes_per_launch": c3["attn_kernel_bytes"],
                "clock": "mean launch duration from the dispatch timestamps (HIP events recorded by hipExtLaunchKernelGGL "
                         "at the kernel's own start and end, on its launch stream) over a profiled pass of the step's "
                         "one-layer calls, without rocprofv3; profiles/attn_cfg3.md holds the rocprofv3 kernel trace of "
                         "the same calls (bench.py --configs 3 --no-cpu --step-only)",
                "duration_us": c3["attn_kernel_avg_s"] * 1e6}
        tr = rocprof_duration("attn_cfg3_duration.json")
        if tr:
            roof["rocprof_mean_us"] = tr
            roof["frac_rocprof"] = c3["attn_kernel_bytes"] / (tr * 1e-6) / HBM_PEAK
    line = {
        "metric": METRIC,
        "value": c3["positions_per_s"] if c3 else None,
        "unit": "KV positions/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": c3["step_s"] * 1e3 if c3 else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8 codes -> f16 mfma, f32 softmax",
        "data": "synthetic (seeded N(0,1) K/V with 4 outlier K channels per head x12; N(0,1) Q)",
        "config": {"workload": "cfg3: preset F (K5r/V6, win 2048) decode attention, L=101,600, 16 layers, T=1",
                   "layers": 16, "context": 101600, "kv_heads": 4, "q_heads": 24, "head_dim": 256,
                   "parallelism": "single GPU"},
        "step_note": "one decode step = the 16 one-layer mk_kv_attend calls at L = 101,600, captured once as a HIP graph "
                     "and replayed (every attention and combine kernel runs; the context length is the one fixed at "
                     "capture, so a decoder whose L grows recaptures or updates the kernel nodes); the same calls issued "
                     "eagerly from Python: extra.cfg3.eager_step_s",
        "gbps": c3["gbps"] if c3 else None,
        "hbm_frac": c3["gbps"] * 1e9 / HBM_PEAK if c3 else None,
        "append_us_per_step": extra.get("cfg2_append", {}).get("us_per_step"),
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
