#!/usr/bin/env python3
"""Benchmark of the GQA attention hot path on one MI355X.

Headline (one JSON line on stdout): fused decode step -- RoPE of q and the new
k, KV append, split-K attention -- of one layer of the BitNet b1.58 2B shape
(20 q heads, 5 kv heads, d=128) at position 4095 (4096 attended rows), in
GB/s of algorithmic bytes (5120*L + 30720 per step).  Inputs are resident in
HBM; 32 layer caches (671 MB) are used round-robin so the 256 MB
Infinity Cache cannot hold the working set.

Secondary (same line, key "prefill"): causal prefill of 2048 tokens of one
layer, in TFLOP/s of causal algorithmic FLOPs (4*d*Hq*N(N+1)/2), against the
FP32 matrix-core peak.

cpu_baseline: the oracle (C restatement of the reference's CPU path:
rope_embed -> store_kv -> masked_attention with AVX2/FMA, heads across
threads) timed on a bounded sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HQ, HKV, D, THETA = 20, 5, 128, 500000.0
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E
FP32_MATRIX_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix
METRIC = "GQA decode attn GB/s (% HBM peak) @4096 ctx; causal prefill attn TFLOP/s"


def decode_bytes(L: int) -> int:
    """K and V over L rows (5120 B per row at 5 kv heads x 128 x 2 x 4 B), plus
    q in, out, new k/v in and the appended cache row (30720 B)."""
    return 5120 * L + 30720


def prefill_flops(n: int) -> int:
    """QK^T and PV over causal pairs only, 2 FLOP per FMA."""
    return 4 * D * HQ * n * (n + 1) // 2


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def per_launch_ms(torch, launch, n: int) -> float:
    """Mean GPU duration of one launch, from an event pair around each launch.
    A spin kernel first holds the queue so that every launch is enqueued
    before the GPU reaches it (no host gaps inside a pair)."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)]
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2e8))
    for i in range(n):
        evs[i][0].record()
        launch(i)
        evs[i][1].record()
    torch.cuda.synchronize()
    ds = sorted(a.elapsed_time(b) for a, b in evs)
    return sum(ds) / len(ds)


def bench_decode(torch, be, steps: int, warmup: int, n_layers: int = 32, eager: bool = False,
                 reps: int = 100):
    L, pos, cap = 4096, 4095, 4096
    g = torch.Generator(device="cuda").manual_seed(0xB17E7020)
    kc = torch.randn(n_layers, HKV, cap, D, device="cuda", generator=g)
    vc = torch.randn(n_layers, HKV, cap, D, device="cuda", generator=g)
    q = torch.randn(n_layers, HQ * D, device="cuda", generator=g) * 4.0
    k = torch.randn(n_layers, HKV * D, device="cuda", generator=g)
    v = torch.randn(n_layers, HKV * D, device="cuda", generator=g)
    out = torch.zeros(n_layers, HQ * D, device="cuda")

    def step(i):
        r = i % n_layers
        be.dev_decode_step(q[r], k[r], v[r], pos, HQ, HKV, D, THETA, kc[r], vc[r], cap, out[r])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()

    # Timed region: K steps captured in one HIP graph (removes host launch
    # overhead; the GPU still runs K separate kernels), replayed `reps` times;
    # each replay is bracketed by device synchronisations and the median
    # replay gives the per-step time.
    graph = None
    try:
        if eager:
            raise RuntimeError("eager timing requested")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(3):
                step(i)
        torch.cuda.current_stream().wait_stream(side)
        graph = capture(torch, step, steps)
        graph.replay()
        torch.cuda.synchronize()
    except Exception as e:  # capture unsupported: time eager launches
        log(f"graph capture failed ({e}); timing eager launches")
        graph = None
    if graph is not None:
        st = replay_stats(torch, graph, steps, reps=reps)
    else:
        per = []
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        for _ in range(reps):
            torch.cuda.synchronize()
            t0.record()
            for i in range(steps):
                step(i)
            t1.record()
            torch.cuda.synchronize()
            per.append(t0.elapsed_time(t1) / steps)
        per.sort()
        st = {"median": per[len(per) // 2], "min": per[0], "p90": per[(9 * len(per)) // 10],
              "replays": reps}
    ms_step = st["median"]
    # Event pairs around eager launches (spin-held queue), beside the graph.
    pair_ms = per_launch_ms(torch, step, min(steps, 200))
    floor = stream_floor(torch, be, kc, vc, steps)
    nbytes = decode_bytes(L)
    res = {
        "ms_per_step": ms_step,
        "stats": st,
        "gbs": nbytes / (ms_step * 1e-3) / 1e9,
        "pair_ms": pair_ms,
        "bytes_per_step": nbytes,
        "floor": floor,
        "graph": graph is not None,
        # layer 0's inputs and the output of its last timed step, for the
        # parity stamp (the appended row 4095 holds the rotated k, which the
        # reference's store_kv writes there too)
        "host": {"q": q[0].cpu().numpy(), "k": k[0].cpu().numpy(), "v": v[0].cpu().numpy(),
                 "k_cache": kc[0].cpu().numpy(), "v_cache": vc[0].cpu().numpy(),
                 "out": out[0].cpu().numpy()},
    }
    del graph, kc, vc
    torch.cuda.empty_cache()
    return res


# Shapes of the streaming floor: (threads per workgroup, 16-byte loads in
# flight per lane, non-temporal).  (512, 1, False) is the plain one-load
# kernel (bnr_dev_stream_read's shape).
STREAM_SHAPES = [(512, 1, False), (256, 4, False), (256, 8, False), (256, 16, False),
                 (512, 4, False), (512, 8, False), (1024, 2, False), (1024, 4, False),
                 (256, 8, True), (512, 4, True), (1024, 4, True)]


def stream_floor(torch, be, kc, vc, steps: int, nbytes: int | None = None, reps: int = 50) -> dict:
    """Streaming reads of the same rotated K and V caches (one layer's K and
    V per launch, the layers round-robin as in the decode timing; or, with
    nbytes, the first nbytes/2 of all the K and of all the V caches), timed
    the same way as the decode (median of `reps` graph replays), in every
    shape of STREAM_SHAPES: the fastest is what one launch of that many
    bytes can reach on this part."""
    n_layers = kc.shape[0]
    if nbytes is not None:
        half = nbytes // 2 // 16 * 4  # floats, whole 16-byte words
        ka, va = kc.reshape(-1)[:half], vc.reshape(-1)[:half]
    res = {}
    for threads, loads, nt in STREAM_SHAPES:
        if nbytes is None:
            def read(i):
                r = i % n_layers
                be.dev_stream_read_shape(kc[r], vc[r], threads, loads, nt)
        else:
            def read(i):
                be.dev_stream_read_shape(ka, va, threads, loads, nt)
        for i in range(8):
            read(i)
        torch.cuda.synchronize()
        graph = capture(torch, read, steps)
        res[f"{threads}x{loads}{'nt' if nt else ''}"] = replay_stats(torch, graph, steps, reps=reps)["median"]
        del graph
    best = min(res, key=res.get)
    return {"ms": res[best], "shape": best, "plain_ms": res["512x1"],
            "shapes_us": {k: round(v * 1e3, 3) for k, v in res.items()}}


def bench_trait_path(be, steps: int = 300, pos_end: int = 4095):
    """The path an unchanged bitnet-inference drives (bitnet-model/src/lib.rs:
    1004-1036): per token and layer, Backend::rope_embed on host q/k slices,
    store_kv into the host KVCache, Backend::masked_attention over the host
    caches -- here through the C ABI's host-slice entry points, timed at
    positions pos_end-steps+1 .. pos_end after 10 untimed ones (the HBM
    mirror takes one new row per call).
    Also one rms_norm and one sqrelu_gate host call of the 2B shape."""
    import numpy as np

    rng = np.random.default_rng(0xB17E7090)
    cap = 4096
    kc = rng.standard_normal((HKV, cap, D), dtype=np.float32)
    vc = rng.standard_normal((HKV, cap, D), dtype=np.float32)
    q0 = rng.standard_normal(HQ * D, dtype=np.float32)
    k0 = rng.standard_normal(HKV * D, dtype=np.float32)
    v0 = rng.standard_normal(HKV * D, dtype=np.float32)
    out = np.zeros(HQ * D, np.float32)
    kcf, vcf = kc.reshape(-1), vc.reshape(-1)
    warm = 10
    p0 = pos_end - steps + 1
    be.mirror_invalidate()
    # first call syncs the mirror (rows 0..p0-warm-1 uploaded once), then
    # `warm` positions untimed (first-use staging allocations)
    q, k = q0.copy(), k0.copy()
    be.rope_embed(q, k, p0 - warm - 1, D, HQ, HKV, THETA)
    be.masked_attention(q, kcf, vcf, out, HQ, HKV, D, p0 - warm - 1)
    t_rope = t_attn = 0.0
    # The library is an FFI boundary (the reference's caller is Rust): Python's
    # cyclic garbage collector, whose full passes take tens of ms in a process
    # holding torch, stays off while the calls are timed.
    gc.collect()
    gc.disable()
    for pos in range(p0 - warm, pos_end + 1):
        q, k = q0.copy(), k0.copy()
        t0 = time.perf_counter()
        be.rope_embed(q, k, pos, D, HQ, HKV, THETA)
        t1 = time.perf_counter()
        kc[:, pos] = k.reshape(HKV, D)
        vc[:, pos] = v0.reshape(HKV, D)
        t2 = time.perf_counter()
        be.masked_attention(q, kcf, vcf, out, HQ, HKV, D, pos)
        t3 = time.perf_counter()
        if pos >= p0:
            t_rope += t1 - t0
            t_attn += t3 - t2
    gc.enable()
    hidden, ffn = 2560, 6912
    x = rng.standard_normal(hidden, dtype=np.float32)
    g = rng.uniform(0.8, 1.2, hidden).astype(np.float32)
    y = np.zeros(hidden, np.float32)
    gate = rng.standard_normal(ffn, dtype=np.float32)
    up = rng.standard_normal(ffn, dtype=np.float32)
    inner = np.zeros(ffn, np.float32)
    n_glue = 200
    for _ in range(5):
        be.rms_norm(x, g, 1e-5, y)
        be.sqrelu_gate(gate, up, inner)
    gc.collect()
    gc.disable()
    t0 = time.perf_counter()
    for _ in range(n_glue):
        be.rms_norm(x, g, 1e-5, y)
    t1 = time.perf_counter()
    for _ in range(n_glue):
        be.sqrelu_gate(gate, up, inner)
    t2 = time.perf_counter()
    gc.enable()
    return {"rope_us": t_rope / steps * 1e6, "attn_us": t_attn / steps * 1e6,
            "token_layer_us": (t_rope + t_attn) / steps * 1e6, "steps": steps,
            "rms_norm_us": (t1 - t0) / n_glue * 1e6, "sqrelu_gate_us": (t2 - t1) / n_glue * 1e6}


def trait_timer(steps: int = 300, pos_end: int = 4095):
    """The host-slice trait path driven from a compiled caller
    (bitnetrs_amd/trait_timer, built with the library): what the reference's
    Rust decode loop would pay per call through an extern "C" block, with no
    Python between the calls.  None if the program is not built."""
    exe = os.path.join(ROOT, "bitnetrs_amd", "trait_timer")
    if not os.path.exists(exe):
        log("trait_timer is not built; the trait path is timed from Python only")
        return None
    res = subprocess.run([exe, str(steps), str(pos_end)], capture_output=True, text=True,
                         timeout=300)
    if res.returncode != 0:
        raise RuntimeError(f"trait_timer failed ({res.returncode}): {res.stderr.strip()}")
    return json.loads(res.stdout.strip().splitlines()[-1])


def replay_stats(torch, graph, steps: int, reps: int = 100, restore=None, warm: int = 3) -> dict:
    """Per-launch time of a HIP graph of `steps` launches: `warm` untimed
    replays (a short graph's first replays after the host-side setup run
    below the part's steady clock), then `reps` timed replays, each
    bracketed by device synchronisations and preceded by `restore()`
    (untimed) when given.  Returns the median, minimum and 90th percentile
    over the replays of (replay time / steps), in ms."""
    for _ in range(warm):
        if restore is not None:
            restore()
        graph.replay()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    per = []
    for _ in range(reps):
        if restore is not None:
            restore()
        torch.cuda.synchronize()
        t0.record()
        graph.replay()
        t1.record()
        torch.cuda.synchronize()
        per.append(t0.elapsed_time(t1) / steps)
    per.sort()
    return {"median": per[len(per) // 2] if len(per) % 2 else 0.5 * (per[len(per) // 2 - 1]
                                                                       + per[len(per) // 2]),
            "min": per[0], "p90": per[min(len(per) - 1, (9 * len(per)) // 10)], "replays": reps}


def capture(torch, launch, steps: int):
    """`steps` launches captured in one HIP graph."""
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            launch(i)
    return graph


def graph_ms(torch, launch, steps: int, reps: int = 50, restore=None, warm: int = 3) -> float:
    """Median per-launch time of `steps` launches captured in one HIP graph
    over `reps` timed replays (replay_stats)."""
    graph = capture(torch, launch, steps)
    st = replay_stats(torch, graph, steps, reps=reps, restore=restore, warm=warm)
    del graph
    return st["median"]


def bench_decode_contexts(torch, be, contexts, steps: int = 200):
    """Single-sequence fused decode step of the 2B shape at other context
    lengths: graph-timed over enough rotated layer caches (>= 700 MB in
    total, at least 8) that the 256 MB MALL cannot hold them."""
    res = {}
    for L in contexts:
        pos, cap = L - 1, L
        n_layers = max(8, min(64, 700_000_000 // (5120 * L)))
        g = torch.Generator(device="cuda").manual_seed(0xB17E7021)
        kc = torch.randn(n_layers, HKV, cap, D, device="cuda", generator=g)
        vc = torch.randn(n_layers, HKV, cap, D, device="cuda", generator=g)
        q = torch.randn(n_layers, HQ * D, device="cuda", generator=g) * 4.0
        k = torch.randn(n_layers, HKV * D, device="cuda", generator=g)
        v = torch.randn(n_layers, HKV * D, device="cuda", generator=g)
        out = torch.zeros(n_layers, HQ * D, device="cuda")

        def step(i):
            r = i % n_layers
            be.dev_decode_step(q[r], k[r], v[r], pos, HQ, HKV, D, THETA, kc[r], vc[r], cap,
                               out[r])

        for i in range(2 * n_layers):
            step(i)
        torch.cuda.synchronize()
        ms = graph_ms(torch, step, steps)
        res[L] = {"us_per_step": round(ms * 1e3, 3),
                  "gbs": round(decode_bytes(L) / (ms * 1e-3) / 1e9, 1),
                  "frac_hbm": round(decode_bytes(L) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"decode L={L}: {ms * 1e3:.2f} us/step, {res[L]['gbs']:.0f} GB/s")
        del kc, vc
        torch.cuda.empty_cache()
    return res


def bench_prefill_shapes(torch, be, shapes, steps: int = 10):
    """Prefill attention (dev_prefill_attention) at other (tokens, cached
    rows) shapes, graph-timed over 4 rotated layers."""
    res = {}
    for n, sp in shapes:
        cap, nl = n + sp, 4
        g = torch.Generator(device="cuda").manual_seed(0xB17E7031)
        q = torch.randn(nl, n, HQ * D, device="cuda", generator=g)
        kc = torch.randn(nl, HKV, cap, D, device="cuda", generator=g)
        vc = torch.randn(nl, HKV, cap, D, device="cuda", generator=g)
        out = torch.zeros(nl, n, HQ * D, device="cuda")

        def attn(i):
            r = i % nl
            be.dev_prefill_attention(q[r], kc[r], vc[r], cap, out[r], n, sp, HQ, HKV, D)

        for i in range(2 * nl):
            attn(i)
        torch.cuda.synchronize()
        ms = graph_ms(torch, attn, max(steps, nl))
        flops = 4 * D * HQ * (n * sp + n * (n + 1) / 2)
        key = f"{n}@{sp}"
        res[key] = {"us": round(ms * 1e3, 2), "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                    "frac_fp32_matrix_peak": round(flops / (ms * 1e-3) / 1e12
                                                   / FP32_MATRIX_PEAK_TFLOPS, 4)}
        log(f"prefill attention {n} tokens after {sp}: {ms * 1e3:.1f} us, "
            f"{res[key]['tflops']:.1f} TFLOP/s")
        del q, kc, vc, out
        torch.cuda.empty_cache()
    return res


def bench_prefill(torch, be, steps: int, warmup: int, n: int = 2048):
    """2048-token causal prefill of one layer: RoPE + append + attention
    (dev_prefill) and attention alone, each as a HIP graph of one launch per
    layer over `steps` layers (q and k restored before every replay,
    untimed), like the decode; the attention kernel's event-pair duration of
    eager launches beside it."""
    n_layers = steps
    cap = n
    g = torch.Generator(device="cuda").manual_seed(0xB17E7030)
    q0 = torch.randn(n_layers, n, HQ * D, device="cuda", generator=g)
    k0 = torch.randn(n_layers, n, HKV * D, device="cuda", generator=g)
    v = torch.randn(n_layers, n, HKV * D, device="cuda", generator=g)
    q, k = q0.clone(), k0.clone()
    kc = torch.zeros(n_layers, HKV, cap, D, device="cuda")
    vc = torch.zeros_like(kc)
    out = torch.zeros(n_layers, n, HQ * D, device="cuda")

    def step(i):
        r = i % n_layers
        be.dev_prefill(q[r], k[r], v[r], n, 0, HQ, HKV, D, THETA, kc[r], vc[r], cap, out[r])

    def restore():
        q.copy_(q0)
        k.copy_(k0)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ms_step = graph_ms(torch, step, steps, restore=restore)

    def attn_only(i):
        r = i % n_layers
        be.dev_prefill_attention(q[r], kc[r], vc[r], cap, out[r], n, 0, HQ, HKV, D)

    attn_ms = graph_ms(torch, attn_only, steps)
    pair_ms = per_launch_ms(torch, attn_only, max(steps, 3))
    torch.cuda.synchronize()
    flops = prefill_flops(n)
    # layer 0's raw inputs and the output of its last timed launch (parity)
    host = {"q": q0[0].cpu().numpy(), "k": k0[0].cpu().numpy(), "v": v[0].cpu().numpy(),
            "out": out[0].cpu().numpy()}
    return {"ms_per_step": ms_step, "tflops": flops / (ms_step * 1e-3) / 1e12,
            "attn_ms": attn_ms, "attn_tflops": flops / (attn_ms * 1e-3) / 1e12,
            "pair_ms": pair_ms, "flops": flops, "host": host}


def bench_stack(torch, be, n_layers: int = 30, n_pre: int = 1024, n_dec: int = 256,
                dec_reps: int = 20):
    """The 30-layer stack at the 2B shape: 1024-token causal prefill of every
    layer, then 256 decode steps (every layer each step), seeded N(0,1)
    projections per layer and step.  The prefill is timed as one HIP graph
    of the 30 layers' launches after one untimed warm-up prefill; decode as
    one HIP graph of all n_layers * n_dec fused decode launches."""
    import bitnetrs_amd

    g = torch.Generator(device="cuda").manual_seed(0xB17E7050)
    qp = torch.randn(n_layers, n_pre, HQ * D, device="cuda", generator=g)
    kp = torch.randn(n_layers, n_pre, HKV * D, device="cuda", generator=g)
    vp = torch.randn(n_layers, n_pre, HKV * D, device="cuda", generator=g)
    qd = torch.randn(n_dec, n_layers, HQ * D, device="cuda", generator=g)
    kd = torch.randn(n_dec, n_layers, HKV * D, device="cuda", generator=g)
    vd = torch.randn(n_dec, n_layers, HKV * D, device="cuda", generator=g)
    out_p = torch.zeros_like(qp)
    out_d = torch.zeros_like(qd)
    st = bitnetrs_amd.AttentionStack(be, n_layers, HQ, HKV, D, n_pre + n_dec, THETA)
    # Untimed warm-up prefill on copies (q and k are rotated in place): the
    # first call builds the RoPE table and sizes the prefill workspace.  Then
    # the 30 layers' prefill (RoPE + append + attention per layer) as one
    # HIP graph, replayed from restored q and k (restore untimed).
    q_in, k_in = qp.clone(), kp.clone()
    st.prefill(q_in.clone(), k_in.clone(), vp, out_p)
    st.cache.clear()
    torch.cuda.synchronize()
    pre_ms = graph_ms(torch, lambda i: st.prefill(qp, kp, vp, out_p), 1,
                      restore=lambda: (qp.copy_(q_in), kp.copy_(k_in)))
    start = st.position
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # one eager step on a side stream before capture
        st.decode(qd[0], kd[0], vd[0], out_d[0])
    torch.cuda.current_stream().wait_stream(side)
    st.cache.filled_positions = start
    st.cache.layer_lengths = [start] * n_layers
    with torch.cuda.graph(graph):
        for s in range(n_dec):
            st.decode(qd[s], kd[s], vd[s], out_d[s])
    graph.replay()  # first replay writes the cache rows; replays are idempotent
    torch.cuda.synchronize()
    dec_ms = replay_stats(torch, graph, 1, reps=dec_reps, warm=1)["median"]
    dec_bytes = n_layers * sum(decode_bytes(n_pre + s + 1) for s in range(n_dec))
    pre_flops = n_layers * prefill_flops(n_pre)
    # layer 0's raw inputs (prefill then decode tokens) and the outputs of
    # its last timed launches (parity)
    host = {"q": torch.cat([q_in[0], qd[:, 0]]).cpu().numpy(),
            "k": torch.cat([k_in[0], kd[:, 0]]).cpu().numpy(),
            "v": torch.cat([vp[0], vd[:, 0]]).cpu().numpy(),
            "out": torch.cat([out_p[0], out_d[:, 0]]).cpu().numpy()}
    return {"prefill_ms": pre_ms, "prefill_tflops": pre_flops / (pre_ms * 1e-3) / 1e12,
            "decode_ms": dec_ms, "decode_gbs": dec_bytes / (dec_ms * 1e-3) / 1e9,
            "decode_tok_s": n_dec / (dec_ms * 1e-3), "decode_bytes": dec_bytes,
            "prefill_flops": pre_flops, "launches": n_layers * n_dec, "host": host,
            "decode_replays": dec_reps}


def bench_batched(torch, be, steps: int = 50, n_seq: int = 32, cap: int = 4096, reps: int = 50):
    """32 independent sequences, cached lengths ~ U[128, 4096) (seeded), one
    fused decode step each per launch (ragged split-K)."""
    import numpy as np

    lens = np.random.default_rng(0xB17E7040).integers(128, 4096, size=n_seq).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(0xB17E7041)
    kc = torch.randn(n_seq, HKV, cap, D, device="cuda", generator=g)
    vc = torch.randn(n_seq, HKV, cap, D, device="cuda", generator=g)
    q = torch.randn(n_seq, HQ * D, device="cuda", generator=g)
    k = torch.randn(n_seq, HKV * D, device="cuda", generator=g)
    v = torch.randn(n_seq, HKV * D, device="cuda", generator=g)
    out = torch.zeros(n_seq, HQ * D, device="cuda")

    def step(i):
        be.dev_decode_step_batched(q, k, v, lens, HQ, HKV, D, THETA, kc, vc, cap, out)

    for i in range(5):
        step(i)
    torch.cuda.synchronize()
    graph = capture(torch, step, steps)
    graph.replay()
    torch.cuda.synchronize()
    ms = replay_stats(torch, graph, steps, reps=reps)["median"]
    del graph
    nbytes = int(sum(decode_bytes(int(L) + 1) for L in lens))
    floor = stream_floor(torch, be, kc, vc, steps, nbytes=nbytes)
    # inputs and the outputs of the last timed launch, for the parity stamp:
    # each sequence's rows 0..len-1 (row len is the appended one)
    host = {"lens": lens, "q": q.cpu().numpy(), "k": k.cpu().numpy(), "v": v.cpu().numpy(),
            "k_cache": [kc[b, :, :int(L)].cpu().numpy() for b, L in enumerate(lens)],
            "v_cache": [vc[b, :, :int(L)].cpu().numpy() for b, L in enumerate(lens)],
            "out": out.cpu().numpy()}
    del kc, vc
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes,
            "floor": floor, "host": host,
            "lengths_min_max_mean": [int(lens.min()), int(lens.max()), float(lens.mean())]}


# The seven ternary projections of one BitNet b1.58 2B layer for one token:
# (out_features, in_features) of q, k, v, o, gate, up, down.
GEMV_SHAPES = [(2560, 2560), (640, 2560), (640, 2560), (2560, 2560), (6912, 2560),
               (6912, 2560), (2560, 6912)]


def gemv_bytes(m: int, k: int) -> int:
    """Packed weights (ceil(k/4) bytes per row) + int8 activations + f32 outputs."""
    return m * ((k + 3) // 4) + k + 4 * m


def bench_gemv(torch, be, steps: int = 20, n_layers: int = 30):
    """W2A8 ternary GEMV: the 7 projections of every layer for one decode
    token (30 layers x 17.4 MB of packed weights = 522 MB, more than the
    256 MB MALL), one HIP graph of 210 launches per token.  Weights are
    random bytes (every 2-bit code, 0b11 included), activations random int8."""
    g = torch.Generator(device="cuda").manual_seed(0xB17E7060)
    ws = [[torch.randint(0, 256, (m * ((k + 3) // 4),), dtype=torch.uint8, device="cuda",
                         generator=g) for (m, k) in GEMV_SHAPES] for _ in range(n_layers)]
    acts = [torch.randint(-128, 128, (k,), dtype=torch.int8, device="cuda", generator=g)
            for (_, k) in GEMV_SHAPES]
    outs = [torch.zeros(m, device="cuda") for (m, _) in GEMV_SHAPES]

    def token():  # q/k/v and gate/up share their activation: one grouped launch each
        for layer in range(n_layers):
            w = ws[layer]
            be.dev_ternary_gemv_preq_group(w[0:3], [0.75] * 3, acts[0], 11.0, outs[0:3],
                                           [2560, 640, 640], 2560)
            be.dev_ternary_gemv_preq(w[3], 0.75, acts[3], 11.0, outs[3], 2560, 2560)
            be.dev_ternary_gemv_preq_group(w[4:6], [0.75] * 2, acts[4], 11.0, outs[4:6],
                                           [6912, 6912], 2560)
            be.dev_ternary_gemv_preq(w[6], 0.75, acts[6], 11.0, outs[6], 2560, 6912)

    def token_separate():  # one launch per projection, as the trait calls them
        for layer in range(n_layers):
            for i, (m, k) in enumerate(GEMV_SHAPES):
                be.dev_ternary_gemv_preq(ws[layer][i], 0.75, acts[i], 11.0, outs[i], m, k)

    def gate_only():  # the dominant launch (6912 x 2560), over the 30 layers' gate weights
        for layer in range(n_layers):
            be.dev_ternary_gemv_preq(ws[layer][4], 0.75, acts[4], 11.0, outs[4], 6912, 2560)

    res = {}
    for name, fn, launches in (("token", token, n_layers * 4),
                               ("separate", token_separate, n_layers * len(GEMV_SHAPES)),
                               ("gate", gate_only, n_layers)):
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        graph.replay()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            graph.replay()
        t1.record()
        torch.cuda.synchronize()
        res[name] = t0.elapsed_time(t1) / steps
        res[name + "_launches"] = launches
    tok_bytes = n_layers * sum(gemv_bytes(m, k) for (m, k) in GEMV_SHAPES)
    gate_bytes = gemv_bytes(6912, 2560)
    gate_us = res["gate"] * 1e3 / n_layers
    del ws
    torch.cuda.empty_cache()
    return {"token_ms": res["token"], "token_bytes": tok_bytes,
            "gbs": tok_bytes / (res["token"] * 1e-3) / 1e9,
            "launch_us": res["token"] * 1e3 / res["token_launches"],
            "separate_ms": res["separate"],
            "gate_us": gate_us, "gate_bytes": gate_bytes,
            "gate_gbs": gate_bytes / (gate_us * 1e-6) / 1e9}


LM_VOCAB, LM_HIDDEN = 128256, 2560  # BitNet b1.58 2B (LLaMA 3 tokenizer)


def lm_head_bytes(v: int, h: int) -> int:
    """i8 weights + f32 hidden in + f32 scales + f32 logits out."""
    return v * h + 4 * h + 8 * v


def bench_lm_head(torch, be, steps: int = 20):
    """LM head with i8 weights at the 2B shape: 128256 x 2560 (328 MB, more
    than the 256 MB MALL, so every launch streams it from HBM)."""
    g = torch.Generator(device="cuda").manual_seed(0xB17E7070)
    w = torch.randint(-128, 128, (LM_VOCAB * LM_HIDDEN,), dtype=torch.int8, device="cuda",
                      generator=g)
    hid = torch.randn(LM_HIDDEN, device="cuda", generator=g)
    sc = torch.rand(LM_VOCAB, device="cuda", generator=g) * 0.02
    out = torch.zeros(LM_VOCAB, device="cuda")

    def run():
        be.dev_lm_head_matmul_i8(hid, w, sc, out, LM_VOCAB, LM_HIDDEN)

    for _ in range(3):
        run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            run()
    graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    graph.replay()
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / steps
    nbytes = lm_head_bytes(LM_VOCAB, LM_HIDDEN)
    del w
    torch.cuda.empty_cache()
    return {"us": us, "bytes": nbytes, "gbs": nbytes / (us * 1e-6) / 1e9}


def bench_model(torch, be, position: int = 1024, steps: int = 10, fused: bool = True):
    """One decode token through the whole 2B stack on the device (30 layers:
    norm/quantise, grouped ternary GEMVs, fused decode attention at context
    `position`, residuals; final norm; i8 LM head), captured as one HIP graph
    (fused: 5 launches per layer, each projection computing its input's
    RMSNorm and quantisation; otherwise 9, the glue as launches of its own).
    Synthetic weights (random packed bytes, every 2-bit code), random cache
    rows 0..position-1."""
    from bitnetrs_amd.model import DecodeModel, LayerWeights, ModelShape

    s = ModelShape()
    cap = 4096
    g = torch.Generator(device="cuda").manual_seed(0xB17E7080)
    q_dim, kv_dim = s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim
    shapes = [(q_dim, s.hidden), (kv_dim, s.hidden), (kv_dim, s.hidden), (s.hidden, q_dim),
              (s.ffn, s.hidden), (s.ffn, s.hidden), (s.hidden, s.ffn)]

    def packed(m, k):
        return torch.randint(0, 256, (m * ((k + 3) // 4),), dtype=torch.uint8, device="cuda",
                             generator=g)

    def norm(n):
        return 0.8 + 0.4 * torch.rand(n, device="cuda", generator=g)

    layers = [LayerWeights(*[packed(m, k) for (m, k) in shapes], scales=(0.05,) * 7,
                           attention_norm=norm(s.hidden), attn_sub_norm=norm(q_dim),
                           ffn_norm=norm(s.hidden), ffn_sub_norm=norm(s.ffn))
              for _ in range(s.n_layers)]
    lm_w = torch.randint(-128, 128, (s.vocab * s.hidden,), dtype=torch.int8, device="cuda",
                         generator=g)
    dm = DecodeModel(be, s, layers, norm(s.hidden), lm_w,
                     torch.rand(s.vocab, device="cuda", generator=g) * 0.01, cap, fused=fused)
    for li in range(s.n_layers):
        dm.cache.k[li][:, :position].normal_(generator=g)
        dm.cache.v[li][:, :position].normal_(generator=g)
    dm.cache.layer_lengths = [position] * s.n_layers
    dm.cache.filled_positions = position
    emb = torch.randn(s.hidden, device="cuda", generator=g)
    h = emb.clone()
    logits = torch.zeros(s.vocab, device="cuda")
    dm.step(h, logits, position=position)  # eager warm-up (every launch once)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        h.copy_(emb)
        dm.step(h, logits, position=position)
    graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    nbytes = (s.n_layers * sum(gemv_bytes(m, k) for (m, k) in shapes)
              + s.n_layers * decode_bytes(position + 1) + lm_head_bytes(s.vocab, s.hidden))
    del layers, lm_w, dm
    torch.cuda.empty_cache()
    return {"ms": ms, "tok_s": 1e3 / ms, "bytes": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9,
            "position": position}


def cpu_baseline_lm_head(budget_s: float):
    """The oracle's lm_head_matmul_i8 (AVX2+FMA rows over all host cores) at
    the 2B shape."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(0xB17E7071)
    w = rng.integers(-128, 128, size=LM_VOCAB * LM_HIDDEN, dtype=np.int8)
    hid = rng.standard_normal(LM_HIDDEN).astype(np.float32)
    sc = rng.uniform(0.0, 0.02, size=LM_VOCAB).astype(np.float32)
    out = np.zeros(LM_VOCAB, np.float32)
    n, t_start = 0, time.perf_counter()
    while True:
        oracle.lm_head_matmul_i8(hid, w, sc, out, LM_VOCAB, LM_HIDDEN)
        n += 1
        if time.perf_counter() - t_start > budget_s:
            break
    dt = (time.perf_counter() - t_start) / n
    return {"value": lm_head_bytes(LM_VOCAB, LM_HIDDEN) / dt / 1e9, "unit": "GB/s",
            "cores": oracle.get_threads(), "kind": "port",
            "sample": f"{n} x the 128256 x 2560 i8 LM head, {dt * 1e3:.2f} ms each"}


def cpu_baseline_gemv(budget_s: float):
    """The oracle's ternary_gemv_preq (AVX2 integer dot, rows over all host
    cores) on the 7 projections of one layer for one token, repeated."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(0xB17E7061)
    mats = [(rng.integers(0, 256, size=m * ((k + 3) // 4)).astype(np.uint8),
             rng.integers(-128, 128, size=k).astype(np.int8), np.zeros(m, np.float32), m, k)
            for (m, k) in GEMV_SHAPES]
    n, t_start = 0, time.perf_counter()
    while True:
        for w, a, o, m, k in mats:
            oracle.ternary_gemv_preq(w, 0.75, a, 11.0, o, m, k)
        n += 1
        if time.perf_counter() - t_start > budget_s:
            break
    dt = (time.perf_counter() - t_start) / n
    layer_bytes = sum(gemv_bytes(m, k) for (m, k) in GEMV_SHAPES)
    return {"value": layer_bytes / dt / 1e9, "unit": "GB/s", "cores": oracle.get_threads(),
            "kind": "port",
            "sample": f"{n} x the 7 ternary projections of one 2B layer for one token "
                      f"({layer_bytes} B), {dt * 1e3:.3f} ms each"}


def copy_calibration(torch, nbytes: int = 256 << 20, reps: int = 5) -> None:
    """Plain device-to-device copies of a known size: the reference for
    scaling FETCH_SIZE / WRITE_SIZE counters in a --pmc run of this script."""
    src = torch.empty(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1.0)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: {reps} copies of {nbytes} bytes")


def load_traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, scaled by the copy calibration), if recorded."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def parity(got, ref) -> dict:
    """Error of timed outputs against the oracle on the same inputs:
    max-abs and max-rel separately, and whether every element is within
    |gpu - ref| <= 2e-3 + 1e-3 |ref|."""
    import numpy as np

    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    err = np.abs(got - ref)
    rel = err / np.maximum(np.abs(ref), 1e-30)
    ok = bool(np.all(np.isfinite(got)) and np.all(err <= 2e-3 + 1e-3 * np.abs(ref)))
    return {"max_abs": float(err.max()), "max_rel": float(rel.max()), "within_tol": ok,
            "elements": int(ref.size)}


def oracle_decode_out(host, pos: int = 4095):
    """The reference's rope_embed -> store_kv -> masked_attention for one token
    of one layer (bitnet-model/src/lib.rs:1004-1036), on the oracle."""
    import numpy as np

    import oracle

    be = oracle.CpuBackend()
    q, k = host["q"].copy(), host["k"].copy()
    be.rope_embed(q, k, pos, D, HQ, HKV, THETA)
    kc, vc = host["k_cache"].copy(), host["v_cache"].copy()
    kc[:, pos] = k.reshape(HKV, D)
    vc[:, pos] = host["v"].reshape(HKV, D)
    out = np.zeros(HQ * D, np.float32)
    be.masked_attention(q, kc.reshape(-1), vc.reshape(-1), out, HQ, HKV, D, pos)
    return out


def oracle_tokens_out(q, k, v, start_pos: int = 0, cap: int | None = None):
    """n serial per-token calls of one layer from start_pos (the reference's
    prefill loop, bitnet-model/src/lib.rs:684-718) on the oracle; returns
    the outputs [n, HQ*D]."""
    import oracle

    n = q.shape[0]
    cache = oracle.KVCache(1, HKV, D, cap or start_pos + n)
    return oracle.layer_tokens(oracle.CpuBackend(), cache, 0, q.copy(), k.copy(), v.copy(),
                               start_pos, HQ, HKV, D, THETA)


def cpu_baseline_decode(host, budget_s: float):
    """Reference call sequence for one decode token of one layer at pos 4095."""
    import numpy as np

    import oracle

    be = oracle.CpuBackend()
    kc = host["k_cache"].copy()
    vc = host["v_cache"].copy()
    out = np.zeros(HQ * D, np.float32)
    n, t_start = 0, time.perf_counter()
    while True:
        q, k = host["q"].copy(), host["k"].copy()
        be.rope_embed(q, k, 4095, D, HQ, HKV, THETA)
        kc[:, 4095] = k.reshape(HKV, D)
        vc[:, 4095] = host["v"].reshape(HKV, D)
        be.masked_attention(q, kc.reshape(-1), vc.reshape(-1), out, HQ, HKV, D, 4095)
        n += 1
        el = time.perf_counter() - t_start
        if el >= budget_s or n >= 20000:
            break
    per = el / n
    return {"value": decode_bytes(4096) / per / 1e9, "unit": "GB/s",
            "cores": min(oracle.get_threads(), HQ), "kind": "port",
            "sample": f"{n} decode steps (rope_embed, store_kv, masked_attention) of one layer "
                      f"at pos 4095, {per * 1e3:.3f} ms each"}


def cpu_baseline_prefill(budget_s: float, n: int = 2048):
    import numpy as np

    import oracle

    g = np.random.default_rng(7)
    q = g.standard_normal((n, HQ * D), dtype=np.float32)
    k = g.standard_normal((n, HKV * D), dtype=np.float32)
    v = g.standard_normal((n, HKV * D), dtype=np.float32)
    reps, t_start = 0, time.perf_counter()
    while True:
        cache = oracle.KVCache(1, HKV, D, n)
        be = oracle.CpuBackend()
        oracle.layer_tokens(be, cache, 0, q.copy(), k.copy(), v, 0, HQ, HKV, D, THETA)
        reps += 1
        el = time.perf_counter() - t_start
        if el >= budget_s:
            break
    per = el / reps
    return {"value": prefill_flops(n) / per / 1e12, "unit": "TFLOP/s",
            "cores": min(oracle.get_threads(), HQ), "kind": "port",
            "sample": f"{reps} x 2048-token causal prefill of one layer as 2048 serial "
                      f"(rope_embed, store_kv, masked_attention) calls, {per:.3f} s each"}


TIMELINE_PHASES = ["issue", "read", "barrier", "combine", "sums", "ticket", "merge"]


def decode_timeline_main(args) -> int:
    """Per-phase timeline of the fused decode step at 4096 rows (the headline
    workload, 32 rotated layer caches, a HIP graph of --steps launches
    replayed --replays times).  Loads the measurement build
    libbitnet_hip_timeline.so, whose decode kernel stores eight 100 MHz
    s_memrealtime stamps per workgroup: entry, loads issued, rows consumed,
    path barrier passed, combine done (sums sent), sums complete, ticket
    returned, merge done (merging workgroup).  Prints one JSON line of
    medians over launches (us): the phases of the workgroup that finishes
    last (the critical path), the same phases over all workgroups, the
    dispatch spread, and the gap from one launch's last stamp to the next
    launch's first.  With --batched-timeline: the same for the 32-sequence
    batched decode (one launch per step; splits past a sequence's end are
    left out)."""
    import ctypes

    import numpy as np
    import torch

    from bitnetrs_amd import _lib

    path = os.path.join(ROOT, "bitnetrs_amd", "libbitnet_hip_timeline.so")
    if not os.path.exists(path):
        log("libbitnet_hip_timeline.so is not built (make -C bitnetrs_amd/csrc)")
        return 1
    _lib.LIB_PATH = path
    import bitnetrs_amd

    lib = _lib.load()
    lib.bnr_debug_decode_timeline.restype = ctypes.c_int
    lib.bnr_debug_decode_timeline.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    be = bitnetrs_amd.HipBackend(0)
    log(f"device: {be.device_name()} (timeline build)")
    steps, reps = args.steps, args.replays
    batched = args.batched_timeline
    if batched:
        # the batched workload: 32 sequences, lengths ~ U[128, 4096), one launch a step
        n_seq, cap = 32, 4096
        lens = np.random.default_rng(0xB17E7040).integers(128, 4096, size=n_seq).astype(np.int32)
        g = torch.Generator(device="cuda").manual_seed(0xB17E7041)
        kc = torch.randn(n_seq, HKV, cap, D, device="cuda", generator=g)
        vc = torch.randn(n_seq, HKV, cap, D, device="cuda", generator=g)
        q = torch.randn(n_seq, HQ * D, device="cuda", generator=g)
        k = torch.randn(n_seq, HKV * D, device="cuda", generator=g)
        v = torch.randn(n_seq, HKV * D, device="cuda", generator=g)
        out = torch.zeros(n_seq, HQ * D, device="cuda")
        max_wg = 256 * HKV * n_seq
    else:
        n_layers, pos, cap = 32, 4095, 4096
        g = torch.Generator(device="cuda").manual_seed(0xB17E7020)
        kc = torch.randn(n_layers, HKV, cap, D, device="cuda", generator=g)
        vc = torch.randn(n_layers, HKV, cap, D, device="cuda", generator=g)
        q = torch.randn(n_layers, HQ * D, device="cuda", generator=g) * 4.0
        k = torch.randn(n_layers, HKV * D, device="cuda", generator=g)
        v = torch.randn(n_layers, HKV * D, device="cuda", generator=g)
        out = torch.zeros(n_layers, HQ * D, device="cuda")
        max_wg = 256 * HKV  # at most 256 splits per kv head
    stamps = torch.zeros(steps, max_wg * 8, dtype=torch.int64, device="cuda")

    def step(i, rec=True):
        _lib.check(lib.bnr_debug_decode_timeline(be._h, stamps[i].data_ptr() if rec else None))
        if batched:
            be.dev_decode_step_batched(q, k, v, lens, HQ, HKV, D, THETA, kc, vc, cap, out)
        else:
            r = i % n_layers
            be.dev_decode_step(q[r], k[r], v[r], pos, HQ, HKV, D, THETA, kc[r], vc[r], cap,
                               out[r])

    for i in range(args.warmup):
        step(i, rec=False)
    torch.cuda.synchronize()
    graph = capture(torch, step, steps)
    _lib.check(lib.bnr_debug_decode_timeline(be._h, None))
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    per_step, samples, gaps, ticks_per_us = [], [], [], []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0.record()
        graph.replay()
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1)
        per_step.append(ms / steps)
        st = stamps.cpu().numpy().reshape(steps, max_wg, 8)
        firsts, lasts = [], []
        for i in range(steps):
            rows = st[i][st[i][:, 0] != 0]
            t_first = rows[:, 0].min()
            rows = rows[rows[:, 2] != 0]  # ragged launches: splits past a sequence's end exit
            end = rows[:, 1:].max()
            firsts.append(t_first)
            lasts.append(end)
            crit = rows[np.argmax(rows[:, 7])]
            d = np.diff(rows[:, :7], axis=1)  # issue .. ticket, every workgroup
            merger = rows[rows[:, 7] != 0]
            samples.append({
                "span": end - t_first,
                "dispatch_spread": rows[:, 0].max() - t_first,
                "last_rows": rows[:, 2].max() - t_first,
                "last_sums": rows[:, 5].max() - t_first,
                "crit_start": crit[0] - t_first,
                **{f"crit_{p}": crit[j + 1] - crit[j] for j, p in enumerate(TIMELINE_PHASES)},
                **{f"all_{p}": np.median(d[:, j]) for j, p in enumerate(TIMELINE_PHASES[:6])},
                **{f"all90_{p}": np.percentile(d[:, j], 90) for j, p in enumerate(TIMELINE_PHASES[:6])},
                "all_merge": np.median(merger[:, 7] - merger[:, 6]),
                # when the workgroups pass their path barrier (all rows in), from the first entry
                "rows_in_p10": np.percentile(rows[:, 3] - t_first, 10),
                "rows_in_p50": np.percentile(rows[:, 3] - t_first, 50),
                "rows_in_p90": np.percentile(rows[:, 3] - t_first, 90),
                "rows_in_max": rows[:, 3].max() - t_first,
                "entry_p90": np.percentile(rows[:, 0] - t_first, 90),
                "wgs": len(rows)})
        gaps += [firsts[i + 1] - lasts[i] for i in range(steps - 1)]
        ticks_per_us.append((lasts[-1] - firsts[0]) / (ms * 1e3))
    # s_memrealtime counts at 100 MHz; the ratio of the stamps' extent to the
    # event-timed replay checks it (a little below 100: the replay also holds
    # the first launch's dispatch and the last one's end)
    tick_us = 1.0 / 100.0
    med = lambda xs: float(np.median(xs))  # noqa: E731
    res = {"workload": ("gqa_decode_step_batch32_ragged_len_U128_4096_hq20_hkv5_d128_fp32"
                        if batched else "gqa_decode_step_L4096_hq20_hkv5_d128_fp32")
                       + " (timeline build)",
           "launches": len(samples), "steps": steps, "replays": reps,
           "wgs_per_launch": int(samples[0]["wgs"]),
           "graph_step_us": round(med(per_step) * 1e3, 3),
           "stamp_ticks_per_us": round(med(ticks_per_us), 2),
           "gap_to_next_launch_us": round(med(gaps) * tick_us, 3)}
    for key in samples[0]:
        if key != "wgs":
            res[key + "_us"] = round(med([x[key] for x in samples]) * tick_us, 3)
    # The phases' hardware floors: one lane's chain of dependent device-scope
    # operations (the merge chain is made of them), and a graph of empty
    # launches of the same grid (the launch-to-launch cost).
    lib.bnr_debug_rt_probe.restype = ctypes.c_int
    lib.bnr_debug_rt_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_void_p, ctypes.c_void_p]
    lib.bnr_debug_empty_launch.restype = ctypes.c_int
    lib.bnr_debug_empty_launch.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    buf = torch.zeros(256, dtype=torch.int32, device="cuda")
    out = torch.zeros(2, dtype=torch.int64, device="cuda")
    n_ops = 2000
    for mode, name in enumerate(["fetch_add_return", "add_then_wait", "exchange", "agent_load"]):
        ticks = []
        for _ in range(5):
            _lib.check(lib.bnr_debug_rt_probe(be._h, buf.data_ptr(), n_ops, mode, out.data_ptr(), None))
            torch.cuda.synchronize()
            ticks.append(int(out[0].item()))
        res[f"rt_{name}_us"] = round(med(ticks) * tick_us / n_ops, 4)
    wgs = int(samples[0]["wgs"])
    wbuf = torch.zeros(64 * 256, dtype=torch.int32, device="cuda")
    for mode, name in enumerate(["bare", "args", "lds64k", "args_lds64k", "store", "nt_store",
                                 "atomic_add", "system_store", "decode_footprint"]):
        # on the capturing stream (a NULL stream would not be captured)
        empty = capture(torch, lambda i: _lib.check(lib.bnr_debug_empty_launch(
            be._h, wgs, 256 if batched else 512, mode, wbuf.data_ptr(),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))), steps)
        res[f"empty_launch_{name}_graph_step_us"] = round(
            replay_stats(torch, empty, steps, reps=reps)["median"] * 1e3, 3)
        del empty
    print(json.dumps(res), flush=True)
    be.close()
    return 0


# Words of a prefill workgroup's timeline record (PfStamp in bnr_internal.h).
PF_ENTRY, PF_READY, PF_TILES, PF_TICKET, PF_MERGED, PF_STORED, PF_HWID, PF_ITEM = range(8)


def prefill_launch_stats(rows, tick_us):
    """One launch's records (rows of 8 words, one per workgroup) -> phase
    statistics in us: span, start latency, per-key-tile time, partial-state
    store + ticket, merge, output store; per-CU residency and how many
    workgroups are still running as the launch drains; and per CU, the
    (key tiles, chunks) of its workgroups in entry order with its end."""
    import numpy as np

    t0 = rows[:, PF_ENTRY].min()
    ends = np.maximum.reduce([rows[:, PF_TICKET], rows[:, PF_MERGED], rows[:, PF_STORED]])
    span = ends.max() - t0
    ntiles = (rows[:, PF_ITEM] & 0xFFFF).astype(np.float64)
    nch = (rows[:, PF_ITEM] >> 16) & 0xFFFF
    split = nch > 1
    merger = rows[:, PF_MERGED] != 0
    writer = rows[:, PF_STORED] != 0
    hw = rows[:, PF_HWID]
    # XCC_ID, then HW_ID's SE / SH / CU fields (bits 8..15): one CU
    cu_key = ((hw >> 32) << 8) | ((hw >> 8) & 0xFF)
    cus = np.unique(cu_key)
    # per CU: time with >= 1 workgroup in its key-tile phase, mean residents
    busy, resident = [], []
    for c in cus:
        sel = cu_key == c
        iv = sorted(zip(rows[sel, PF_READY], rows[sel, PF_TILES]))
        tot, cur_s, cur_e = 0, None, None
        for a, b in iv:
            if cur_e is None or a > cur_e:
                if cur_e is not None:
                    tot += cur_e - cur_s
                cur_s, cur_e = a, b
            else:
                cur_e = max(cur_e, b)
        if cur_e is not None:
            tot += cur_e - cur_s
        busy.append(tot / span)
        resident.append((ends[sel] - rows[sel, PF_ENTRY]).sum() / span)
    rel_end = (ends - t0) / span
    med = lambda x: float(np.median(x)) if len(x) else 0.0  # noqa: E731
    out = {
        "span": span * tick_us,
        "wgs": int(len(rows)),
        "cus": int(len(cus)),
        "entry_spread": (rows[:, PF_ENTRY].max() - t0) * tick_us,
        "start_latency": med(rows[:, PF_READY] - rows[:, PF_ENTRY]) * tick_us,
        "start_latency_p90": float(np.percentile(rows[:, PF_READY] - rows[:, PF_ENTRY], 90)) * tick_us,
        "tile": med((rows[:, PF_TILES] - rows[:, PF_READY]) / ntiles) * tick_us,
        "key_tiles_mean": float(ntiles.mean()),
        "ticket": med(rows[split, PF_TICKET] - rows[split, PF_TILES]) * tick_us,
        "merge": med(rows[merger, PF_MERGED] - rows[merger, PF_TICKET]) * tick_us,
        "store": med(rows[writer, PF_STORED] - np.maximum(rows[writer, PF_MERGED],
                                                           rows[writer, PF_TILES])) * tick_us,
        "cu_tile_busy": med(busy),
        "cu_residents": med(resident),
        "first_end": (ends.min() - t0) * tick_us,
        "end_p50": float(np.percentile(rel_end, 50)) * span * tick_us,
        "end_p90": float(np.percentile(rel_end, 90)) * span * tick_us,
    }
    # workgroups still running at tenths of the span
    out["running_by_tenth"] = [int(((rows[:, PF_ENTRY] <= t0 + f * span) & (ends > t0 + f * span)).sum())
                               for f in np.arange(0.0, 1.0, 0.1)]
    # what each CU ran: its workgroups' (key tiles, chunks of their query
    # unit) in the order they entered, and when its last one ended
    bins = []
    for c in cus:
        sel = np.nonzero(cu_key == c)[0]
        sel = sel[np.argsort(rows[sel, PF_ENTRY], kind="stable")]
        bins.append((tuple((int(ntiles[j]), int(nch[j])) for j in sel),
                     float(ends[sel].max() - t0) * tick_us))
    return out, bins, t0, ends.max()


def prefill_timeline_main(args) -> int:
    """Per-workgroup timeline of the grid-mapped prefill kernel on the
    30-layer stack's prefill (N = --prefill-tokens from an empty cache of
    N + 256 rows, RoPE + append + attention per layer, the planner's chunks)
    as a HIP graph of 30 layers' launches replayed --replays times (q and k
    restored between replays, untimed).  Loads the measurement build
    libbitnet_hip_timeline.so, whose prefill kernel stores eight words per
    workgroup (PfStamp).  Prints one JSON line of medians over launches."""
    import ctypes

    import numpy as np
    import torch

    from bitnetrs_amd import _lib

    path = os.path.join(ROOT, "bitnetrs_amd", "libbitnet_hip_timeline.so")
    if not os.path.exists(path):
        log("libbitnet_hip_timeline.so is not built (make -C bitnetrs_amd/csrc)")
        return 1
    _lib.LIB_PATH = path
    import bitnetrs_amd

    lib = _lib.load()
    lib.bnr_debug_decode_timeline.restype = ctypes.c_int
    lib.bnr_debug_decode_timeline.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    be = bitnetrs_amd.HipBackend(0)
    log(f"device: {be.device_name()} (timeline build)")
    n_layers, n = 30, args.prefill_tokens
    cap, reps = n + 256, args.replays
    g = torch.Generator(device="cuda").manual_seed(0xB17E7050)
    qp = torch.randn(n_layers, n, HQ * D, device="cuda", generator=g)
    kp = torch.randn(n_layers, n, HKV * D, device="cuda", generator=g)
    vp = torch.randn(n_layers, n, HKV * D, device="cuda", generator=g)
    kc = torch.zeros(n_layers, HKV, cap, D, device="cuda")
    vc = torch.zeros_like(kc)
    out = torch.zeros_like(qp)
    q_in, k_in = qp.clone(), kp.clone()
    max_wg = 8192
    stamps = torch.zeros(n_layers, max_wg * 8, dtype=torch.int64, device="cuda")

    def layer(i, rec=True):
        _lib.check(lib.bnr_debug_decode_timeline(be._h, stamps[i].data_ptr() if rec else None))
        be.dev_prefill(qp[i], kp[i], vp[i], n, 0, HQ, HKV, D, THETA, kc[i], vc[i], cap, out[i])

    layer(0, rec=False)  # sizes the table and workspace
    torch.cuda.synchronize()
    qp.copy_(q_in)
    kp.copy_(k_in)
    graph = capture(torch, layer, n_layers)
    _lib.check(lib.bnr_debug_decode_timeline(be._h, None))
    tick_us = 1.0 / 100.0
    t0e = torch.cuda.Event(enable_timing=True)
    t1e = torch.cuda.Event(enable_timing=True)
    samples, gaps, per_layer, cu_bins = [], [], [], {}
    for r in range(reps):
        qp.copy_(q_in)
        kp.copy_(k_in)
        stamps.zero_()
        torch.cuda.synchronize()
        t0e.record()
        graph.replay()
        t1e.record()
        torch.cuda.synchronize()
        per_layer.append(t0e.elapsed_time(t1e) / n_layers)
        st = stamps.cpu().numpy().reshape(n_layers, max_wg, 8)
        bounds = []
        for i in range(n_layers):
            rows = st[i][st[i][:, PF_ENTRY] != 0]
            stats, bins, first, last = prefill_launch_stats(rows, tick_us)
            samples.append(stats)
            for comp, end in bins:
                cu_bins.setdefault(comp, []).append(end)
            bounds.append((first, last))
        gaps += [(bounds[i + 1][0] - bounds[i][1]) * tick_us for i in range(n_layers - 1)]
    med = lambda xs: float(np.median(xs))  # noqa: E731
    flops = prefill_flops(n)
    res = {"workload": f"bitnet_2b_attention_stack_30L_prefill{n}_fp32 (timeline build)",
           "launches": len(samples), "replays": reps,
           "graph_layer_us": round(med(per_layer) * 1e3, 3),
           "graph_layer_tflops": round(flops / (med(per_layer) * 1e-3) / 1e12, 2),
           "gap_to_next_launch_us": round(med(gaps), 3)}
    for key in samples[0]:
        if key == "running_by_tenth":
            res[key] = [int(np.median([x[key][j] for x in samples])) for j in range(10)]
        else:
            res[key if key in ("wgs", "cus", "key_tiles_mean", "cu_tile_busy", "cu_residents")
                else key + "_us"] = round(med([x[key] for x in samples]), 3)
    res["span_tflops"] = round(flops / (res["span_us"] * 1e-6) / 1e12, 2)
    # the CU workloads that end last: [(key tiles, chunks) per workgroup in
    # entry order], CUs per launch running it, median end (us from launch start)
    slow = sorted(cu_bins.items(), key=lambda kv: -np.median(kv[1]))[:10]
    res["cu_bins_slowest"] = [[[list(w) for w in comp], round(len(ends) / len(samples), 2),
                               round(med(ends), 2)] for comp, ends in slow]
    print(json.dumps(res), flush=True)
    be.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--decode-contexts", default="",
                    help="comma-separated context lengths: also time the decode step at each")
    ap.add_argument("--prefill-shapes", default="",
                    help="comma-separated tokens@cached shapes: also time prefill attention")
    ap.add_argument("--prefill-tokens", type=int, default=2048,
                    help="tokens of the single-layer prefill workload (profiling other shapes)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-stack", action="store_true", help="skip the 30-layer stack workload")
    ap.add_argument("--no-batched", action="store_true", help="skip the 32-sequence batched decode")
    ap.add_argument("--no-gemv", action="store_true", help="skip the ternary GEMV workload")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the i8 LM head workload")
    ap.add_argument("--no-model", action="store_true", help="skip the whole-model decode token")
    ap.add_argument("--no-trait", action="store_true",
                    help="skip the host-slice (Backend trait) path timing")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds per CPU baseline")
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches instead of a captured graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run plain copies of a known size (for --pmc scaling)")
    ap.add_argument("--replays", type=int, default=100,
                    help="timed replays of the decode graph (the median is reported)")
    ap.add_argument("--decode-timeline", action="store_true",
                    help="only the per-phase timeline of the decode kernel (loads the "
                         "measurement build libbitnet_hip_timeline.so)")
    ap.add_argument("--batched-timeline", action="store_true",
                    help="with --decode-timeline: the 32-sequence batched decode instead")
    ap.add_argument("--prefill-timeline", action="store_true",
                    help="only the per-workgroup timeline of the stack-shape prefill (loads the "
                         "measurement build libbitnet_hip_timeline.so; --prefill-tokens sets N)")
    ap.add_argument("--no-parity", action="store_true",
                    help="skip the oracle checks of the timed outputs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (asked for --gpus {args.gpus}); the attention "
              "path runs on a single GPU and has no multi-GPU launch",
              file=sys.stderr)
        return 2

    if args.decode_timeline:
        return decode_timeline_main(args)
    if args.prefill_timeline:
        return prefill_timeline_main(args)

    import torch

    import bitnetrs_amd

    be = bitnetrs_amd.HipBackend(0)
    log(f"device: {be.device_name()}")
    if args.copy_calibration:
        copy_calibration(torch)
    traffic = load_traffic()
    dec = bench_decode(torch, be, args.steps, args.warmup, eager=args.eager, reps=args.replays)
    fl = dec["floor"]
    log(f"decode: {dec['ms_per_step'] * 1e3:.2f} us/step (median of {dec['stats']['replays']} "
        f"replays; min {dec['stats']['min'] * 1e3:.2f}, p90 {dec['stats']['p90'] * 1e3:.2f}), "
        f"{dec['gbs']:.0f} GB/s; event pair {dec['pair_ms'] * 1e3:.2f} us; streaming floor "
        f"{fl['ms'] * 1e3:.2f} us ({fl['shape']}; plain one-load {fl['plain_ms'] * 1e3:.2f} us)")
    line = {
        "metric": METRIC,
        "value": round(dec["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dec["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) q/k/v and caches, q x4)",
        "config": {"workload": "gqa_decode_step_L4096_hq20_hkv5_d128_fp32",
                   "context": 4096, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                   "rope_theta": THETA, "layers_rotated": 32,
                   "timed": f"hip graph of {args.steps} fused rope+append+split-K attention "
                            f"launches; ms_per_step = median over {dec['stats']['replays']} "
                            "timed replays, each bracketed by device synchronisations"},
        "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("decode_reg_kernel", {}).get("bytes_per_launch"),
                     "kernel": "decode_reg_kernel",
                     "graph_step_us": round(dec["ms_per_step"] * 1e3, 3),
                     "graph_step_us_min": round(dec["stats"]["min"] * 1e3, 3),
                     "graph_step_us_p90": round(dec["stats"]["p90"] * 1e3, 3),
                     "event_pair_us": round(dec["pair_ms"] * 1e3, 3),
                     "bytes_per_launch": dec["bytes_per_step"],
                     "stream_floor_us": round(fl["ms"] * 1e3, 3),
                     "stream_floor_shape": fl["shape"],
                     "stream_floor_gbs": round(dec["bytes_per_step"] / (fl["ms"] * 1e-3) / 1e9, 1),
                     "stream_plain_us": round(fl["plain_ms"] * 1e3, 3),
                     "stream_shapes_us": fl["shapes_us"],
                     "frac_of_stream_floor": round(fl["ms"] / dec["ms_per_step"], 4)},
    }
    if args.decode_contexts:
        line["decode_contexts"] = bench_decode_contexts(
            torch, be, [int(x) for x in args.decode_contexts.split(",")])
    if args.prefill_shapes:
        line["prefill_shapes"] = bench_prefill_shapes(
            torch, be, [tuple(int(y) for y in x.split("@")) for x in args.prefill_shapes.split(",")])
    if not args.no_trait:
        tp = bench_trait_path(be)
        log(f"trait path (Python caller) at pos 4095: rope_embed {tp['rope_us']:.1f} us + "
            f"masked_attention {tp['attn_us']:.1f} us = {tp['token_layer_us']:.1f} us per token "
            f"and layer; rms_norm {tp['rms_norm_us']:.1f} us, sqrelu_gate "
            f"{tp['sqrelu_gate_us']:.1f} us")
        ct = trait_timer()
        if ct is not None:
            log(f"trait path (compiled caller) at pos 4095: rope_embed {ct['rope_us']:.1f} us + "
                f"masked_attention {ct['attn_us']:.1f} us = {ct['token_layer_us']:.1f} us; "
                f"rms_norm {ct['rms_norm_us']:.1f} us, sqrelu_gate {ct['sqrelu_gate_us']:.1f} us")
        main_tp = ct if ct is not None else tp
        line["trait_path"] = {
            "workload": "host_slice_rope_embed_masked_attention_pos4095_hq20_hkv5_d128_fp32",
            "caller": "compiled C over the C ABI (bitnetrs_amd/trait_timer)" if ct is not None
                      else "Python ctypes (trait_timer not built)",
            "us_per_token_layer": round(main_tp["token_layer_us"], 2),
            "rope_embed_us": round(main_tp["rope_us"], 2),
            "masked_attention_us": round(main_tp["attn_us"], 2),
            "rms_norm_host_us": round(main_tp["rms_norm_us"], 2),
            "sqrelu_gate_host_us": round(main_tp["sqrelu_gate_us"], 2),
            "python_caller_us_per_token_layer": round(tp["token_layer_us"], 2),
            "timed": f"{tp['steps']} consecutive positions after 10 untimed, wall clock per "
                     "host call (PCIe included); Python caller with its GC off"}
        if ct is not None and "kv_decode_us" in ct:
            # bnr_kv_decode: the same token and layer through the backend-owned
            # cache (rope_embed, store_kv and masked_attention in one call)
            line["trait_path"]["owned_cache_kv_decode_us"] = round(ct["kv_decode_us"], 2)
            log(f"owned-cache decode (bnr_kv_decode, compiled caller) at pos 4095: "
                f"{ct['kv_decode_us']:.1f} us per token and layer")
    if not args.no_prefill:
        pre = bench_prefill(torch, be, args.prefill_steps, 2, n=args.prefill_tokens)
        log(f"prefill: {pre['ms_per_step']:.3f} ms/step, {pre['tflops']:.2f} TFLOP/s; attention "
            f"{pre['attn_ms']:.3f} ms, {pre['attn_tflops']:.2f} TFLOP/s (graph); eager event "
            f"pair {pre['pair_ms']:.3f} ms")
        line["prefill"] = {
            "workload": f"gqa_causal_prefill_N{args.prefill_tokens}_hq20_hkv5_d128_fp32",
            "value": round(pre["tflops"], 3), "unit": "TFLOP/s",
            "ms_per_step": pre["ms_per_step"],
            "roofline": {"bound": "mfma", "achieved": round(pre["attn_tflops"], 3),
                         "peak": FP32_MATRIX_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pre["attn_tflops"] / FP32_MATRIX_PEAK_TFLOPS, 4),
                         "traffic": traffic.get("prefill_kernel", {}).get("bytes_per_launch"),
                         "kernel": "prefill_kernel",
                         "graph_launch_us": round(pre["attn_ms"] * 1e3, 3),
                         "event_pair_us": round(pre["pair_ms"] * 1e3, 3),
                         "flops_per_launch": pre["flops"]},
            "timed": "HIP graph of one launch per layer over rotated layers, median of 50 "
                     "timed replays (q/k restored between replays, untimed)"}
    if not args.no_batched:
        bat = bench_batched(torch, be)
        log(f"batched decode (32 seqs, ragged): {bat['ms_per_step'] * 1e3:.2f} us/step, "
            f"{bat['gbs']:.0f} GB/s; streaming floor of as many bytes "
            f"{bat['floor']['ms'] * 1e3:.2f} us ({bat['floor']['shape']})")
        line["batched"] = {
            "workload": "gqa_decode_step_batch32_ragged_len_U128_4096_hq20_hkv5_d128_fp32",
            "value": round(bat["gbs"], 2), "unit": "GB/s", "ms_per_step": bat["ms_per_step"],
            "bytes_per_step": bat["bytes"], "frac_hbm": round(bat["gbs"] / HBM_PEAK_GBS, 4),
            "stream_floor_us": round(bat["floor"]["ms"] * 1e3, 3),
            "stream_floor_shape": bat["floor"]["shape"],
            "frac_of_stream_floor": round(bat["floor"]["ms"] / bat["ms_per_step"], 4),
            "lengths_min_max_mean": bat["lengths_min_max_mean"],
            "timed": "HIP graph of 50 batched launches, median of 50 timed replays"}
    if not args.no_stack:
        stk = bench_stack(torch, be)
        log(f"stack: prefill 30x1024 {stk['prefill_ms']:.2f} ms ({stk['prefill_tflops']:.1f} TFLOP/s); "
            f"decode 256 steps x 30 layers {stk['decode_ms']:.2f} ms ({stk['decode_gbs']:.0f} GB/s, "
            f"{stk['decode_tok_s']:.0f} tok/s attention-only)")
        line["stack"] = {
            "workload": "bitnet_2b_attention_stack_30L_prefill1024_decode256_fp32",
            "prefill_ms": round(stk["prefill_ms"], 3), "prefill_tflops": round(stk["prefill_tflops"], 2),
            "decode_ms": round(stk["decode_ms"], 3), "decode_gbs": round(stk["decode_gbs"], 1),
            "decode_tok_s": round(stk["decode_tok_s"], 1), "decode_bytes": stk["decode_bytes"],
            "prefill_flops": stk["prefill_flops"],
            "note": "prefill: one HIP graph of 60 launches, median of 50 replays; decode: one "
                    f"HIP graph of 7680 fused decode launches, median of {stk['decode_replays']} "
                    "replays; caches total 197 MB, which fits the 256 MB MALL"}
    if not args.no_gemv:
        gm = bench_gemv(torch, be)
        log(f"ternary gemv: token (30 layers x 7 projections, 4 launches per layer) "
            f"{gm['token_ms']:.3f} ms, {gm['gbs']:.0f} GB/s; 7 launches per layer "
            f"{gm['separate_ms']:.3f} ms; gate 6912x2560 {gm['gate_us']:.2f} us, "
            f"{gm['gate_gbs']:.0f} GB/s")
        line["gemv"] = {
            "workload": "bitnet_2b_ternary_gemv_token_30L_x7proj_w2a8",
            "value": round(gm["gbs"], 2), "unit": "GB/s", "ms_per_token": round(gm["token_ms"], 4),
            "bytes_per_token": gm["token_bytes"], "launch_us": round(gm["launch_us"], 3),
            "launches_per_layer": 4, "ms_per_token_7_launches": round(gm["separate_ms"], 4),
            "roofline": {"bound": "hbm", "achieved": round(gm["gate_gbs"], 2),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gm["gate_gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": traffic.get("ternary_gemv_kernel", {}).get("bytes_per_launch"),
                         "kernel": "ternary_gemv_kernel (6912 x 2560)",
                         "kernel_us": round(gm["gate_us"], 3), "bytes_per_launch": gm["gate_bytes"]}}
    if not args.no_lm_head:
        lm = bench_lm_head(torch, be)
        log(f"lm head i8 128256x2560: {lm['us']:.2f} us, {lm['gbs']:.0f} GB/s")
        line["lm_head"] = {
            "workload": "bitnet_2b_lm_head_i8_128256x2560",
            "value": round(lm["gbs"], 2), "unit": "GB/s", "us_per_token": round(lm["us"], 3),
            "roofline": {"bound": "hbm", "achieved": round(lm["gbs"], 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(lm["gbs"] / HBM_PEAK_GBS, 4),
                         "traffic": traffic.get("lm_head_i8_kernel", {}).get("bytes_per_launch"),
                         "kernel": "lm_head_i8_kernel", "kernel_us": round(lm["us"], 3),
                         "bytes_per_launch": lm["bytes"]}}
    if not args.no_model:
        md = bench_model(torch, be)
        mg = bench_model(torch, be, fused=False)
        log(f"model decode token, glue as launches of its own (9 per layer): {mg['ms']:.3f} ms")
        log(f"model decode token (30 layers + LM head, context {md['position']}): "
            f"{md['ms']:.3f} ms = {md['tok_s']:.0f} tok/s, {md['gbs']:.0f} GB/s")
        line["model"] = {
            "workload": "bitnet_2b_decode_token_30L_ctx1024_w2a8_i8head",
            "value": round(md["tok_s"], 1), "unit": "tokens/s", "ms_per_token": round(md["ms"], 4),
            "bytes_per_token": md["bytes"], "gbs": round(md["gbs"], 1),
            "frac_hbm": round(md["gbs"] / HBM_PEAK_GBS, 4),
            "ms_per_token_glue_launches": round(mg["ms"], 4),
            "timed": "one HIP graph per token: 30 x 5 launches (glue in the projections' "
                     "prologues) + residual, final norm, LM head"}
    if not args.no_parity:
        # The timed launches' outputs against the oracle on the same inputs
        # (outside every timed region).
        line["parity"] = parity(dec["host"]["out"], oracle_decode_out(dec["host"]))
        log(f"parity decode: {line['parity']}")
        if not args.no_prefill:
            h = pre["host"]
            line["prefill"]["parity"] = parity(
                h["out"], oracle_tokens_out(h["q"], h["k"], h["v"]).reshape(h["out"].shape))
            log(f"parity prefill: {line['prefill']['parity']}")
        if not args.no_batched:
            import numpy as np

            h = bat["host"]
            ref = []
            for b, L in enumerate(h["lens"]):
                L = int(L)
                kc = np.zeros((HKV, L + 1, D), np.float32)
                vc = np.zeros_like(kc)
                kc[:, :L], vc[:, :L] = h["k_cache"][b], h["v_cache"][b]
                ref.append(oracle_decode_out({"q": h["q"][b], "k": h["k"][b], "v": h["v"][b],
                                              "k_cache": kc, "v_cache": vc}, pos=L))
            line["batched"]["parity"] = parity(h["out"], np.stack(ref))
            log(f"parity batched: {line['batched']['parity']}")
        if not args.no_stack:
            h = stk["host"]
            ref = oracle_tokens_out(h["q"], h["k"], h["v"])
            line["stack"]["parity_layer0"] = parity(h["out"], ref.reshape(h["out"].shape))
            log(f"parity stack layer 0 (1024 prefill + 256 decode outputs): "
                f"{line['stack']['parity_layer0']}")
    if not args.no_cpu:
        log("cpu baseline (oracle) ...")
        line["cpu_baseline"] = cpu_baseline_decode(dec["host"], args.cpu_budget)
        if "trait_path" in line:
            cb = line["cpu_baseline"]
            line["trait_path"]["cpu_oracle_us_per_token_layer"] = round(
                decode_bytes(4096) / (cb["value"] * 1e9) * 1e6, 2)
        if not args.no_prefill:
            line["prefill"]["cpu_baseline"] = cpu_baseline_prefill(args.cpu_budget)
        if not args.no_gemv:
            line["gemv"]["cpu_baseline"] = cpu_baseline_gemv(min(args.cpu_budget, 5.0))
        if not args.no_lm_head:
            line["lm_head"]["cpu_baseline"] = cpu_baseline_lm_head(min(args.cpu_budget, 5.0))
    be.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
