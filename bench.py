#!/usr/bin/env python3
"""Benchmark of the ragged paged-attention path on one MI355X.

Headline (BASELINE.json metric): paged decode KV GB/s on configuration c2 (GQA
fp16 ragged decode, B=64, L~U[128,4096], 32 query / 8 KV heads, d=128, bs=16,
32768-block shuffled pool with a shared 512-token prefix), plus the chunked
prefill TFLOP/s of the c3 mixed continuous-batching step.  A step is one decode
of the whole batch with Q, pools and tables already resident in HBM.

  python bench.py [--steps K] [--warmup W] [--no-configs] [--no-trace] [--no-cpu]

Prints one JSON line.  "configs" holds the c1, c4 and c5 decode lines (skipped
with --no-configs); "trace_c5" the 200-step scheduler trace of c5 (skipped with
--no-trace); "next_rows" the fused prefill, backward, copy-on-write and adapter
measurements (skipped with --no-next).  Every configuration carries a CPU baseline: the oracle on
the host's cores over a bounded sample of the same inputs (skipped with
--no-cpu).  The roofline block times the dominant kernel (the decode attention
kernel) with HIP events on the stream it is launched on.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
# untimed steps before any timed loop (the ramp from idle clocks measured
# 4-16% slow over the first ~100 steps)
MIN_WARMUP = 200
METRIC = "paged decode KV GB/s (% HBM peak) + chunked-prefill TFLOP/s, 1 MI355X"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_setup(k, torch, api, workloads):
    """Device tensors for decode workload k (FP8 pools are quantised by the append kernel)."""
    w = workloads.config(k)
    q, kp, vp = workloads.device_pools(w)
    eng = api.PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    bt = torch.from_numpy(w.block_tables).cuda()
    lens = torch.from_numpy(w.seq_lens.view("int32")).cuda()
    ks = vs = None
    if w.data_type == 2:
        # quantise-on-append: every sequence's tokens go through the FP8 append kernel
        src_k, src_v = kp, vp
        kp = torch.zeros(src_k.shape, dtype=torch.uint8, device="cuda")
        vp = torch.zeros_like(kp)
        ks = torch.zeros(w.pool_blocks, dtype=torch.float16, device="cuda")
        vs = torch.zeros_like(ks)
        lay = api.PagedLayerSpec(w.head_dim, w.num_kv_heads, w.num_kv_heads, w.block_size, 2)
        for b in range(w.batch):
            L = int(w.seq_lens[b])
            tok = torch.arange(L, device="cuda")
            phys = bt[b][tok // w.block_size].long()
            keys = src_k[phys, tok % w.block_size].contiguous()
            vals = src_v[phys, tok % w.block_size].contiguous()
            eng.append_to_cache(keys, vals, kp, vp, bt[b].contiguous(), 0, L, lay, k_scale=ks, v_scale=vs)
        del src_k, src_v
        torch.cuda.synchronize()
    layer = api.PagedLayerSpec(w.head_dim, w.num_heads, w.num_kv_heads, w.block_size, w.data_type, w.window)
    out = torch.empty(q.shape, dtype=q.dtype, device="cuda")
    return w, eng, (q, kp, vp, bt, lens, out, layer, ks, vs)


def event_steps(torch, stream, step, n, depth=2):
    """Per-step GPU times (ms) from HIP events recorded on `stream` around each
    step, with at most `depth` steps in flight (a serving loop waits for each
    step's output; a queue thousands of launches deep is not a serving loop and
    measured unsteady).  Returns the list of n durations."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i in range(n):
        if i >= depth:
            ev[i - depth][1].synchronize()
        ev[i][0].record(stream)
        step()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def median(xs):
    xs = sorted(xs)
    n = len(xs)
    return xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])


def time_decode(torch, eng, w, t, steps, warmup):
    q, kp, vp, bt, lens, out, layer, ks, vs = t
    stream = torch.cuda.current_stream()
    eng.set_stream(stream)
    eng.synchronous = False

    def step():
        eng.decode(q, kp, vp, bt, lens, out, w.batch, w.max_num_blocks, layer, k_scale=ks, v_scale=vs)

    # the timed steps run as a serving loop would: no per-call timing events.
    # At least MIN_WARMUP untimed steps whatever --warmup says: the GPU leaves the
    # host-side set-up at idle clocks and a short warm-up times the ramp
    eng.set_gpu_timing(False)
    for _ in range(max(warmup, MIN_WARMUP)):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # BASELINE's timing rule: HIP events around each step, median of the steps
    med = median(event_steps(torch, stream, step, max(steps, 100)))
    eng.set_gpu_timing(True)
    # per-kernel durations: HIP events recorded by the engine around each launch
    kern, red = [], []
    for _ in range(steps):
        step()
        s = eng.last_stats
        kern.append(s["kernel_ms"])
        red.append(s["reduce_ms"])
    torch.cuda.synchronize()
    kern_ms = sum(kern) / len(kern)
    red_ms = sum(red) / len(red)
    return ms, kern_ms, red_ms, med


def mixed_setup(torch, api, workloads):
    """Device tensors for the c3 mixed step: cached context in the pool, new tokens to append."""
    w = workloads.mixed_config()
    kp, vp, q, nk, nv = workloads.mixed_pools(w)
    bt = torch.from_numpy(w.block_tables).cuda()
    out = torch.empty_like(q)
    eng = api.PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    layer = api.PagedLayerSpec(w.head_dim, w.num_heads, w.num_kv_heads, w.block_size, 1)
    return w, eng, (q, kp, vp, bt, nk, nv, out, layer)


def time_mixed(torch, eng, w, t, steps, warmup):
    """Whole mixed step (append + prefill chunks + decode rows), then the prefill
    chunks alone (the dense prefill kernel, timed by the engine's HIP events);
    both the median over the timed steps."""
    q, kp, vp, bt, nk, nv, out, layer = t
    stream = torch.cuda.current_stream()
    eng.set_stream(stream)
    eng.synchronous = False
    ctx, ql = w.context_lens, w.query_lens
    nch = int((ql > 1).sum())
    rows_ch = int(ql[:nch].sum())

    def step():
        eng.mixed_step(q, out, kp, vp, bt, ctx, ql, layer, new_keys=nk, new_values=nv)

    def prefill_only():
        eng.mixed_step(q[:rows_ch], out[:rows_ch], kp, vp, bt[:nch], ctx[:nch], ql[:nch], layer)

    assert (ql[:nch] > 1).all() and (ql[nch:] == 1).all()
    # the timed steps run as a serving loop would: no per-call timing events,
    # each step's output awaited before the step after next is issued (event_steps)
    eng.set_gpu_timing(False)
    for _ in range(max(warmup, MIN_WARMUP)):
        step()
    torch.cuda.synchronize()
    ms = median(event_steps(torch, stream, step, max(steps, 100)))
    eng.set_gpu_timing(True)
    for _ in range(max(warmup, MIN_WARMUP // 4)):
        prefill_only()
    kern = []
    for _ in range(steps):
        prefill_only()
        kern.append(eng.last_stats["kernel_ms"])
    torch.cuda.synchronize()
    return ms, median(kern)


def compact_rows(torch, w, t, B):
    """Host copies of the pool blocks that rows 0..B-1 read (their window only),
    gathered on the device, and the tables renumbered to them."""
    import numpy as np
    q, kp, vp, bt, lens, out, layer, ks, vs = t
    L = w.seq_lens[:B].astype(np.int64)
    bs = w.block_size
    need = {}
    new_bt = np.zeros((B, w.max_num_blocks), np.int32)
    for b in range(B):
        first = max(0, int(L[b]) - w.window) // bs if w.window > 0 else 0
        for i in range(first, (int(L[b]) + bs - 1) // bs):
            new_bt[b, i] = need.setdefault(int(w.block_tables[b, i]), len(need))
    order = torch.tensor(sorted(need, key=need.get), dtype=torch.long, device=kp.device)
    kh, vh = kp.index_select(0, order).cpu().numpy(), vp.index_select(0, order).cpu().numpy()
    if w.data_type == 2:
        ksh = ks.index_select(0, order).cpu().numpy().view(np.uint16)
        vsh = vs.index_select(0, order).cpu().numpy().view(np.uint16)
    else:
        ksh = vsh = None
    return q[:B].cpu().numpy(), kh, vh, ksh, vsh, new_bt


def cpu_baseline_decode(torch, w, t, threads, batch=None, min_seconds=2.0, max_reps=5):
    """The oracle (C restatement of the reference's paged attention) on host cores:
    the first `batch` sequences of the step (all by default), repeated until
    `min_seconds` of wall time (at most `max_reps` passes); returns GB/s, seconds
    and passes."""
    import numpy as np

    import oracle
    B = w.batch if batch is None else batch
    qh, kh, vh, ksh, vsh, bt = compact_rows(torch, w, t, B)
    L = w.seq_lens[:B].astype(np.int64)
    if w.window > 0:
        L = np.minimum(L, w.window)
    elem = {0: 4, 1: 2, 2: 1}[w.data_type]
    nbytes = int(L.sum()) * w.num_kv_heads * w.head_dim * 2 * elem
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.decode(w.data_type, qh, kh, vh, bt, w.seq_lens[:B], w.num_heads, window=w.window,
                      k_scale=ksh, v_scale=vsh, n_threads=threads)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds or reps >= max_reps:
            break
    return nbytes * reps / dt / 1e9, dt, reps


def cpu_baseline_prefill(torch, w3, t3, threads, rows=64, min_seconds=1.0, max_reps=5):
    """The oracle's causal prefill on host cores for the first `rows` rows of the
    first c3 chunk (its cached context included); returns TFLOP/s, seconds,
    passes and the sample's description."""
    import numpy as np

    import oracle
    q, kp, vp, bt, nk, nv, out, layer = t3
    ctx, ql = int(w3.context_lens[0]), int(w3.query_lens[0])
    T = min(rows, ql)
    kv_len = ctx + T
    nb = (kv_len + w3.block_size - 1) // w3.block_size
    blocks = torch.from_numpy(w3.block_tables[0, :nb].astype(np.int64)).to(kp.device)
    kh, vh = kp.index_select(0, blocks).cpu().numpy(), vp.index_select(0, blocks).cpu().numpy()
    qh = q[:T].cpu().numpy()
    flops = 4 * w3.head_dim * w3.num_heads * (T * ctx + T * (T + 1) // 2)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.prefill(1, qh, kh, vh, np.arange(nb, dtype=np.int32), ctx, causal=True, n_threads=threads)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds or reps >= max_reps:
            break
    return flops * reps / dt / 1e12, dt, reps, f"rows [{ctx}, {ctx + T}) of a causal prefill at context {ctx} (chunk 0)"


def run_next_rows(torch, api, workloads, cpu=True, threads=16):
    """The rows after the hot path, each on one shape with its roofline and a CPU
    baseline: fused append + prefill (one 4096-token prompt), the backward (a
    4096-token sequence), copy-on-write of a shared prefix block, and the
    framework adapter's decode step."""
    import numpy as np

    out = {}
    H, hkv, d, bs = 32, 8, 128, 16
    eng = api.PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    stream = torch.cuda.current_stream()
    eng.set_stream(stream)
    layer = api.PagedLayerSpec(d, H, hkv, bs, 1)
    seed = workloads.SEED_BASE + 6

    def timed(fn, reps, warm=3):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        ms = median(event_steps(torch, stream, fn, reps))
        return ms

    # f2: fused append + prefill of one prompt (PagedAttentionEngine.fusedPrefill)
    T = 4096
    nbl = T // bs
    perm = torch.from_numpy(workloads.permutation(seed, 2 * nbl)[:nbl].astype(np.int32)).cuda()
    kp = torch.zeros((2 * nbl, bs, hkv, d), dtype=torch.float16, device="cuda")
    vp = torch.zeros_like(kp)
    q = workloads.device_normals((T, H, d), torch.float16, seed, workloads.S_Q)
    rk = workloads.device_normals((T, hkv, d), torch.float16, seed, workloads.S_NEW_K, 0.5)
    rv = workloads.device_normals((T, hkv, d), torch.float16, seed, workloads.S_NEW_V, 0.5)
    o = torch.empty_like(q)
    eng.synchronous = False
    eng.set_gpu_timing(False)
    # 200 warm-up calls each: the first calls after the set-up run at ramping
    # clocks (measured 6% slow with 30)
    fused_ms = timed(lambda: eng.fused_prefill(q, rk, rv, perm, kp, vp, o, T, layer), 30, warm=200)
    sep_ms = timed(lambda: (eng.append_to_cache(rk, rv, kp, vp, perm, 0, T, layer),
                            eng.prefill(q, kp, vp, perm, o, T, layer, causal=True)), 30, warm=200)
    flops = 4 * d * H * T * (T + 1) // 2
    f2 = {"workload": f"one {T}-token causal prompt, append of its K/V included, {H}/{hkv} heads, d={d}, bs={bs}, f16",
          "ms": round(fused_ms, 4), "tflops": round(flops / (fused_ms * 1e-3) / 1e12, 1),
          "peak_tflops": 2500.0, "frac": round(flops / (fused_ms * 1e-3) / 1e12 / 2500.0, 4),
          "append_then_prefill_ms": round(sep_ms, 4)}
    if cpu:
        import oracle
        rows = 32
        qh, kh, vh = q[T - rows:].cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy()
        bth = perm.cpu().numpy()
        cf = 4 * d * H * (rows * (T - rows) + rows * (rows + 1) // 2)
        t0, reps = time.perf_counter(), 0
        while True:
            oracle.prefill(1, qh, kh, vh, bth, T - rows, causal=True, n_threads=threads)
            reps += 1
            if time.perf_counter() - t0 >= 2.0 or reps >= 50:
                break
        dt = time.perf_counter() - t0
        f2["cpu_baseline"] = {"value": round(cf * reps / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
                              "kind": "port",
                              "sample": f"{reps} x the last {rows} rows of the prompt through the C oracle, {dt:.2f} s"}
    out["f2_fused_prefill"] = f2

    # f4: backward of one sequence (PagedAttentionEngine.backward)
    go = workloads.device_normals((T, H, d), torch.float16, seed, 9)
    m = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    lsum = torch.full((T, H), float(T), dtype=torch.float32, device="cuda")
    dq = torch.empty_like(q)
    dk, dv = torch.zeros_like(kp), torch.zeros_like(vp)
    bwd_ms = timed(lambda: eng.backward(q, kp, vp, perm, go, m, lsum, dq, dk, dv, T, layer), 10, warm=2)
    bflops = 10 * T * T * d * H
    f4 = {"workload": f"non-causal backward of one {T}-token sequence, {H}/{hkv} heads, d={d}, f16 "
                      "(dQ, dK, dV; flops 10 T^2 d H)",
          "ms": round(bwd_ms, 4), "tflops": round(bflops / (bwd_ms * 1e-3) / 1e12, 1), "peak_tflops": 2500.0,
          "frac": round(bflops / (bwd_ms * 1e-3) / 1e12 / 2500.0, 4)}
    if cpu:
        import oracle
        Ts = 256
        rng = np.random.default_rng(1)
        qs = rng.standard_normal((Ts, H, d)).astype(np.float16)
        ks = rng.standard_normal((Ts // bs, bs, hkv, d)).astype(np.float16)
        vs = rng.standard_normal((Ts // bs, bs, hkv, d)).astype(np.float16)
        gs = rng.standard_normal((Ts, H, d)).astype(np.float16)
        bts = np.arange(Ts // bs, dtype=np.int32)
        mm, ll, _ = oracle.forward_stats(qs, ks, vs, bts)
        t0, reps = time.perf_counter(), 0
        while True:
            oracle.backward(qs, ks, vs, bts, gs, mm, ll)
            reps += 1
            if time.perf_counter() - t0 >= 2.0 or reps >= 20:
                break
        dt = time.perf_counter() - t0
        f4["cpu_baseline"] = {"value": round(10 * Ts * Ts * d * H * reps / dt / 1e12, 6), "unit": "TFLOP/s",
                              "cores": 1, "kind": "port",
                              "sample": f"{reps} x the backward of a {Ts}-token sequence (same heads) through the "
                                        f"oracle, {dt:.2f} s"}
    out["f4_backward"] = f4
    eng.synchronous = True
    eng.set_gpu_timing(True)

    # f1: copy-on-write of a shared prefix block (KVCacheManager.ensureExclusiveAccess)
    nseq = 64
    cache = api.KVCacheManager(eng, 4 * nseq, bs, d, hkv, 1)
    cache.allocate_sequence(0)
    cache.append_tokens(0, bs, block_hashes=[0xC0FFEE])
    for sid in range(1, nseq + 1):
        cache.allocate_sequence(sid)
        cache.append_tokens(sid, bs, block_hashes=[0xC0FFEE])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for sid in range(1, nseq + 1):
        cache.ensure_exclusive_access(sid, 0)
    torch.cuda.synchronize()
    cow_us = (time.perf_counter() - t0) / nseq * 1e6
    out["f1_copy_on_write"] = {"workload": f"{nseq} sequences sharing one {bs}-token f16 prefix block "
                                           f"({hkv} kv heads, d={d}) each made exclusive",
                               "us_per_call": round(cow_us, 2), "bytes_per_call": 2 * bs * hkv * d * 2,
                               "note": "one synchronous call per block: host bookkeeping plus a device copy"}

    # f3: the adapter's decode step (PagedMetalKVCache.pagedAttention)
    from pagedattentionmetal_amd.adapter import PagedTorchKVCache
    ctx_len = 4096
    ad = PagedTorchKVCache(1, layer, (ctx_len + 512) // bs + 2)  # its own engine, on the torch stream
    qp = workloads.device_normals((1, H, ctx_len, d), torch.float16, seed, 10)
    kpf = workloads.device_normals((1, hkv, ctx_len, d), torch.float16, seed, 11, 0.5)
    vpf = workloads.device_normals((1, hkv, ctx_len, d), torch.float16, seed, 12, 0.5)
    ad.paged_attention(qp, kpf, vpf, mask="causal")
    q1, k1, v1 = qp[:, :, :1].contiguous(), kpf[:, :, :1].contiguous(), vpf[:, :, :1].contiguous()
    # the first step creates the sequence's device table (one allocation); the
    # warm-up steps also take the clocks out of idle
    for _ in range(50):
        ad.paged_attention(q1, k1, v1)
    steps = 200
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        ad.paged_attention(q1, k1, v1)
    t_issue = time.perf_counter() - t0
    torch.cuda.synchronize()
    step_us = (time.perf_counter() - t0) / steps * 1e6
    out["f3_adapter"] = {"workload": f"decode steps of one sequence after a {ctx_len}-token prompt through "
                                     "PagedTorchKVCache.paged_attention (append + decode, batch 1)",
                         "us_per_step": round(step_us, 1),
                         "host_us_per_step": round(t_issue / steps * 1e6, 1),
                         "kv_bytes_per_step": (ctx_len + 50 + steps // 2) * hkv * d * 2 * 2,
                         "note": "batch 1 is launch- and host-bound; the step includes the cache bookkeeping"}
    return out


def run_trace_c5(torch, api, steps=200, seed=0x5EED0005):
    """BASELINE c5's serving trace: `steps` ContinuousBatchingScheduler steps with
    Poisson(2) arrivals, prompts U[64,8192], outputs U[16,512], max batch 32,
    on the c5 layer (64/8 heads, d=128, bs=16, fp16, 4096-token window) with a
    block pool of 60% of the GPU's memory.  Each step is one mixed prefill +
    decode launch set on synthetic Q and K/V.

    Two passes over the same seeded trace: the first in the engine's default
    synchronous mode with per-call HIP events (GPU time per step); the second
    as a serving loop runs, asynchronous and without events, for the
    wall-clock rate (host scheduling overlapping the GPU)."""
    import gc
    from pagedattentionmetal_amd.inference import PagedAttentionInference, poisson_trace
    H, hkv, d, bs, W = 64, 8, 128, 16, 4096
    _, total = torch.cuda.mem_get_info()
    blocks = int(0.6 * total / (2 * bs * hkv * d * 2))

    def one_pass(timed):
        eng = api.PagedAttentionEngine()
        eng.set_graceful_degradation(False)
        eng.set_stream(torch.cuda.current_stream())
        if not timed:
            eng.synchronous = False
            eng.set_gpu_timing(False)
        cache = api.KVCacheManager(eng, blocks, bs, d, hkv, 1)
        sched = api.ContinuousBatchingScheduler(32, 1024)  # maxSequences raised: completed ones still count
        inf = PagedAttentionInference(eng, cache, sched, api.PagedLayerSpec(d, H, hkv, bs, 1, W), seed=seed)
        gpu_ms = []
        seen = [None]

        def on_step(i):
            if timed and inf.last_launch is not seen[0]:  # the step launched work
                gpu_ms.append(eng.last_stats["kernel_ms"])
                seen[0] = inf.last_launch

        torch.cuda.synchronize()
        t0 = time.perf_counter()
        admitted = poisson_trace(inf, steps, 2.0, (64, 8192), (16, 512), seed, on_step=on_step)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        res = dict(admitted=admitted, completed=inf.completed_count, preemptions=inf.preemptions,
                   prefill=inf.prefill_tokens, decoded=inf.decoded_tokens, wall=wall, gpu=sum(gpu_ms) * 1e-3,
                   flops=4 * d * H * inf.attended_pairs)
        inf = None
        cache.close()
        eng.close()
        gc.collect()
        torch.cuda.empty_cache()
        return res

    a = one_pass(True)
    b = one_pass(False)
    assert (a["prefill"], a["decoded"], a["preemptions"]) == (b["prefill"], b["decoded"], b["preemptions"])
    tokens = b["prefill"] + b["decoded"]
    return {"workload": f"c5 trace: {steps} scheduler steps, Poisson(2) arrivals, prompts U[64,8192], outputs "
                        f"U[16,512], max batch 32, 64/8 heads, d=128, bs=16, fp16, window {W}, pool {blocks} blocks "
                        f"(60% of HBM); one mixed prefill + decode launch set per step",
            "requests_admitted": b["admitted"], "completed": b["completed"], "preemptions": b["preemptions"],
            "prefill_tokens": b["prefill"], "decoded_tokens": b["decoded"],
            "wall_s": round(b["wall"], 4), "tokens_per_s_wall": round(tokens / b["wall"], 1),
            "wall_s_synchronous": round(a["wall"], 4),
            "gpu_s": round(a["gpu"], 4), "tokens_per_s_gpu": round(tokens / a["gpu"], 1) if a["gpu"] > 0 else None,
            # 4 d H flops per unmasked (row, key) pair over all the steps' kernels (append and decode included)
            "attention_flops": a["flops"],
            "attention_tflops_gpu": round(a["flops"] / a["gpu"] / 1e12, 1) if a["gpu"] > 0 else None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # the GPU comes out of the host-side set-up at idle clocks; the first ~100
    # steps after it run 4-6% slower (measured), so the default warms up past that
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--all", action="store_true", help="measure c1, c4, c5 too (the default; kept for old command lines)")
    ap.add_argument("--no-configs", action="store_true", help="skip the c1, c4, c5 lines")
    ap.add_argument("--no-trace", action="store_true", help="skip the c5 scheduler trace")
    ap.add_argument("--trace-only", action="store_true",
                    help="run only the c5 scheduler trace and print its JSON object (for profiling it)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-next", action="store_true",
                    help="skip the next rows (fused prefill, backward, copy-on-write, adapter)")
    ap.add_argument("--only", choices=("c1", "c2", "c3", "c4", "c5", "next"),
                    help="time one configuration alone and print its JSON object (for profiling it)")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run the 1 GiB read and copy calibration streams (achievable HBM rate; "
                         "the byte counters of a profiling run are scaled by what they read on these)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the paged-attention path runs on a single GPU "
              "(sharding is a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from pagedattentionmetal_amd import api, workloads

    torch.cuda.set_device(0)
    if args.trace_only:
        print(json.dumps({"trace_c5": run_trace_c5(torch, api)}), flush=True)
        return
    if args.only and args.calibrate:
        # the calibration streams in the same process, for scaling the byte counters
        gib = 1 << 30
        src = torch.empty(gib, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        ec = api.PagedAttentionEngine()
        for _ in range(3):
            ec.calib_stream_read(src)
            ec.calib_stream_copy(src, dst)
        del src, dst, ec
        torch.cuda.empty_cache()
    if args.only == "next":
        print(json.dumps({"next_rows": run_next_rows(torch, api, workloads, cpu=False)}), flush=True)
        return
    if args.only == "c3":
        w3, e3, t3 = mixed_setup(torch, api, workloads)
        ms3, pk_ms = time_mixed(torch, e3, w3, t3, args.steps, args.warmup)
        print(json.dumps({"c3": {"mixed_step_ms": round(ms3, 5), "prefill_kernel_ms": round(pk_ms, 5),
                                 "tflops": round(w3.prefill_flops() / (pk_ms * 1e-3) / 1e12, 2)}}), flush=True)
        return
    if args.only:
        k = int(args.only[1])
        wk, ek, tk = decode_setup(k, torch, api, workloads)
        msk, kk, rk, mk = time_decode(torch, ek, wk, tk, args.steps, args.warmup)
        print(json.dumps({args.only: {"ms_per_step": round(msk, 5), "kernel_ms": round(kk, 5),
                                      "kernel_ms_median": round(mk, 5),
                                      "kv_GBps": round(wk.kv_bytes() / (msk * 1e-3) / 1e9, 2)}}), flush=True)
        return
    log("bench: c2 decode setup")
    w, eng, t = decode_setup(2, torch, api, workloads)
    ms, kern_ms, red_ms, med_ms = time_decode(torch, eng, w, t, args.steps, args.warmup)
    kv = w.kv_bytes()
    gbs = kv / (ms * 1e-3) / 1e9
    # A c2 step is exactly one launch of the decode kernel (stream-K: no reduce,
    # no staging), so the timed loop's time per step is that kernel's average
    # launch duration over the timed region.  The engine's per-launch events
    # (kern_ms) bracket each launch with their own packets and read a few us more.
    achieved = kv / (ms * 1e-3) / 1e9
    log(f"bench: c2 {ms:.4f} ms/step ({gbs:.1f} GB/s), decode kernel {kern_ms:.4f} ms, after it {red_ms:.4f} ms")

    log("bench: c3 mixed step setup")
    w3, e3, t3 = mixed_setup(torch, api, workloads)
    ms3, pk_ms = time_mixed(torch, e3, w3, t3, args.steps, args.warmup)
    pflops = w3.prefill_flops()
    tflops = pflops / (pk_ms * 1e-3) / 1e12
    log(f"bench: c3 mixed step {ms3:.4f} ms; prefill kernel {pk_ms:.4f} ms = {tflops:.1f} TFLOP/s")
    # the dense f16 MFMA rate this part sustains at its power-limited clock
    # (pam_calib_mfma: MFMAs only, one 8-wave workgroup per CU), beside the
    # published peak the roofline uses
    e3.calib_mfma(20000)  # untimed: clocks settle over the first milliseconds
    mfma_ceiling = e3.calib_mfma(60000)
    log(f"bench: MFMA-only loop {mfma_ceiling:.0f} TFLOP/s")
    cpu3 = None
    if not args.no_cpu:
        threads = max(1, min(16, os.cpu_count() or 1))
        log("bench: CPU baseline for the c3 prefill rows")
        ctf, cdt, creps, what = cpu_baseline_prefill(torch, w3, t3, threads, min_seconds=5.0, max_reps=100)
        cpu3 = {"value": round(ctf, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
                "sample": f"{creps} x {what} through the C oracle on {threads} host threads, {cdt:.2f} s"}
    del t3, e3
    torch.cuda.empty_cache()

    traffic = None
    tp = os.path.join(ROOT, "profiles", "decode_c2_traffic.json")
    if os.path.exists(tp):
        with open(tp) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        threads = max(1, min(16, os.cpu_count() or 1))
        log(f"bench: CPU baseline (oracle, {threads} threads) on the full c2 batch")
        cgbs, cdt, creps = cpu_baseline_decode(torch, w, t, threads, min_seconds=10.0, max_reps=200)
        log(f"bench: CPU baseline single-threaded on the first 8 sequences")
        sgbs, sdt, sreps = cpu_baseline_decode(torch, w, t, 1, batch=8)
        cpu = {"value": round(cgbs, 4), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{creps} x one full c2 decode step (B=64, {kv / 1e9:.3f} GB of KV) through the C "
                         f"oracle, OpenMP over (sequence, head) on {threads} host threads, {cdt:.2f} s",
               "single_thread": {"value": round(sgbs, 4), "unit": "GB/s", "cores": 1,
                                 "sample": f"{sreps} x the first 8 sequences of the c2 step, {sdt:.2f} s"}}
    del t, eng

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (SplitMix64 counter-based generator, seed 0x5EED0002; K/V ~ N(0, 0.5^2), shuffled pool)",
        "config": {"workload": "c2: GQA fp16 ragged paged decode, B=64, L~U[128,4096] (sharers U[513,4096]), "
                               "32 q / 8 kv heads, d=128, bs=16, 32768-block shuffled pool, 32 shared "
                               "prefix blocks in 32 tables",
                   "batch": w.batch, "kv_bytes_per_step": kv,
                   "tokens_per_s": round(w.batch / (ms * 1e-3), 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "attn_mfma_streamk<f16,128,bs16> (stream-K split, partials merged in the "
                               "kernel; no reduce launch)",
                     "kernel_ms": round(ms, 5),
                     "kernel_ms_median": round(med_ms, 5),
                     "kernel_ms_per_launch_events": round(kern_ms, 5)},
        "cpu_baseline": cpu,
        "prefill": {"workload": "c3: mixed continuous-batching step, 8 chunks x 512 new tokens (context "
                                "U[0,3584], causal) + 56 decodes (context U[256,4096]), 32 q / 8 kv heads, "
                                "d=128, bs=16, fp16, append of the new K/V included in the step",
                    "mixed_step_ms": round(ms3, 5),
                    "mixed_step_form": "automatic: one launch with the prefill and the decode rows side by side "
                                       "on CUs of their own when its estimate wins (c3: it does), else separate",
                    "step_tflops": round(pflops / (ms3 * 1e-3) / 1e12, 2),
                    "tokens_per_s": round(w3.total_rows / (ms3 * 1e-3), 1),
                    "prefill_kernel": "prefill_mfma_kernel<128>", "prefill_kernel_ms": round(pk_ms, 5),
                    "flops_per_launch": pflops, "tflops": round(tflops, 2), "peak_tflops": FP16_PEAK_TFLOPS,
                    "frac": round(tflops / FP16_PEAK_TFLOPS, 4),
                    "mfma_loop_tflops": round(mfma_ceiling, 1),
                    "frac_of_mfma_loop": round(tflops / mfma_ceiling, 4) if mfma_ceiling > 0 else None,
                    "cpu_baseline": cpu3},
    }

    if args.calibrate:
        import torch as _t
        gib = 1 << 30
        src = _t.empty(gib, dtype=_t.uint8, device="cuda").fill_(1)
        dst = _t.empty_like(src)
        ec = api.PagedAttentionEngine()
        rd = min(ec.calib_stream_read(src) for _ in range(5))
        cp = min(ec.calib_stream_copy(src, dst) for _ in range(5))
        result["calibration"] = {"stream_read_GBps": round(gib / (rd * 1e-3) / 1e9, 1),
                                 "stream_copy_GBps": round(2 * gib / (cp * 1e-3) / 1e9, 1),
                                 "bytes": gib}
        del src, dst

    if not args.no_configs:
        # the other decode configurations, each beside the oracle on a bounded
        # sample of its rows (c1 whole; c4 and c5 the first 16 and 4 rows)
        cfgs = {}
        for k, sample in ((1, None), (4, 16), (5, 4)):
            log(f"bench: c{k} decode")
            wk, ek, tk = decode_setup(k, torch, api, workloads)
            msk, kk, rk, mk = time_decode(torch, ek, wk, tk, args.steps, args.warmup)
            b = wk.kv_bytes()
            # c4 and c5 are one launch per step (stream-K, no reduce): the loop's
            # time per step is the kernel's; c1 adds the reduce kernel
            cfgs[f"c{k}"] = {"ms_per_step": round(msk, 5), "kv_GBps": round(b / (msk * 1e-3) / 1e9, 2),
                             "kernel_ms": round(kk, 5), "reduce_ms": round(rk, 5),
                             "kernel_ms_median": round(mk, 5),
                             "kernel_frac_hbm": round(b / (msk * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                             "tokens_per_s": round(wk.batch / (msk * 1e-3), 1)}
            if not args.no_cpu:
                threads = max(1, min(16, os.cpu_count() or 1))
                # (c1 is a few MB: its passes repeat until half a second has passed)
                cg, cd, cr = cpu_baseline_decode(torch, wk, tk, threads, batch=sample,
                                                 min_seconds=0.5 if sample is None else 1.0,
                                                 max_reps=100000 if sample is None else 5)
                rows = wk.batch if sample is None else sample
                cfgs[f"c{k}"]["cpu_baseline"] = {
                    "value": round(cg, 4), "unit": "GB/s", "cores": threads, "kind": "port",
                    "sample": f"{cr} x the first {rows} rows of the c{k} step through the C oracle, {cd:.2f} s"}
            del tk, ek
            torch.cuda.empty_cache()
        result["configs"] = cfgs
    if not args.no_trace:
        log("bench: c5 scheduler trace")
        result["trace_c5"] = run_trace_c5(torch, api)
    if not args.no_next:
        log("bench: next rows (fused prefill, backward, copy-on-write, adapter)")
        result["next_rows"] = run_next_rows(torch, api, workloads, cpu=not args.no_cpu)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
