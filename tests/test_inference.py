"""The serving-loop driver (inference.py), the semantics of the reference's
PagedAttentionInference (PagedAttentionInference.swift:119-299) over the native
scheduler and cache manager.

CPU: bookkeeping with a host-only cache and a pool small enough to force the
scheduler's memory-pressure preemption (which pauses every running sequence,
Scheduler.swift:135-152), run to completion.  GPU: a short Poisson trace whose
steps run as mixed prefill + decode launches on the real pools.
"""
import numpy as np
import pytest

from pagedattentionmetal_amd.api import SequenceStatus


def _driver(max_blocks, max_batch=8, max_sequences=64, attend=False, layer_kw=None):
    from pagedattentionmetal_amd import api
    from pagedattentionmetal_amd.inference import PagedAttentionInference
    kw = dict(head_dim=128, num_heads=8, num_kv_heads=2, block_size=16, data_type=1)
    kw.update(layer_kw or {})
    eng = api.PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    cache = api.KVCacheManager(eng, max_blocks, kw["block_size"], kw["head_dim"], kw["num_kv_heads"],
                               kw["data_type"], device=attend)
    sched = api.ContinuousBatchingScheduler(max_batch, max_sequences)
    layer = api.PagedLayerSpec(kw["head_dim"], kw["num_heads"], kw["num_kv_heads"], kw["block_size"],
                               kw["data_type"], kw.get("window", 0))
    return PagedAttentionInference(eng, cache, sched, layer, attend=attend), cache, sched


def test_driver_preempts_under_pressure_and_completes():
    inf, cache, sched = _driver(max_blocks=40)
    a = inf.add_request(300, 40)  # 19 blocks each: two fit in 40, their growth (22 each) does not
    b = inf.add_request(300, 40)
    assert (a, b) == (0, 1)
    # runAll (PagedAttentionInference.swift:151-157) stops once no sequence is
    # waiting or running: the pressure event pauses both, and it returns
    inf.run_all(max_steps=500)
    assert inf.preemptions == 2 and inf.completed_count == 0
    assert sched.count(SequenceStatus.paused) == 2
    # stepping on resumes the paused sequences (re-prefilled) until they finish
    for _ in range(500):
        if not inf.step():
            break
    assert inf.completed_count == 2 and inf.waiting_count == 0 and inf.running_count == 0
    assert cache.available_blocks == 40  # every block returned
    assert inf.decoded_tokens == 80  # 40 per request; re-prefills keep the generated count
    # every prefill (first ones and the re-prefills after preemption) counts its prompt
    assert inf.prefill_tokens % 300 == 0 and inf.prefill_tokens >= 600
    assert inf.total_tokens_generated == inf.prefill_tokens + inf.decoded_tokens


def test_driver_rejects_past_max_sequences():
    inf, cache, sched = _driver(max_blocks=100, max_sequences=2)
    assert inf.add_request(10, 2) == 0 and inf.add_request(10, 2) == 1
    assert inf.add_request(10, 2) == -1  # Scheduler.swift:59-70: completed ones still count
    inf.run_all()
    assert inf.completed_count == 2
    assert inf.add_request(10, 2) == -1


def test_driver_out_of_blocks_for_a_prompt_that_cannot_fit():
    from pagedattentionmetal_amd.inference import OutOfBlocks
    inf, cache, sched = _driver(max_blocks=4)
    inf.add_request(200, 3)  # 13 blocks
    with pytest.raises(OutOfBlocks):
        inf.step()


def test_preempted_newcomers_hold_no_blocks():
    """A newcomer that memory pressure pauses in its own step (the handler pauses
    every running sequence, Scheduler.swift:135-152) is not allocated: after the
    step no paused sequence holds blocks."""
    inf, cache, sched = _driver(max_blocks=30)
    inf.add_request(300, 4)  # 19 blocks each: the first fits, the second's pressure pauses both
    inf.add_request(300, 4)
    inf.step()
    assert inf.preemptions == 2
    assert sched.count(SequenceStatus.paused) == 2
    assert cache.available_blocks == 30
    for _ in range(200):
        if not inf.step():
            break
    assert cache.available_blocks == 30


@pytest.mark.gpu
def test_poisson_trace_on_the_gpu():
    W = 256
    import torch
    from pagedattentionmetal_amd.inference import poisson_trace
    inf, cache, sched = _driver(max_blocks=600, max_batch=16, max_sequences=256, attend=True,
                                layer_kw=dict(num_heads=32, num_kv_heads=8, window=W))
    checked = []

    def on_step(i):
        # every row is finite except a prompt's first len - W rows, which see no key under the
        # prefill's single window start len - W (kernels.metal:116-154)
        if inf.last_launch is None:
            return
        ctx, ql = inf.last_launch
        o = inf._out[:int(ql.sum())].float()
        nan_rows = torch.isnan(o).any(-1).any(-1).cpu().numpy()
        want = np.concatenate([np.arange(q) < (q - W if c == 0 else 0) for c, q in zip(ctx, ql)])
        assert (nan_rows == want).all(), (i, ctx, ql)
        assert torch.isfinite(o[torch.from_numpy(~want).cuda()]).all()
        # the step's host mirrors agree with the cache and the scheduler
        for sid in inf.prefilled:
            assert inf._length[sid] == cache.get_sequence_length(sid), (i, sid)
            assert inf._generated[sid] == sched.sequence(sid)["generated"], (i, sid)
        checked.append(i)

    admitted = poisson_trace(inf, steps=40, rate=2.0, prompt_range=(16, 700), output_range=(4, 24), seed=3,
                             on_step=on_step)
    assert admitted > 40 and 30 < inf.step_count <= 40  # an empty batch is not a step (PagedAttentionInference.swift:120)
    assert inf.decoded_tokens > 0 and inf.prefill_tokens > 0 and inf.completed_count > 0
    assert len(checked) > 30
    assert inf.preemptions > 0  # the pool was sized to force it


def test_attended_pairs_match_brute_force():
    """The pair count of a mixed step equals an enumeration of the masks: a chunk's
    rows see keys from its one window start max(0, ctx + T - W) up to their own
    position (causal), a decode row its last min(L + 1, W) keys."""
    rng = np.random.default_rng(5)
    for W in (0, 1, 7, 64):
        inf, _, _ = _driver(max_blocks=8, layer_kw=dict(window=W))
        ctx = rng.integers(0, 100, 12).astype(np.int32)
        ql = rng.integers(1, 90, 12).astype(np.int32)
        ql[::3] = 1
        want = 0
        for c, q in zip(ctx.tolist(), ql.tolist()):
            kv = c + q
            ws = max(0, kv - W) if W else 0
            want += sum(1 for p in range(c, kv) for j in range(kv) if ws <= j <= p)
        assert inf._pairs(ctx, ql) == want


@pytest.mark.gpu
def test_asynchronous_serving_loop_matches_synchronous():
    """The serving loop with the engine asynchronous and untimed (as bench.py's
    wall-clock pass runs it) gives the same bookkeeping and the same outputs of
    its last step as the synchronous, timed default."""
    import torch
    from pagedattentionmetal_amd.inference import poisson_trace
    res = []
    for asynchronous in (False, True):
        inf, cache, sched = _driver(max_blocks=600, max_batch=16, max_sequences=256, attend=True,
                                    layer_kw=dict(num_heads=32, num_kv_heads=8, window=0))
        if asynchronous:
            inf.engine.synchronous = False
            inf.engine.set_gpu_timing(False)
        poisson_trace(inf, steps=25, rate=2.0, prompt_range=(16, 500), output_range=(4, 16), seed=11)
        torch.cuda.synchronize()
        rows = int(inf.last_launch[1].sum())
        res.append((inf.prefill_tokens, inf.decoded_tokens, inf.preemptions, inf.completed_count,
                    inf._out[:rows].float().cpu()))
        inf.engine.synchronize()
    assert res[0][:4] == res[1][:4]
    assert torch.isfinite(res[0][4]).all() and torch.equal(res[0][4], res[1][4])


def _gather(torch, pool, tables):
    """Host copy of the pool blocks the given tables name, and the tables renumbered to it."""
    need = {}
    new = []
    for t in tables:
        new.append([need.setdefault(int(b), len(need)) for b in t])
    order = torch.tensor(sorted(need, key=need.get), dtype=torch.long, device=pool.device)
    host = pool.index_select(0, order).cpu().numpy()
    width = max(len(t) for t in new)
    bt = np.zeros((len(new), width), np.int32)
    for i, t in enumerate(new):
        bt[i, :len(t)] = t
    return host, bt


@pytest.mark.gpu
def test_c5_shape_trace_step_against_oracle():
    """A serving trace at BASELINE c5's layer shape (64 q / 8 kv heads, d 128,
    bs 16, fp16, 4096-token window; prompts U[64, 8192], outputs U[16, 512]):
    an early, a middle and a late step of a 40-step trace (the first step with
    both prompts and decode rows at or after steps 4, 20 and 36) are checked
    against the oracle - every decode row, and the last 16 rows of the longest
    prompt."""
    import torch
    import oracle
    from helpers import TOL, row_rel_err
    from pagedattentionmetal_amd.inference import poisson_trace
    W = 4096
    inf, cache, sched = _driver(max_blocks=16384, max_batch=32, max_sequences=1024, attend=True,
                                layer_kw=dict(num_heads=64, num_kv_heads=8, window=W))
    eng = inf.engine
    orig = eng.mixed_step
    targets = [4, 20, 36]
    seen = {"checked": [], "steps": 0}

    def checked_step(q, out, k_pool, v_pool, bt, ctx, ql, layer, **kw):
        orig(q, out, k_pool, v_pool, bt, ctx, ql, layer, **kw)
        seen["steps"] += 1
        dec = np.nonzero(ql == 1)[0]
        pre = np.nonzero(ql > 1)[0]
        due = [t for t in targets if t <= seen["steps"]]
        if len(due) <= len(seen["checked"]) or len(dec) == 0 or len(pre) == 0:
            return
        torch.cuda.synchronize()
        bs, H, d = layer.block_size, layer.num_heads, layer.head_dim
        cu = np.concatenate([[0], np.cumsum(ql)])
        bth = bt.cpu().numpy()
        # decode rows: key range [max(0, L - W), L) with L = ctx + 1
        lens = (ctx[dec] + 1).astype(np.int64)
        tables = [bth[s, :(int(L) + bs - 1) // bs] for s, L in zip(dec, lens)]
        kh, btd = _gather(torch, k_pool, tables)
        vh, _ = _gather(torch, v_pool, tables)
        qd = q[torch.from_numpy(cu[dec]).cuda()].cpu().numpy()
        ref = oracle.decode(1, qd, kh, vh, btd, lens.astype(np.uint32), H, window=W, n_threads=8)
        got = out[torch.from_numpy(cu[dec]).cuda()].cpu().numpy().astype(np.float64)
        assert row_rel_err(got, ref) <= TOL[1], "decode rows"
        # the last 16 rows of the longest prompt (one window start P - W for all its rows)
        s = int(pre[np.argmax(ql[pre])])
        P = int(ctx[s] + ql[s])
        kh, btp = _gather(torch, k_pool, [bth[s, :(P + bs - 1) // bs]])
        vh, _ = _gather(torch, v_pool, [bth[s, :(P + bs - 1) // bs]])
        rows = slice(int(cu[s] + ql[s] - 16), int(cu[s] + ql[s]))
        qp = q[rows].cpu().numpy()
        refp = oracle.prefill(1, qp, kh, vh, btp[0], P - 16, causal=True, window=W, n_threads=8)
        gotp = out[rows].cpu().numpy().astype(np.float64)
        assert row_rel_err(gotp, refp) <= TOL[1], f"step {seen['steps']}: prompt of {P} tokens"
        seen["checked"].append((seen["steps"], len(dec), P))

    eng.mixed_step = checked_step
    poisson_trace(inf, steps=40, rate=2.0, prompt_range=(64, 8192), output_range=(16, 512), seed=0x5EED0005)
    assert len(seen["checked"]) == 3, seen
    print("checked (step, decode rows, prompt tokens):", seen["checked"])


@pytest.mark.gpu
def test_multi_layer_driver_calls_layers_and_matches_oracle():
    """With several layer specs the driver makes the reference's calls
    (prefill_layers per newcomer, one decode_layers per step); one step's decode
    rows of every layer are checked against the oracle."""
    import torch
    import oracle
    from helpers import TOL, row_rel_err
    from pagedattentionmetal_amd import api
    from pagedattentionmetal_amd.inference import PagedAttentionInference, poisson_trace
    eng = api.PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    H, hkv, d, bs = 32, 8, 128, 16
    cache = api.KVCacheManager(eng, 2048, bs, d, hkv, 1)
    sched = api.ContinuousBatchingScheduler(16, 256)
    layers = [api.PagedLayerSpec(d, H, hkv, bs, 1) for _ in range(3)]
    inf = PagedAttentionInference(eng, cache, sched, layers)
    calls = {"prefill": 0, "decode": 0, "checked": 0}
    orig_p, orig_d = eng.prefill_layers, eng.decode_layers

    def prefill_layers(*a, **kw):
        calls["prefill"] += 1
        return orig_p(*a, **kw)

    def decode_layers(qs, k_pool, v_pool, bt, sl, outs, B, width, lays, **kw):
        calls["decode"] += 1
        orig_d(qs, k_pool, v_pool, bt, sl, outs, B, width, lays, **kw)
        if calls["decode"] != 3:
            return
        torch.cuda.synchronize()
        lens = sl.cpu().numpy().astype(np.uint32)
        bth = bt.cpu().numpy()
        tables = [bth[b, :(int(L) + bs - 1) // bs] for b, L in enumerate(lens)]
        kh, btd = _gather(torch, k_pool, tables)
        vh, _ = _gather(torch, v_pool, tables)
        for i in range(len(lays)):
            ref = oracle.decode(1, qs[i].cpu().numpy(), kh, vh, btd, lens, H, n_threads=8)
            assert row_rel_err(outs[i].cpu().numpy().astype(np.float64), ref) <= TOL[1], f"layer {i}"
        calls["checked"] += 1

    eng.prefill_layers, eng.decode_layers = prefill_layers, decode_layers
    poisson_trace(inf, steps=12, rate=1.5, prompt_range=(16, 600), output_range=(4, 12), seed=21)
    assert calls["checked"] == 1
    assert calls["prefill"] > 0 and calls["decode"] >= 3
    assert inf.decoded_tokens > 0
