"""libpam's C++ host logic against the reference semantics (CPU only, no GPU calls).

Known answers come from the reference's own tests
(Tests/PagedAttentionMetalTests/PagedAttentionMetalTests.swift: cabiLifecycle :586,
prefillWithZeroBlocks :736, allocateThenImmediateFree :755,
appendBeyondBlockBoundary :794); randomized sequences compare the C++ allocator
and scheduler with the restatements in oracle/allocator.py and oracle/scheduler.py.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

from oracle.allocator import BEST_FIT, FIFO, LIFO, OutOfMemory, RefAllocator
from oracle.scheduler import PAUSED, RUNNING, WAITING, COMPLETED, RefScheduler

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def pam():
    from pagedattentionmetal_amd import _lib
    return _lib.load()


@pytest.fixture()
def ctx(pam):
    c = pam.pam_create_context()
    assert c
    yield c
    pam.pam_destroy_context(c)


def host_cache(pam, ctx, max_blocks, bs=16, hd=32, hkv=1, dtype=0):
    c = pam.pam_create_cache_host(ctx, max_blocks, bs, hd, hkv, dtype)
    assert c, pam.pam_last_error(ctx)
    return c


def table(pam, ctx, cache, sid):
    n = pam.pam_block_table(ctx, cache, sid, None, 0)
    assert n >= 0
    buf = (C.c_int32 * max(n, 1))()
    pam.pam_block_table(ctx, cache, sid, buf, n)
    return list(buf[:n])


# ---------------------------------------------------------------- C ABI surface

def test_library_exports_every_declared_symbol(pam):
    header = open(os.path.join(ROOT, "include", "pam.h")).read()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    names = set(re.findall(r"\b(pam_[a-z0-9_]+)\s*\(", header))
    assert len(names) > 60
    for n in sorted(names):
        assert hasattr(pam, n), f"{n} declared in include/pam.h but not exported"
    from pagedattentionmetal_amd import _lib
    assert names == set(_lib.SIGNATURES), "ctypes bindings out of sync with include/pam.h"


def test_error_convention(pam, ctx):
    assert pam.pam_last_error(ctx) is None
    assert pam.pam_reserve_sequence(ctx, None, 1) == -1
    c = host_cache(pam, ctx, 4)
    assert pam.pam_reserve_sequence(ctx, c, 7) == 0
    assert pam.pam_reserve_sequence(ctx, c, 7) == -1
    assert b"sequenceAlreadyExists" in pam.pam_last_error(ctx)
    assert pam.pam_sequence_length(ctx, c, 99) == -1
    assert b"sequenceNotFound" in pam.pam_last_error(ctx)
    assert pam.pam_sequence_length(ctx, c, 7) == 0
    assert pam.pam_last_error(ctx) is None  # success clears the error
    assert pam.pam_append_tokens(ctx, c, 7, -1) == -1
    assert b"non-negative" in pam.pam_last_error(ctx)
    assert not pam.pam_create_cache_host(ctx, 4, 16, 32, 1, 7)
    assert b"unknown dtype" in pam.pam_last_error(ctx)
    assert not pam.pam_create_cache_host(ctx, 0, 16, 32, 1, 0)
    assert b"maxBlocks" in pam.pam_last_error(ctx)
    pam.pam_destroy_cache(c)
    # tuning setters check their arguments on the host
    assert pam.pam_set_mixed_launch(ctx, 3, 0, 0) == -1
    assert b"mixed launch mode" in pam.pam_last_error(ctx)
    assert pam.pam_set_mixed_launch(ctx, 2, -1, 0) == -1
    assert pam.pam_set_mixed_launch(ctx, 2, 200, 56) == 0
    assert pam.pam_set_mixed_launch(ctx, 0, 0, 0) == 0


def test_no_gpu_paths_fail_cleanly(pam, ctx):
    """Without a device, device entry points report an error instead of crashing."""
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert not pam.pam_create_cache(ctx, 8, 4, 16, 1, 0)
    assert pam.pam_last_error(ctx)
    assert not pam.pam_buffer_alloc(ctx, 1024)


# ---------------------------------------------------------------- known answers

def test_cabi_lifecycle_known_answer(pam, ctx):
    # pam_create_cache(context, 8, 4, 16, 1, float32) in the reference test; the
    # bookkeeping is the same on a host cache
    c = host_cache(pam, ctx, 8, bs=4, hd=16, hkv=1)
    assert pam.pam_reserve_sequence(ctx, c, 42) == 0
    assert pam.pam_append_tokens(ctx, c, 42, 5) == 0
    assert pam.pam_sequence_length(ctx, c, 42) == 5
    assert pam.pam_available_blocks(c) == 6
    pam.pam_free_sequence(c, 42)
    assert pam.pam_available_blocks(c) == 8
    pam.pam_destroy_cache(c)


def test_allocator_known_answers(pam, ctx):
    c = host_cache(pam, ctx, 1)
    assert pam.pam_reserve_sequence(ctx, c, 1) == 0
    assert pam.pam_append_tokens(ctx, c, 1, 16) == 0
    assert pam.pam_available_blocks(c) == 0
    assert pam.pam_append_tokens(ctx, c, 1, 1) == -1
    assert b"outOfMemory" in pam.pam_last_error(ctx)
    pam.pam_destroy_cache(c)

    c = host_cache(pam, ctx, 4)
    pam.pam_reserve_sequence(ctx, c, 1)
    pam.pam_append_tokens(ctx, c, 1, 16)
    assert pam.pam_available_blocks(c) == 3
    pam.pam_free_sequence(c, 1)
    assert pam.pam_available_blocks(c) == 4
    pam.pam_reserve_sequence(ctx, c, 2)
    pam.pam_append_tokens(ctx, c, 2, 32)
    assert len(table(pam, ctx, c, 2)) == 2
    pam.pam_destroy_cache(c)

    c = host_cache(pam, ctx, 16)
    pam.pam_reserve_sequence(ctx, c, 1)
    pam.pam_append_tokens(ctx, c, 1, 16 * 3 + 7)
    assert len(table(pam, ctx, c, 1)) == 4
    assert table(pam, ctx, c, 1) == [0, 1, 2, 3]  # Deque(reversed(0..<N)).removeLast
    pam.pam_append_tokens(ctx, c, 1, 16 * 2)
    assert len(table(pam, ctx, c, 1)) == 6 and pam.pam_sequence_length(ctx, c, 1) == 16 * 5 + 7
    pam.pam_destroy_cache(c)


# ---------------------------------------------------------------- randomized

def run_random(pam, ctx, seed, policy, steps=400):
    rng = np.random.default_rng(seed)
    nb, bs = 48, 4
    c = host_cache(pam, ctx, nb, bs=bs)
    ref = RefAllocator(nb, bs)
    if policy != FIFO:
        assert pam.pam_set_eviction_policy(c, policy) == 0
        ref.set_policy(policy)
    live = []
    next_id = 0
    for _ in range(steps):
        op = rng.choice(["new", "append", "hashed", "free", "excl", "policy"], p=[.15, .35, .2, .15, .1, .05])
        if op == "new" or not live:
            rc = pam.pam_reserve_sequence(ctx, c, next_id)
            ref.allocate_sequence(next_id)
            assert rc == 0
            live.append(next_id)
            next_id += 1
        elif op in ("append", "hashed"):
            sid = int(rng.choice(live))
            n = int(rng.integers(0, 12))
            hashes = None
            if op == "hashed":
                hashes = [int(h) for h in rng.integers(0, 6, size=int(rng.integers(1, 4)))]
            try:
                ref.append_tokens(sid, n, hashes)
                ok = True
            except OutOfMemory:
                ok = False
            if hashes is None:
                rc = pam.pam_append_tokens(ctx, c, sid, n)
            else:
                arr = (C.c_uint64 * len(hashes))(*hashes)
                rc = pam.pam_append_tokens_hashed(ctx, c, sid, n, arr, len(hashes))
            assert (rc == 0) == ok
        elif op == "free":
            sid = int(rng.choice(live))
            live.remove(sid)
            pam.pam_free_sequence(c, sid)
            ref.free_sequence(sid)
        elif op == "excl":
            sid = int(rng.choice(live))
            nblk = len(ref.block_table(sid))
            if nblk:
                idx = int(rng.integers(0, nblk))
                try:
                    ref.ensure_exclusive(sid, idx)
                    ok = True
                except OutOfMemory:
                    ok = False
                assert (pam.pam_ensure_exclusive(ctx, c, sid, idx) == 0) == ok
        elif op == "policy":
            p = int(rng.integers(0, 3))
            pam.pam_set_eviction_policy(c, p)
            ref.set_policy(p)
        assert pam.pam_available_blocks(c) == ref.available
        for sid in live:
            assert table(pam, ctx, c, sid) == ref.block_table(sid)
            assert pam.pam_sequence_length(ctx, c, sid) == ref.seq_len(sid)
    from pagedattentionmetal_amd import _lib
    st = _lib.MemoryStats()
    assert pam.pam_cache_memory_stats(c, C.byref(st)) == 0
    rs = ref.stats(bs * 1 * 32 * 4 * 2)
    for k in ("total_blocks", "used_blocks", "free_blocks", "active_sequences", "total_memory_bytes",
              "used_memory_bytes", "partially_filled_blocks", "prefix_cache_hits", "prefix_cache_entries",
              "shared_blocks"):
        assert getattr(st, k) == rs[k], k
    assert abs(st.fragmentation_ratio - rs["fragmentation_ratio"]) < 1e-6
    pam.pam_destroy_cache(c)


@pytest.mark.parametrize("policy", [FIFO, LIFO, BEST_FIT])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_allocator_matches_reference_semantics(pam, ctx, policy, seed):
    run_random(pam, ctx, seed * 10 + policy, policy)


def test_prefix_sharing_and_copy_on_write(pam, ctx):
    c = host_cache(pam, ctx, 16, bs=4)
    ref = RefAllocator(16, 4)
    hashes = (C.c_uint64 * 2)(11, 22)
    for sid in (1, 2):
        assert pam.pam_reserve_sequence(ctx, c, sid) == 0
        ref.allocate_sequence(sid)
        assert pam.pam_append_tokens_hashed(ctx, c, sid, 6, hashes, 2) == 0  # 2 blocks, hashed
        ref.append_tokens(sid, 6, [11, 22])
    assert table(pam, ctx, c, 1) == table(pam, ctx, c, 2) == [0, 1]
    # appending into the shared partial tail block copies it first
    assert pam.pam_append_tokens(ctx, c, 2, 1) == 0
    ref.append_tokens(2, 1)
    assert table(pam, ctx, c, 2) == ref.block_table(2) == [0, 2]
    assert ref.copies == [(1, 2)]
    pam.pam_destroy_cache(c)


# ---------------------------------------------------------------- scheduler

def sched_state(pam, s, ids):
    out = {}
    for i in ids:
        st, gen, pr = C.c_int32(), C.c_int32(), C.c_int32()
        assert pam.pam_scheduler_sequence(s, i, C.byref(st), C.byref(gen), C.byref(pr)) == 0
        out[i] = (st.value, gen.value, pr.value)
    return out


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_scheduler_matches_reference_semantics(pam, ctx, seed):
    rng = np.random.default_rng(seed)
    max_batch, max_seqs = 5, 12
    s = pam.pam_scheduler_create(max_batch, max_seqs)
    ref = RefScheduler(max_batch, max_seqs)
    cache = host_cache(pam, ctx, 32, bs=4)
    ids = []
    buf = (C.c_int32 * 64)()
    for _ in range(200):
        op = rng.choice(["add", "step", "decode", "prefill", "complete", "preempt", "pressure"],
                        p=[.2, .3, .2, .1, .07, .05, .08])
        if op == "add":
            a, b = int(rng.integers(1, 50)), int(rng.integers(1, 6))
            sid = pam.pam_scheduler_add_request(s, a, b)
            assert sid == ref.add_request(a, b)
            if sid >= 0:
                ids.append(sid)
        elif op == "step":
            n = pam.pam_scheduler_step(s, buf, 64)
            assert list(buf[:n]) == ref.step()
        elif ids:
            sid = int(rng.choice(ids))
            if op == "decode":
                pam.pam_scheduler_mark_decoded(s, sid)
                ref.mark_decoded(sid)
            elif op == "prefill":
                pam.pam_scheduler_mark_prefilled(s, sid)
                ref.mark_prefilled(sid)
            elif op == "complete":
                pam.pam_scheduler_complete(s, sid)
                ref.complete(sid)
            elif op == "preempt":
                pam.pam_scheduler_preempt(s, sid)
                ref.preempt(sid)
            else:
                need = int(rng.integers(0, 40))
                n = pam.pam_scheduler_handle_memory_pressure(s, need, cache, buf, 64)
                avail = pam.pam_available_blocks(cache)
                assert list(buf[:n]) == ref.handle_memory_pressure(need, lambda: avail)
        want = {i: (r.status, r.generated, r.prompt) for i, r in ref.seqs.items()}
        assert sched_state(pam, s, ids) == want
        for st in (WAITING, RUNNING, PAUSED, COMPLETED):
            assert pam.pam_scheduler_count(s, st) == ref.count(st)
    pam.pam_scheduler_destroy(s)
    pam.pam_destroy_cache(cache)


def test_scheduler_quirks(pam, ctx):
    # completed sequences stay in the table: the 3rd request is rejected
    s = pam.pam_scheduler_create(4, 2)
    assert pam.pam_scheduler_add_request(s, 10, 1) == 0
    assert pam.pam_scheduler_add_request(s, 10, 1) == 1
    pam.pam_scheduler_complete(s, 0)
    assert pam.pam_scheduler_add_request(s, 10, 1) == -1
    pam.pam_scheduler_destroy(s)
    # one memory-pressure event pauses every running sequence when the caller
    # frees the victims only afterwards (Scheduler.swift:135-152)
    s = pam.pam_scheduler_create(8, 16)
    for _ in range(5):
        pam.pam_scheduler_add_request(s, 10, 3)
    buf = (C.c_int32 * 16)()
    assert pam.pam_scheduler_step(s, buf, 16) == 5
    cache = host_cache(pam, ctx, 4, bs=4)
    n = pam.pam_scheduler_handle_memory_pressure(s, 10, cache, buf, 16)
    assert list(buf[:n]) == [4, 3, 2, 1, 0]
    assert pam.pam_scheduler_count(s, RUNNING) == 0 and pam.pam_scheduler_count(s, PAUSED) == 5
    # paused sequences resume in arrival order on the next step
    assert pam.pam_scheduler_step(s, buf, 16) == 5 and list(buf[:5]) == [0, 1, 2, 3, 4]
    pam.pam_scheduler_destroy(s)
    pam.pam_destroy_cache(cache)


def test_fused_prefill_validation(pam, ctx):
    """fusedPrefill checks (PagedAttentionEngine.swift:633-641) run before any device
    work: seqLen must be positive, the block table and output must be large enough."""
    from pagedattentionmetal_amd import _lib
    lay = _lib.LayerSpec(64, 4, 2, 16, 0, 0)
    fake = 0x10000  # never dereferenced: validation fails first
    def req(seq_len, bt_bytes=0, out_bytes=0):
        return _lib.FusedPrefillRequest(fake, fake, fake, fake, fake, fake, fake, seq_len, lay, False, None, None,
                                        0, 0, 0, 0, 0, bt_bytes, out_bytes)
    r = req(0)
    assert pam.pam_engine_fused_prefill(ctx, C.byref(r)) == -1
    assert b"seqLen must be positive." in pam.pam_last_error(ctx)
    r = req(40, bt_bytes=8)  # 3 blocks of 16 need 12 bytes
    assert pam.pam_engine_fused_prefill(ctx, C.byref(r)) == -1
    assert b"blockTable" in pam.pam_last_error(ctx)
    r = req(40, out_bytes=40 * 4 * 64 * 4 - 4)
    assert pam.pam_engine_fused_prefill(ctx, C.byref(r)) == -1
    assert b"output" in pam.pam_last_error(ctx)
    bad = _lib.LayerSpec(64, 3, 2, 16, 0, 0)  # H % Hkv != 0
    r = _lib.FusedPrefillRequest(fake, fake, fake, fake, fake, fake, fake, 16, bad, False, None, None,
                                 0, 0, 0, 0, 0, 0, 0)
    assert pam.pam_engine_fused_prefill(ctx, C.byref(r)) == -1
    assert pam.pam_last_error(ctx)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one MI355X: --gpus N > 1 (or a multi-rank launch) exits
    with a message before touching the GPU."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "single GPU" in r.stderr
    env = dict(os.environ, WORLD_SIZE="4")
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py")], capture_output=True, text=True, timeout=120,
                       env=env)
    assert r.returncode == 2 and "single GPU" in r.stderr


def test_mixed_step_validation(pam, ctx):
    """The mixed step checks every buffer against the step's rows before any
    launch: q / output / new K,V rows, block-table rows and the pools."""
    from pagedattentionmetal_amd import _lib
    lay = _lib.LayerSpec(64, 4, 2, 16, 1, 0)
    fake = 0x10000  # never dereferenced: validation fails first
    cl = (C.c_int32 * 3)(10, 0, 40)
    ql = (C.c_int32 * 3)(1, 20, 1)  # 22 rows; longest sequence 41 tokens = 3 blocks
    row_q = 4 * 64 * 2
    row_kv = 2 * 64 * 2
    good = dict(q_bytes=22 * row_q, output_bytes=22 * row_q, new_keys_bytes=22 * row_kv,
                new_values_bytes=22 * row_kv, k_pool_bytes=3 * 16 * row_kv, v_pool_bytes=3 * 16 * row_kv,
                block_tables_bytes=3 * 4 * 4)

    def req(**kw):
        b = dict(good, **kw)
        return _lib.MixedRequest(fake, fake, fake, fake, fake, fake, None, None, fake, 4, 3,
                                 C.cast(cl, C.c_void_p), C.cast(ql, C.c_void_p), lay, b["q_bytes"],
                                 b["output_bytes"], b["new_keys_bytes"], b["new_values_bytes"], b["k_pool_bytes"],
                                 b["v_pool_bytes"], b["block_tables_bytes"])
    for field, name in (("q_bytes", b"Q"), ("output_bytes", b"output"), ("new_keys_bytes", b"new keys"),
                        ("new_values_bytes", b"new values"), ("k_pool_bytes", b"K pool"),
                        ("v_pool_bytes", b"V pool"), ("block_tables_bytes", b"blockTables")):
        r = req(**{field: good[field] - 1})
        assert pam.pam_engine_mixed_step(ctx, C.byref(r)) == -1, field
        err = pam.pam_last_error(ctx)
        assert name in err and b"too small" in err, (field, err)
    # a table row narrower than a sequence's blocks
    r = req()
    r.bt_stride = 2
    assert pam.pam_engine_mixed_step(ctx, C.byref(r)) == -1
    assert b"blockTables" in pam.pam_last_error(ctx)


def test_mixed_step_python_checks():
    """api.mixed_step refuses mismatched length arrays and short block tables
    before calling the library."""
    import torch
    from pagedattentionmetal_amd import api
    eng = api.PagedAttentionEngine()
    lay = api.PagedLayerSpec(64, 4, 2, 16, 1)
    q = torch.zeros((3, 4, 64), dtype=torch.float16)
    kp = torch.zeros((4, 16, 2, 64), dtype=torch.float16)
    bt = torch.zeros((2, 4), dtype=torch.int32)
    with pytest.raises(api.PagedAttentionError, match="one entry per sequence"):
        eng.mixed_step(q, q, kp, kp, bt, [1, 2], [1, 1, 1], lay)
    with pytest.raises(api.PagedAttentionError, match="one row per"):
        eng.mixed_step(q, q, kp, kp, bt, [1, 2, 3], [1, 1, 1], lay)
    with pytest.raises(api.PagedAttentionError, match="Q buffer is too small"):
        eng.mixed_step(q[:2], q, kp, kp, torch.zeros((3, 4), dtype=torch.int32), [1, 2, 3], [1, 1, 1], lay)
    eng.close()


def test_injected_launch_failure_enqueues_nothing(pam, ctx):
    """pam_debug_fail_next_launches reports the failure in place of the launch,
    like a launch the runtime refuses: the retry path then launches once."""
    src = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                            "pagedattentionmetal_amd", "csrc", "runtime", "engine.cpp")).read()
    i = src.index("void Context::check_launch(F &&launch")
    body = src[i:src.index("\n}\n", i)]
    # the injected failure throws before launch() is called
    assert body.index("fail_next_launches--") < body.index("launch()")


def test_engine_config_surface():
    """splitThreshold / defaultWindowSize / defaultChunkSize (PagedAttentionEngine.swift:116-121):
    reference defaults, settable, negative values refused."""
    from pagedattentionmetal_amd import api
    eng = api.PagedAttentionEngine()
    assert (eng.split_threshold, eng.default_window_size, eng.default_chunk_size) == (1024, 0, 0)
    eng.split_threshold = 4096
    eng.default_window_size = 256
    eng.default_chunk_size = 512
    assert (eng.split_threshold, eng.default_window_size, eng.default_chunk_size) == (4096, 256, 512)
    with pytest.raises(api.PagedAttentionError, match="non-negative"):
        eng.default_chunk_size = -1
    assert eng.default_chunk_size == 512
    eng.close()


def test_layers_calls_validate_before_any_launch(pam, ctx):
    """decodeLayers / prefillLayers / appendLayers: count mismatches raise the
    reference's error; zero layers is a no-op; a bad layer fails validation
    before any device work."""
    from pagedattentionmetal_amd import _lib, api
    eng = api.PagedAttentionEngine()
    lay = api.PagedLayerSpec(64, 4, 2, 16, 1)
    with pytest.raises(api.PagedAttentionError, match="buffer/layer count mismatch"):
        eng.decode_layers([0x1000], 0x1000, 0x1000, 0x1000, 0x1000, [], 1, 1, [lay])
    with pytest.raises(api.PagedAttentionError, match="buffer/layer count mismatch"):
        eng.prefill_layers([0x1000, 0x1000], 0x1000, 0x1000, 0x1000, [0x1000], 4, [lay, lay])
    with pytest.raises(api.PagedAttentionError, match="kScaleBuffers count"):
        eng.append_layers([0x1000], [0x1000], 0x1000, 0x1000, 0x1000, 0, 4, [lay], k_scale_buffers=[])
    r = _lib.DecodeLayersRequest()
    assert pam.pam_engine_decode_layers(ctx, C.byref(r)) == 0  # zero layers
    bad = api.PagedLayerSpec(64, 3, 2, 16, 1)  # H % Hkv != 0
    with pytest.raises(api.PagedAttentionError, match="divisible"):
        eng.decode_layers([0x1000], 0x1000, 0x1000, 0x1000, 0x1000, [0x1000], 1, 1, [bad])
    eng.close()


def test_code_object_is_built_beside_the_library(pam, ctx):
    """libpam_kernels.hsaco is a gfx950 ELF code object beside libpam.so with the
    named entries; loading it needs a GPU and fails cleanly without one."""
    path = pam.pam_module_default_path().decode()
    assert path.endswith("libpam_kernels.hsaco") and os.path.exists(path)
    with open(path, "rb") as f:
        head = f.read(4)
        data = head + f.read()
    assert head == b"\x7fELF"
    for name in (b"pam_decode_streamk_f16_d128", b"pam_decode_streamk_e4m3_d128", b"pam_decode_layers_streamk_f16_d128",
                 b"pam_prefill_f16_d128", b"pam_prefill_fused_f16_d128", b"pam_prefill_e4m3_d128",
                 b"pam_prefill_f16_d64", b"pam_prefill_fused_f16_d64", b"pam_prefill_e4m3_d64",
                 b"pam_decode_valu_wg_f32_h1", b"pam_decode_valu_wg_e4m3_h2", b"pam_fill_u32"):
        assert name in data, name
    import torch
    if not torch.cuda.is_available():
        assert pam.pam_module_load(ctx, path.encode()) == -1
        assert pam.pam_last_error(ctx)
