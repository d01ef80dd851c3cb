// engine.cpp - PagedAttentionEngine on HIP: validation, kernel choice, launch,
// retry / circuit breaker, graceful degradation and stats.
//
// Reference: Sources/PagedAttentionMetal/PagedAttentionEngine.swift
//   prefill / decode / appendToCache entry points  :405-418, :533-546, :585-597
//   withRetry (3 attempts, 10 ms * 2^k backoff, breaker at 2*maxRetries)  :375-400
//   validatePrefill / validateDecode / validateAppend  :1897-1950
//   PagedLayerSpec.validate  PagedAttentionTypes.swift:126-142
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "runtime.h"

namespace pam {

// Every HIP failure reaches the caller as this exception; the thread's last
// error is cleared so that an unrelated later hipGetLastError does not report it
// again (a device fault stays sticky in the runtime regardless).
void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw ExecutionError(std::string("GPU command execution failed: ") + what + ": " + hipGetErrorString(e));
    }
}

// ------------------------------------------------------------------ helpers

static int32_t elem_bytes(int32_t dtype) { return dtype == kF32 ? 4 : (dtype == kF16 ? 2 : 1); }
static int32_t io_bytes(int32_t dtype) { return dtype == kF32 ? 4 : 2; }  // Q / O / new K,V element

static void validate_layer(const pam_layer_spec &l) {
    if (l.head_dim <= 0) throw invalid_configuration("headDim must be positive.");
    if (l.num_heads <= 0) throw invalid_configuration("numHeads must be positive.");
    if (l.num_kv_heads <= 0) throw invalid_configuration("numKVHeads must be positive.");
    if (l.num_heads % l.num_kv_heads != 0)
        throw invalid_configuration("numHeads must be divisible by numKVHeads for GQA/MQA mapping.");
    if (l.block_size <= 0) throw invalid_configuration("blockSize must be positive.");
    if (l.data_type < 0 || l.data_type > 2) throw invalid_configuration("unknown dtype");
    if (l.window_size < 0) throw invalid_configuration("windowSize must be non-negative.");
    // kernel envelope: 4-element slices per lane, at most 64 lanes per token row
    if (l.head_dim % 4 != 0 || l.head_dim > 256)
        throw PamError("Unsupported paged attention path: headDim must be a multiple of 4 and at most 256.");
}

static void require(size_t actual, const char *name, int64_t expected) {
    if (actual != 0 && (int64_t)actual < expected) throw buffer_too_small(name, expected, (int64_t)actual);
}

static int64_t q_bytes_per_token(const pam_layer_spec &l) { return (int64_t)l.num_heads * l.head_dim * io_bytes(l.data_type); }
static int64_t kv_bytes_per_token(const pam_layer_spec &l) {
    return (int64_t)l.num_kv_heads * l.head_dim * elem_bytes(l.data_type);
}
static int64_t pool_bytes_for(int64_t blocks, const pam_layer_spec &l) { return blocks * l.block_size * kv_bytes_per_token(l); }
static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The prefill regime lastStats.operation names, by the reference's rule
// (PagedAttentionEngine.swift:420-433, 436-438, 512-516, 1952-1958): MMA for f16
// with headDim a multiple of 64 up to 256, else flash for f16/f32 up to headDim
// 64, else the tiled pass when its single-pass form would not fit a threadgroup
// (blockSize * headDim * 12 bytes over 32 KiB, or blockSize * headDim threads
// over 1024 - Apple GPU limits, kept so the same call reports the same regime)
// or seqLen exceeds splitThreshold, else the single pass.  The kernels that run
// here are chosen separately; usedSplitPass says whether the work was split.
int32_t Context::prefill_operation(const pam_layer_spec &l, int32_t seq_len) const {
    if (l.data_type == kF16 && l.head_dim <= 256 && l.head_dim % 64 == 0) return PAM_OP_PREFILL_MMA;
    if (l.data_type != kFP8 && l.head_dim <= 64) return PAM_OP_PREFILL_FLASH;
    const int64_t cells = (int64_t)l.block_size * l.head_dim;
    if (cells * 12 > 32768 || cells > 1024 || seq_len > split_threshold) return PAM_OP_PREFILL_TILED_PASS;
    return PAM_OP_PREFILL_SINGLE_PASS;
}

// ------------------------------------------------------------------ context

Context::Context() {}

Context::~Context() {
    if (!device_ready_) return;
    (void)hipSetDevice(device_);
    module_unload();
    if (own_stream_) (void)hipStreamSynchronize(own_stream_);
    if (workspace_.ptr) (void)hipFree(workspace_.ptr);
    if (seg_count_.ptr) (void)hipFree(seg_count_.ptr);
    for (auto &s : scratch_)
        if (s.ptr) (void)hipFree(s.ptr);
    if (pinned_) (void)hipHostFree(pinned_);
    if (ev0_) (void)hipEventDestroy(ev0_);
    if (ev1_) (void)hipEventDestroy(ev1_);
    if (evmid_) (void)hipEventDestroy(evmid_);
    if (handoff_) (void)hipEventDestroy(handoff_);
    if (zero_page_) (void)hipFree(zero_page_);
    for (auto &e : seg_event_)
        if (e) (void)hipEventDestroy(e);
    if (own_stream_) (void)hipStreamDestroy(own_stream_);
}

void Context::ensure_device() {
    if (device_ready_) return;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) throw PamError("GPU device or stream could not be initialized.");
    hip_check(hipGetDevice(&device_), "hipGetDevice");
    hip_check(hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, device_), "hipDeviceGetAttribute");
    // A blocking stream: work the caller queued on the legacy default stream (the
    // usual producer of the buffers passed in) completes before ours starts, and
    // the other way round, as for the reference's synchronous command buffers.
    hip_check(hipStreamCreateWithFlags(&own_stream_, hipStreamDefault), "hipStreamCreate");
    hip_check(hipEventCreate(&ev0_), "hipEventCreate");
    hip_check(hipEventCreate(&ev1_), "hipEventCreate");
    hip_check(hipEventCreate(&evmid_), "hipEventCreate");
    hip_check(hipEventCreateWithFlags(&handoff_, hipEventDisableTiming), "hipEventCreate");
    for (auto &e : seg_event_) hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
    // zeros that masked lanes of the attention kernels load instead of pool rows
    hip_check(hipMalloc(&zero_page_, kZeroPageBytes), "hipMalloc zero page");
    hip_check(hipMemset(zero_page_, 0, kZeroPageBytes), "hipMemset zero page");
    device_ready_ = true;
}

hipStream_t Context::stream() { return use_ext_stream_ ? ext_stream_ : own_stream_; }

void Context::switch_stream(bool use_ext, hipStream_t s) {
    const hipStream_t old = stream();
    ext_stream_ = use_ext ? s : nullptr;
    use_ext_stream_ = use_ext;
    if (device_ready_ && stream() != old) {
        hip_check(hipEventRecord(handoff_, old), "stream handoff");
        hip_check(hipStreamWaitEvent(stream(), handoff_, 0), "stream handoff");
    }
}

void Context::finish(const char *what) {
    hip_check(hipGetLastError(), what);
    if (synchronous) hip_check(hipStreamSynchronize(stream()), what);
}

// Device buffers that grow with the requests grow by at least half their size
// (rounded up to 1 MiB), so that a serving loop whose steps grow slowly
// reallocates, and drains the stream for it, only a few times.
static size_t grown(size_t bytes, size_t have) {
    const size_t want = std::max(bytes, have + have / 2);
    return (want + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
}

void Context::reserve_workspace(size_t bytes) {
    ensure_device();
    if (bytes <= workspace_.bytes) return;
    hip_check(hipStreamSynchronize(stream()), "workspace resize");
    const size_t want = grown(bytes, workspace_.bytes);
    if (workspace_.ptr) (void)hip_check(hipFree(workspace_.ptr), "hipFree");
    workspace_.ptr = nullptr;
    workspace_.bytes = 0;
    hip_check(hipMalloc(&workspace_.ptr, want), "hipMalloc workspace");
    workspace_.bytes = want;
}

void *Context::device_scratch(int slot, size_t bytes) {
    DeviceBuffer &b = scratch_[slot];
    if (bytes > b.bytes) {
        hip_check(hipStreamSynchronize(stream()), "scratch resize");
        if (b.ptr) hip_check(hipFree(b.ptr), "hipFree");
        b.ptr = nullptr;
        b.bytes = 0;
        const size_t want = bytes <= 4096 && b.bytes == 0 ? 4096 : grown(bytes, b.bytes);
        hip_check(hipMalloc(&b.ptr, want), "hipMalloc scratch");
        b.bytes = want;
    }
    return b.ptr;
}

// Host bytes -> pinned staging -> device memory, ordered on the stream.  The
// pinned arena is a ring of kStageSegs segments; each segment's last copy
// records an event, and a segment is refilled only after the event it recorded
// on its previous use, so the host waits for copies several calls old (already
// done in a steady serving loop) instead of draining the stream when the arena
// wraps.
void *Context::stage_into(void *dst, const void *host, size_t bytes) {
    if (bytes == 0) return dst;
    const size_t need = (bytes + 255) & ~(size_t)255;
    const size_t seg = pinned_bytes_ / kStageSegs;
    if (need > seg) {
        // grow: every staged copy must be done with the old arena
        for (int i = 0; i < kStageSegs; i++)
            if (seg_used_[i]) hip_check(hipEventSynchronize(seg_event_[i]), "staging wait");
        if (pinned_) hip_check(hipHostFree(pinned_), "hipHostFree");
        pinned_ = nullptr;
        pinned_bytes_ = 0;
        const size_t want = std::max<size_t>(need * kStageSegs, (size_t)4 << 20);
        hip_check(hipHostMalloc(&pinned_, want, hipHostMallocMapped), "hipHostMalloc");
        hip_check(hipHostGetDevicePointer(&pinned_dev_, pinned_, 0), "hipHostGetDevicePointer");
        pinned_bytes_ = want;
        for (int i = 0; i < kStageSegs; i++) seg_used_[i] = false;
        cur_seg_ = 0;
        pinned_used_ = 0;
    } else if (pinned_used_ + need > seg) {
        cur_seg_ = (cur_seg_ + 1) % kStageSegs;
        pinned_used_ = 0;
        if (seg_used_[cur_seg_]) hip_check(hipEventSynchronize(seg_event_[cur_seg_]), "staging wait");
    }
    const size_t off = (size_t)cur_seg_ * (pinned_bytes_ / kStageSegs) + pinned_used_;
    char *src = static_cast<char *>(pinned_) + off;
    std::memcpy(src, host, bytes);
    // a copy kernel on this stream (a DMA-engine copy would cost an engine
    // hand-off around the call); destinations are 256-byte aligned allocations
    const char *src_dev = static_cast<const char *>(pinned_dev_) + off;
    pinned_used_ += need;
    if (((uintptr_t)dst & 15) == 0)
        hip_check(launch_stage_copy(src_dev, dst, bytes, stream(), ktab()), "staging copy");
    else
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()), "hipMemcpyAsync staging");
    hip_check(hipEventRecord(seg_event_[cur_seg_], stream()), "hipEventRecord");
    seg_used_[cur_seg_] = true;
    return dst;
}

void *Context::stage(int slot, const void *host, size_t bytes) {
    return stage_into(device_scratch(slot, bytes), host, bytes);
}

template <class F>
void Context::with_retry(const char *op, F &&fn) {
    std::string last = std::string("operation '") + op + "' failed";
    for (int32_t attempt = 0; attempt < max_retries; attempt++) {
        try {
            fn();
            consecutive_failures = 0;
            return;
        } catch (const ScratchLimitError &) {
            throw;  // a size limit: the same request would fail again
        } catch (const ExecutionError &) {
            // work that reached the GPU and failed there is not replayed
            consecutive_failures += 1;
            throw;
        } catch (const PamError &e) {
            last = e.what();
            consecutive_failures += 1;
            if (consecutive_failures >= max_retries * 2)
                throw PamError(std::string("Recurring failure in '") + op + "' after " +
                               std::to_string(consecutive_failures) + " attempts - circuit breaker engaged.");
            if (attempt > 0) usleep((useconds_t)(10000u << attempt));
        }
    }
    throw PamError(last);
}

// An injected failure (pam_debug_fail_next_launches) stands in for a launch the
// runtime refused: it is reported before the launch, so nothing is enqueued.
template <class F>
void Context::check_launch(F &&launch, const char *what) {
    if (fail_next_launches > 0) {
        fail_next_launches--;
        throw PamError(std::string("GPU command encoding failed: injected launch failure in ") + what);
    }
    const hipError_t e = launch();
    if (e != hipSuccess) throw PamError(std::string("GPU command encoding failed: ") + what + ": " + hipGetErrorString(e));
}

void Context::zero_output(void *ptr, size_t bytes) {
    if (ptr == nullptr || bytes == 0) return;
    (void)hipMemsetAsync(ptr, 0, bytes, stream());
    (void)hipStreamSynchronize(stream());
}

void Context::record_stats(int32_t op, int32_t batch, int32_t seq_len, int32_t blocks, int64_t tmp, bool split,
                           bool has_mid) {
    last_stats.operation = op;
    last_stats.batch_size = batch;
    last_stats.sequence_length = seq_len;
    last_stats.num_blocks = blocks;
    last_stats.temporary_bytes = tmp;
    last_stats.used_split_pass = split ? 1 : 0;
    last_stats.chunks = (op >= PAM_OP_PREFILL_SINGLE_PASS && op <= PAM_OP_PREFILL_TILED_PASS) ? 1 : 0;
    last_stats.elapsed_ms = last_stats.kernel_ms = last_stats.reduce_ms = -1.0;
    stats_pending_ = gpu_timing;
    stats_has_mid_ = has_mid;
    if (synchronous) stats();
}

pam_stats Context::stats() {
    if (stats_pending_ && device_ready_) {
        stats_pending_ = false;
        if (hipEventSynchronize(ev1_) == hipSuccess) {
            float ms = -1.0f;
            if (hipEventElapsedTime(&ms, ev0_, ev1_) == hipSuccess) last_stats.elapsed_ms = ms;
            if (stats_has_mid_) {
                float a = -1.0f, b = -1.0f;
                if (hipEventElapsedTime(&a, ev0_, evmid_) == hipSuccess) last_stats.kernel_ms = a;
                if (hipEventElapsedTime(&b, evmid_, ev1_) == hipSuccess) last_stats.reduce_ms = b;
            } else {
                last_stats.kernel_ms = last_stats.elapsed_ms;
                last_stats.reduce_ms = 0.0;
            }
        }
    }
    return last_stats;
}

// Split-context partition length (tokens, a multiple of 16) for the forms that
// use fixed partitions (the stream-K form splits rows itself).
//  MFMA workgroup form (more than 2048 rows): one workgroup per (row, kv head,
//  partition).  Long partitions (up to 1024 tokens) keep the waves' load
//  pipelines full between per-item start-ups and keep the partials small; they
//  shrink until there are about three items per CU.
//  VALU kernel: one wave per (row, head group, partition); a few thousand waves
//  keep all CUs busy.
int32_t Context::choose_part_tokens(int64_t items_per_part, int64_t max_tiles, bool mfma) {
    if (max_tiles <= 0) return 16;
    if (part_tokens_override > 0) return std::max<int32_t>(16, part_tokens_override / 16 * 16);
    if (mfma) {
        int64_t tpp = 64;
        while (tpp > 16 && items_per_part * ceil_div(max_tiles, tpp) < 3 * (int64_t)cus_) tpp /= 2;
        if (tpp >= max_tiles) tpp = max_tiles;
        return (int32_t)(tpp * 16);
    }
    if (items_per_part >= 8192) return (int32_t)(max_tiles * 16);  // enough rows: one partition per row
    // VALU kernel: a wave works through its tokens in batches of 8 steps whose
    // loads are in flight together; few rows are split down to one-tile
    // partitions, so each wave's latency chain stays short
    int64_t tpp = 16;
    while (tpp > 1 && items_per_part * ceil_div(max_tiles, tpp) < 4096) tpp /= 2;
    if (tpp >= max_tiles) tpp = max_tiles;
    return (int32_t)(tpp * 16);
}

// Split-context set-up of a row launch (p.rows and the shape already filled).
// The MFMA kernel runs in its stream-K form when the rows fit it: partial slots
// in the workspace plus the counters, no reduce kernel.  Otherwise rows are cut
// into fixed partitions merged by the reduce kernel.  Returns the workspace
// bytes used (0: none).
int64_t Context::plan_split(AttnParams &p, int32_t dtype, bool use_mfma, int64_t max_tiles, int64_t waves,
                            char *fixed) {
    p.seg_count = nullptr;
    p.valu_wg = 0;
    int64_t slots = 0, counters = 0;
    // `fixed`: the allocation-free scratch (kNoAllocScratchBytes, laid out as
    // zero page | counters | partials); requests that do not fit it are refused
    const int64_t fixed_parts = (int64_t)(kNoAllocScratchBytes - kNoAllocZeroBytes - kNoAllocCounterBytes);
    auto too_big = [](const char *what, int64_t need, int64_t have) {
        return ScratchLimitError(std::string("Unsupported paged attention path: the allocation-free decode's ") + what +
                        " needs " + std::to_string(need) + " bytes of its fixed " + std::to_string(have) +
                        "-byte scratch.");
    };
    // a partition length set through pam_set_partition_tokens selects the
    // partitioned form.  So do few (row, kv head) pairs with long contexts:
    // there the stream-K form's last unit of a pair merges many partials one
    // batch after another, where fixed partitions, split over a workgroup's
    // waves and merged by the reduce kernel, keep every step short.  Measured
    // on gfx950 (32/8 heads, f16, µs per call, stream-K -> partitions):
    //   1 row:  2K tokens 20.8 -> 14.5, 4K 23.8 -> 15.1, 16K 43.5 -> 27.2, 64K 87.6 -> 65.9
    //   2 rows: 4K 24.3 -> 16.3, 16K 49.2 -> 44.0, 64K 99.1 -> 103.2
    //   4 rows: 2K 22.1 -> 16.3, 4K 27.6 -> 25.1, 16K 56.6 -> 58.9, 64K 168 -> 201
    const int64_t pairs = (int64_t)p.rows * p.num_kv_heads;
    const bool few_pairs = p.fused_layers <= 1 && max_tiles >= 128 &&
                           (pairs <= 8 || (pairs <= 16 && max_tiles <= 2048) || (pairs <= 32 && max_tiles <= 256));
    if (use_mfma && part_tokens_override == 0 && !few_pairs && mfma_streamk_plan(p, dtype, &slots, &counters)) {
        p.part_tokens = (int32_t)(max_tiles * 16);
        p.max_parts = 1;
        const int64_t bytes = slots * ((int64_t)p.head_dim + 2) * 4;
        if (bytes >= ((int64_t)1 << 31)) throw PamError("stream-K workspace exceeds 2 GiB");
        if (fixed) {
            if (bytes > fixed_parts) throw too_big("split-context partials", bytes, fixed_parts);
            if (counters * 8 > (int64_t)kNoAllocCounterBytes)
                throw too_big("merge counters", counters * 8, (int64_t)kNoAllocCounterBytes);
            p.part_o = reinterpret_cast<float *>(fixed + kNoAllocZeroBytes + kNoAllocCounterBytes);
            p.seg_count = reinterpret_cast<uint64_t *>(fixed + kNoAllocZeroBytes);
        } else {
            reserve_workspace((size_t)bytes);
            p.part_o = static_cast<float *>(workspace_.ptr);
            reserve_counters(seg_count_, (size_t)counters * 8);
            p.seg_count = static_cast<uint64_t *>(seg_count_.ptr);
        }
        p.part_ml = p.part_o + slots * p.head_dim;
        p.part_bytes = (uint32_t)bytes;
        return bytes;
    }
    p.part_tokens = choose_part_tokens(waves, max_tiles, use_mfma);
    p.max_parts = (int32_t)std::max<int64_t>(1, ceil_div(max_tiles, p.part_tokens / 16));
    if (p.max_parts <= 1) return 0;
    // VALU rows of one or two heads per wave split into at most kValuWgMaxParts
    // partitions: a (row, head group)'s partitions run as the waves of one
    // workgroup and merge in LDS, with no partials in memory and no counters
    if (!use_mfma && p.heads_per_wave <= 2 && p.max_parts <= kValuWgMaxParts) {
        p.valu_wg = 1;
        return 0;
    }
    const int64_t slots_p = (int64_t)p.rows * p.num_heads * p.max_parts;
    const int64_t bytes = slots_p * ((int64_t)p.head_dim + 2) * 4;
    if (bytes >= ((int64_t)1 << 31)) throw PamError("split-context workspace exceeds 2 GiB");
    // The VALU kernel merges its partitions itself (one counter per row and
    // head group; no reduce launch); the MFMA workgroup form leaves them to
    // attn_reduce_kernel.
    const int64_t merge_counters = use_mfma ? 0 : (int64_t)p.rows * (p.num_heads / p.heads_per_wave);
    if (fixed) {
        if (bytes > fixed_parts) throw too_big("split-context partials", bytes, fixed_parts);
        if (merge_counters * 8 > (int64_t)kNoAllocCounterBytes)
            throw too_big("merge counters", merge_counters * 8, (int64_t)kNoAllocCounterBytes);
        p.part_o = reinterpret_cast<float *>(fixed + kNoAllocZeroBytes + kNoAllocCounterBytes);
        if (merge_counters) p.seg_count = reinterpret_cast<uint64_t *>(fixed + kNoAllocZeroBytes);
    } else {
        reserve_workspace((size_t)bytes);
        p.part_o = static_cast<float *>(workspace_.ptr);
        if (merge_counters) {
            reserve_counters(seg_count_, (size_t)merge_counters * 8);
            p.seg_count = static_cast<uint64_t *>(seg_count_.ptr);
        }
    }
    p.part_ml = p.part_o + slots_p * p.head_dim;
    p.part_bytes = (uint32_t)bytes;
    return bytes;
}

void Context::reserve_counters(DeviceBuffer &b, size_t bytes) {
    if (bytes <= b.bytes) return;
    hip_check(hipStreamSynchronize(stream()), "counter resize");
    const size_t want = grown(bytes, b.bytes);
    if (b.ptr) hip_check(hipFree(b.ptr), "hipFree");
    b.ptr = nullptr;
    b.bytes = 0;
    hip_check(hipMalloc(&b.ptr, want), "hipMalloc counters");
    hip_check(hipMemsetAsync(b.ptr, 0, want, stream()), "counter clear");
    hip_check(hipStreamSynchronize(stream()), "counter clear");
    b.bytes = want;
}

void Context::dirty_counters(int32_t arrivals) {
    ensure_device();
    const uint64_t v = ((uint64_t)next_launch_epoch() << 32) | (uint32_t)arrivals;
    for (DeviceBuffer *b : {&seg_count_, &pf_count_}) {
        if (!b->ptr) continue;
        std::vector<uint64_t> h(b->bytes / 8, v);
        hip_check(hipStreamSynchronize(stream()), "dirty counters");
        hip_check(hipMemcpy(b->ptr, h.data(), h.size() * 8, hipMemcpyHostToDevice), "dirty counters");
    }
}

Context::DensePlan Context::plan_dense_prefill(AttnParams &p, const int4 *chunks, int32_t n, StageList &sl,
                                              int32_t groups) {
    // splitThreshold (PagedAttentionEngine.swift:116-117, :1952-1958): only
    // prefills past it may use the multi-pass form, here items cut into pieces
    // whose partial states are merged in the kernel
    int64_t longest = 0;
    for (int32_t c = 0; c < n; c++) longest = std::max<int64_t>(longest, (int64_t)chunks[c].y + chunks[c].z);
    PrefillSplit ps;
    prefill_split_plan(chunks, n, p, groups > 0 ? groups : cus_, ps, longest > split_threshold);
    DensePlan d;
    d.o_work = sl.add(ps.work.data(), ps.work.size() * sizeof(int4));
    d.o_range = sl.add(ps.range.data(), ps.range.size() * sizeof(int2));
    p.pf_part = nullptr;
    p.pf_count = nullptr;
    p.pf_part_bytes = 0;
    if (ps.slots > 0) {
        const int64_t bytes = ps.slots * kPrefillSlotBytes;
        if (bytes >= ((int64_t)1 << 31)) throw PamError("prefill split workspace exceeds 2 GiB");
        if ((size_t)bytes > pf_part_.bytes) {
            hip_check(hipStreamSynchronize(stream()), "prefill workspace resize");
            if (pf_part_.ptr) hip_check(hipFree(pf_part_.ptr), "hipFree");
            pf_part_.ptr = nullptr;
            pf_part_.bytes = 0;
            const size_t want = grown((size_t)bytes, pf_part_.bytes);
            hip_check(hipMalloc(&pf_part_.ptr, want), "hipMalloc prefill workspace");
            pf_part_.bytes = want;
        }
        reserve_counters(pf_count_, (size_t)ps.slots * 8);
        p.pf_part = static_cast<float *>(pf_part_.ptr);
        p.pf_count = static_cast<uint64_t *>(pf_count_.ptr);
        p.pf_part_bytes = (uint32_t)bytes;
        d.tmp = bytes;
    }
    return d;
}

void Context::bind_dense_prefill(AttnParams &p, const DensePlan &d, const char *base) {
    p.pf_work = reinterpret_cast<const int4 *>(base + d.o_work);
    p.pf_range = reinterpret_cast<const int2 *>(base + d.o_range);
}

static int32_t heads_per_wave(int32_t group) {
    for (int32_t nh : {8, 4, 2})
        if (group % nh == 0) return nh;
    return 1;
}

// ------------------------------------------------------------------ code object

// The reference's pipeline manager (PagedAttentionEngine.swift:151-198, 248-333)
// compiles its shader library at start-up and looks kernels up by name; here a
// gfx950 code object is loaded with hipModuleLoad and its named entries are
// bound for this context's launches.
void Context::module_load(const char *path) {
    ensure_device();
    if (!path || !*path) throw invalid_configuration("code object path is empty.");
    module_unload();
    hipModule_t m = nullptr;
    const hipError_t e = hipModuleLoad(&m, path);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // the failure is reported here, not to the caller's next launch check
        throw PamError(std::string("GPU device or stream could not be initialized: hipModuleLoad(") + path +
                       "): " + hipGetErrorString(e));
    }
    // unloaded on every way out until the context takes it over below
    struct ModuleGuard {
        hipModule_t m;
        ~ModuleGuard() {
            if (m) (void)hipModuleUnload(m);
        }
    } guard{m};
    KernelTable t{};
    auto get = [&](const char *name) {
        hipFunction_t f = nullptr;
        if (hipModuleGetFunction(&f, m, name) == hipSuccess) return f;
        // an absent entry leaves hipErrorNotFound as the thread's last error,
        // which a later hipGetLastError (torch's launch check) would report
        (void)hipGetLastError();
        return (hipFunction_t) nullptr;
    };
    t.streamk[0][0] = get("pam_decode_streamk_f16_d128");
    t.streamk[1][0] = get("pam_decode_streamk_e4m3_d128");
    t.streamk[0][1] = get("pam_decode_layers_streamk_f16_d128");
    t.streamk[1][1] = get("pam_decode_layers_streamk_e4m3_d128");
    t.prefill[0][0] = get("pam_prefill_f16_d128");
    t.prefill[0][1] = get("pam_prefill_fused_f16_d128");
    t.prefill[0][2] = get("pam_prefill_e4m3_d128");
    t.prefill[1][0] = get("pam_prefill_f16_d64");
    t.prefill[1][1] = get("pam_prefill_fused_f16_d64");
    t.prefill[1][2] = get("pam_prefill_e4m3_d64");
    t.mfma_wg[0] = get("pam_decode_wg_f16_d128");
    t.mfma_wg[1] = get("pam_decode_wg_e4m3_d128");
    t.mixed[0] = get("pam_mixed_step_f16_d128");
    t.mixed[1] = get("pam_mixed_step_e4m3_d128");
    static const char *kv_names[3] = {"f32", "f16", "e4m3"};
    static const int heads[4] = {1, 2, 4, 8};
    for (int k = 0; k < 3; k++)
        for (int h = 0; h < 4; h++)
            t.valu[k][h] = get(("pam_decode_valu_" + std::string(kv_names[k]) + "_h" + std::to_string(heads[h])).c_str());
    for (int k = 0; k < 3; k++)
        for (int h = 0; h < 2; h++)
            t.valu_wg[k][h] = get(("pam_decode_valu_wg_" + std::string(kv_names[k]) + "_h" + std::to_string(heads[h])).c_str());
    t.reduce[0] = get("pam_reduce_f32");
    t.reduce[1] = get("pam_reduce_f16");
    static const char *piece[3] = {"16", "4", "2"};
    for (int w = 0; w < 3; w++) {
        t.append[w] = get(("pam_append_b" + std::string(piece[w])).c_str());
        t.append_batch[w] = get(("pam_append_batch_b" + std::string(piece[w])).c_str());
    }
    t.append_fp8 = get("pam_append_fp8");
    t.stage = get("pam_stage_copy");
    t.block_copy = get("pam_block_copy");
    t.strict = module_strict_;
    // a stream-K launch is planned for the library kernel's resident grid: an
    // entry with another occupancy would not fit the plan's partial slots
    for (int dt = 0; dt < 2; dt++)
        for (int fl = 0; fl < 2; fl++) {
            if (!t.streamk[dt][fl]) continue;
            int lib = 0, mod = 0;
            hip_check(streamk_occupancy(dt == 0 ? kF16 : kFP8, fl != 0, &lib), "stream-K occupancy");
            hip_check(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&mod, t.streamk[dt][fl], 256, 0),
                      "code object occupancy");
            if (mod != lib) {
                throw PamError("Unsupported paged attention path: the code object's stream-K entry runs " +
                               std::to_string(mod) + " workgroups per CU, the library's kernel " +
                               std::to_string(lib) + ".");
            }
        }
    guard.m = nullptr;
    module_ = m;
    ktab_ = t;
}

void Context::module_unload() {
    if (!module_) return;
    if (device_ready_) (void)hipStreamSynchronize(stream());
    (void)hipModuleUnload(module_);
    module_ = nullptr;
    ktab_ = KernelTable{};
}

void *Context::module_function(const char *name) {
    if (!module_) throw invalid_configuration("no code object is loaded.");
    hipFunction_t f = nullptr;
    if (!name || hipModuleGetFunction(&f, module_, name) != hipSuccess) {
        (void)hipGetLastError();  // reported by this exception, not by the caller's next launch check
        throw invalid_configuration(std::string("the code object has no entry '") + (name ? name : "") + "'.");
    }
    return (void *)f;
}

void Context::module_launch_raw(void *function, const uint32_t grid[3], const uint32_t block[3], uint32_t shared_bytes,
                                void *args, size_t args_bytes) {
    if (!module_ || !function) throw invalid_configuration("no code object entry to launch.");
    ensure_device();
    void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &args_bytes,
                      HIP_LAUNCH_PARAM_END};
    check_launch([&] {
        return hipModuleLaunchKernel((hipFunction_t)function, grid[0], grid[1], grid[2], block[0], block[1], block[2],
                                     shared_bytes, stream(), nullptr, args_bytes ? config : nullptr);
    }, "module launch");
    finish("module launch");
}

// ------------------------------------------------------------------ decode

void Context::setup_noalloc() {
    ensure_device();
    void *ptr = nullptr;
    hip_check(noalloc_scratch_setup(device_, stream(), &ptr), "allocation-free scratch set-up");
}

void Context::decode(const pam_decode_request &r) { decode_checked(r, false); }

void Context::decode_noalloc(const pam_decode_request &r) { decode_checked(r, true); }

// validateDecode (PagedAttentionEngine.swift:1916-1934)
static void validate_decode(const pam_decode_request &r) {
    validate_layer(r.layer);
    if (r.batch_size <= 0) throw invalid_configuration("batchSize must be positive.");
    if (r.max_num_blocks <= 0) throw invalid_configuration("maxNumBlocks must be positive.");
    if (r.block_tables_bytes != 0 &&
        (int64_t)r.max_num_blocks > (int64_t)(r.block_tables_bytes / ((size_t)r.batch_size * 4)))
        throw invalid_configuration("maxNumBlocks exceeds blockTables buffer capacity");
    const pam_layer_spec &l = r.layer;
    require(r.q_bytes, "Q", r.batch_size * q_bytes_per_token(l));
    require(r.block_tables_bytes, "blockTables", (int64_t)r.batch_size * r.max_num_blocks * 4);
    require(r.seq_lengths_bytes, "seqLengths", (int64_t)r.batch_size * 4);
    require(r.output_bytes, "output", r.batch_size * q_bytes_per_token(l));
    require(r.k_pool_bytes, "K pool", pool_bytes_for(r.max_num_blocks, l));
    require(r.v_pool_bytes, "V pool", pool_bytes_for(r.max_num_blocks, l));
    if (l.data_type == kFP8 && (r.k_scale == nullptr || r.v_scale == nullptr))
        throw invalid_configuration("FP8 decode needs the K and V scale pools.");
    if (!r.q || !r.k_pool || !r.v_pool || !r.block_tables || !r.seq_lengths || !r.output)
        throw invalid_configuration("decode request has a null buffer.");
}

void Context::decode_checked(const pam_decode_request &r, bool noalloc) {
    validate_decode(r);
    char *fixed = nullptr;
    if (noalloc) {
        // set up by pam_engine_setup_noalloc: this path creates nothing itself
        if (!device_ready_ || (fixed = static_cast<char *>(noalloc_scratch(device_))) == nullptr)
            throw PamError("GPU device or stream could not be initialized: call pam_engine_setup_noalloc first.");
    }
    ensure_device();
    if (graceful_degradation) {
        try {
            decode_gpu(r, fixed);
        } catch (const ScratchLimitError &) {
            throw;  // a size limit of the fixed scratch, not a failure to degrade from
        } catch (const PamError &e) {
            std::fprintf(stderr, "[pam] decode failed: %s\n", e.what());
            zero_output(r.output, (size_t)(r.batch_size * q_bytes_per_token(r.layer)));
        }
    } else {
        decode_gpu(r, fixed);
    }
}

// Kernel choice, parameters and split workspace of one decode launch.  With
// `fused` > 1 the launch serves that many consecutive layers of `layers_q` /
// `layers_out` (same spec, shared pool): the stream-K MFMA kernel reads each K/V
// tile once for all of their heads.
Context::DecodePlan Context::plan_decode(const pam_decode_request &r, char *fixed, int32_t fused,
                                         const void *const *layers_q, void *const *layers_out) {
    const pam_layer_spec &l = r.layer;
    const int32_t G = l.num_heads / l.num_kv_heads;
    DecodePlan d{};
    bool use_mfma = mfma_supported(l.data_type, l.head_dim, G, l.block_size) && G >= 4;
    if (decode_kernel_choice == 1) use_mfma = false;
    if (decode_kernel_choice == 2) use_mfma = mfma_supported(l.data_type, l.head_dim, G, l.block_size);
    const int32_t nh = heads_per_wave(G);

    AttnParams &p = d.p;
    p.q = r.q;
    p.out = r.output;
    p.k_pool = r.k_pool;
    p.v_pool = r.v_pool;
    p.k_scale = r.k_scale;
    p.v_scale = r.v_scale;
    p.block_tables = r.block_tables;
    p.seq_lengths = r.seq_lengths;
    p.rows = r.batch_size;
    p.bt_stride = r.max_num_blocks;
    p.max_num_blocks = r.max_num_blocks;
    p.num_heads = l.num_heads;
    p.num_kv_heads = l.num_kv_heads;
    p.head_dim = l.head_dim;
    p.block_size = l.block_size;
    p.window = l.window_size;
    p.mode = kRowDecode;
    p.heads_per_wave = nh;
    p.scale_log2 = kLog2eHost / std::sqrt((float)l.head_dim);
    p.zero_page = fixed ? static_cast<const void *>(fixed) : zero_page_;
    if (fused > 1) {
        if (!use_mfma || fused > kMaxFusedLayers || G * fused > 16) throw PamError("decode layers cannot be fused");
        p.fused_layers = fused;
        for (int32_t i = 0; i < fused; i++) {
            p.layer_q[i] = layers_q[i];
            p.layer_out[i] = layers_out[i];
        }
    }

    const int64_t cap_tokens = (int64_t)r.max_num_blocks * l.block_size;
    int64_t max_tiles = ceil_div(cap_tokens, 16);
    if (l.window_size > 0) max_tiles = std::min<int64_t>(max_tiles, l.window_size / 16 + 2);
    const int64_t waves = (int64_t)r.batch_size * (use_mfma ? l.num_kv_heads : l.num_heads / nh);
    d.tmp = plan_split(p, l.data_type, use_mfma, max_tiles, waves, fixed);
    if (fused > 1 && p.seg_count == nullptr) throw PamError("decode layers cannot be fused");
    d.use_mfma = use_mfma;
    return d;
}

// Layers that one stream-K launch can serve together (0: this layer cannot be
// fused with others).
int32_t Context::fusable_layers(const pam_decode_request &r) {
    const pam_layer_spec &l = r.layer;
    const int32_t G = l.num_heads / l.num_kv_heads;
    if (decode_kernel_choice == 1 || part_tokens_override != 0 || G < 4) return 0;
    if (!mfma_supported(l.data_type, l.head_dim, G, l.block_size)) return 0;
    AttnParams p{};
    p.rows = r.batch_size;
    p.num_heads = l.num_heads;
    p.num_kv_heads = l.num_kv_heads;
    p.head_dim = l.head_dim;
    p.block_size = l.block_size;
    int64_t slots = 0, counters = 0;
    if (!mfma_streamk_plan(p, l.data_type, &slots, &counters)) return 0;
    return std::min<int32_t>(kMaxFusedLayers, 16 / G);
}

void Context::decode_gpu(const pam_decode_request &r, char *fixed) {
    const DecodePlan d = plan_decode(r, fixed, 1, nullptr, nullptr);
    const pam_layer_spec &l = r.layer;
    with_retry("decodeFlat", [&] {
        mark(ev0_);
        check_launch([&] { return launch_attention(d.p, l.data_type, d.use_mfma, stream(), gpu_timing ? evmid_ : nullptr, ktab()); }, "decode");
        mark(ev1_);
        finish("decode");
    });
    record_stats(PAM_OP_DECODE, r.batch_size, 0, r.max_num_blocks, d.tmp, d.p.max_parts > 1 || d.p.seg_count != nullptr,
                 true);
}

// decodeLayers (PagedAttentionEngine.swift:1641-1741): every layer decodes its
// own Q into its own output over the one pool, table and lengths; a window
// argument > 0 overrides each layer's window.  Consecutive layers of one spec
// that the stream-K kernel serves run as one launch per group (each K/V tile
// read once for all of their heads); the others run one launch per layer.  All
// launches of the call are one retried unit on the context's stream.
void Context::decode_layers(const pam_decode_layers_request &r) {
    if (r.num_layers < 0 || (r.num_layers > 0 && (!r.q || !r.output || !r.layers)))
        throw invalid_configuration("buffer/layer count mismatch");
    const int32_t n = r.num_layers;
    if (n == 0) return;
    std::vector<pam_decode_request> reqs((size_t)n);
    for (int32_t i = 0; i < n; i++) {
        pam_decode_request &q = reqs[i];
        q = pam_decode_request{};
        q.q = r.q[i];
        q.output = r.output[i];
        q.k_pool = r.k_pool;
        q.v_pool = r.v_pool;
        q.block_tables = r.block_tables;
        q.seq_lengths = r.seq_lengths;
        q.batch_size = r.batch_size;
        q.max_num_blocks = r.max_num_blocks;
        q.layer = r.layers[i];
        if (r.window_size > 0) q.layer.window_size = r.window_size;
        q.k_scale = r.k_scale;
        q.v_scale = r.v_scale;
        q.q_bytes = r.q_bytes ? r.q_bytes[i] : 0;
        q.output_bytes = r.output_bytes ? r.output_bytes[i] : 0;
        q.k_pool_bytes = r.k_pool_bytes;
        q.v_pool_bytes = r.v_pool_bytes;
        q.block_tables_bytes = r.block_tables_bytes;
        q.seq_lengths_bytes = r.seq_lengths_bytes;
        validate_decode(q);
    }
    ensure_device();
    if (graceful_degradation) {
        try {
            decode_layers_gpu(reqs);
        } catch (const PamError &e) {
            std::fprintf(stderr, "[pam] decodeLayers failed: %s\n", e.what());
            for (const auto &q : reqs) zero_output(q.output, (size_t)(q.batch_size * q_bytes_per_token(q.layer)));
        }
    } else {
        decode_layers_gpu(reqs);
    }
}

static bool same_spec(const pam_layer_spec &a, const pam_layer_spec &b) {
    return a.head_dim == b.head_dim && a.num_heads == b.num_heads && a.num_kv_heads == b.num_kv_heads &&
           a.block_size == b.block_size && a.data_type == b.data_type && a.window_size == b.window_size;
}

void Context::decode_layers_gpu(const std::vector<pam_decode_request> &reqs) {
    // groups of consecutive layers: [first, first + count)
    std::vector<std::pair<int32_t, int32_t>> groups;
    for (int32_t i = 0; i < (int32_t)reqs.size();) {
        const int32_t cap = std::max<int32_t>(1, fusable_layers(reqs[i]));
        int32_t j = i + 1;
        while (j < (int32_t)reqs.size() && j - i < cap && same_spec(reqs[j].layer, reqs[i].layer)) j++;
        groups.emplace_back(i, j - i);
        i = j;
    }
    int64_t tmp = 0;
    bool split = false;
    with_retry("decodeLayers", [&] {
        mark(ev0_);
        for (const auto &g : groups) {
            std::vector<const void *> qs;
            std::vector<void *> outs;
            for (int32_t k = 0; k < g.second; k++) {
                qs.push_back(reqs[g.first + k].q);
                outs.push_back(reqs[g.first + k].output);
            }
            // launches of the call run in stream order, so they share the workspace
            const DecodePlan d = plan_decode(reqs[g.first], nullptr, g.second, qs.data(), outs.data());
            tmp = std::max(tmp, d.tmp);
            split = split || d.p.max_parts > 1 || d.p.seg_count != nullptr;
            check_launch([&] { return launch_attention(d.p, reqs[g.first].layer.data_type, d.use_mfma, stream(), nullptr, ktab()); },
                         "decodeLayers");
        }
        mark(ev1_);
        finish("decodeLayers");
    });
    last_fused_groups = (int32_t)groups.size();
    record_stats(PAM_OP_DECODE, reqs[0].batch_size, 0, reqs[0].max_num_blocks, tmp, split, false);
}

// prefillLayers (PagedAttentionEngine.swift:1433-1639): causal (or full)
// prefill of rows 0 .. seq_len-1 of every layer over the one pool and table; a
// window argument > 0 overrides each layer's window.  One launch per layer (the
// prefill is MFMA-bound: sharing K/V reads across layers would save little),
// all in one retried unit on the context's stream.
void Context::prefill_layers(const pam_prefill_layers_request &r) {
    if (r.num_layers < 0 || (r.num_layers > 0 && (!r.q || !r.output || !r.layers)))
        throw invalid_configuration("buffer/layer count mismatch");
    const int32_t n = r.num_layers;
    if (n == 0) return;
    std::vector<pam_prefill_request> reqs((size_t)n);
    for (int32_t i = 0; i < n; i++) {
        pam_prefill_request &q = reqs[i];
        q = pam_prefill_request{};
        q.q = r.q[i];
        q.output = r.output[i];
        q.k_pool = r.k_pool;
        q.v_pool = r.v_pool;
        q.block_table = r.block_table;
        q.seq_len = r.seq_len;
        q.q_offset = 0;
        q.layer = r.layers[i];
        if (r.window_size > 0) q.layer.window_size = r.window_size;
        q.causal = r.causal;
        q.k_scale = r.k_scale;
        q.v_scale = r.v_scale;
        q.q_bytes = r.q_bytes ? r.q_bytes[i] : 0;
        q.output_bytes = r.output_bytes ? r.output_bytes[i] : 0;
        q.k_pool_bytes = r.k_pool_bytes;
        q.v_pool_bytes = r.v_pool_bytes;
        q.block_table_bytes = r.block_table_bytes;
        validate_prefill(q);
    }
    ensure_device();
    auto run = [&] {
        int64_t tmp = 0;
        bool split = false;
        with_retry("prefillLayers", [&] {
            mark(ev0_);
            for (const auto &q : reqs) {
                // a layer's work list is staged on the stream ahead of its launch
                const PrefillPlan pl = plan_prefill(q);
                tmp = std::max(tmp, pl.tmp);
                split = split || (pl.dense ? pl.p.pf_part != nullptr : (pl.p.max_parts > 1 || pl.p.seg_count != nullptr));
                launch_prefill_plan(pl, q.layer.data_type, false);
            }
            mark(ev1_);
            finish("prefillLayers");
        });
        record_stats(prefill_operation(reqs[0].layer, r.seq_len), 1, r.seq_len,
                     (int32_t)ceil_div(r.seq_len, reqs[0].layer.block_size), tmp,
                     split, false);
    };
    if (graceful_degradation) {
        try {
            run();
        } catch (const PamError &e) {
            std::fprintf(stderr, "[pam] prefillLayers failed: %s\n", e.what());
            for (const auto &q : reqs) zero_output(q.output, (size_t)(q.seq_len * q_bytes_per_token(q.layer)));
        }
    } else {
        run();
    }
}

// appendLayers (PagedAttentionEngine.swift:1744-1895): every layer's new keys and
// values are appended, in layer order, at the same positions of the one pool
// (FP8: with that layer's scale pools), so a later layer's rows replace an
// earlier one's, as in the reference.  One retried unit on the stream.
void Context::append_layers(const pam_append_layers_request &r) {
    if (r.num_layers < 0 || (r.num_layers > 0 && (!r.keys || !r.values || !r.layers)))
        throw invalid_configuration("buffer/layer count mismatch");
    const int32_t n = r.num_layers;
    if (n == 0) return;
    std::vector<pam_append_request> reqs((size_t)n);
    for (int32_t i = 0; i < n; i++) {
        pam_append_request &a = reqs[i];
        a = pam_append_request{};
        a.keys = r.keys[i];
        a.values = r.values[i];
        a.k_pool = r.k_pool;
        a.v_pool = r.v_pool;
        a.block_table = r.block_table;
        a.token_offset = r.token_offset;
        a.num_new_tokens = r.num_new_tokens;
        a.layer = r.layers[i];
        a.k_scale = r.k_scale ? r.k_scale[i] : nullptr;
        a.v_scale = r.v_scale ? r.v_scale[i] : nullptr;
        a.keys_bytes = r.keys_bytes ? r.keys_bytes[i] : 0;
        a.values_bytes = r.values_bytes ? r.values_bytes[i] : 0;
        a.k_pool_bytes = r.k_pool_bytes;
        a.v_pool_bytes = r.v_pool_bytes;
        a.block_table_bytes = r.block_table_bytes;
        validate_append(a);
    }
    ensure_device();
    auto run = [&] {
        with_retry("appendLayers", [&] {
            mark(ev0_);
            for (const auto &a : reqs) {
                const AppendParams ap = append_params(a);
                check_launch([&] { return launch_append(ap, a.layer.data_type, stream(), ktab()); }, "appendLayers");
            }
            mark(ev1_);
            finish("appendLayers");
        });
        record_stats(PAM_OP_APPEND, 1, r.num_new_tokens, 0, 0, false, false);
    };
    if (graceful_degradation) {
        try {
            run();
        } catch (const PamError &e) {
            std::fprintf(stderr, "[pam] appendLayers failed: %s\n", e.what());
        }
    } else {
        run();
    }
}

// ------------------------------------------------------------------ flat overloads

static int32_t effective(int32_t arg, int32_t dflt) { return arg > 0 ? arg : dflt; }

void Context::decode_flat(const pam_decode_request &r, int32_t window_size) {
    pam_decode_request q = r;
    q.layer.window_size = effective(window_size, default_window_size);
    decode(q);
}

void Context::append_flat(const pam_append_request &r, int32_t window_size) {
    pam_append_request a = r;
    a.layer.window_size = effective(window_size, default_window_size);
    append(a);
}

// The reference's chunk loop (:740-756) prefills rows [0, end) for every chunk
// end in turn; each pass overwrites the rows of the one before, so its result is
// the last pass, the unchunked prefill.  Here a causal prefill without window
// runs its chunks as query-offset pieces [start, end) - one launch per chunk,
// every row computed once, each exactly as the unchunked prefill computes it
// (a causal row reads only keys up to itself).  A full or windowed prefill, whose
// rows depend on the final length, runs as the one pass that decides the result.
void Context::prefill_flat(const pam_prefill_request &r, int32_t window_size, int32_t chunk_size) {
    pam_prefill_request q = r;
    q.layer.window_size = effective(window_size, default_window_size);
    const int32_t chunk = effective(chunk_size, default_chunk_size);
    if (chunk <= 0 || r.seq_len <= chunk || !r.causal || q.layer.window_size > 0 || r.q_offset != 0) {
        prefill(q);
        last_stats.chunks = chunk > 0 && r.seq_len > chunk ? (int32_t)ceil_div(r.seq_len, chunk) : 1;
        return;
    }
    validate_prefill(q);
    const int64_t qrow = q_bytes_per_token(q.layer);
    int32_t n = 0;
    for (int32_t start = 0; start < r.seq_len; start += chunk, n++) {
        pam_prefill_request c = q;
        c.seq_len = std::min(chunk, r.seq_len - start);
        c.q_offset = start;
        c.q = static_cast<const char *>(r.q) + start * qrow;
        c.output = static_cast<char *>(r.output) + start * qrow;
        c.q_bytes = r.q_bytes ? r.q_bytes - (size_t)(start * qrow) : 0;
        c.output_bytes = r.output_bytes ? r.output_bytes - (size_t)(start * qrow) : 0;
        prefill(c);
    }
    last_stats.chunks = n;
}

// ------------------------------------------------------------------ prefill

void Context::prefill(const pam_prefill_request &r) {
    validate_prefill(r);
    const pam_layer_spec &l = r.layer;
    ensure_device();
    if (graceful_degradation) {
        try {
            prefill_gpu(r);
        } catch (const PamError &e) {
            std::fprintf(stderr, "[pam] prefill failed: %s\n", e.what());
            zero_output(r.output, (size_t)(r.seq_len * q_bytes_per_token(l)));
        }
    } else {
        prefill_gpu(r);
    }
}

// validatePrefill (PagedAttentionEngine.swift:1897-1914)
void Context::validate_prefill(const pam_prefill_request &r) {
    validate_layer(r.layer);
    if (r.seq_len <= 0) throw invalid_configuration("seqLen must be positive.");
    if (r.q_offset < 0) throw invalid_configuration("qOffset must be non-negative.");
    const pam_layer_spec &l = r.layer;
    const int64_t kv_len = (int64_t)r.q_offset + r.seq_len;
    const int64_t nb = ceil_div(kv_len, l.block_size);
    require(r.q_bytes, "Q", r.seq_len * q_bytes_per_token(l));
    require(r.block_table_bytes, "blockTable", nb * 4);
    require(r.output_bytes, "output", r.seq_len * q_bytes_per_token(l));
    require(r.k_pool_bytes, "K pool", pool_bytes_for(nb, l));
    require(r.v_pool_bytes, "V pool", pool_bytes_for(nb, l));
    if (l.data_type == kFP8 && (r.k_scale == nullptr || r.v_scale == nullptr))
        throw invalid_configuration("FP8 prefill needs the K and V scale pools.");
    if (!r.q || !r.k_pool || !r.v_pool || !r.block_table || !r.output)
        throw invalid_configuration("prefill request has a null buffer.");
}

Context::PrefillPlan Context::plan_prefill(const pam_prefill_request &r) {
    const pam_layer_spec &l = r.layer;
    const int32_t G = l.num_heads / l.num_kv_heads;
    PrefillPlan pl{};
    AttnParams &p = pl.p;
    p.q = r.q;
    p.out = r.output;
    p.k_pool = r.k_pool;
    p.v_pool = r.v_pool;
    p.k_scale = r.k_scale;
    p.v_scale = r.v_scale;
    p.block_tables = r.block_table;
    p.rows = r.seq_len;
    p.num_heads = l.num_heads;
    p.num_kv_heads = l.num_kv_heads;
    p.head_dim = l.head_dim;
    p.block_size = l.block_size;
    p.window = l.window_size;
    p.q_offset = r.q_offset;
    p.causal = r.causal ? 1 : 0;
    p.mode = kRowPrefill;
    p.scale_log2 = kLog2eHost / std::sqrt((float)l.head_dim);
    p.zero_page = zero_page_;

    pl.dense = prefill_mfma_supported(l.data_type, l.head_dim, G, l.block_size) && decode_kernel_choice != 1;
    pl.use_mfma = mfma_supported(l.data_type, l.head_dim, G, l.block_size) && decode_kernel_choice != 1;
    const int32_t nh = heads_per_wave(G);
    p.heads_per_wave = nh;
    pl.kv_len = (int64_t)r.q_offset + r.seq_len;
    const int64_t max_tiles = ceil_div(pl.kv_len, 16) + 1;
    if (pl.dense) {
        const int4 ch = make_int4(0, r.q_offset, r.seq_len, 0);
        p.bt_stride = 0;
        p.max_parts = 1;
        StageList sl;
        const DensePlan d = plan_dense_prefill(p, &ch, 1, sl);
        bind_dense_prefill(p, d, static_cast<const char *>(stage(4, sl.blob.data(), sl.blob.size())));
        pl.tmp = d.tmp;
    } else {
        const int64_t waves = (int64_t)r.seq_len * (pl.use_mfma ? l.num_kv_heads : l.num_heads / nh);
        pl.tmp = plan_split(p, l.data_type, pl.use_mfma, max_tiles, waves);
    }
    return pl;
}

void Context::launch_prefill_plan(const PrefillPlan &pl, int32_t dtype, bool mark_mid) {
    hipEvent_t mid = gpu_timing && mark_mid ? evmid_ : nullptr;
    if (pl.dense)
        check_launch([&] { return launch_prefill_mfma(pl.p, dtype, stream(), ktab()); }, "prefill");
    else
        check_launch([&] { return launch_attention(pl.p, dtype, pl.use_mfma, stream(), mid, ktab()); }, "prefill");
}

void Context::prefill_gpu(const pam_prefill_request &r) {
    const pam_layer_spec &l = r.layer;
    const PrefillPlan pl = plan_prefill(r);
    with_retry("prefill", [&] {
        mark(ev0_);
        launch_prefill_plan(pl, l.data_type);
        mark(ev1_);
        finish("prefill");
    });
    const int32_t op = prefill_operation(l, r.seq_len);
    // split: the dense kernel cut items into pieces merged in the kernel, or the
    // row kernels used split-context partitions
    const bool split = pl.dense ? pl.p.pf_part != nullptr : (pl.p.max_parts > 1 || pl.p.seg_count != nullptr);
    record_stats(op, 1, r.seq_len, (int32_t)ceil_div(pl.kv_len, l.block_size), pl.tmp, split, !pl.dense);
}

// fusedPrefill (PagedAttentionEngine.swift:633-710).  The reference runs one kernel
// that writes the raw rows into the pool and then attends over them; here the
// append kernel and the prefill kernel run back to back on the stream within one
// call (the append moves seq_len rows, a small fraction of the prefill's time).
// FP8 blocks get the append's per-block scale rule, so the pool bytes equal a
// separate append's.
void Context::fused_prefill(const pam_fused_prefill_request &r) {
    validate_layer(r.layer);
    const pam_layer_spec &l = r.layer;
    if (r.seq_len <= 0) throw invalid_configuration("seqLen must be positive.");
    const int64_t nb = ceil_div(r.seq_len, l.block_size);
    require(r.block_table_bytes, "blockTable", nb * 4);
    require(r.output_bytes, "output", r.seq_len * q_bytes_per_token(l));
    require(r.q_bytes, "Q", r.seq_len * q_bytes_per_token(l));
    const int64_t in_row = (int64_t)l.num_kv_heads * l.head_dim * io_bytes(l.data_type);
    require(r.raw_k_bytes, "raw keys", r.seq_len * in_row);
    require(r.raw_v_bytes, "raw values", r.seq_len * in_row);
    require(r.k_pool_bytes, "K pool", pool_bytes_for(nb, l));
    require(r.v_pool_bytes, "V pool", pool_bytes_for(nb, l));
    if (l.data_type == kFP8 && (r.k_scale == nullptr || r.v_scale == nullptr))
        throw invalid_configuration("FP8 fused prefill needs the K and V scale pools.");
    if (!r.q || !r.raw_k || !r.raw_v || !r.block_table || !r.k_pool || !r.v_pool || !r.output)
        throw invalid_configuration("fused prefill request has a null buffer.");
    ensure_device();
    fused_prefill_gpu(r);
}

void Context::fused_prefill_gpu(const pam_fused_prefill_request &r) {
    const pam_layer_spec &l = r.layer;
    pam_append_request a{};
    a.keys = r.raw_k;
    a.values = r.raw_v;
    a.k_pool = r.k_pool;
    a.v_pool = r.v_pool;
    a.block_table = r.block_table;
    a.token_offset = 0;
    a.num_new_tokens = r.seq_len;
    a.layer = l;
    a.k_scale = r.k_scale;
    a.v_scale = r.v_scale;
    pam_prefill_request q{};
    q.q = r.q;
    q.k_pool = r.k_pool;
    q.v_pool = r.v_pool;
    q.block_table = r.block_table;
    q.output = r.output;
    q.seq_len = r.seq_len;
    q.q_offset = 0;
    q.layer = l;
    q.causal = r.causal;
    q.k_scale = r.k_scale;
    q.v_scale = r.v_scale;
    const AppendParams ap = append_params(a);
    PrefillPlan pl = plan_prefill(q);
    // the dense f16 kernel appends as it reads: one launch; other cases append
    // first, then attend
    const bool one_kernel = fused_one_kernel && pl.dense && l.data_type == kF16;
    if (one_kernel) {
        pl.p.fuse_k = r.raw_k;
        pl.p.fuse_v = r.raw_v;
    }
    with_retry("fusedPrefill", [&] {
        mark(ev0_);
        if (!one_kernel) check_launch([&] { return launch_append(ap, l.data_type, stream(), ktab()); }, "fused prefill append");
        launch_prefill_plan(pl, l.data_type);
        mark(ev1_);
        finish("fusedPrefill");
    });
    // the reference reports its fused kernel as prefillSinglePass
    record_stats(PAM_OP_PREFILL_SINGLE_PASS, 1, r.seq_len, (int32_t)ceil_div(r.seq_len, l.block_size), pl.tmp,
                 pl.p.max_parts > 1 || pl.p.seg_count != nullptr, false);
}

// ------------------------------------------------------------------ backward

// backward(q:kPool:vPool:...) (PagedAttentionEngine.swift:1340-1396): withRetry,
// no degradation, f32 or f16.
void Context::backward(const pam_backward_request &r) {
    validate_layer(r.layer);
    const pam_layer_spec &l = r.layer;
    if (r.seq_len <= 0) throw invalid_configuration("seqLen must be positive.");
    if (l.data_type == kFP8) throw PamError("Unsupported paged attention path: backward takes f32 or f16 caches.");
    if (l.head_dim > 256) throw PamError("Unsupported paged attention path: backward needs headDim <= 256.");
    if (!r.q || !r.k_pool || !r.v_pool || !r.block_table || !r.d_out || !r.m || !r.l || !r.d_q || !r.d_k_pool ||
        !r.d_v_pool)
        throw invalid_configuration("backward request has a null buffer.");
    ensure_device();
    // refused before any work or retry: the same request would be refused again
    if (ktab() && ktab()->strict)
        throw PamError("Unsupported paged attention path: the backward kernels are not in the code object.");
    BackwardParams p{};
    p.q = r.q;
    p.k_pool = r.k_pool;
    p.v_pool = r.v_pool;
    p.d_out = r.d_out;
    p.block_table = r.block_table;
    p.m = r.m;
    p.l = r.l;
    p.d_q = r.d_q;
    p.d_k_pool = r.d_k_pool;
    p.d_v_pool = r.d_v_pool;
    p.seq_len = r.seq_len;
    p.window_start = l.window_size > 0 ? std::max(0, r.seq_len - l.window_size) : 0;
    p.num_heads = l.num_heads;
    p.num_kv_heads = l.num_kv_heads;
    p.head_dim = l.head_dim;
    p.block_size = l.block_size;
    p.scale = 1.0f / std::sqrt((float)l.head_dim);
    const int64_t tmp = (int64_t)r.seq_len * l.num_heads * 4 * 2;
    reserve_workspace((size_t)tmp);
    p.row_d = static_cast<float *>(workspace_.ptr);
    p.row_c = p.row_d + (int64_t)r.seq_len * l.num_heads;
    with_retry("backward", [&] {
        mark(ev0_);
        check_launch([&] { return launch_backward(p, l.data_type, stream()); }, "backward");
        mark(ev1_);
        finish("backward");
    });
    record_stats(PAM_OP_BACKWARD, 1, r.seq_len, (int32_t)ceil_div(r.seq_len, l.block_size), tmp, false, false);
}

// ------------------------------------------------------------------ append

void Context::append(const pam_append_request &r) {
    validate_append(r);
    ensure_device();
    if (graceful_degradation) {
        try {
            append_gpu(r);
        } catch (const PamError &e) {
            std::fprintf(stderr, "[pam] appendToCache failed: %s\n", e.what());
        }
    } else {
        append_gpu(r);
    }
}

// validateAppend (PagedAttentionEngine.swift:1936-1950)
void Context::validate_append(const pam_append_request &r) {
    validate_layer(r.layer);
    if (r.token_offset < 0) throw invalid_configuration("tokenOffset must be non-negative.");
    if (r.num_new_tokens <= 0) throw invalid_configuration("numNewTokens must be positive.");
    const pam_layer_spec &l = r.layer;
    const int64_t final_len = (int64_t)r.token_offset + r.num_new_tokens;
    const int64_t nb = ceil_div(final_len, l.block_size);
    const int64_t in_row = (int64_t)l.num_kv_heads * l.head_dim * io_bytes(l.data_type);
    require(r.keys_bytes, "new keys", r.num_new_tokens * in_row);
    require(r.values_bytes, "new values", r.num_new_tokens * in_row);
    if (!r.slot_mapping) require(r.block_table_bytes, "blockTable", nb * 4);
    require(r.k_pool_bytes, "K pool", pool_bytes_for(nb, l));
    require(r.v_pool_bytes, "V pool", pool_bytes_for(nb, l));
    if (l.data_type == kFP8 && (r.k_scale == nullptr || r.v_scale == nullptr))
        throw invalid_configuration("FP8 append needs the K and V scale pools.");
    if (l.data_type == kFP8 && r.slot_mapping)
        throw PamError("Unsupported paged attention path: FP8 append takes a block table, not a slot mapping.");
    if (!r.keys || !r.values || !r.k_pool || !r.v_pool || (!r.block_table && !r.slot_mapping))
        throw invalid_configuration("append request has a null buffer.");
}

bool Context::decode_step(const pam_append_request &a, const AppendParams &ap, const pam_decode_request &d) {
    validate_append(a);
    validate_decode(d);
    if (a.num_new_tokens != 1 || a.layer.data_type == kFP8)
        throw invalid_configuration("the decode step appends one f32 or f16 token.");
    ensure_device();
    auto run = [&] {
        const DecodePlan dp = plan_decode(d, nullptr, 1, nullptr, nullptr);
        with_retry("decodeStep", [&] {
            mark(ev0_);
            check_launch([&] { return launch_append(ap, a.layer.data_type, stream(), ktab()); }, "decode step append");
            check_launch([&] { return launch_attention(dp.p, d.layer.data_type, dp.use_mfma, stream(),
                                                       gpu_timing ? evmid_ : nullptr, ktab()); },
                         "decode step");
            mark(ev1_);
            finish("decode step");
        });
        record_stats(PAM_OP_DECODE, 1, 0, d.max_num_blocks, dp.tmp, dp.p.max_parts > 1 || dp.p.seg_count != nullptr,
                     true);
    };
    if (graceful_degradation) {
        try {
            run();
        } catch (const PamError &e) {
            std::fprintf(stderr, "[pam] decode step failed: %s\n", e.what());
            zero_output(d.output, (size_t)q_bytes_per_token(d.layer));
            return false;
        }
    } else {
        run();
    }
    return true;
}

AppendParams Context::append_params(const pam_append_request &r) {
    const pam_layer_spec &l = r.layer;
    AppendParams p{};
    p.keys = r.keys;
    p.values = r.values;
    p.k_pool = r.k_pool;
    p.v_pool = r.v_pool;
    p.k_scale = r.k_scale;
    p.v_scale = r.v_scale;
    p.block_table = r.block_table;
    p.slot_mapping = r.slot_mapping;
    p.token_offset = r.token_offset;
    p.num_tokens = r.num_new_tokens;
    p.num_kv_heads = l.num_kv_heads;
    p.head_dim = l.head_dim;
    p.block_size = l.block_size;
    p.fixed_slot = -1;
    return p;
}

void Context::append_gpu(const pam_append_request &r) {
    const pam_layer_spec &l = r.layer;
    const AppendParams p = append_params(r);
    with_retry(l.data_type == kFP8 ? "appendToCacheCheckedFP8" : "appendToCacheFlat", [&] {
        mark(ev0_);
        check_launch([&] { return launch_append(p, l.data_type, stream(), ktab()); }, "append");
        mark(ev1_);
        finish("append");
    });
    record_stats(PAM_OP_APPEND, 1, r.num_new_tokens, 0, 0, false, false);
}

// ------------------------------------------------------------------ mixed step

void Context::mixed_step(const pam_mixed_request &r) {
    const pam_layer_spec &l = r.layer;
    validate_layer(l);
    if (r.num_seqs <= 0) throw invalid_configuration("numSeqs must be positive.");
    if (!r.context_lens || !r.query_lens) throw invalid_configuration("mixed step needs host context/query lengths.");
    if (!r.q || !r.output || !r.k_pool || !r.v_pool || !r.block_tables)
        throw invalid_configuration("mixed step request has a null buffer.");
    if (l.data_type == kFP8 && (!r.k_scale || !r.v_scale))
        throw invalid_configuration("FP8 mixed step needs the K and V scale pools.");
    if (r.bt_stride <= 0) throw invalid_configuration("btStride must be positive.");
    // buffer sizes, before any launch (every kernel below indexes them by row)
    {
        int64_t total_rows = 0, max_blocks = 0;
        for (int32_t s = 0; s < r.num_seqs; s++) {
            if (r.context_lens[s] < 0 || r.query_lens[s] < 0)
                throw invalid_configuration("negative context or query length");
            total_rows += r.query_lens[s];
            const int64_t nb = ceil_div((int64_t)r.context_lens[s] + r.query_lens[s], l.block_size);
            if (nb > r.bt_stride) throw buffer_too_small("blockTables row", nb * 4, (int64_t)r.bt_stride * 4);
            max_blocks = std::max<int64_t>(max_blocks, nb);
        }
        const int64_t in_row = (int64_t)l.num_kv_heads * l.head_dim * io_bytes(l.data_type);
        require(r.q_bytes, "Q", total_rows * q_bytes_per_token(l));
        require(r.output_bytes, "output", total_rows * q_bytes_per_token(l));
        if (r.new_keys || r.new_values) {
            if (!r.new_keys || !r.new_values) throw invalid_configuration("mixed step needs both new keys and new values.");
            require(r.new_keys_bytes, "new keys", total_rows * in_row);
            require(r.new_values_bytes, "new values", total_rows * in_row);
        }
        require(r.block_tables_bytes, "blockTables", (int64_t)r.num_seqs * r.bt_stride * 4);
        require(r.k_pool_bytes, "K pool", pool_bytes_for(max_blocks, l));
        require(r.v_pool_bytes, "V pool", pool_bytes_for(max_blocks, l));
    }
    ensure_device();
    const int32_t bs = l.block_size, W = l.window_size;
    const int32_t G = l.num_heads / l.num_kv_heads;
    // multi-token chunks go to the dense prefill kernel where it applies
    const bool dense = prefill_mfma_supported(l.data_type, l.head_dim, G, l.block_size) && decode_kernel_choice != 1;
    std::vector<int4> rows, chunks;
    std::vector<int32_t> cu(r.num_seqs + 1, 0);
    int64_t max_tiles = 1;
    for (int32_t s = 0; s < r.num_seqs; s++) {
        const int64_t c = r.context_lens[s], T = r.query_lens[s];
        if (c < 0 || T < 0) throw invalid_configuration("negative context or query length");
        const int64_t kv_len = c + T;
        if (ceil_div(kv_len, bs) > r.bt_stride) throw buffer_too_small("blockTables row", ceil_div(kv_len, bs) * 4, (int64_t)r.bt_stride * 4);
        const int64_t ws = W > 0 ? std::max<int64_t>(0, kv_len - W) : 0;
        if (dense && T > 1) {
            chunks.push_back(make_int4(s, (int32_t)c, (int32_t)T, cu[s]));
            cu[s + 1] = cu[s] + (int32_t)T;
            continue;
        }
        for (int64_t i = 0; i < T; i++) {
            int4 ri;
            ri.x = s;
            ri.y = (int32_t)ws;
            ri.z = (int32_t)(c + i + 1);
            ri.w = cu[s] + (int32_t)i;
            rows.push_back(ri);
        }
        max_tiles = std::max<int64_t>(max_tiles, ceil_div(kv_len, 16) - ws / 16);
        cu[s + 1] = cu[s] + (int32_t)T;
    }
    const int32_t total = cu[r.num_seqs];
    if (total == 0) return;
    const int32_t ragged_rows = (int32_t)rows.size();
    bool use_mfma = mfma_supported(l.data_type, l.head_dim, G, l.block_size) && G >= 4;
    if (decode_kernel_choice == 1) use_mfma = false;
    const int32_t nh = heads_per_wave(G);

    // device-side descriptors, staged with one copy (StageList)
    StageList sl;
    const size_t o_rows = sl.add(rows.data(), rows.size() * sizeof(int4));
    AppendBatchParams ab{};
    std::vector<int2> tok;
    std::vector<int4> work;
    size_t o_cu = 0, o_ctx = 0, o_work = 0, o_tok = 0;
    const bool appending = r.new_keys && r.new_values;
    if (appending) {
        o_cu = sl.add(cu.data(), cu.size() * 4);
        o_ctx = sl.add(r.context_lens, (size_t)r.num_seqs * 4);
        if (l.data_type == kFP8) {
            for (int32_t s = 0; s < r.num_seqs; s++) {
                const int64_t c = r.context_lens[s], T = r.query_lens[s];
                if (T <= 0) continue;
                for (int64_t lb = c / bs; lb <= (c + T - 1) / bs; lb++) work.push_back(make_int4(s, (int)lb, 0, 0));
            }
            o_work = sl.add(work.data(), work.size() * sizeof(int4));
        } else {
            // per-token (sequence, position); the kernel resolves slots from the device table
            for (int32_t s = 0; s < r.num_seqs; s++)
                for (int64_t i = 0; i < r.query_lens[s]; i++) tok.push_back(make_int2(s, (int)(r.context_lens[s] + i)));
            o_tok = sl.add(tok.data(), tok.size() * sizeof(int2));
        }
    }
    AttnParams pf{};  // the dense prefill's work list and split workspace
    pf.num_heads = l.num_heads;
    pf.num_kv_heads = l.num_kv_heads;
    pf.window = W;
    pf.causal = 1;
    // One launch for the chunks and the decode rows (mixed.hip): the prefill's
    // workgroups first, the decode's after them, on CUs of their own (a
    // workgroup of either part fills a CU).  The split follows a cost estimate:
    // the prefill's key tiles (plus the per-item cost of the planner) at
    // kPfUnitUs per tile per CU, the decode rows' K/V bytes at kDecodeCuGBs per
    // CU; the decode gets the CUs (a multiple of 8, one per XCD in turn) that
    // balance the two.  Automatic mode takes it when its estimate beats
    // separate launches (prefill on every CU, then the decode at the chip's
    // rate) by 5%.  c3 measured 0.224-0.227 ms with 64-72 decode CUs against
    // 0.258 ms for separate launches.
    const bool one_ok = !chunks.empty() && ragged_rows > 0 && use_mfma && part_tokens_override == 0 &&
                        mixed_launch_supported(l.data_type, l.head_dim, G, bs, ragged_rows);
    bool one_launch = false;
    int32_t mix_pf_groups = mixed_prefill_groups, mix_dec_groups = mixed_decode_groups;
    if (one_ok && mixed_launch_mode != 1) {
        constexpr double kPfUnitUs = 1.0, kDecodeCuGBs = 40.0, kChipGBs = 5800.0;
        const int32_t tpw = 256 / G;  // a prefill item: 256 query rows (token, head) of one kv head
        double units = 0.0;
        for (const int4 &c : chunks) {
            const int64_t kv_len = (int64_t)c.y + c.z;
            const int64_t ws = W > 0 ? std::max<int64_t>(0, kv_len - W) : 0;
            for (int32_t tok0 = 0; tok0 < c.z; tok0 += tpw) {
                const int64_t key_end = (int64_t)c.y + std::min(c.z, tok0 + tpw);
                units += (double)(ceil_div(key_end, 32) - ws / 32 + 12) * l.num_kv_heads;
            }
        }
        double dec_bytes = 0.0;
        const double row_bytes = (double)l.num_kv_heads * l.head_dim * (l.data_type == kFP8 ? 1 : 2) * 2;
        for (const int4 &ri : rows) dec_bytes += (double)(ri.z - ri.y) * row_bytes;
        auto est_one = [&](int32_t dec) {
            return std::max(units * kPfUnitUs / (cus_ - dec), dec_bytes / (dec * kDecodeCuGBs * 1e3)) + 13.0;
        };
        int32_t best = 0;
        double best_t = 1e300;
        for (int32_t dec = 8; dec + 8 <= cus_; dec += 8) {
            const double t = est_one(dec);
            if (t < best_t) best_t = t, best = dec;
        }
        const double t_sep = units * kPfUnitUs / cus_ + dec_bytes / (kChipGBs * 1e3) + 17.0;
        if (mixed_launch_mode == 2 || (best > 0 && best_t < 0.95 * t_sep)) {
            one_launch = true;
            // groups not set by the caller: the estimate's split, or (a device
            // too small to split) every CU for each part, the decode after the prefill
            if (mix_dec_groups <= 0) mix_dec_groups = best > 0 ? best : cus_;
            if (mix_pf_groups <= 0) mix_pf_groups = best > 0 ? cus_ - mix_dec_groups : cus_;
        }
    }
    DensePlan dense_plan;
    if (!chunks.empty())
        dense_plan = plan_dense_prefill(pf, chunks.data(), (int32_t)chunks.size(), sl, one_launch ? mix_pf_groups : 0);
    const char *sbase = static_cast<const char *>(stage(0, sl.blob.data(), sl.blob.size()));
    const int4 *d_rows = ragged_rows ? reinterpret_cast<const int4 *>(sbase + o_rows) : nullptr;
    if (appending) {
        ab.keys = r.new_keys;
        ab.values = r.new_values;
        ab.k_pool = r.k_pool;
        ab.v_pool = r.v_pool;
        ab.k_scale = r.k_scale;
        ab.v_scale = r.v_scale;
        ab.block_tables = r.block_tables;
        ab.bt_stride = r.bt_stride;
        ab.seqs = r.num_seqs;
        ab.total_tokens = total;
        ab.num_kv_heads = l.num_kv_heads;
        ab.head_dim = l.head_dim;
        ab.block_size = bs;
        ab.cu_tokens = reinterpret_cast<const int32_t *>(sbase + o_cu);
        ab.token_offsets = reinterpret_cast<const int32_t *>(sbase + o_ctx);
        if (l.data_type == kFP8) {
            ab.work = reinterpret_cast<const int4 *>(sbase + o_work);
            ab.num_work = (int32_t)work.size();
        } else {
            ab.token_pos = reinterpret_cast<const int2 *>(sbase + o_tok);
        }
    }

    AttnParams p{};
    p.q = r.q;
    p.out = r.output;
    p.k_pool = r.k_pool;
    p.v_pool = r.v_pool;
    p.k_scale = r.k_scale;
    p.v_scale = r.v_scale;
    p.block_tables = r.block_tables;
    p.row_info = d_rows;
    p.rows = ragged_rows;
    p.bt_stride = r.bt_stride;
    p.max_num_blocks = r.bt_stride;
    p.num_heads = l.num_heads;
    p.num_kv_heads = l.num_kv_heads;
    p.head_dim = l.head_dim;
    p.block_size = bs;
    p.window = W;
    p.mode = kRowRagged;
    p.causal = 1;  // prefill chunks are causal within the chunk (ragged rows carry it in k_hi)
    if (!chunks.empty()) {
        p.pf_part = pf.pf_part;
        p.pf_count = pf.pf_count;
        p.pf_part_bytes = pf.pf_part_bytes;
        p.pf_groups = pf.pf_groups;
        bind_dense_prefill(p, dense_plan, sbase);
    }
    p.heads_per_wave = nh;
    p.scale_log2 = kLog2eHost / std::sqrt((float)l.head_dim);
    p.zero_page = zero_page_;
    const int64_t waves = (int64_t)ragged_rows * (use_mfma ? l.num_kv_heads : l.num_heads / nh);
    int64_t tmp = 0;
    if (one_launch) {
        int64_t slots = 0, counters = 0;
        mixed_decode_slots(p, mix_dec_groups, &slots, &counters);
        const int64_t bytes = slots * ((int64_t)l.head_dim + 2) * 4;
        if (bytes >= ((int64_t)1 << 31)) throw PamError("stream-K workspace exceeds 2 GiB");
        reserve_workspace((size_t)bytes);
        reserve_counters(seg_count_, (size_t)counters * 8);
        p.part_o = static_cast<float *>(workspace_.ptr);
        p.part_ml = p.part_o + slots * l.head_dim;
        p.part_bytes = (uint32_t)bytes;
        p.seg_count = static_cast<uint64_t *>(seg_count_.ptr);
        p.part_tokens = (int32_t)((max_tiles + 1) * 16);
        p.max_parts = 1;
        tmp = bytes;
    } else if (ragged_rows > 0) {
        tmp = plan_split(p, l.data_type, use_mfma, max_tiles + 1, waves);
    }
    with_retry("mixedStep", [&] {
        mark(ev0_);
        if (ab.keys) check_launch([&] { return launch_append_batch(ab, l.data_type, stream(), ktab()); }, "mixed append");
        if (one_launch) {
            check_launch([&] { return launch_mixed_step(p, l.data_type, mix_dec_groups, stream(), ktab()); }, "mixed attention");
            mark(evmid_);
            mark(ev1_);
            finish("mixed step");
            return;
        }
        if (!chunks.empty()) check_launch([&] { return launch_prefill_mfma(p, l.data_type, stream(), ktab()); }, "mixed prefill");
        if (ragged_rows > 0)
            check_launch([&] { return launch_attention(p, l.data_type, use_mfma, stream(), gpu_timing ? evmid_ : nullptr, ktab()); }, "mixed attention");
        else
            mark(evmid_);
        mark(ev1_);
        finish("mixed step");
    });
    record_stats(PAM_OP_DECODE, r.num_seqs, total, r.bt_stride, tmp, p.max_parts > 1 || p.seg_count != nullptr, true);
}

// ------------------------------------------------------------------ codec

void Context::fp8_quantize(const uint16_t *v, const uint16_t *s, uint8_t *o, int64_t n) {
    ensure_device();
    check_launch([&] { return launch_fp8_quantize(v, s, o, n, stream()); }, "fp8 quantize");
    finish("fp8 quantize");
}

void Context::fp8_dequant(const uint8_t *c, const uint16_t *s, uint16_t *o, int64_t n) {
    ensure_device();
    check_launch([&] { return launch_fp8_dequant(c, s, o, n, stream()); }, "fp8 dequant");
    finish("fp8 dequant");
}

}  // namespace pam
