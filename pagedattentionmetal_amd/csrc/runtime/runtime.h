// runtime.h - host runtime of libpam: the engine context and the device KV cache.
//
// Context  ~ PagedAttentionEngine (Sources/PagedAttentionMetal/PagedAttentionEngine.swift):
//            request validation (:1897-2006), kernel selection, launch on one HIP
//            stream, retry with backoff + circuit breaker (:375-400), graceful
//            degradation that zero-fills the output (:405-418, :533-546), lastStats.
// KVCache  ~ KVCacheManager / BatchKVCacheManager (KVCacheManager.swift): a
//            BlockAllocator plus K/V pools (and FP8 scale pools) resident in HBM.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/pam.h"
#include "../kernels/kernels.h"
#include "block_allocator.h"

namespace pam {

void hip_check(hipError_t e, const char *what);

// A growable device buffer owned by a context.
struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
};

class Context;

// Several host arrays staged to the device with one copy: parts are packed at
// 16-byte offsets into one blob; after Context::stage of the blob, part i lives
// at base + offset(i).
struct StageList {
    std::vector<char> blob;
    size_t add(const void *p, size_t bytes) {
        const size_t off = (blob.size() + 15) & ~(size_t)15;
        blob.resize(off + bytes);
        if (bytes) std::memcpy(blob.data() + off, p, bytes);
        return off;
    }
};

class KVCache {
   public:
    KVCache(Context *ctx, int32_t max_blocks, int32_t block_size, int32_t head_dim, int32_t num_kv_heads,
            int32_t dtype, bool with_device);
    ~KVCache();

    std::mutex mu;
    BlockAllocator alloc;
    int32_t head_dim, num_kv_heads, dtype;
    bool has_device;
    int device = 0;
    void *k_pool = nullptr, *v_pool = nullptr;
    uint16_t *k_scale = nullptr, *v_scale = nullptr;
    size_t pool_bytes = 0;

    size_t bytes_per_block() const;  // one pool (K or V)
    // perform copy-on-write block copies in HBM on the given stream
    void copy_blocks(const BlockCopies &copies, hipStream_t stream, const KernelTable *kt = nullptr);

    // A sequence's block table and length kept in HBM for the decode step
    // (pam_decode_step): [length | table entries ...], capacity `cap` entries.
    // `shadow` is what the device copy holds; a step whose table only grew by
    // its last entry patches that entry in the append kernel, any other change
    // re-stages the whole table.
    struct DeviceTable {
        int32_t *ptr = nullptr;
        int32_t cap = 0;
        std::vector<int32_t> shadow;
        uint32_t length = 0;
    };
    std::unordered_map<int64_t, DeviceTable> device_tables;
    void drop_device_table(int64_t id);
};

class Context {
   public:
    Context();
    ~Context();

    std::mutex mu;
    std::string last_error;
    bool has_error = false;

    void set_error(const std::string &m) {
        last_error = m;
        has_error = true;
    }
    void clear_error() {
        last_error.clear();
        has_error = false;
    }

    // --- device state (created on first GPU use)
    void ensure_device();
    hipStream_t stream();
    // Launch on a caller's stream (or back on the context's own).  Work the
    // context already issued on the previous stream is ordered before anything
    // it issues on the new one: its launches share the split workspace and the
    // stream-K counters, so they must never overlap.
    void set_stream(hipStream_t s) { switch_stream(true, s); }
    void use_own_stream() { switch_stream(false, nullptr); }
    void switch_stream(bool use_ext, hipStream_t s);
    bool synchronous = true;
    void finish(const char *what);  // synchronise when synchronous, surface GPU errors

    // --- engine (PagedAttentionEngine)
    void decode(const pam_decode_request &r);
    // decode with the split-context workspace, counters and zero page in the
    // library's fixed per-device scratch: no allocation (setup_noalloc first)
    void decode_noalloc(const pam_decode_request &r);
    // decodeLayers / prefillLayers / appendLayers: per-layer buffers over one
    // shared pool
    void decode_layers(const pam_decode_layers_request &r);
    void prefill_layers(const pam_prefill_layers_request &r);
    void append_layers(const pam_append_layers_request &r);
    static void validate_prefill(const pam_prefill_request &r);
    static void validate_append(const pam_append_request &r);
    int32_t last_fused_groups = 0;  // launches the last decode_layers call made
    void setup_noalloc();
    void prefill(const pam_prefill_request &r);
    void append(const pam_append_request &r);
    // one decode step of a sequence: the append of its new token (`ap`, one
    // token, with its table and length patches) then the decode of `d`, which
    // reads the table and length the append wrote; validated as append + decode.
    // False: the work failed and graceful degradation zeroed the output
    bool decode_step(const pam_append_request &a, const AppendParams &ap, const pam_decode_request &d);
    void mixed_step(const pam_mixed_request &r);
    void fused_prefill(const pam_fused_prefill_request &r);
    void backward(const pam_backward_request &r);
    void fp8_quantize(const uint16_t *v, const uint16_t *s, uint8_t *o, int64_t n);
    void fp8_dequant(const uint8_t *c, const uint16_t *s, uint16_t *o, int64_t n);

    pam_stats last_stats{};
    pam_stats stats();  // last_stats with event timings resolved
    bool graceful_degradation = true;
    // splitThreshold, defaultWindowSize, defaultChunkSize
    // (PagedAttentionEngine.swift:116-121)
    int32_t split_threshold = 1024;
    int32_t default_window_size = 0;
    int32_t default_chunk_size = 0;
    // the flat overloads: prefill(q:...:windowSize:chunkSize:) (:713-760),
    // decode(q:...:windowSize:) (:1012-1046), appendToCache(keys:...:windowSize:)
    // (:1167-1201)
    void prefill_flat(const pam_prefill_request &r, int32_t window_size, int32_t chunk_size);
    void decode_flat(const pam_decode_request &r, int32_t window_size);
    void append_flat(const pam_append_request &r, int32_t window_size);
    int32_t max_retries = 3;
    int32_t consecutive_failures = 0;
    int32_t fail_next_launches = 0;
    int32_t part_tokens_override = 0;
    int32_t decode_kernel_choice = 0;
    // mixed step: 0 automatic, 1 separate launches, 2 one launch; its groups (0: automatic)
    int32_t mixed_launch_mode = 0, mixed_prefill_groups = 0, mixed_decode_groups = 0;
    // fused prefill, f16 with d = 128: false appends then prefills (two launches,
    // the faster on gfx950), true runs the one kernel that appends as it reads
    bool fused_one_kernel = false;
    // HIP events around each call's kernels (the timings of last_stats); off
    // saves their queue packets between back-to-back launches
    bool gpu_timing = true;
    void mark(hipEvent_t e) {
        if (gpu_timing) (void)hipEventRecord(e, stream());
    }

    // Test hook: every merge counter the context owns is set to `arrivals`
    // arrivals of an abandoned launch (a consumed epoch).
    void dirty_counters(int32_t arrivals);

    // --- code object (libpam_kernels.hsaco): named entries loaded with
    // hipModuleLoad and used for this context's launches while loaded
    void module_load(const char *path);
    void module_unload();
    void *module_function(const char *name);
    void module_launch_raw(void *function, const uint32_t grid[3], const uint32_t block[3], uint32_t shared_bytes,
                           void *args, size_t args_bytes);
    const KernelTable *ktab() const { return module_ ? &ktab_ : nullptr; }
    // strict: launches the code object has no entry for fail instead of
    // running the library's kernel
    void module_set_strict(bool strict) {
        module_strict_ = strict;
        ktab_.strict = strict;
    }

    // --- scratch
    void reserve_workspace(size_t bytes);
    // stage host bytes into a context-owned device region (slot selects one of
    // several independent regions); returns the device pointer
    void *stage(int slot, const void *host, size_t bytes);
    void *stage_into(void *device_dst, const void *host, size_t bytes);
    void *device_scratch(int slot, size_t bytes);

   private:
    template <class F>
    void with_retry(const char *op, F &&fn);
    template <class F>
    void check_launch(F &&launch, const char *what);
    void zero_output(void *ptr, size_t bytes);
    void decode_checked(const pam_decode_request &r, bool noalloc);
    void decode_gpu(const pam_decode_request &r, char *fixed);
    struct DecodePlan {
        AttnParams p;
        bool use_mfma;
        int64_t tmp;
    };
    DecodePlan plan_decode(const pam_decode_request &r, char *fixed, int32_t fused, const void *const *layers_q,
                           void *const *layers_out);
    int32_t fusable_layers(const pam_decode_request &r);
    void decode_layers_gpu(const std::vector<pam_decode_request> &reqs);
    void prefill_gpu(const pam_prefill_request &r);
    void append_gpu(const pam_append_request &r);
    void fused_prefill_gpu(const pam_fused_prefill_request &r);
    // a prefill's launch, planned (parameters, kernel choice, split workspace)
    struct PrefillPlan {
        AttnParams p;
        bool dense, use_mfma;
        int64_t tmp, kv_len;
    };
    PrefillPlan plan_prefill(const pam_prefill_request &r);
    void launch_prefill_plan(const PrefillPlan &pl, int32_t dtype, bool mark_mid = true);
    AppendParams append_params(const pam_append_request &r);
    int32_t choose_part_tokens(int64_t items_per_part, int64_t max_tiles, bool mfma);
    int64_t plan_split(AttnParams &p, int32_t dtype, bool use_mfma, int64_t max_tiles, int64_t waves,
                       char *fixed = nullptr);
    // dense prefill: work list of host chunks (the order staged as p.chunks) added
    // to `sl`, partial slots and counters reserved; after staging `sl` at `base`,
    // bind_dense_prefill points p at the list
    struct DensePlan {
        size_t o_work = 0, o_range = 0;
        int64_t tmp = 0;
    };
    DensePlan plan_dense_prefill(AttnParams &p, const int4 *chunks, int32_t n, StageList &sl, int32_t groups = 0);
    static void bind_dense_prefill(AttnParams &p, const DensePlan &d, const char *base);
    int32_t prefill_operation(const pam_layer_spec &l, int32_t seq_len) const;
    void record_stats(int32_t op, int32_t batch, int32_t seq_len, int32_t blocks, int64_t tmp, bool split,
                      bool has_mid);

    bool device_ready_ = false;
    int device_ = 0;
    int cus_ = 256;  // compute units of the device (set in ensure_device)
    hipStream_t own_stream_ = nullptr, ext_stream_ = nullptr;
    bool use_ext_stream_ = false;
    hipEvent_t ev0_ = nullptr, ev1_ = nullptr, evmid_ = nullptr, handoff_ = nullptr;
    // pinned staging ring: kStageSegs segments, each with the event of its last copy
    static constexpr int kStageSegs = 4;
    hipEvent_t seg_event_[kStageSegs] = {};
    bool seg_used_[kStageSegs] = {};
    int cur_seg_ = 0;
    void *zero_page_ = nullptr;
    hipModule_t module_ = nullptr;
    bool module_strict_ = false;
    KernelTable ktab_{};
    bool stats_pending_ = false;
    bool stats_has_mid_ = false;
    DeviceBuffer workspace_;
    DeviceBuffer seg_count_;  // stream-K merge counters (epoch-tagged, never reset)
    DeviceBuffer pf_part_;    // dense prefill: partial slots of split items
    DeviceBuffer pf_count_;   // dense prefill: merge counters (epoch-tagged, never reset)
    void reserve_counters(DeviceBuffer &b, size_t bytes);
    DeviceBuffer scratch_[6];
    void *pinned_ = nullptr;
    void *pinned_dev_ = nullptr;  // the device's address of pinned_
    size_t pinned_bytes_ = 0;
    size_t pinned_used_ = 0;
};

}  // namespace pam
