// capi.cpp - extern "C" exports declared in include/pam.h.
//
// Handles are heap objects (the reference retains Swift objects with
// Unmanaged.passRetained, PagedAttentionCABI.swift:75,127).  Every context call
// runs under the context mutex; cache state under the cache mutex (context
// first, then cache).  Failures set the context's last error and return -1
// (PagedAttentionCABI.swift:18-37); success clears it.
#include <dlfcn.h>

#include <mutex>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <exception>
#include <memory>
#include <vector>

#include "runtime.h"
#include "scheduler.h"

using namespace pam;

#define PAM_API extern "C" __attribute__((visibility("default")))

namespace {

Context *ctx_of(void *p) { return static_cast<Context *>(p); }
KVCache *cache_of(void *p) { return static_cast<KVCache *>(p); }
Scheduler *sched_of(void *p) { return static_cast<Scheduler *>(p); }

template <class F>
int32_t guarded(void *context, F &&f) {
    Context *ctx = ctx_of(context);
    if (!ctx) return -1;
    std::lock_guard<std::mutex> g(ctx->mu);
    try {
        f(ctx);
        ctx->clear_error();
        return 0;
    } catch (const std::exception &e) {
        ctx->set_error(e.what());
        return -1;
    }
}

int32_t elem_bytes(int32_t dtype) { return dtype == kF32 ? 4 : (dtype == kF16 ? 2 : 1); }

pam_layer_spec layer_of(const KVCache *c, int32_t num_heads) {
    pam_layer_spec l{};
    l.head_dim = c->head_dim;
    l.num_heads = num_heads;
    l.num_kv_heads = c->num_kv_heads;
    l.block_size = c->alloc.block_size();
    l.data_type = c->dtype;
    l.window_size = 0;
    return l;
}

void require_device(const KVCache *c) {
    if (!c->has_device) throw PamError("Invalid engine state: cache has no device pools.");
}

// the sequence's block table staged to the device (an empty table reads as [0],
// KVCacheManager.swift:310); returns the table length in bytes
size_t stage_table(Context *ctx, KVCache *c, int64_t id, int slot, const int32_t **dev) {
    std::vector<int32_t> t = c->alloc.sequence(id).block_table;
    if (t.empty()) t.push_back(0);
    *dev = static_cast<const int32_t *>(ctx->stage(slot, t.data(), t.size() * 4));
    return t.size() * 4;
}

void *create_cache(void *context, int32_t maxBlocks, int32_t blockSize, int32_t headDim, int32_t numKVHeads,
                   int32_t dataType, bool device) {
    Context *ctx = ctx_of(context);
    if (!ctx) return nullptr;
    std::lock_guard<std::mutex> g(ctx->mu);
    try {
        if (dataType < 0 || dataType > 2)
            throw invalid_configuration("unknown dtype " + std::to_string(dataType) +
                                        "; use 0 for float32, 1 for float16 or 2 for float8");
        // PagedLayerSpec(numHeads: numKVHeads).validate() (PagedAttentionCABI.swift:107-114)
        if (headDim <= 0) throw invalid_configuration("headDim must be positive.");
        if (numKVHeads <= 0) throw invalid_configuration("numHeads must be positive.");
        if (blockSize <= 0) throw invalid_configuration("blockSize must be positive.");
        if (maxBlocks <= 0) throw invalid_configuration("maxBlocks must be positive");
        KVCache *c = new KVCache(ctx, maxBlocks, blockSize, headDim, numKVHeads, dataType, device);
        ctx->clear_error();
        return c;
    } catch (const std::exception &e) {
        ctx->set_error(e.what());
        return nullptr;
    }
}

}  // namespace

// ====================================================================== Part 1

PAM_API void *pam_create_context(void) {
    try {
        return new Context();
    } catch (...) {
        return nullptr;
    }
}

PAM_API void pam_destroy_context(void *context) { delete ctx_of(context); }

PAM_API const char *pam_last_error(void *context) {
    Context *ctx = ctx_of(context);
    if (!ctx || !ctx->has_error) return nullptr;
    return ctx->last_error.c_str();
}

PAM_API void *pam_create_cache(void *context, int32_t maxBlocks, int32_t blockSize, int32_t headDim,
                               int32_t numKVHeads, int32_t dataType) {
    return create_cache(context, maxBlocks, blockSize, headDim, numKVHeads, dataType, true);
}

PAM_API void pam_destroy_cache(void *cache) { delete cache_of(cache); }

PAM_API int32_t pam_reserve_sequence(void *context, void *cache, int64_t sequenceID) {
    KVCache *c = cache_of(cache);
    if (!c) return -1;
    return guarded(context, [&](Context *) {
        std::lock_guard<std::mutex> g(c->mu);
        c->alloc.allocate_sequence(sequenceID);
    });
}

PAM_API int32_t pam_append_tokens(void *context, void *cache, int64_t sequenceID, int32_t count) {
    return pam_append_tokens_hashed(context, cache, sequenceID, count, nullptr, 0);
}

PAM_API void pam_free_sequence(void *cache, int64_t sequenceID) {
    KVCache *c = cache_of(cache);
    if (!c) return;
    std::lock_guard<std::mutex> g(c->mu);
    c->alloc.free_sequence(sequenceID);
    c->drop_device_table(sequenceID);
}

PAM_API int32_t pam_available_blocks(void *cache) {
    KVCache *c = cache_of(cache);
    if (!c) return -1;
    std::lock_guard<std::mutex> g(c->mu);
    return c->alloc.available();
}

PAM_API int32_t pam_sequence_length(void *context, void *cache, int64_t sequenceID) {
    KVCache *c = cache_of(cache);
    if (!c) return -1;
    int64_t len = 0;
    const int32_t rc = guarded(context, [&](Context *) {
        std::lock_guard<std::mutex> g(c->mu);
        len = c->alloc.sequence(sequenceID).length;
    });
    return rc == 0 ? (int32_t)len : -1;
}

PAM_API int32_t pam_append_kv(void *context, void *cache, int64_t sequenceID, void *keys, void *values,
                              int32_t tokenOffset, int32_t numNewTokens, int32_t numHeads) {
    KVCache *c = cache_of(cache);
    if (!c || !keys || !values) return -1;
    return guarded(context, [&](Context *ctx) {
        std::lock_guard<std::mutex> g(c->mu);
        require_device(c);
        pam_append_request r{};
        const int32_t *bt = nullptr;
        r.block_table_bytes = stage_table(ctx, c, sequenceID, 0, &bt);
        r.block_table = bt;
        r.keys = keys;
        r.values = values;
        r.k_pool = c->k_pool;
        r.v_pool = c->v_pool;
        r.k_scale = c->k_scale;
        r.v_scale = c->v_scale;
        r.token_offset = tokenOffset;
        r.num_new_tokens = numNewTokens;
        r.layer = layer_of(c, numHeads);
        r.k_pool_bytes = r.v_pool_bytes = c->pool_bytes;
        ctx->append(r);
    });
}

PAM_API int32_t pam_prefill(void *context, void *cache, int64_t sequenceID, void *query, void *output,
                            int32_t seqLen, int32_t numHeads, bool causal) {
    KVCache *c = cache_of(cache);
    if (!c || !query || !output) return -1;
    return guarded(context, [&](Context *ctx) {
        std::lock_guard<std::mutex> g(c->mu);
        require_device(c);
        pam_prefill_request r{};
        const int32_t *bt = nullptr;
        r.block_table_bytes = stage_table(ctx, c, sequenceID, 0, &bt);
        r.block_table = bt;
        r.q = query;
        r.output = output;
        r.k_pool = c->k_pool;
        r.v_pool = c->v_pool;
        r.k_scale = c->k_scale;
        r.v_scale = c->v_scale;
        r.seq_len = seqLen;
        r.q_offset = 0;
        r.causal = causal;
        r.layer = layer_of(c, numHeads);
        r.k_pool_bytes = r.v_pool_bytes = c->pool_bytes;
        ctx->prefill(r);
    });
}

PAM_API int32_t pam_decode(void *context, void *cache, const int64_t *batchIDs, int32_t batchSize, void *query,
                           void *output, int32_t numHeads) {
    KVCache *c = cache_of(cache);
    if (!c || !batchIDs || !query || !output) return -1;
    return guarded(context, [&](Context *ctx) {
        std::lock_guard<std::mutex> g(c->mu);
        require_device(c);
        // BatchKVCacheView (PagedAttentionCABI.swift:339-372): zero-padded slab,
        // maxNumBlocks = max(1, longest table)
        int32_t max_nb = 1;
        for (int32_t i = 0; i < batchSize; i++)
            max_nb = std::max<int32_t>(max_nb, (int32_t)c->alloc.sequence(batchIDs[i]).block_table.size());
        const int32_t n = std::max<int32_t>(batchSize, 0);
        std::vector<int32_t> slab((size_t)n * max_nb, 0);
        std::vector<uint32_t> lens((size_t)n, 0);
        for (int32_t i = 0; i < n; i++) {
            const LogicalSequence &s = c->alloc.sequence(batchIDs[i]);
            std::copy(s.block_table.begin(), s.block_table.end(), slab.begin() + (size_t)i * max_nb);
            lens[i] = (uint32_t)s.length;
        }
        pam_decode_request r{};
        StageList sl;
        const size_t o_slab = sl.add(slab.data(), slab.size() * 4), o_lens = sl.add(lens.data(), lens.size() * 4);
        const char *base = static_cast<const char *>(ctx->stage(1, sl.blob.data(), sl.blob.size()));
        r.block_tables = reinterpret_cast<const int32_t *>(base + o_slab);
        r.seq_lengths = reinterpret_cast<const uint32_t *>(base + o_lens);
        r.block_tables_bytes = slab.size() * 4;
        r.seq_lengths_bytes = lens.size() * 4;
        r.q = query;
        r.output = output;
        r.k_pool = c->k_pool;
        r.v_pool = c->v_pool;
        r.k_scale = c->k_scale;
        r.v_scale = c->v_scale;
        r.batch_size = batchSize;
        r.max_num_blocks = max_nb;
        r.layer = layer_of(c, numHeads);
        r.k_pool_bytes = r.v_pool_bytes = c->pool_bytes;
        ctx->decode(r);
    });
}

// The adapter's decode step (PagedMetalKVCache.swift:94-129 at seqLen 1):
// appendTokens(count: 1), appendToCache of the token's K/V, decode of its query.
// The sequence's table and length stay in HBM between steps (KVCache::
// DeviceTable): the append kernel writes the token at a slot the host computes,
// patches a new last table entry and the length, and the decode reads them, so
// a step is two launches and no staging.  Any other table change (a first step,
// copy-on-write, a prefix hit) re-stages the table first.
PAM_API int32_t pam_decode_step(void *context, void *cache, int64_t sequenceID, const void *keys, const void *values,
                                const void *query, void *output, int32_t numHeads) {
    KVCache *c = cache_of(cache);
    if (!c || !keys || !values || !query || !output) return -1;
    return guarded(context, [&](Context *ctx) {
        std::lock_guard<std::mutex> g(c->mu);
        require_device(c);
        if (c->dtype == kFP8) throw invalid_configuration("the decode step appends one f32 or f16 token.");
        BlockCopies copies;
        try {
            c->alloc.append_tokens(sequenceID, 1, nullptr, 0, &copies);
        } catch (...) {
            c->copy_blocks(copies, ctx->stream(), ctx->ktab());  // CoW done before an OOM stays done
            throw;
        }
        c->copy_blocks(copies, ctx->stream(), ctx->ktab());
        const LogicalSequence &s = c->alloc.sequence(sequenceID);
        const std::vector<int32_t> &t = s.block_table;
        const int32_t nb = (int32_t)t.size(), bs = c->alloc.block_size();
        KVCache::DeviceTable &m = c->device_tables[sequenceID];
        if (m.cap < nb) {
            int32_t cap = 64;
            while (cap < nb) cap *= 2;
            int32_t *p = nullptr;
            hip_check(hipMalloc(&p, ((size_t)cap + 1) * 4), "hipMalloc decode-step table");
            if (m.ptr) {
                (void)hipStreamSynchronize(ctx->stream());
                (void)hipFree(m.ptr);
            }
            m.ptr = p;
            m.cap = cap;
            m.shadow.clear();
        }
        AppendParams ap{};
        ap.keys = keys;
        ap.values = values;
        ap.k_pool = c->k_pool;
        ap.v_pool = c->v_pool;
        ap.token_offset = (int32_t)s.length - 1;
        ap.num_tokens = 1;
        ap.num_kv_heads = c->num_kv_heads;
        ap.head_dim = c->head_dim;
        ap.block_size = bs;
        const int64_t pos = s.length - 1;
        ap.fixed_slot = (int64_t)t[(size_t)(pos / bs)] * bs + pos % bs;
        ap.length_patch = reinterpret_cast<uint32_t *>(m.ptr);
        ap.length_value = (uint32_t)s.length;
        const bool grew_by_one = m.shadow.size() + 1 == t.size() && std::equal(m.shadow.begin(), m.shadow.end(), t.begin());
        const bool same = m.shadow.size() == t.size() && std::equal(m.shadow.begin(), m.shadow.end(), t.begin());
        if (grew_by_one) {
            ap.table_patch = m.ptr + 1;
            ap.patch_index = nb - 1;
            ap.patch_block = t.back();
        } else if (!same) {
            std::vector<int32_t> img((size_t)nb + 1);
            img[0] = (int32_t)s.length;
            std::copy(t.begin(), t.end(), img.begin() + 1);
            ctx->stage_into(m.ptr, img.data(), img.size() * 4);
        }
        m.shadow.clear();  // unknown until the step's work is enqueued
        pam_append_request a{};
        a.keys = keys;
        a.values = values;
        a.k_pool = c->k_pool;
        a.v_pool = c->v_pool;
        a.block_table = m.ptr + 1;
        a.block_table_bytes = (size_t)nb * 4;
        a.token_offset = ap.token_offset;
        a.num_new_tokens = 1;
        a.layer = layer_of(c, c->num_kv_heads);
        a.k_pool_bytes = a.v_pool_bytes = c->pool_bytes;
        pam_decode_request d{};
        d.q = query;
        d.output = output;
        d.k_pool = c->k_pool;
        d.v_pool = c->v_pool;
        d.block_tables = m.ptr + 1;
        d.seq_lengths = reinterpret_cast<const uint32_t *>(m.ptr);
        d.block_tables_bytes = (size_t)nb * 4;
        d.seq_lengths_bytes = 4;
        d.batch_size = 1;
        d.max_num_blocks = nb;
        d.layer = layer_of(c, numHeads);
        d.k_pool_bytes = d.v_pool_bytes = c->pool_bytes;
        if (ctx->decode_step(a, ap, d)) m.shadow = t;
    });
}

// ====================================================================== Part 2

PAM_API int32_t pam_engine_decode(void *context, const pam_decode_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->decode(*request); });
}

PAM_API int32_t pam_engine_set_config(void *context, const pam_engine_config *config) {
    if (!config) return -1;
    return guarded(context, [&](Context *ctx) {
        if (config->split_threshold < 0 || config->default_window_size < 0 || config->default_chunk_size < 0)
            throw invalid_configuration("engine settings must be non-negative.");
        ctx->split_threshold = config->split_threshold;
        ctx->default_window_size = config->default_window_size;
        ctx->default_chunk_size = config->default_chunk_size;
    });
}

PAM_API int32_t pam_engine_get_config(void *context, pam_engine_config *out) {
    if (!out) return -1;
    return guarded(context, [&](Context *ctx) {
        out->split_threshold = ctx->split_threshold;
        out->default_window_size = ctx->default_window_size;
        out->default_chunk_size = ctx->default_chunk_size;
    });
}

PAM_API int32_t pam_engine_prefill_flat(void *context, const pam_prefill_request *request, int32_t window_size,
                                        int32_t chunk_size) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->prefill_flat(*request, window_size, chunk_size); });
}

PAM_API int32_t pam_engine_decode_flat(void *context, const pam_decode_request *request, int32_t window_size) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->decode_flat(*request, window_size); });
}

PAM_API int32_t pam_engine_append_flat(void *context, const pam_append_request *request, int32_t window_size) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->append_flat(*request, window_size); });
}

PAM_API int32_t pam_engine_decode_layers(void *context, const pam_decode_layers_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->decode_layers(*request); });
}

PAM_API int32_t pam_engine_prefill_layers(void *context, const pam_prefill_layers_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->prefill_layers(*request); });
}

PAM_API int32_t pam_engine_append_layers(void *context, const pam_append_layers_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->append_layers(*request); });
}

PAM_API int32_t pam_module_load(void *context, const char *path) {
    return guarded(context, [&](Context *ctx) { ctx->module_load(path); });
}

PAM_API int32_t pam_module_set_strict(void *context, int32_t strict) {
    return guarded(context, [&](Context *ctx) { ctx->module_set_strict(strict != 0); });
}

PAM_API int32_t pam_module_unload(void *context) {
    return guarded(context, [&](Context *ctx) { ctx->module_unload(); });
}

PAM_API int32_t pam_module_function(void *context, const char *name, void **function) {
    if (!function) return -1;
    return guarded(context, [&](Context *ctx) { *function = ctx->module_function(name); });
}

PAM_API int32_t pam_module_launch(void *context, void *function, uint32_t grid_x, uint32_t grid_y, uint32_t grid_z,
                                  uint32_t block_x, uint32_t block_y, uint32_t block_z, uint32_t shared_bytes,
                                  void *args, size_t args_bytes) {
    const uint32_t g[3] = {grid_x, grid_y, grid_z}, b[3] = {block_x, block_y, block_z};
    return guarded(context, [&](Context *ctx) { ctx->module_launch_raw(function, g, b, shared_bytes, args, args_bytes); });
}

PAM_API const char *pam_module_default_path(void) {
    // libpam_kernels.hsaco beside this library
    static std::string path;
    static std::once_flag once;
    std::call_once(once, [] {
        Dl_info info{};
        if (dladdr((void *)&pam_module_default_path, &info) && info.dli_fname) {
            path = info.dli_fname;
            const size_t slash = path.rfind('/');
            path = (slash == std::string::npos ? std::string() : path.substr(0, slash + 1)) + "libpam_kernels.hsaco";
        }
    });
    return path.c_str();
}

PAM_API int32_t pam_engine_setup_noalloc(void *context) {
    return guarded(context, [&](Context *ctx) { ctx->setup_noalloc(); });
}

PAM_API int32_t pam_engine_decode_noalloc(void *context, const pam_decode_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->decode_noalloc(*request); });
}

PAM_API int32_t pam_engine_prefill(void *context, const pam_prefill_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->prefill(*request); });
}

PAM_API int32_t pam_engine_append(void *context, const pam_append_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->append(*request); });
}

PAM_API int32_t pam_engine_fused_prefill(void *context, const pam_fused_prefill_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->fused_prefill(*request); });
}

PAM_API int32_t pam_engine_backward(void *context, const pam_backward_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->backward(*request); });
}

PAM_API int32_t pam_engine_last_stats(void *context, pam_stats *out) {
    if (!out) return -1;
    return guarded(context, [&](Context *ctx) { *out = ctx->stats(); });
}

PAM_API int32_t pam_engine_set_graceful_degradation(void *context, bool enabled) {
    return guarded(context, [&](Context *ctx) { ctx->graceful_degradation = enabled; });
}

PAM_API int32_t pam_engine_set_max_retries(void *context, int32_t retries) {
    return guarded(context, [&](Context *ctx) {
        if (retries < 1) throw invalid_configuration("maxRetries must be positive.");
        ctx->max_retries = retries;
    });
}

PAM_API int32_t pam_append_tokens_hashed(void *context, void *cache, int64_t sequenceID, int32_t count,
                                         const uint64_t *blockHashes, int32_t numHashes) {
    KVCache *c = cache_of(cache);
    if (!c) return -1;
    return guarded(context, [&](Context *ctx) {
        std::lock_guard<std::mutex> g(c->mu);
        BlockCopies copies;
        try {
            c->alloc.append_tokens(sequenceID, count, blockHashes, numHashes, &copies);
        } catch (...) {
            if (c->has_device) c->copy_blocks(copies, ctx->stream(), ctx->ktab());  // CoW done before an OOM stays done
            throw;
        }
        if (c->has_device && !copies.empty()) {
            c->copy_blocks(copies, ctx->stream(), ctx->ktab());
            ctx->finish("copy-on-write");
        }
    });
}

PAM_API int32_t pam_ensure_exclusive(void *context, void *cache, int64_t sequenceID, int32_t logicalBlock) {
    KVCache *c = cache_of(cache);
    if (!c) return -1;
    return guarded(context, [&](Context *ctx) {
        std::lock_guard<std::mutex> g(c->mu);
        BlockCopies copies;
        c->alloc.ensure_exclusive(sequenceID, logicalBlock, &copies);
        if (c->has_device && !copies.empty()) {
            c->copy_blocks(copies, ctx->stream(), ctx->ktab());
            ctx->finish("copy-on-write");
        }
    });
}

PAM_API int32_t pam_register_block_hash(void *cache, uint64_t hash, int32_t physicalBlock) {
    KVCache *c = cache_of(cache);
    if (!c || physicalBlock < 0 || physicalBlock >= c->alloc.max_blocks()) return -1;
    std::lock_guard<std::mutex> g(c->mu);
    c->alloc.register_block_hash(hash, physicalBlock);
    return 0;
}

PAM_API int32_t pam_set_eviction_policy(void *cache, int32_t policy) {
    KVCache *c = cache_of(cache);
    if (!c || policy < 0 || policy > 2) return -1;
    std::lock_guard<std::mutex> g(c->mu);
    c->alloc.set_policy(static_cast<EvictionPolicy>(policy));
    return 0;
}

PAM_API int32_t pam_block_table(void *context, void *cache, int64_t sequenceID, int32_t *out, int32_t capacity) {
    KVCache *c = cache_of(cache);
    if (!c) return -1;
    int32_t n = 0;
    const int32_t rc = guarded(context, [&](Context *) {
        std::lock_guard<std::mutex> g(c->mu);
        const auto &t = c->alloc.sequence(sequenceID).block_table;
        n = (int32_t)t.size();
        if (out)
            for (int32_t i = 0; i < std::min(n, capacity); i++) out[i] = t[i];
    });
    return rc == 0 ? n : -1;
}

PAM_API int32_t pam_cache_memory_stats(void *cache, pam_memory_stats *out) {
    KVCache *c = cache_of(cache);
    if (!c || !out) return -1;
    std::lock_guard<std::mutex> g(c->mu);
    const AllocatorStats s = c->alloc.stats();
    const int64_t bpb = (int64_t)c->bytes_per_block() * 2;  // K + V (KVCacheManager.swift:357)
    out->total_blocks = s.total_blocks;
    out->used_blocks = s.used_blocks;
    out->free_blocks = s.free_blocks;
    out->active_sequences = s.active_sequences;
    out->total_memory_bytes = s.total_blocks * bpb;
    out->used_memory_bytes = s.used_blocks * bpb;
    out->partially_filled_blocks = s.partially_filled_blocks;
    out->fragmentation_ratio = s.fragmentation_ratio;
    out->prefix_cache_hits = s.prefix_cache_hits;
    out->prefix_cache_entries = s.prefix_cache_entries;
    out->shared_blocks = s.shared_blocks;
    out->eviction_policy = (int32_t)c->alloc.policy();
    return 0;
}

PAM_API void *pam_cache_k_pool(void *cache) { return cache ? cache_of(cache)->k_pool : nullptr; }
PAM_API void *pam_cache_v_pool(void *cache) { return cache ? cache_of(cache)->v_pool : nullptr; }
PAM_API void *pam_cache_k_scale(void *cache) { return cache ? cache_of(cache)->k_scale : nullptr; }
PAM_API void *pam_cache_v_scale(void *cache) { return cache ? cache_of(cache)->v_scale : nullptr; }

PAM_API int32_t pam_cache_batch_view(void *context, void *cache, const int64_t *ids, int32_t n, int32_t max_num_blocks,
                                     int32_t *device_block_tables, uint32_t *device_seq_lengths) {
    KVCache *c = cache_of(cache);
    if (!c || (n > 0 && !ids)) return -1;
    int32_t used = 0;
    const int32_t rc = guarded(context, [&](Context *ctx) {
        std::lock_guard<std::mutex> g(c->mu);
        int32_t width = max_num_blocks;
        if (width <= 0) {
            width = 1;
            for (int32_t i = 0; i < n; i++)
                width = std::max<int32_t>(width, (int32_t)c->alloc.sequence(ids[i]).block_table.size());
        }
        std::vector<int32_t> slab((size_t)std::max(n, 0) * width, 0);
        std::vector<uint32_t> lens((size_t)std::max(n, 0), 0);
        for (int32_t i = 0; i < n; i++) {
            const LogicalSequence &s = c->alloc.sequence(ids[i]);
            if ((int32_t)s.block_table.size() > width)
                throw invalid_request("sequence " + std::to_string(ids[i]) + " requires " +
                                      std::to_string(s.block_table.size()) + " blocks, maxSequenceBlocks is " +
                                      std::to_string(width));
            std::copy(s.block_table.begin(), s.block_table.end(), slab.begin() + (size_t)i * width);
            lens[i] = (uint32_t)s.length;
        }
        ctx->ensure_device();
        if (device_block_tables) ctx->stage_into(device_block_tables, slab.data(), slab.size() * 4);
        if (device_seq_lengths) ctx->stage_into(device_seq_lengths, lens.data(), lens.size() * 4);
        ctx->finish("batch view");
        used = width;
    });
    return rc == 0 ? used : -1;
}

// ---------------------------------------------------------------------- scheduler

PAM_API void *pam_scheduler_create(int32_t maxBatchSize, int32_t maxSequences) {
    try {
        return new Scheduler(maxBatchSize, maxSequences);
    } catch (...) {
        return nullptr;
    }
}
PAM_API void pam_scheduler_destroy(void *s) { delete sched_of(s); }
PAM_API int32_t pam_scheduler_add_request(void *s, int32_t prompt, int32_t max_new) {
    return s ? sched_of(s)->add_request(prompt, max_new) : -1;
}
PAM_API void pam_scheduler_complete(void *s, int32_t id) {
    if (s) sched_of(s)->complete(id);
}
PAM_API int32_t pam_scheduler_step(void *s, int32_t *ids, int32_t capacity) {
    if (!s) return -1;
    const auto b = sched_of(s)->step();
    if (ids)
        for (size_t i = 0; i < b.size() && (int32_t)i < capacity; i++) ids[i] = b[i];
    return (int32_t)b.size();
}
PAM_API void pam_scheduler_mark_prefilled(void *s, int32_t id) {
    if (s) sched_of(s)->mark_prefilled(id);
}
PAM_API void pam_scheduler_mark_decoded(void *s, int32_t id) {
    if (s) sched_of(s)->mark_decoded(id);
}
PAM_API void pam_scheduler_preempt(void *s, int32_t id) {
    if (s) sched_of(s)->preempt(id);
}
PAM_API int32_t pam_scheduler_handle_memory_pressure(void *s, int32_t requiredBlocks, void *cache, int32_t *ids,
                                                     int32_t capacity) {
    KVCache *c = cache_of(cache);
    if (!s || !c) return -1;
    const auto v = sched_of(s)->handle_memory_pressure(requiredBlocks, [&] {
        std::lock_guard<std::mutex> g(c->mu);
        return c->alloc.available();
    });
    if (ids)
        for (size_t i = 0; i < v.size() && (int32_t)i < capacity; i++) ids[i] = v[i];
    return (int32_t)v.size();
}
PAM_API int32_t pam_scheduler_count(void *s, int32_t status) {
    if (!s || status < 0 || status > 3) return -1;
    return sched_of(s)->count(static_cast<SeqStatus>(status));
}
PAM_API int32_t pam_scheduler_sequence(void *s, int32_t id, int32_t *status, int32_t *generated, int32_t *prompt) {
    if (!s) return -1;
    SchedulerSequence q{};
    if (!sched_of(s)->get(id, &q)) return -1;
    if (status) *status = (int32_t)q.status;
    if (generated) *generated = q.generated;
    if (prompt) *prompt = q.prompt_length;
    return 0;
}

// ====================================================================== Part 3

PAM_API void *pam_create_cache_host(void *context, int32_t maxBlocks, int32_t blockSize, int32_t headDim,
                                    int32_t numKVHeads, int32_t dataType) {
    return create_cache(context, maxBlocks, blockSize, headDim, numKVHeads, dataType, false);
}

PAM_API void *pam_buffer_alloc(void *context, size_t bytes) {
    void *p = nullptr;
    const int32_t rc = guarded(context, [&](Context *ctx) {
        ctx->ensure_device();
        hip_check(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc");
    });
    return rc == 0 ? p : nullptr;
}

PAM_API void pam_buffer_free(void *context, void *ptr) {
    guarded(context, [&](Context *ctx) {
        if (!ptr) return;
        ctx->ensure_device();
        hip_check(hipStreamSynchronize(ctx->stream()), "hipStreamSynchronize");
        hip_check(hipFree(ptr), "hipFree");
    });
}

PAM_API int32_t pam_buffer_upload(void *context, void *dst, const void *src, size_t bytes) {
    return guarded(context, [&](Context *ctx) {
        ctx->ensure_device();
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream()), "upload");
        hip_check(hipStreamSynchronize(ctx->stream()), "upload");
    });
}

PAM_API int32_t pam_buffer_download(void *context, void *dst, const void *src, size_t bytes) {
    return guarded(context, [&](Context *ctx) {
        ctx->ensure_device();
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream()), "download");
        hip_check(hipStreamSynchronize(ctx->stream()), "download");
    });
}

PAM_API int32_t pam_buffer_zero(void *context, void *ptr, size_t bytes) {
    return guarded(context, [&](Context *ctx) {
        ctx->ensure_device();
        hip_check(hipMemsetAsync(ptr, 0, bytes, ctx->stream()), "zero");
        ctx->finish("zero");
    });
}

PAM_API int32_t pam_set_stream(void *context, void *hip_stream) {
    return guarded(context, [&](Context *ctx) {
        ctx->ensure_device();
        ctx->set_stream(static_cast<hipStream_t>(hip_stream));
    });
}

PAM_API int32_t pam_use_own_stream(void *context) {
    return guarded(context, [&](Context *ctx) { ctx->use_own_stream(); });
}

PAM_API int32_t pam_set_synchronous(void *context, bool synchronous) {
    return guarded(context, [&](Context *ctx) { ctx->synchronous = synchronous; });
}

PAM_API int32_t pam_synchronize(void *context) {
    return guarded(context, [&](Context *ctx) {
        ctx->ensure_device();
        hip_check(hipStreamSynchronize(ctx->stream()), "hipStreamSynchronize");
    });
}

PAM_API int32_t pam_reserve_workspace(void *context, size_t bytes) {
    return guarded(context, [&](Context *ctx) { ctx->reserve_workspace(bytes); });
}

PAM_API int32_t pam_set_partition_tokens(void *context, int32_t tokens) {
    return guarded(context, [&](Context *ctx) {
        if (tokens < 0 || tokens % 16 != 0) throw invalid_configuration("partition tokens must be a multiple of 16");
        ctx->part_tokens_override = tokens;
    });
}

PAM_API int32_t pam_set_mixed_launch(void *context, int32_t mode, int32_t prefill_groups, int32_t decode_groups) {
    return guarded(context, [&](Context *ctx) {
        if (mode < 0 || mode > 2) throw invalid_configuration("mixed launch mode must be 0, 1 or 2");
        if (prefill_groups < 0 || decode_groups < 0) throw invalid_configuration("workgroup counts must be >= 0");
        ctx->mixed_launch_mode = mode;
        ctx->mixed_prefill_groups = prefill_groups;
        ctx->mixed_decode_groups = decode_groups;
    });
}

PAM_API int32_t pam_set_fused_prefill_kernel(void *context, bool one_kernel) {
    return guarded(context, [&](Context *ctx) { ctx->fused_one_kernel = one_kernel; });
}

PAM_API int32_t pam_set_decode_kernel(void *context, int32_t choice) {
    return guarded(context, [&](Context *ctx) {
        if (choice < 0 || choice > 2) throw invalid_configuration("decode kernel choice must be 0, 1 or 2");
        ctx->decode_kernel_choice = choice;
    });
}

PAM_API int32_t pam_set_gpu_timing(void *context, bool enabled) {
    return guarded(context, [&](Context *ctx) { ctx->gpu_timing = enabled; });
}

PAM_API int32_t pam_engine_mixed_step(void *context, const pam_mixed_request *request) {
    if (!request) return -1;
    return guarded(context, [&](Context *ctx) { ctx->mixed_step(*request); });
}

PAM_API int32_t pam_fp8_quantize(void *context, const uint16_t *values, const uint16_t *scales, uint8_t *out,
                                 int64_t n) {
    return guarded(context, [&](Context *ctx) { ctx->fp8_quantize(values, scales, out, n); });
}

PAM_API int32_t pam_fp8_dequant(void *context, const uint8_t *codes, const uint16_t *scales, uint16_t *out,
                                int64_t n) {
    return guarded(context, [&](Context *ctx) { ctx->fp8_dequant(codes, scales, out, n); });
}

static int32_t calib_blocks(int32_t blocks) {
    if (blocks > 0) return blocks;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                 hipSuccess)
        cus = 256;
    return 4 * cus;
}

PAM_API int32_t pam_synth_normal(void *context, void *dst, int32_t dtype, uint64_t n, uint64_t seed, uint64_t stream,
                                 float stddev, int64_t outlier_stream, float outlier_frac) {
    return guarded(context, [&](Context *ctx) {
        if (n > 0 && !dst) throw invalid_configuration("synthetic data needs a destination buffer.");
        if (dtype != kF32 && dtype != kF16) throw invalid_configuration("synthetic data is float32 or float16.");
        if (stream >= ((uint64_t)1 << 23) || outlier_stream >= ((int64_t)1 << 23) || n >= ((uint64_t)1 << 39))
            throw invalid_configuration("synthetic data: stream ids must be < 2^23 and n < 2^39.");
        ctx->ensure_device();
        hip_check(launch_synth_normal(dst, dtype, n, seed, stream, stddev, outlier_stream, outlier_frac, ctx->stream()),
                  "synthetic data");
        ctx->finish("synthetic data");
    });
}

// Two events around work on `stream`; both are released however the caller
// leaves (a failed create or record throws).
struct TimedSpan {
    hipEvent_t a = nullptr, b = nullptr;
    hipStream_t stream;
    explicit TimedSpan(hipStream_t s) : stream(s) {
        // a constructor that throws runs no destructor: release here
        try {
            hip_check(hipEventCreate(&a), "hipEventCreate");
            hip_check(hipEventCreate(&b), "hipEventCreate");
            hip_check(hipEventRecord(a, stream), "hipEventRecord");
        } catch (...) {
            release();
            throw;
        }
    }
    void release() {
        if (a) (void)hipEventDestroy(a);
        if (b) (void)hipEventDestroy(b);
        a = b = nullptr;
    }
    // milliseconds from the first event to now on the stream (-1 if not measurable)
    float end() {
        float t = -1.0f;
        if (hipEventRecord(b, stream) == hipSuccess && hipEventSynchronize(b) == hipSuccess)
            (void)hipEventElapsedTime(&t, a, b);
        return t;
    }
    ~TimedSpan() { release(); }
    TimedSpan(const TimedSpan &) = delete;
    TimedSpan &operator=(const TimedSpan &) = delete;
};

PAM_API int32_t pam_calib_mfma(void *context, int32_t iters, double *tflops) {
    return guarded(context, [&](Context *ctx) {
        if (iters <= 0 || !tflops) throw invalid_configuration("the MFMA calibration needs iters > 0 and an output.");
        ctx->ensure_device();
        const int32_t nb = calib_blocks(0) / 4;  // one 8-wave workgroup per CU
        float *sink = static_cast<float *>(ctx->device_scratch(5, (size_t)nb * 4));
        hip_check(launch_mfma_loop(nb, iters, sink, ctx->stream()), "MFMA calibration");  // warm-up
        TimedSpan span(ctx->stream());
        const hipError_t e = launch_mfma_loop(nb, iters, sink, ctx->stream());
        const float t = span.end();
        hip_check(e, "MFMA calibration");
        *tflops = t > 0 ? (double)nb * 8 * iters * 4 * 32768.0 / (t * 1e-3) / 1e12 : -1.0;
    });
}

PAM_API int32_t pam_calib_stream_read(void *context, const void *src, size_t bytes, int32_t blocks, float *ms) {
    return guarded(context, [&](Context *ctx) {
        ctx->ensure_device();
        const int32_t nb = calib_blocks(blocks);
        uint32_t *sink = static_cast<uint32_t *>(ctx->device_scratch(5, (size_t)nb * 4));
        TimedSpan span(ctx->stream());
        const hipError_t e = launch_stream_read(src, bytes, sink, nb, ctx->stream());
        const float t = span.end();
        hip_check(e, "stream read");
        if (ms) *ms = t;
    });
}

PAM_API int32_t pam_calib_stream_copy(void *context, const void *src, void *dst, size_t bytes, int32_t blocks,
                                      float *ms) {
    return guarded(context, [&](Context *ctx) {
        ctx->ensure_device();
        const int32_t nb = calib_blocks(blocks);
        TimedSpan span(ctx->stream());
        const hipError_t e = launch_stream_copy(src, dst, bytes, nb, ctx->stream());
        const float t = span.end();
        hip_check(e, "stream copy");
        if (ms) *ms = t;
    });
}

PAM_API int32_t pam_debug_fail_next_launches(void *context, int32_t n) {
    return guarded(context, [&](Context *ctx) { ctx->fail_next_launches = n < 0 ? 0 : n; });
}

PAM_API int32_t pam_debug_dirty_counters(void *context, int32_t arrivals) {
    return guarded(context, [&](Context *ctx) { ctx->dirty_counters(arrivals); });
}

PAM_API const char *pam_version(void) { return "pam-mi355x 0.1.0 (gfx950)"; }
