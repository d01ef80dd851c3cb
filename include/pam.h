/*
 * pam.h - C ABI of libpam, the MI355X (gfx950) paged-attention library.
 *
 * Part 1 is a drop-in for the reference's flat C ABI
 * (Sources/PagedAttentionMetal/PagedAttentionCABI.swift, abderahmane-ai/PagedAttentionMetal):
 * same names, argument order, meaning and status convention (0 = success, -1 =
 * failure with the message available from pam_last_error until the next call
 * on that context).  The one change of meaning: buffer arguments that were
 * opaque MTLBuffer handles are device pointers (from pam_buffer_alloc,
 * hipMalloc or any framework allocator) on the context's GPU.
 *
 * Part 2 adds what the Swift API layer (PagedAttentionEngine, KVCacheManager,
 * ContinuousBatchingScheduler) needs to sit on this library, each entry citing
 * the Swift method it carries.  Part 3 holds entry points with no reference
 * counterpart (split-context / chunked / mixed-step paths, device buffers,
 * streams, codec checks).
 *
 * Threading: a context and each cache serialise their calls with a mutex, as
 * the reference's unfair locks do.  By default every call returns after the GPU
 * work it enqueued has completed (the reference's commitAndWait); a context
 * switched to asynchronous mode returns after enqueueing on its stream.
 */
#ifndef PAM_H
#define PAM_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* data type codes: PagedAttentionDataType (PagedAttentionTypes.swift:67-73) */
enum { PAM_FLOAT32 = 0, PAM_FLOAT16 = 1, PAM_FLOAT8 = 2 };
/* BlockEvictionPolicy (KVCacheManager.swift:13-17) */
enum { PAM_EVICT_FIFO = 0, PAM_EVICT_LIFO = 1, PAM_EVICT_BEST_FIT = 2 };

/* ======================================================================
 * Part 1 - drop-in for PagedAttentionCABI.swift
 * ==================================================================== */

/* PagedAttentionCABI.swift:71-79 */
void *pam_create_context(void);
/* PagedAttentionCABI.swift:81-85 */
void pam_destroy_context(void *context);
/* PagedAttentionCABI.swift:87-90 */
const char *pam_last_error(void *context);
/* PagedAttentionCABI.swift:92-132 (layer numHeads = numKVHeads, dtype 0/1/2).
 * Allocates the K/V pools (and, for FP8, zeroed per-block half scale pools) in HBM. */
void *pam_create_cache(void *context, int32_t maxBlocks, int32_t blockSize, int32_t headDim,
                       int32_t numKVHeads, int32_t dataType);
/* PagedAttentionCABI.swift:134-138 */
void pam_destroy_cache(void *cache);
/* PagedAttentionCABI.swift:140-154 -> KVCacheManager.allocateSequence (KVCacheManager.swift:106-113) */
int32_t pam_reserve_sequence(void *context, void *cache, int64_t sequenceID);
/* PagedAttentionCABI.swift:156-171 -> KVCacheManager.appendTokens (KVCacheManager.swift:115-174) */
int32_t pam_append_tokens(void *context, void *cache, int64_t sequenceID, int32_t count);
/* PagedAttentionCABI.swift:173-179 -> KVCacheManager.freeSequence (KVCacheManager.swift:216-239) */
void pam_free_sequence(void *cache, int64_t sequenceID);
/* PagedAttentionCABI.swift:181-185 */
int32_t pam_available_blocks(void *cache);
/* PagedAttentionCABI.swift:187-201 */
int32_t pam_sequence_length(void *context, void *cache, int64_t sequenceID);
/* PagedAttentionCABI.swift:203-244: keys/values [numNewTokens][numKVHeads][headDim]
 * (f32 for f32 caches, f16 for f16 and FP8 caches) -> PagedAttentionEngine.appendToCache */
int32_t pam_append_kv(void *context, void *cache, int64_t sequenceID, void *keys, void *values,
                      int32_t tokenOffset, int32_t numNewTokens, int32_t numHeads);
/* PagedAttentionCABI.swift:246-287: query/output [seqLen][numHeads][headDim]
 * -> PagedAttentionEngine.prefill */
int32_t pam_prefill(void *context, void *cache, int64_t sequenceID, void *query, void *output,
                    int32_t seqLen, int32_t numHeads, bool causal);
/* PagedAttentionCABI.swift:289-337: query/output [batchSize][numHeads][headDim]
 * -> PagedAttentionEngine.decode over a zero-padded batch view (:339-372) */
int32_t pam_decode(void *context, void *cache, const int64_t *batchIDs, int32_t batchSize, void *query,
                   void *output, int32_t numHeads);

/* ======================================================================
 * Part 2 - Swift API layer support
 * ==================================================================== */

/* PagedLayerSpec (PagedAttentionTypes.swift:94-152) */
typedef struct pam_layer_spec {
    int32_t head_dim;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t block_size;
    int32_t data_type;
    int32_t window_size; /* 0 = full context */
} pam_layer_spec;

/* PagedAttentionStats (PagedAttentionTypes.swift:169-207).  elapsed_ms is GPU time
 * between hipEvents around the launch sequence of the last call; kernel_ms and
 * reduce_ms split it per kernel.  In asynchronous mode pam_engine_last_stats waits
 * for the last call's end event before reading them. */
enum {
    PAM_OP_NONE = 0,
    PAM_OP_PREFILL_SINGLE_PASS = 1,
    PAM_OP_PREFILL_MMA = 2,
    PAM_OP_PREFILL_FLASH = 3,
    PAM_OP_PREFILL_TILED_PASS = 4,
    PAM_OP_DECODE = 5,
    PAM_OP_APPEND = 6,
    PAM_OP_BACKWARD = 7
};
typedef struct pam_stats {
    int32_t operation;
    int32_t batch_size;
    int32_t sequence_length;
    int32_t num_blocks;
    int64_t temporary_bytes;
    int32_t used_split_pass;
    double elapsed_ms;
    double kernel_ms; /* attention kernel alone (decode / prefill / mixed), -1 if not timed */
    double reduce_ms; /* split-context reduce kernel, 0 when not launched */
    int32_t chunks;   /* prefill passes of the call (the chunk loop of the flat prefill), 0 for other ops */
} pam_stats;

/* PagedAttentionDecodeRequest (PagedAttentionTypes.swift:259-315).  *_bytes are the
 * buffer lengths used for PagedAttentionEngine.validateDecode (Engine.swift:1916-1934);
 * a length of 0 skips that buffer's size check. */
typedef struct pam_decode_request {
    const void *q;
    const void *k_pool;
    const void *v_pool;
    const int32_t *block_tables; /* [batch_size][max_num_blocks] */
    const uint32_t *seq_lengths; /* [batch_size] */
    void *output;
    int32_t batch_size;
    int32_t max_num_blocks;
    pam_layer_spec layer;
    const uint16_t *k_scale; /* FP8: one half per physical block */
    const uint16_t *v_scale;
    size_t q_bytes, k_pool_bytes, v_pool_bytes, block_tables_bytes, seq_lengths_bytes, output_bytes;
} pam_decode_request;

/* PagedAttentionPrefillRequest (PagedAttentionTypes.swift:210-256) plus q_offset:
 * the request's rows are query positions [q_offset, q_offset + seq_len) of a
 * sequence whose first q_offset tokens are already cached (q_offset = 0 is the
 * reference's prefill). */
typedef struct pam_prefill_request {
    const void *q; /* [seq_len][num_heads][head_dim] */
    const void *k_pool;
    const void *v_pool;
    const int32_t *block_table;
    void *output;
    int32_t seq_len;
    int32_t q_offset;
    pam_layer_spec layer;
    bool causal;
    const uint16_t *k_scale;
    const uint16_t *v_scale;
    size_t q_bytes, k_pool_bytes, v_pool_bytes, block_table_bytes, output_bytes;
} pam_prefill_request;

/* PagedKVAppendRequest (PagedAttentionTypes.swift:318-364); slot_mapping (optional,
 * f32/f16 only) gives each token's pool slot explicitly, overriding the table. */
typedef struct pam_append_request {
    const void *keys;
    const void *values;
    void *k_pool;
    void *v_pool;
    const int32_t *block_table;
    int32_t token_offset;
    int32_t num_new_tokens;
    pam_layer_spec layer;
    uint16_t *k_scale;
    uint16_t *v_scale;
    const int64_t *slot_mapping;
    size_t keys_bytes, values_bytes, k_pool_bytes, v_pool_bytes, block_table_bytes;
} pam_append_request;

/* PagedAttentionFusedPrefillRequest (PagedAttentionTypes.swift:366-421): the new
 * tokens' raw K/V [seq_len][num_kv_heads][head_dim] are appended at positions
 * 0 .. seq_len-1 of the sequence's block table (FP8: quantised with the per-block
 * scale rule of the append), then rows 0 .. seq_len-1 attend over the pool. */
typedef struct pam_fused_prefill_request {
    const void *q; /* [seq_len][num_heads][head_dim] */
    const void *raw_k;
    const void *raw_v;
    const int32_t *block_table;
    void *k_pool;
    void *v_pool;
    void *output;
    int32_t seq_len;
    pam_layer_spec layer;
    bool causal;
    uint16_t *k_scale;
    uint16_t *v_scale;
    size_t q_bytes, raw_k_bytes, raw_v_bytes, k_pool_bytes, v_pool_bytes, block_table_bytes, output_bytes;
} pam_fused_prefill_request;

/* PagedAttentionEngine.backward (PagedAttentionEngine.swift:1340-1396): gradients of
 * non-causal attention of rows 0 .. seq_len-1 over keys [max(0, seq_len - W),
 * seq_len), given the forward's row max m and sum l ([seq_len][num_heads] float,
 * natural-log units).  d_q is written; d_k_pool / d_v_pool (pool layout) are
 * accumulated into.  f32 and f16 caches. */
typedef struct pam_backward_request {
    const void *q;
    const void *k_pool;
    const void *v_pool;
    const int32_t *block_table;
    const void *d_out;
    const float *m;
    const float *l;
    void *d_q;
    void *d_k_pool;
    void *d_v_pool;
    int32_t seq_len;
    pam_layer_spec layer;
} pam_backward_request;

/* PagedAttentionEngine.decode(_:) (PagedAttentionEngine.swift:533-546) */
int32_t pam_engine_decode(void *context, const pam_decode_request *request);
/* PagedAttentionEngine.prefill(_:) (PagedAttentionEngine.swift:405-418) */
int32_t pam_engine_prefill(void *context, const pam_prefill_request *request);
/* PagedAttentionEngine.appendToCache(_:) (PagedAttentionEngine.swift:585-597) */
int32_t pam_engine_append(void *context, const pam_append_request *request);
/* PagedAttentionEngine.fusedPrefill(_:) (PagedAttentionEngine.swift:633-710): append
 * and prefill as one call on the context's stream.  f16 caches with head_dim 64 or 128
 * run one kernel that reads the new keys and values from raw_k / raw_v and writes
 * them into the pools; other shapes and dtypes append first, then attend.  The
 * pools end up equal to a separate append in every case. */
int32_t pam_engine_fused_prefill(void *context, const pam_fused_prefill_request *request);
/* PagedAttentionEngine.backward(q:kPool:...) (PagedAttentionEngine.swift:1340-1396) */
int32_t pam_engine_backward(void *context, const pam_backward_request *request);
/* Multi-layer calls over one shared pool, block table(s) and lengths; every
 * layer has its own Q and output (and, for appends, its own keys, values and
 * FP8 scale pools).  Arrays hold num_layers entries; *_bytes arrays may be
 * NULL (no size check).  window_size > 0 overrides every layer's window. */
typedef struct pam_decode_layers_request {
    const void *const *q;       /* [num_layers] -> [batch_size][num_heads][head_dim] */
    void *const *output;        /* [num_layers] */
    const pam_layer_spec *layers;
    int32_t num_layers;
    const void *k_pool;
    const void *v_pool;
    const int32_t *block_tables; /* [batch_size][max_num_blocks] */
    const uint32_t *seq_lengths;
    int32_t batch_size;
    int32_t max_num_blocks;
    int32_t window_size;
    const uint16_t *k_scale;
    const uint16_t *v_scale;
    const size_t *q_bytes, *output_bytes;
    size_t k_pool_bytes, v_pool_bytes, block_tables_bytes, seq_lengths_bytes;
} pam_decode_layers_request;
typedef struct pam_prefill_layers_request {
    const void *const *q;       /* [num_layers] -> [seq_len][num_heads][head_dim] */
    void *const *output;
    const pam_layer_spec *layers;
    int32_t num_layers;
    const void *k_pool;
    const void *v_pool;
    const int32_t *block_table;
    int32_t seq_len;
    bool causal;
    int32_t window_size;
    const uint16_t *k_scale;
    const uint16_t *v_scale;
    const size_t *q_bytes, *output_bytes;
    size_t k_pool_bytes, v_pool_bytes, block_table_bytes;
} pam_prefill_layers_request;
typedef struct pam_append_layers_request {
    const void *const *keys;    /* [num_layers] -> [num_new_tokens][num_kv_heads][head_dim] */
    const void *const *values;
    const pam_layer_spec *layers;
    int32_t num_layers;
    void *k_pool;
    void *v_pool;
    const int32_t *block_table;
    int32_t token_offset;
    int32_t num_new_tokens;
    uint16_t *const *k_scale;   /* [num_layers] FP8 scale pools, or NULL */
    uint16_t *const *v_scale;
    const size_t *keys_bytes, *values_bytes;
    size_t k_pool_bytes, v_pool_bytes, block_table_bytes;
} pam_append_layers_request;
/* PagedAttentionEngine.decodeLayers (PagedAttentionEngine.swift:1641-1741).
 * Consecutive layers of one spec that the stream-K MFMA decode serves (G >= 4)
 * share one launch, up to 16 query heads per kv head: each K/V tile is read
 * once for all of their heads. */
int32_t pam_engine_decode_layers(void *context, const pam_decode_layers_request *request);
/* PagedAttentionEngine.prefillLayers (PagedAttentionEngine.swift:1433-1639) */
int32_t pam_engine_prefill_layers(void *context, const pam_prefill_layers_request *request);
/* PagedAttentionEngine.appendLayers (PagedAttentionEngine.swift:1744-1895): layers
 * append in order at the same positions of the one pool. */
int32_t pam_engine_append_layers(void *context, const pam_append_layers_request *request);

/* PagedAttentionEngine.splitThreshold / defaultWindowSize / defaultChunkSize
 * (PagedAttentionEngine.swift:116-121).  split_threshold (tokens, default 1024):
 * only prefills whose longest key range exceeds it may run the multi-pass form
 * (items cut over workgroups, partial states merged in the kernel).  The
 * defaults apply to the flat overloads below when their argument is 0. */
typedef struct pam_engine_config {
    int32_t split_threshold;
    int32_t default_window_size;
    int32_t default_chunk_size;
} pam_engine_config;
int32_t pam_engine_set_config(void *context, const pam_engine_config *config);
int32_t pam_engine_get_config(void *context, pam_engine_config *out);
/* The flat overloads: the request's layer window is replaced by window_size,
 * or defaultWindowSize when window_size is 0.
 * prefill(q:kPool:...:windowSize:chunkSize:) (PagedAttentionEngine.swift:713-760):
 * chunk_size (or defaultChunkSize) > 0 below seq_len runs the chunk loop, whose
 * result equals the unchunked prefill; pam_stats.chunks counts its passes. */
int32_t pam_engine_prefill_flat(void *context, const pam_prefill_request *request, int32_t window_size,
                                int32_t chunk_size);
/* decode(q:kPool:...:windowSize:) (PagedAttentionEngine.swift:1012-1046) */
int32_t pam_engine_decode_flat(void *context, const pam_decode_request *request, int32_t window_size);
/* appendToCache(keys:values:...:windowSize:) (PagedAttentionEngine.swift:1167-1201) */
int32_t pam_engine_append_flat(void *context, const pam_append_request *request, int32_t window_size);

/* PagedAttentionEngine.lastStats (PagedAttentionEngine.swift:136-141) */
int32_t pam_engine_last_stats(void *context, pam_stats *out);
/* PagedAttentionEngine.enableGracefulDegradation / maxRetries (Engine.swift:126-129) */
int32_t pam_engine_set_graceful_degradation(void *context, bool enabled);
int32_t pam_engine_set_max_retries(void *context, int32_t retries);

/* KVCacheManager extras */
/* appendTokens(toSequence:count:blockHashes:) (KVCacheManager.swift:115-174) */
int32_t pam_append_tokens_hashed(void *context, void *cache, int64_t sequenceID, int32_t count,
                                 const uint64_t *blockHashes, int32_t numHashes);
/* ensureExclusiveAccess (KVCacheManager.swift:200-214); the copy is a device D2D copy */
int32_t pam_ensure_exclusive(void *context, void *cache, int64_t sequenceID, int32_t logicalBlock);
/* registerBlockHash (KVCacheManager.swift:196-198) */
int32_t pam_register_block_hash(void *cache, uint64_t hash, int32_t physicalBlock);
/* evictionPolicy setter (KVCacheManager.swift:65-67) */
int32_t pam_set_eviction_policy(void *cache, int32_t policy);
/* getBlockTable(forSequence:) (KVCacheManager.swift:299-303): copies up to capacity
 * entries to out (host) and returns the table length, or -1. */
int32_t pam_block_table(void *context, void *cache, int64_t sequenceID, int32_t *out, int32_t capacity);
/* KVCacheMemoryStats (KVCacheManager.swift:19-32, 353-378) */
typedef struct pam_memory_stats {
    int64_t total_blocks, used_blocks, free_blocks, active_sequences;
    int64_t total_memory_bytes, used_memory_bytes, partially_filled_blocks;
    float fragmentation_ratio;
    int64_t prefix_cache_hits, prefix_cache_entries, shared_blocks;
    int32_t eviction_policy;
} pam_memory_stats;
int32_t pam_cache_memory_stats(void *cache, pam_memory_stats *out);
/* kPoolBuffer / vPoolBuffer (KVCacheManager.swift:59-60) and the FP8 scale pools
 * the reference's callers allocate beside them (Tests/...Tests.swift:669-680). */
void *pam_cache_k_pool(void *cache);
void *pam_cache_v_pool(void *cache);
void *pam_cache_k_scale(void *cache);
void *pam_cache_v_scale(void *cache);
/* BatchKVCacheManager.getBatchBlockTableBuffer + getSeqLengthsBuffer
 * (KVCacheManager.swift:661-703) into caller device buffers, zero padded to
 * max_num_blocks (0 = longest table in the batch, as PagedAttentionCABI.swift:308).
 * Staged through pinned host memory and copied on the context stream.
 * Returns the max_num_blocks used, or -1. */
int32_t pam_cache_batch_view(void *context, void *cache, const int64_t *ids, int32_t n, int32_t max_num_blocks,
                             int32_t *device_block_tables, uint32_t *device_seq_lengths);

/* ContinuousBatchingScheduler (Scheduler.swift:42-177) */
void *pam_scheduler_create(int32_t maxBatchSize, int32_t maxSequences);
void pam_scheduler_destroy(void *scheduler);
int32_t pam_scheduler_add_request(void *scheduler, int32_t promptTokenCount, int32_t maxNewTokens);
void pam_scheduler_complete(void *scheduler, int32_t id);
/* step(): writes up to capacity ids in batch order; returns the batch size */
int32_t pam_scheduler_step(void *scheduler, int32_t *ids, int32_t capacity);
void pam_scheduler_mark_prefilled(void *scheduler, int32_t id);
void pam_scheduler_mark_decoded(void *scheduler, int32_t id);
void pam_scheduler_preempt(void *scheduler, int32_t id);
/* handleMemoryPressure(requiredBlocks:availableBlocks:) with the closure bound to a
 * cache's availableBlocks; writes preempted ids, returns their count */
int32_t pam_scheduler_handle_memory_pressure(void *scheduler, int32_t requiredBlocks, void *cache, int32_t *ids,
                                             int32_t capacity);
/* status: 0 waiting, 1 running, 2 paused, 3 completed */
int32_t pam_scheduler_count(void *scheduler, int32_t status);
/* per-sequence state: status, generated tokens, prompt length; -1 if unknown */
int32_t pam_scheduler_sequence(void *scheduler, int32_t id, int32_t *status, int32_t *generated, int32_t *prompt);

/* ======================================================================
 * Part 3 - no reference counterpart
 * ==================================================================== */

/* A cache with block bookkeeping only (no HBM pools): allocator / scheduler
 * planning on any host, e.g. without a GPU. */
void *pam_create_cache_host(void *context, int32_t maxBlocks, int32_t blockSize, int32_t headDim,
                            int32_t numKVHeads, int32_t dataType);

/* Device memory and streams of the context's GPU. */
void *pam_buffer_alloc(void *context, size_t bytes);
void pam_buffer_free(void *context, void *ptr);
int32_t pam_buffer_upload(void *context, void *device_dst, const void *host_src, size_t bytes);
int32_t pam_buffer_download(void *context, void *host_dst, const void *device_src, size_t bytes);
int32_t pam_buffer_zero(void *context, void *device_ptr, size_t bytes);
/* Launch on an external hipStream_t (NULL = the device's default stream).  Work the
 * context issued on its previous stream is ordered before its work on the new one
 * (an event wait), since its launches share one workspace. */
int32_t pam_set_stream(void *context, void *hip_stream);
/* Go back to launching on the context's own stream (a blocking stream: ordered
 * against work on the legacy default stream). */
int32_t pam_use_own_stream(void *context);
/* true (default): calls wait for their GPU work; false: calls return once enqueued. */
int32_t pam_set_synchronous(void *context, bool synchronous);
int32_t pam_synchronize(void *context);
/* Pre-size the split-context workspace so that no later call allocates. */
int32_t pam_reserve_workspace(void *context, size_t bytes);
/* Tokens per split-context partition (multiple of 16; 0 = automatic). */
int32_t pam_set_partition_tokens(void *context, int32_t tokens);
/* Kernel choice for decode: 0 automatic, 1 force VALU, 2 force MFMA (when supported). */
int32_t pam_set_decode_kernel(void *context, int32_t choice);
/* How pam_engine_mixed_step runs its attention: 1 the prefill chunks and the
 * decode rows as separate launches, 2 one launch holding both (when supported:
 * f16 or e4m3, d = 128, blocks of 16 tokens or more, G >= 4, at most 1024
 * decode rows), 0 automatic (separate launches, the faster on gfx950).
 * prefill_groups / decode_groups set the one launch's workgroups of each part
 * (0 = automatic: one per CU each). */
int32_t pam_set_mixed_launch(void *context, int32_t mode, int32_t prefill_groups, int32_t decode_groups);
/* pam_engine_fused_prefill for f16 caches with d = 128: false (default) appends
 * then prefills, two launches in the one call; true runs one kernel that writes
 * the new rows into the pools as it reads them.  Results are identical. */
int32_t pam_set_fused_prefill_kernel(void *context, bool one_kernel);
/* true (default): time every call's kernels with HIP events (the elapsed, kernel
 * and reduce times of pam_engine_last_stats); false: no events are recorded and
 * those times read -1. */
int32_t pam_set_gpu_timing(void *context, bool enabled);

/* Mixed continuous-batching step: every sequence s appends query_lens[s] new
 * tokens after context_lens[s] cached ones (query_lens = 1 is a decode), the new
 * K/V are written into the pool through each sequence's block-table row, then
 * every new token attends causally to its sequence's keys.  q/output rows are the
 * sequences' new tokens concatenated in order.  context_lens / query_lens are host
 * arrays; block_tables is a device [num_seqs][bt_stride] table. */
typedef struct pam_mixed_request {
    const void *q;           /* [total_rows][num_heads][head_dim] */
    void *output;
    const void *new_keys;    /* [total_rows][num_kv_heads][head_dim] or NULL (already appended) */
    const void *new_values;
    void *k_pool;
    void *v_pool;
    uint16_t *k_scale;
    uint16_t *v_scale;
    const int32_t *block_tables;
    int32_t bt_stride;
    int32_t num_seqs;
    const int32_t *context_lens;
    const int32_t *query_lens;
    pam_layer_spec layer;
    /* buffer lengths in bytes (0 skips that buffer's check): q and output need
     * total_rows rows, new K/V total_rows token rows, block_tables num_seqs rows of
     * bt_stride entries, each pool at least as many blocks as the longest
     * sequence spans (the decode request's check) */
    size_t q_bytes, output_bytes, new_keys_bytes, new_values_bytes, k_pool_bytes, v_pool_bytes, block_tables_bytes;
} pam_mixed_request;
int32_t pam_engine_mixed_step(void *context, const pam_mixed_request *request);

/* Code-object loading and launch: the counterpart of the reference's Metal
 * pipeline manager (PagedAttentionEngine.swift:151-198 builds the shader library
 * at start-up, :248-333 looks pipelines up by function name).  The build writes
 * libpam_kernels.hsaco (gfx950 code object, pam_module_default_path gives its
 * path beside libpam.so) with a named entry for every kernel of the forward
 * path:
 *   decode   pam_decode_streamk_{f16,e4m3}_d128, pam_decode_layers_streamk_{f16,e4m3}_d128,
 *            pam_decode_wg_{f16,e4m3}_d128, pam_decode_valu_{f32,f16,e4m3}_h{1,2,4,8},
 *            pam_decode_valu_wg_{f32,f16,e4m3}_h{1,2},
 *            pam_reduce_{f32,f16}
 *   prefill  pam_prefill_{f16,fused_f16,e4m3}_d128, pam_prefill_{f16,fused_f16,e4m3}_d64,
 *            pam_mixed_step_{f16,e4m3}_d128
 *   append   pam_append_b{16,4,2}, pam_append_batch_b{16,4,2}, pam_append_fp8
 *   staging  pam_stage_copy;  copy-on-write  pam_block_copy;
 *   and pam_fill_u32 for callers' own launches.
 * pam_module_load loads one with hipModuleLoad; while it is loaded the context
 * launches every configuration the object holds through hipModuleLaunchKernel
 * (same kernel bodies: the same results bit for bit) and all others (MFMA
 * decode at d != 128 or blocks of 8, the backward) from the library.
 * pam_module_set_strict(ctx, 1) makes those others fail with an error instead,
 * for hosts that must run only from the code object.
 * pam_module_function / pam_module_launch are the thin launch shim a host
 * language binds: any entry, grid and block sizes, and the packed kernel
 * arguments (args_bytes bytes at args, laid out as the kernel's parameters),
 * on the context's stream. */
int32_t pam_module_load(void *context, const char *path);
int32_t pam_module_unload(void *context);
int32_t pam_module_set_strict(void *context, int32_t strict);
int32_t pam_module_function(void *context, const char *name, void **function);
int32_t pam_module_launch(void *context, void *function, uint32_t grid_x, uint32_t grid_y, uint32_t grid_z,
                          uint32_t block_x, uint32_t block_y, uint32_t block_z, uint32_t shared_bytes, void *args,
                          size_t args_bytes);
const char *pam_module_default_path(void);

/* One decode step of a sequence through the framework adapter (PagedMetalKVCache
 * pagedAttention at seqLen 1, PagedMetalKVCache.swift:94-129): appendTokens(1)
 * on the cache's bookkeeping, the token's K/V ([numKVHeads][headDim]) written
 * into the pools and its query ([numHeads][headDim]) decoded into output.  The
 * sequence's block table and length stay in HBM between steps, patched by the
 * append kernel, so a step is two launches and no host-to-device staging.
 * f32 and f16 caches; pam_free_sequence releases the device table. */
int32_t pam_decode_step(void *context, void *cache, int64_t sequenceID, const void *keys, const void *values,
                        const void *query, void *output, int32_t numHeads);

/* Allocation-free decode.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (tight serving loops, harnesses that
 * forbid hipMalloc).  Not for HIP graph capture: the host picks each launch's
 * merge-counter epoch, which a replayed graph would repeat.  pam_engine_decode_noalloc
 * takes the same request and gives the same results as pam_engine_decode, but
 * its kernels keep their split-context partials, merge counters and zero page
 * in one fixed per-GPU array of the library (32 MiB, held until the process
 * ends) and it calls no hipMalloc / hipFree; a request whose workspace does not
 * fit (stream-K partials above 31 MiB - 4 KiB, or more than 131072 merge
 * counters) fails with an error, also under graceful degradation.  Every call on one GPU shares that array:
 * calls that overlap on one GPU (other contexts or streams) race.
 * pam_engine_setup_noalloc prepares the context and the array (it may
 * allocate; call it once, outside the no-allocation region). */
int32_t pam_engine_setup_noalloc(void *context);
int32_t pam_engine_decode_noalloc(void *context, const pam_decode_request *request);

/* FP8 e4m3 codec over n elements (device buffers): the quantize_fp8 / dequant_fp8
 * pair of kernels.metal:553-601 with a per-element half scale. */
int32_t pam_fp8_quantize(void *context, const uint16_t *values, const uint16_t *scales, uint8_t *out, int64_t n);
int32_t pam_fp8_dequant(void *context, const uint8_t *codes, const uint16_t *scales, uint16_t *out, int64_t n);

/* Calibration streams of known size on the context's stream, timed with hipEvents
 * (ms written to *ms): every byte of src read once / copied once with 16-byte
 * accesses by `blocks` workgroups of 256 threads (0 = 4 per CU).  bytes % 16 == 0. */
int32_t pam_calib_stream_read(void *context, const void *src, size_t bytes, int32_t blocks, float *ms);
int32_t pam_calib_stream_copy(void *context, const void *src, void *dst, size_t bytes, int32_t blocks, float *ms);
/* Dense f16 MFMA rate the device sustains (TFLOP/s written to *tflops): one
 * 8-wave workgroup per CU, each wave iters x 4 v_mfma_f32_32x32x16_f16 on
 * independent accumulators and nothing else, timed with hipEvents after one
 * untimed launch.  The power-limited ceiling a matrix-bound kernel is set against. */
int32_t pam_calib_mfma(void *context, int32_t iters, double *tflops);

/* Synthetic data of the measured workloads (no reference counterpart): n
 * normals N(0, stddev^2) into dst (PAM_FLOAT32 or PAM_FLOAT16), element i from
 * SplitMix64 outputs (stream << 40) + 2i and + 2i + 1 of the generator seeded
 * with `seed` (Box-Muller cosine branch in binary64, rounded to binary32, then to
 * the output type).  outlier_stream >= 0: element i is multiplied by 8 when the
 * uniform of output (outlier_stream << 40) + i is below outlier_frac.  Streams
 * < 2^23, n < 2^39.  Enqueued on the context's stream. */
int32_t pam_synth_normal(void *context, void *dst, int32_t dtype, uint64_t n, uint64_t seed, uint64_t stream,
                         float stddev, int64_t outlier_stream, float outlier_frac);

/* Test hook: the next n kernel launches of this context report a launch failure
 * (host-side; no GPU work is faulted). */
int32_t pam_debug_fail_next_launches(void *context, int32_t n);

/* Test hook: every split-merge counter of this context is set to `arrivals`
 * arrivals of a launch that was abandoned part-way (an epoch no later launch
 * uses).  Later launches must be unaffected. */
int32_t pam_debug_dirty_counters(void *context, int32_t arrivals);

/* Library version string. */
const char *pam_version(void);

#ifdef __cplusplus
}
#endif
#endif /* PAM_H */
