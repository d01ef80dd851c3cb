// kv_cache.cpp - KVCacheManager with HBM-resident pools.
//
// Pools: [maxBlocks][blockSize][numKVHeads][headDim] of the cache's element type
// (KVCacheManager.swift:91-99); FP8 caches also own one half scale per block for
// K and for V, zero-initialised as the reference's callers do
// (Tests/PagedAttentionMetalTests/PagedAttentionMetalTests.swift:669-680).
// Copy-on-write (KVCacheManager.swift:176-194) copies the block's K and V bytes
// HBM-to-HBM; FP8 scales travel with the block (the reference copies bytes only,
// which would leave the copy paired with a stale scale).
#include "runtime.h"

namespace pam {

static size_t elem_size(int32_t dtype) { return dtype == kF32 ? 4 : (dtype == kF16 ? 2 : 1); }

KVCache::KVCache(Context *ctx, int32_t max_blocks, int32_t block_size, int32_t head_dim_, int32_t num_kv_heads_,
                 int32_t dtype_, bool with_device)
    : alloc(max_blocks, block_size),
      head_dim(head_dim_),
      num_kv_heads(num_kv_heads_),
      dtype(dtype_),
      has_device(with_device) {
    pool_bytes = (size_t)max_blocks * bytes_per_block();
    if (!with_device) return;
    ctx->ensure_device();
    hip_check(hipGetDevice(&device), "hipGetDevice");
    hipError_t e = hipMalloc(&k_pool, pool_bytes);
    if (e == hipSuccess) e = hipMalloc(&v_pool, pool_bytes);
    if (e == hipSuccess && dtype == kFP8) {
        e = hipMalloc(reinterpret_cast<void **>(&k_scale), (size_t)max_blocks * 2);
        if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&v_scale), (size_t)max_blocks * 2);
        if (e == hipSuccess) e = hipMemset(k_scale, 0, (size_t)max_blocks * 2);
        if (e == hipSuccess) e = hipMemset(v_scale, 0, (size_t)max_blocks * 2);
    }
    if (e != hipSuccess) {
        if (k_pool) (void)hipFree(k_pool);
        if (v_pool) (void)hipFree(v_pool);
        if (k_scale) (void)hipFree(k_scale);
        if (v_scale) (void)hipFree(v_scale);
        k_pool = v_pool = nullptr;
        k_scale = v_scale = nullptr;
        throw PamError(std::string("GPU command encoding failed: Failed to allocate KV pool buffers: ") +
                       hipGetErrorString(e));
    }
}

KVCache::~KVCache() {
    if (!has_device) return;
    (void)hipSetDevice(device);
    (void)hipDeviceSynchronize();
    for (auto &t : device_tables)
        if (t.second.ptr) (void)hipFree(t.second.ptr);
    if (k_pool) (void)hipFree(k_pool);
    if (v_pool) (void)hipFree(v_pool);
    if (k_scale) (void)hipFree(k_scale);
    if (v_scale) (void)hipFree(v_scale);
}

void KVCache::drop_device_table(int64_t id) {
    auto it = device_tables.find(id);
    if (it == device_tables.end()) return;
    if (it->second.ptr) {
        (void)hipSetDevice(device);
        (void)hipFree(it->second.ptr);  // waits for the work that reads it
    }
    device_tables.erase(it);
}

size_t KVCache::bytes_per_block() const {
    return (size_t)alloc.block_size() * num_kv_heads * head_dim * elem_size(dtype);
}

void KVCache::copy_blocks(const BlockCopies &copies, hipStream_t stream, const KernelTable *kt) {
    if (!has_device || copies.empty()) return;
    const size_t bpb = bytes_per_block();
    for (const auto &c : copies) {
        // one kernel for K, V and the scales; a block whose bytes are not
        // whole 16-byte pieces goes through the copy engine
        const hipError_t e = launch_block_copy(k_pool, v_pool, dtype == kFP8 ? k_scale : nullptr,
                                               dtype == kFP8 ? v_scale : nullptr, bpb, c.first, c.second, stream, kt);
        if (e == hipSuccess) continue;
        if (e != hipErrorInvalidValue) hip_check(e, "copy-on-write");
        (void)hipGetLastError();
        char *k = static_cast<char *>(k_pool), *v = static_cast<char *>(v_pool);
        hip_check(hipMemcpyAsync(k + (size_t)c.second * bpb, k + (size_t)c.first * bpb, bpb, hipMemcpyDeviceToDevice,
                                 stream),
                  "copy-on-write K");
        hip_check(hipMemcpyAsync(v + (size_t)c.second * bpb, v + (size_t)c.first * bpb, bpb, hipMemcpyDeviceToDevice,
                                 stream),
                  "copy-on-write V");
        if (dtype == kFP8) {
            hip_check(hipMemcpyAsync(k_scale + c.second, k_scale + c.first, 2, hipMemcpyDeviceToDevice, stream),
                      "copy-on-write K scale");
            hip_check(hipMemcpyAsync(v_scale + c.second, v_scale + c.first, 2, hipMemcpyDeviceToDevice, stream),
                      "copy-on-write V scale");
        }
    }
}

}  // namespace pam
