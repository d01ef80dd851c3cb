// append.hip - KV append into the paged pools, FP8 quantize-on-append, codec.
//
// kv_append (kernels.metal:1804-1874): token t of the append lands at
//   slot = block_table[(token_offset + t) / bs] * bs + (token_offset + t) % bs
// (or at an explicit slot_mapping[t]).  A token's Hkv*d row is contiguous in both
// the input and the pool, so each thread moves one 16-byte piece of a row.
//
// kv_append_fp8 (kernels.metal:1876-1961): one workgroup per physical block the
// append touches reduces max|k|, max|v| over this append's elements in that block
// (all heads), derives the block's new half scale from the old one and quantizes
// the new elements with it.  A deterministic block reduction replaces the
// reference's scratch buffer + CAS atomics, and one launch replaces its two
// synchronous passes.
#include "append_body.h"

namespace pam {

// The kernels (the fat binary's entries); the bodies also back the named
// entries of the code object (module_entry.hip).
template <typename CH>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p, int64_t chunks_per_row, int64_t total) {
    append_body<CH>(p, chunks_per_row, total);
}

__global__ __launch_bounds__(256) void kv_append_fp8_kernel(AppendBatchParams p, int32_t first_lb,
                                                            int32_t single_offset) {
    append_fp8_body(p, first_lb, single_offset);
}

template <typename CH>
__global__ __launch_bounds__(256) void kv_append_batch_kernel(AppendBatchParams p, int64_t chunks_per_row,
                                                              int64_t total) {
    append_batch_body<CH>(p, chunks_per_row, total);
}

hipError_t launch_append(const AppendParams &p, int32_t dtype, hipStream_t stream, const KernelTable *kt) {
    if (p.num_tokens <= 0) return hipSuccess;
    const int64_t row_elems = (int64_t)p.num_kv_heads * p.head_dim;
    if (dtype == kFP8) {
        if (p.slot_mapping) return hipErrorInvalidValue;
        const int32_t first_lb = p.token_offset / p.block_size;
        const int32_t last_lb = (p.token_offset + p.num_tokens - 1) / p.block_size;
        AppendBatchParams b{};
        b.keys = p.keys;
        b.values = p.values;
        b.k_pool = p.k_pool;
        b.v_pool = p.v_pool;
        b.k_scale = p.k_scale;
        b.v_scale = p.v_scale;
        b.block_tables = p.block_table;
        b.cu_tokens = nullptr;
        b.token_offsets = nullptr;
        b.work = nullptr;
        b.seqs = 1;
        b.bt_stride = 0;
        b.total_tokens = p.num_tokens;
        b.num_kv_heads = p.num_kv_heads;
        b.head_dim = p.head_dim;
        b.block_size = p.block_size;
        const dim3 grid(last_lb - first_lb + 1);
        const int32_t off = p.token_offset;
        hipError_t e;
        if (via_module(kt, kt ? kt->append_fp8 : nullptr, &e, grid, dim3(256), stream, b, first_lb, off)) return e;
        hipLaunchKernelGGL(kv_append_fp8_kernel, grid, dim3(256), 0, stream, b, first_lb, off);
        return hipGetLastError();
    }
    const int64_t row_bytes = row_elems * (dtype == kF32 ? 4 : 2);
    const int64_t total_bytes = row_bytes * p.num_tokens;
    const int threads = 256;
    auto blocks_for = [&](int64_t total) {
        int64_t b = (total + threads - 1) / threads;
        return (int)(b < 65536 ? b : 65536);
    };
    // piece width: 16, 4 or 2 bytes, the widest that divides a token row
    const int w = row_bytes % 16 == 0 ? 0 : (row_bytes % 4 == 0 ? 1 : 2);
    const int64_t piece = w == 0 ? 16 : (w == 1 ? 4 : 2);
    const int64_t cpr = row_bytes / piece, total = total_bytes / piece;
    const dim3 grid(blocks_for(total));
    hipError_t e;
    if (via_module(kt, kt ? kt->append[w] : nullptr, &e, grid, dim3(threads), stream, p, cpr, total)) return e;
    if (w == 0)
        hipLaunchKernelGGL(kv_append_kernel<uint4>, grid, dim3(threads), 0, stream, p, cpr, total);
    else if (w == 1)
        hipLaunchKernelGGL(kv_append_kernel<uint32_t>, grid, dim3(threads), 0, stream, p, cpr, total);
    else
        hipLaunchKernelGGL(kv_append_kernel<uint16_t>, grid, dim3(threads), 0, stream, p, cpr, total);
    return hipGetLastError();
}

hipError_t launch_append_batch(const AppendBatchParams &p, int32_t dtype, hipStream_t stream,
                               const KernelTable *kt) {
    if (dtype != kFP8) {
        if (p.token_pos == nullptr) return hipErrorInvalidValue;
        if (p.total_tokens <= 0) return hipSuccess;
        const int64_t row_bytes = (int64_t)p.num_kv_heads * p.head_dim * (dtype == kF32 ? 4 : 2);
        const int64_t total_bytes = row_bytes * p.total_tokens;
        auto blocks_for = [&](int64_t total) {
            int64_t b = (total + 255) / 256;
            return (int)(b < 65536 ? b : 65536);
        };
        const int w = row_bytes % 16 == 0 ? 0 : (row_bytes % 4 == 0 ? 1 : 2);
        const int64_t piece = w == 0 ? 16 : (w == 1 ? 4 : 2);
        const int64_t cpr = row_bytes / piece, total = total_bytes / piece;
        const dim3 grid(blocks_for(total));
        hipError_t e;
        if (via_module(kt, kt ? kt->append_batch[w] : nullptr, &e, grid, dim3(256), stream, p, cpr, total)) return e;
        if (w == 0)
            hipLaunchKernelGGL(kv_append_batch_kernel<uint4>, grid, dim3(256), 0, stream, p, cpr, total);
        else if (w == 1)
            hipLaunchKernelGGL(kv_append_batch_kernel<uint32_t>, grid, dim3(256), 0, stream, p, cpr, total);
        else
            hipLaunchKernelGGL(kv_append_batch_kernel<uint16_t>, grid, dim3(256), 0, stream, p, cpr, total);
        return hipGetLastError();
    }
    if (p.work == nullptr || p.token_offsets == nullptr || p.cu_tokens == nullptr) return hipErrorInvalidValue;
    if (p.num_work <= 0) return hipSuccess;
    const int32_t zero = 0;
    hipError_t e;
    if (via_module(kt, kt ? kt->append_fp8 : nullptr, &e, dim3(p.num_work), dim3(256), stream, p, zero, zero)) return e;
    hipLaunchKernelGGL(kv_append_fp8_kernel, dim3(p.num_work), dim3(256), 0, stream, p, 0, 0);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void block_copy_kernel(uint4 *k_pool, uint4 *v_pool, uint16_t *k_scale,
                                                         uint16_t *v_scale, int64_t n16, int32_t src, int32_t dst) {
    block_copy_body(k_pool, v_pool, k_scale, v_scale, n16, src, dst);
}

hipError_t launch_block_copy(void *k_pool, void *v_pool, uint16_t *k_scale, uint16_t *v_scale, size_t block_bytes,
                             int32_t src, int32_t dst, hipStream_t stream, const KernelTable *kt) {
    if (block_bytes % 16 || (((uintptr_t)k_pool | (uintptr_t)v_pool) & 15)) return hipErrorInvalidValue;
    const int64_t n16 = (int64_t)(block_bytes / 16);
    const dim3 grid((unsigned)((n16 + 255) / 256));
    uint4 *k = static_cast<uint4 *>(k_pool), *v = static_cast<uint4 *>(v_pool);
    hipError_t e;
    if (via_module(kt, kt ? kt->block_copy : nullptr, &e, grid, dim3(256), stream, k, v, k_scale, v_scale, n16, src, dst))
        return e;
    hipLaunchKernelGGL(block_copy_kernel, grid, dim3(256), 0, stream, k, v, k_scale, v_scale, n16, src, dst);
    return hipGetLastError();
}

// ------------------------------------------------------------------ codec kernels

__global__ void fp8_quantize_kernel(const uint16_t *values, const uint16_t *scales, uint8_t *out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (uint8_t)fp8_quantize(bits_to_f16(values[i]), bits_to_f16(scales[i]));
}

__global__ void fp8_dequant_kernel(const uint8_t *codes, const uint16_t *scales, uint16_t *out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f16_to_bits(fp8_dequant(codes[i], bits_to_f16(scales[i])));
}

hipError_t launch_fp8_quantize(const uint16_t *values, const uint16_t *scales, uint8_t *out, int64_t n,
                               hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    int64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(fp8_quantize_kernel, dim3((unsigned)(b < 65536 ? b : 65536)), dim3(256), 0, stream, values,
                       scales, out, n);
    return hipGetLastError();
}

hipError_t launch_fp8_dequant(const uint8_t *codes, const uint16_t *scales, uint16_t *out, int64_t n,
                              hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    int64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(fp8_dequant_kernel, dim3((unsigned)(b < 65536 ? b : 65536)), dim3(256), 0, stream, codes,
                       scales, out, n);
    return hipGetLastError();
}

}  // namespace pam
