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
#include "kernels.h"
#include "pam_device.h"

namespace pam {

template <typename CH>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p, int64_t chunks_per_row, int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t t = i / chunks_per_row, c = i % chunks_per_row;
        int64_t slot;
        if (p.slot_mapping) {
            slot = p.slot_mapping[t];
            if (slot < 0) continue;  // padding token
        } else {
            const int64_t pos = (int64_t)p.token_offset + t;
            slot = (int64_t)p.block_table[pos / p.block_size] * p.block_size + pos % p.block_size;
        }
        const CH *ks = static_cast<const CH *>(p.keys) + t * chunks_per_row + c;
        const CH *vs = static_cast<const CH *>(p.values) + t * chunks_per_row + c;
        static_cast<CH *>(p.k_pool)[slot * chunks_per_row + c] = *ks;
        static_cast<CH *>(p.v_pool)[slot * chunks_per_row + c] = *vs;
    }
}

// One workgroup per touched (sequence, logical block).  The block's new tokens
// are consecutive rows of the input and consecutive slots of the physical block,
// so both passes (the max for the scale rule, then the quantisation) stream one
// contiguous range: 8 halves in, 8 codes out per thread and step when the rows
// are 16-byte multiples, one element at a time otherwise.
__global__ __launch_bounds__(256) void kv_append_fp8_kernel(AppendBatchParams p, int32_t first_lb,
                                                            int32_t single_offset) {
    int seq, lb;
    if (p.work) {
        const int4 w = p.work[blockIdx.x];
        seq = w.x;
        lb = w.y;
    } else {
        seq = 0;
        lb = first_lb + blockIdx.x;
    }
    const int64_t row = (int64_t)p.num_kv_heads * p.head_dim;  // elements per token
    const int64_t tok_base = p.cu_tokens ? p.cu_tokens[seq] : 0;
    const int64_t n_tok = p.cu_tokens ? p.cu_tokens[seq + 1] - tok_base : p.total_tokens;
    const int64_t off = p.token_offsets ? p.token_offsets[seq] : single_offset;
    const int bs = p.block_size;
    int64_t t0 = (int64_t)lb * bs - off, t1 = t0 + bs;
    if (t0 < 0) t0 = 0;
    if (t1 > n_tok) t1 = n_tok;
    const int32_t phys = p.block_tables[(int64_t)seq * p.bt_stride + lb];
    // input elements [t0 * row, t1 * row) -> pool elements from the slot of t0
    const int64_t n = (t1 - t0) * row;
    const f16 *kin = static_cast<const f16 *>(p.keys) + (tok_base + t0) * row;
    const f16 *vin = static_cast<const f16 *>(p.values) + (tok_base + t0) * row;
    const int64_t dst0 = ((int64_t)phys * bs + (off + t0 - (int64_t)lb * bs)) * row;
    uint8_t *kp = static_cast<uint8_t *>(p.k_pool) + dst0;
    uint8_t *vp = static_cast<uint8_t *>(p.v_pool) + dst0;
    // 16-byte input rows and aligned buffers: every token row keeps the alignment
    const bool vec = (row % 8) == 0 && (((uintptr_t)p.keys | (uintptr_t)p.values) & 15) == 0 &&
                     (((uintptr_t)p.k_pool | (uintptr_t)p.v_pool) & 7) == 0;

    float mk = 0.0f, mv = 0.0f;
    if (vec) {
        for (int64_t e = (int64_t)threadIdx.x * 8; e < n; e += (int64_t)blockDim.x * 8) {
            const f16x8 a = *reinterpret_cast<const f16x8 *>(kin + e);
            const f16x8 b = *reinterpret_cast<const f16x8 *>(vin + e);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                mk = fmaxf(mk, fabsf((float)a[i]));
                mv = fmaxf(mv, fabsf((float)b[i]));
            }
        }
    } else {
        for (int64_t e = threadIdx.x; e < n; e += blockDim.x) {
            mk = fmaxf(mk, fabsf((float)kin[e]));
            mv = fmaxf(mv, fabsf((float)vin[e]));
        }
    }
    mk = wave_max_xor(mk, 1, 64);
    mv = wave_max_xor(mv, 1, 64);
    __shared__ float red[2][4];
    __shared__ uint16_t scales[2];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[0][wave] = mk;
        red[1][wave] = mv;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float a = red[0][0], b = red[1][0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) {
            a = fmaxf(a, red[0][w]);
            b = fmaxf(b, red[1][w]);
        }
        scales[0] = f16_to_bits(fp8_scale_rule(a, bits_to_f16(p.k_scale[phys])));
        scales[1] = f16_to_bits(fp8_scale_rule(b, bits_to_f16(p.v_scale[phys])));
    }
    __syncthreads();
    const f16 ks = bits_to_f16(scales[0]), vs = bits_to_f16(scales[1]);
    if (vec) {
        for (int64_t e = (int64_t)threadIdx.x * 8; e < n; e += (int64_t)blockDim.x * 8) {
            const f16x8 a = *reinterpret_cast<const f16x8 *>(kin + e);
            const f16x8 b = *reinterpret_cast<const f16x8 *>(vin + e);
            uint32_t kw[2] = {0u, 0u}, vw[2] = {0u, 0u};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                kw[i >> 2] |= fp8_quantize(a[i], ks) << (8 * (i & 3));
                vw[i >> 2] |= fp8_quantize(b[i], vs) << (8 * (i & 3));
            }
            *reinterpret_cast<uint2 *>(kp + e) = make_uint2(kw[0], kw[1]);
            *reinterpret_cast<uint2 *>(vp + e) = make_uint2(vw[0], vw[1]);
        }
    } else {
        for (int64_t e = threadIdx.x; e < n; e += blockDim.x) {
            kp[e] = (uint8_t)fp8_quantize(kin[e], ks);
            vp[e] = (uint8_t)fp8_quantize(vin[e], vs);
        }
    }
    if (threadIdx.x == 0) {
        p.k_scale[phys] = scales[0];
        p.v_scale[phys] = scales[1];
    }
}

hipError_t launch_append(const AppendParams &p, int32_t dtype, hipStream_t stream) {
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
        hipLaunchKernelGGL(kv_append_fp8_kernel, dim3(last_lb - first_lb + 1), dim3(256), 0, stream, b, first_lb,
                           p.token_offset);
        return hipGetLastError();
    }
    const int64_t row_bytes = row_elems * (dtype == kF32 ? 4 : 2);
    const int64_t total_bytes = row_bytes * p.num_tokens;
    const int threads = 256;
    auto blocks_for = [&](int64_t total) {
        int64_t b = (total + threads - 1) / threads;
        return (int)(b < 65536 ? b : 65536);
    };
    if (row_bytes % 16 == 0) {
        const int64_t cpr = row_bytes / 16, total = total_bytes / 16;
        hipLaunchKernelGGL(kv_append_kernel<uint4>, dim3(blocks_for(total)), dim3(threads), 0, stream, p, cpr, total);
    } else if (row_bytes % 4 == 0) {
        const int64_t cpr = row_bytes / 4, total = total_bytes / 4;
        hipLaunchKernelGGL(kv_append_kernel<uint32_t>, dim3(blocks_for(total)), dim3(threads), 0, stream, p, cpr,
                           total);
    } else {
        const int64_t cpr = row_bytes / 2, total = total_bytes / 2;
        hipLaunchKernelGGL(kv_append_kernel<uint16_t>, dim3(blocks_for(total)), dim3(threads), 0, stream, p, cpr,
                           total);
    }
    return hipGetLastError();
}

template <typename CH>
__global__ __launch_bounds__(256) void kv_append_batch_kernel(AppendBatchParams p, int64_t chunks_per_row,
                                                              int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t t = i / chunks_per_row, c = i % chunks_per_row;
        const int2 tp = p.token_pos[t];
        const int64_t slot =
            (int64_t)p.block_tables[(int64_t)tp.x * p.bt_stride + tp.y / p.block_size] * p.block_size +
            tp.y % p.block_size;
        static_cast<CH *>(p.k_pool)[slot * chunks_per_row + c] = static_cast<const CH *>(p.keys)[i];
        static_cast<CH *>(p.v_pool)[slot * chunks_per_row + c] = static_cast<const CH *>(p.values)[i];
    }
}

hipError_t launch_append_batch(const AppendBatchParams &p, int32_t dtype, hipStream_t stream) {
    if (dtype != kFP8) {
        if (p.token_pos == nullptr) return hipErrorInvalidValue;
        if (p.total_tokens <= 0) return hipSuccess;
        const int64_t row_bytes = (int64_t)p.num_kv_heads * p.head_dim * (dtype == kF32 ? 4 : 2);
        const int64_t total_bytes = row_bytes * p.total_tokens;
        auto blocks_for = [&](int64_t total) {
            int64_t b = (total + 255) / 256;
            return (int)(b < 65536 ? b : 65536);
        };
        if (row_bytes % 16 == 0)
            hipLaunchKernelGGL(kv_append_batch_kernel<uint4>, dim3(blocks_for(total_bytes / 16)), dim3(256), 0, stream,
                               p, row_bytes / 16, total_bytes / 16);
        else if (row_bytes % 4 == 0)
            hipLaunchKernelGGL(kv_append_batch_kernel<uint32_t>, dim3(blocks_for(total_bytes / 4)), dim3(256), 0,
                               stream, p, row_bytes / 4, total_bytes / 4);
        else
            hipLaunchKernelGGL(kv_append_batch_kernel<uint16_t>, dim3(blocks_for(total_bytes / 2)), dim3(256), 0,
                               stream, p, row_bytes / 2, total_bytes / 2);
        return hipGetLastError();
    }
    if (p.work == nullptr || p.token_offsets == nullptr || p.cu_tokens == nullptr) return hipErrorInvalidValue;
    if (p.num_work <= 0) return hipSuccess;
    hipLaunchKernelGGL(kv_append_fp8_kernel, dim3(p.num_work), dim3(256), 0, stream, p, 0, 0);
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
