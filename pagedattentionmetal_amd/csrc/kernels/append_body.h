// append_body.h - device bodies of the KV append kernels (gfx950): the f32 /
// f16 row copy through the block table or a slot mapping, the FP8
// quantize-on-append per physical block, and the mixed step's batched copy.
// Included by append.hip (the library's kernels) and by the code-object
// entries (module_entry.hip), which wrap the same bodies.
#pragma once
#include "kernels.h"
#include "pam_device.h"

namespace pam {

template <typename CH>
__device__ __forceinline__ void append_body(const AppendParams &p, int64_t chunks_per_row, int64_t total) {
    if (p.length_patch && blockIdx.x == 0 && threadIdx.x == 0) {
        if (p.table_patch) p.table_patch[p.patch_index] = p.patch_block;
        *p.length_patch = p.length_value;
    }
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t t = i / chunks_per_row, c = i % chunks_per_row;
        int64_t slot;
        if (p.slot_mapping) {
            slot = p.slot_mapping[t];
            if (slot < 0) continue;  // padding token
        } else if (p.fixed_slot >= 0) {
            slot = p.fixed_slot;  // one token
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
__device__ __forceinline__ void append_fp8_body(const AppendBatchParams &p, int32_t first_lb,
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

template <typename CH>
__device__ __forceinline__ void append_batch_body(const AppendBatchParams &p, int64_t chunks_per_row,
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

// Copy-on-write of one physical block: its K and V bytes (n16 16-byte pieces
// each) from block `src` to block `dst` of the pools, and its FP8 half scales
// when the pools have them.
__device__ __forceinline__ void block_copy_body(uint4 *k_pool, uint4 *v_pool, uint16_t *k_scale, uint16_t *v_scale,
                                                int64_t n16, int32_t src, int32_t dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) {
        k_pool[(int64_t)dst * n16 + i] = k_pool[(int64_t)src * n16 + i];
        v_pool[(int64_t)dst * n16 + i] = v_pool[(int64_t)src * n16 + i];
    }
    if (i == 0 && k_scale) {
        k_scale[dst] = k_scale[src];
        v_scale[dst] = v_scale[src];
    }
}

}  // namespace pam
