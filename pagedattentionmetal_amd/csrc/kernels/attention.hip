// attention.hip - paged attention over query rows for gfx950.
//
// One wave64 owns (row, kv head | head group, split-context partition).  A row is
// a decode query (kernels.metal:1417-1802 semantics), a prefill query position
// (kernels.metal:693-917 semantics with an explicit query offset) or a ragged row
// of a mixed continuous-batching step.  Keys are walked in 16-token tiles of the
// logical sequence; the block table maps each token to its physical block, so
// any block_size works and blocks may sit anywhere in the pool.
//
// Two bodies:
//  * attn_mfma_kernel - GQA groups 4..16, f16 or e4m3 KV.  S^T = K Q^T with
//    v_mfma_f32_16x16x32_f16 (K rows feed the A operand straight from their
//    16-byte HBM loads, query heads are the N columns), then O^T = V^T P^T with
//    v_mfma_f32_16x16x16_f16: the S^T accumulator layout (lane%16 = head,
//    lane/16 = token quad) is exactly the B-operand layout of P^T, so softmax
//    needs no data movement; V is transposed through a padded LDS tile.
//  * attn_valu_kernel - any group and f32 KV: lanes split a token row into
//    4-element slices, dot products reduce across the row's lanes.
// Both keep the online-softmax state of Reference/paged_attention_sim.py:94-123
// (in log2 units) and either finish the row or write a partial (m, l, O) for
// the split-context reduce kernel.
#include "kernels.h"
#include "pam_device.h"

namespace pam {

struct RowCtx {
    const int32_t *bt;
    int64_t k_lo, k_hi;
    int64_t out_row;
};

__device__ __forceinline__ RowCtx row_ctx(const AttnParams &p, int r) {
    RowCtx c;
    if (p.mode == kRowDecode) {
        // kernels.metal:1440-1449: token-granular window, block table clamp
        const int64_t L = p.seq_lengths[r];
        const int64_t ws = (p.window > 0 && L > p.window) ? L - p.window : 0;
        int64_t nlb = (L + p.block_size - 1) / p.block_size;
        if (nlb > p.max_num_blocks) nlb = p.max_num_blocks;
        const int64_t cap = nlb * p.block_size;
        c.bt = p.block_tables + (int64_t)r * p.bt_stride;
        c.k_lo = ws;
        c.k_hi = L < cap ? L : cap;
        c.out_row = r;
    } else if (p.mode == kRowPrefill) {
        // one fixed window start for every row (PagedAttentionEngine.swift:802)
        const int64_t kv_len = (int64_t)p.q_offset + p.rows;
        c.bt = p.block_tables;
        c.k_lo = p.window > 0 ? (kv_len > p.window ? kv_len - p.window : 0) : 0;
        c.k_hi = p.causal ? (int64_t)p.q_offset + r + 1 : kv_len;
        c.out_row = r;
    } else {
        const int4 ri = p.row_info[r];
        c.bt = p.block_tables + (int64_t)ri.x * p.bt_stride;
        c.k_lo = ri.y;
        c.k_hi = ri.z;
        c.out_row = ri.w;
    }
    return c;
}

struct PartRange {
    int64_t t_begin, t_end;  // 16-token tiles
    int nparts;
};

__device__ __forceinline__ PartRange part_range(const RowCtx &c, int part, int part_tokens) {
    PartRange pr;
    const int64_t tile0 = c.k_lo / 16;
    const int64_t tile_end = (c.k_hi + 15) / 16;
    const int64_t ntiles = c.k_hi > c.k_lo ? tile_end - tile0 : 0;
    const int tpp = part_tokens / 16;
    pr.nparts = (int)((ntiles + tpp - 1) / tpp);
    pr.t_begin = tile0 + (int64_t)part * tpp;
    pr.t_end = pr.t_begin + tpp < tile_end ? pr.t_begin + tpp : tile_end;
    return pr;
}

// ------------------------------------------------------------------ KV slices

template <typename KV>
struct KvTraits;
template <>
struct KvTraits<f16> {
    static constexpr int kBytes = 2;
};
template <>
struct KvTraits<uint8_t> {
    static constexpr int kBytes = 1;
};

// Eight consecutive elements of a raw slice as halves (A operand chunk / LDS row).
template <typename KV>
__device__ __forceinline__ f16x8 slice_chunk(const uint4 *raw, int c, f16 scale);

template <>
__device__ __forceinline__ f16x8 slice_chunk<f16>(const uint4 *raw, int c, f16) {
    return __builtin_bit_cast(f16x8, raw[c]);
}

template <>
__device__ __forceinline__ f16x8 slice_chunk<uint8_t>(const uint4 *raw, int c, f16 scale) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(raw) + c * 2;
    f16x8 o;
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = fp8_dequant((w[i >> 2] >> (8 * (i & 3))) & 0xFFu, scale);
    return o;
}

// ------------------------------------------------------------------ MFMA body

template <typename KV, int HD, bool BS16>
__global__ __launch_bounds__(64) void attn_mfma_kernel(AttnParams p) {
    constexpr int DPG = HD / 4;                 // dims held by one lane group (lane / 16)
    constexpr int NC = HD / 32;                 // 16x16x32 chunks per S tile
    constexpr int NO = HD / 16;                 // 16-dim output chunks
    constexpr int RAW = DPG * KvTraits<KV>::kBytes / 16;  // 16-byte loads per slice
    constexpr int LDS = HD + 8;                 // padded V row (halves)
    __shared__ __attribute__((aligned(16))) f16 vt[16 * LDS];

    const int lane = threadIdx.x, row = lane & 15, grp = lane >> 4;
    const int part = blockIdx.x, kvh = blockIdx.y, r = blockIdx.z;
    const int H = p.num_heads;
    const int G = H / p.num_kv_heads;
    const RowCtx c = row_ctx(p, r);
    const PartRange pr = part_range(c, part, p.part_tokens);
    if (part >= (pr.nparts > 1 ? pr.nparts : 1)) return;

    const int h = kvh * G + row;  // this lane's query head (N column)
    const bool head_ok = row < G;
    f16 *out = static_cast<f16 *>(p.out);
    if (pr.nparts == 0) {
        // no keys: 0/0 as in the reference's m/l bookkeeping
        if (head_ok)
            for (int d = grp; d < HD; d += 4) out[(c.out_row * H + h) * (int64_t)HD + d] = (f16)__builtin_nanf("");
        return;
    }

    // Q^T B operand: lane holds Q[h][grp*DPG + 8c .. +8]
    f16x8 qv[NC];
    {
        const f16 *qp = static_cast<const f16 *>(p.q) + ((int64_t)r * H + (head_ok ? h : 0)) * HD + grp * DPG;
#pragma unroll
        for (int i = 0; i < NC; i++) {
            f16x8 v = *reinterpret_cast<const f16x8 *>(qp + 8 * i);
            qv[i] = head_ok ? v : (f16x8)(f16)0.0f;
        }
    }

    const int64_t row_stride = (int64_t)p.num_kv_heads * HD;  // elements per token
    const char *kbase = static_cast<const char *>(p.k_pool);
    const char *vbase = static_cast<const char *>(p.v_pool);
    const int bs = p.block_size;

    auto load_tile = [&](int64_t tile, uint4 *kr, uint4 *vr, f16 &ks, f16 &vs) {
        const int64_t j = tile * 16 + row;
        const bool valid = j >= c.k_lo && j < c.k_hi;
        int64_t phys = 0, slot = 0;
        if (BS16) {
            phys = c.bt[tile];
            slot = row;
        } else if (valid) {
            phys = c.bt[j / bs];
            slot = j % bs;
        }
        const int64_t off = ((phys * bs + slot) * row_stride + (int64_t)kvh * HD + grp * DPG) * KvTraits<KV>::kBytes;
        const uint4 *kp = reinterpret_cast<const uint4 *>(kbase + off);
        const uint4 *vp = reinterpret_cast<const uint4 *>(vbase + off);
#pragma unroll
        for (int i = 0; i < RAW; i++) {
            kr[i] = valid ? kp[i] : make_uint4(0, 0, 0, 0);
            vr[i] = valid ? vp[i] : make_uint4(0, 0, 0, 0);
        }
        if constexpr (KvTraits<KV>::kBytes == 1) {
            ks = valid ? bits_to_f16(p.k_scale[phys]) : (f16)0.0f;
            vs = valid ? bits_to_f16(p.v_scale[phys]) : (f16)0.0f;
        }
    };

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 o[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) o[i] = (f32x4)0.0f;

    uint4 kr[RAW], vr[RAW], kn[RAW], vn[RAW];
    f16 ks = (f16)0.0f, vs = (f16)0.0f, ksn = (f16)0.0f, vsn = (f16)0.0f;
    load_tile(pr.t_begin, kr, vr, ks, vs);

    for (int64_t tile = pr.t_begin; tile < pr.t_end; tile++) {
        if (tile + 1 < pr.t_end) load_tile(tile + 1, kn, vn, ksn, vsn);

        // S^T[token][head] over HD dims
        f32x4 s = (f32x4)0.0f;
#pragma unroll
        for (int i = 0; i < NC; i++)
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(slice_chunk<KV>(kr, i, ks), qv[i], s, 0, 0, 0);

        // stage V rows (token = row) for the transposed read
#pragma unroll
        for (int i = 0; i < NC; i++)
            *reinterpret_cast<f16x8 *>(&vt[row * LDS + grp * DPG + 8 * i]) = slice_chunk<KV>(vr, i, vs);

        // online softmax on this lane's 4 tokens of head `row`
        float sv[4];
        float mt = -INFINITY;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int64_t j = tile * 16 + 4 * grp + q;
            sv[q] = (j >= c.k_lo && j < c.k_hi) ? s[q] * p.scale_log2 : -INFINITY;
            mt = fmaxf(mt, sv[q]);
        }
        mt = fmaxf(mt, shfl_xor(mt, 16));
        mt = fmaxf(mt, shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float corr = exp2f(m_run - m_use);
        f16x4 pb;
        float psum = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float pq = exp2f(sv[q] - m_use);
            psum += pq;
            pb[q] = (f16)pq;
        }
        l_run = l_run * corr + psum;
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < NO; i++) o[i] *= corr;

        __syncthreads();
#pragma unroll
        for (int i = 0; i < NO; i++) {
            f16x4 a;
#pragma unroll
            for (int q = 0; q < 4; q++) a[q] = vt[(4 * grp + q) * LDS + 16 * i + row];
            o[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb, o[i], 0, 0, 0);
        }
        __syncthreads();

#pragma unroll
        for (int i = 0; i < RAW; i++) {
            kr[i] = kn[i];
            vr[i] = vn[i];
        }
        ks = ksn;
        vs = vsn;
    }

    float l_tot = l_run + shfl_xor(l_run, 16);
    l_tot += shfl_xor(l_tot, 32);
    if (!head_ok) return;
    if (pr.nparts == 1) {
        const float inv = 1.0f / l_tot;
        f16 *op = out + (c.out_row * H + h) * (int64_t)HD + 4 * grp;
#pragma unroll
        for (int i = 0; i < NO; i++) {
            f16x4 v;
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = (f16)(o[i][q] * inv);
            *reinterpret_cast<f16x4 *>(op + 16 * i) = v;
        }
    } else {
        const int64_t slot = ((int64_t)r * H + h) * p.max_parts + part;
        float *po = p.part_o + slot * HD + 4 * grp;
#pragma unroll
        for (int i = 0; i < NO; i++) *reinterpret_cast<f32x4 *>(po + 16 * i) = o[i];
        if (grp == 0) {
            p.part_ml[slot * 2 + 0] = m_run;
            p.part_ml[slot * 2 + 1] = l_tot;
        }
    }
}

// ------------------------------------------------------------------ VALU body

template <typename T>
__device__ __forceinline__ void load4(const T *ptr, float *v);
template <>
__device__ __forceinline__ void load4<float>(const float *ptr, float *v) {
    const float4 x = *reinterpret_cast<const float4 *>(ptr);
    v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
}
template <>
__device__ __forceinline__ void load4<f16>(const f16 *ptr, float *v) {
    const f16x4 x = *reinterpret_cast<const f16x4 *>(ptr);
    v[0] = (float)x[0], v[1] = (float)x[1], v[2] = (float)x[2], v[3] = (float)x[3];
}

template <typename T>
__device__ __forceinline__ void store4(T *ptr, const float *v);
template <>
__device__ __forceinline__ void store4<float>(float *ptr, const float *v) {
    *reinterpret_cast<float4 *>(ptr) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store4<f16>(f16 *ptr, const float *v) {
    f16x4 x;
    x[0] = (f16)v[0], x[1] = (f16)v[1], x[2] = (f16)v[2], x[3] = (f16)v[3];
    *reinterpret_cast<f16x4 *>(ptr) = x;
}

// KV element slice of 4 as floats (fp8: dequantised in half, then widened)
template <typename KV>
__device__ __forceinline__ void load_kv4(const KV *ptr, f16 scale, float *v);
template <>
__device__ __forceinline__ void load_kv4<float>(const float *ptr, f16, float *v) {
    load4<float>(ptr, v);
}
template <>
__device__ __forceinline__ void load_kv4<f16>(const f16 *ptr, f16, float *v) {
    load4<f16>(ptr, v);
}
template <>
__device__ __forceinline__ void load_kv4<uint8_t>(const uint8_t *ptr, f16 scale, float *v) {
    const uint32_t w = *reinterpret_cast<const uint32_t *>(ptr);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = (float)fp8_dequant((w >> (8 * i)) & 0xFFu, scale);
}

// lanes_per_row: power of two >= head_dim / 4 (<= 64); heads NH share one kv head.
template <typename KV, typename QT, int NH>
__global__ __launch_bounds__(64) void attn_valu_kernel(AttnParams p, int lanes_per_row) {
    const int lane = threadIdx.x;
    const int part = blockIdx.x, hg = blockIdx.y, r = blockIdx.z;
    const int HD = p.head_dim, H = p.num_heads;
    const int G = H / p.num_kv_heads;
    const int h0 = hg * NH;
    const int kvh = h0 / G;
    const RowCtx c = row_ctx(p, r);
    const PartRange pr = part_range(c, part, p.part_tokens);
    if (part >= (pr.nparts > 1 ? pr.nparts : 1)) return;

    const int LPR = lanes_per_row, TPI = 64 / lanes_per_row;
    const int sub = lane / LPR;
    const int d0 = (lane % LPR) * 4;
    const bool dim_ok = d0 < HD;
    QT *out = static_cast<QT *>(p.out);
    if (pr.nparts == 0) {
        if (sub == 0 && dim_ok) {
            float nanv[4] = {__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
            for (int hh = 0; hh < NH; hh++) store4<QT>(out + (c.out_row * H + h0 + hh) * (int64_t)HD + d0, nanv);
        }
        return;
    }

    float q[NH][4];
#pragma unroll
    for (int hh = 0; hh < NH; hh++) {
        if (dim_ok)
            load4<QT>(static_cast<const QT *>(p.q) + ((int64_t)r * H + h0 + hh) * HD + d0, q[hh]);
        else
            q[hh][0] = q[hh][1] = q[hh][2] = q[hh][3] = 0.0f;
    }

    float m[NH], l[NH], acc[NH][4];
#pragma unroll
    for (int hh = 0; hh < NH; hh++) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
        acc[hh][0] = acc[hh][1] = acc[hh][2] = acc[hh][3] = 0.0f;
    }
    const int64_t row_stride = (int64_t)p.num_kv_heads * HD;
    const KV *kpool = static_cast<const KV *>(p.k_pool);
    const KV *vpool = static_cast<const KV *>(p.v_pool);
    const int bs = p.block_size;

    for (int64_t j0 = pr.t_begin * 16; j0 < pr.t_end * 16; j0 += TPI) {
        const int64_t j = j0 + sub;
        const bool tok_ok = j >= c.k_lo && j < c.k_hi;
        float kv[4] = {0.f, 0.f, 0.f, 0.f}, vv[4] = {0.f, 0.f, 0.f, 0.f};
        if (tok_ok && dim_ok) {
            const int64_t phys = c.bt[j / bs];
            const int64_t off = (phys * bs + j % bs) * row_stride + (int64_t)kvh * HD + d0;
            f16 ks = (f16)1.0f, vs = (f16)1.0f;
            if constexpr (sizeof(KV) == 1) {
                ks = bits_to_f16(p.k_scale[phys]);
                vs = bits_to_f16(p.v_scale[phys]);
            }
            load_kv4<KV>(kpool + off, ks, kv);
            load_kv4<KV>(vpool + off, vs, vv);
        }
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            float s = q[hh][0] * kv[0] + q[hh][1] * kv[1] + q[hh][2] * kv[2] + q[hh][3] * kv[3];
            s = wave_sum_xor(s, 1, LPR);
            s = tok_ok ? s * p.scale_log2 : -INFINITY;
            const float mt = wave_max_xor(s, LPR, 64);
            const float m_new = fmaxf(m[hh], mt);
            // an iteration whose tokens all fall outside the key range keeps the state
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float corr = exp2f(m[hh] - m_use);
            const float pj = exp2f(s - m_use);
            l[hh] = l[hh] * corr + pj;
            m[hh] = m_new;
#pragma unroll
            for (int e = 0; e < 4; e++) acc[hh][e] = acc[hh][e] * corr + pj * vv[e];
        }
    }

#pragma unroll
    for (int hh = 0; hh < NH; hh++) {
        l[hh] = wave_sum_xor(l[hh], LPR, 64);
#pragma unroll
        for (int e = 0; e < 4; e++) acc[hh][e] = wave_sum_xor(acc[hh][e], LPR, 64);
    }
    if (sub != 0 || !dim_ok) return;
    if (pr.nparts == 1) {
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            const float inv = 1.0f / l[hh];
            float v[4] = {acc[hh][0] * inv, acc[hh][1] * inv, acc[hh][2] * inv, acc[hh][3] * inv};
            store4<QT>(out + (c.out_row * H + h0 + hh) * (int64_t)HD + d0, v);
        }
    } else {
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            const int64_t slot = ((int64_t)r * H + h0 + hh) * p.max_parts + part;
            store4<float>(p.part_o + slot * HD + d0, acc[hh]);
            if (d0 == 0) {
                p.part_ml[slot * 2 + 0] = m[hh];
                p.part_ml[slot * 2 + 1] = l[hh];
            }
        }
    }
}

// ------------------------------------------------------------------ split-context reduce
// O = sum_p 2^{m_p - M} O_p / sum_p 2^{m_p - M} l_p over the row's partitions.
template <typename QT>
__global__ __launch_bounds__(64) void attn_reduce_kernel(AttnParams p) {
    const int r = blockIdx.y, h = blockIdx.x;
    const RowCtx c = row_ctx(p, r);
    const PartRange pr = part_range(c, 0, p.part_tokens);
    if (pr.nparts <= 1) return;
    const int HD = p.head_dim, H = p.num_heads;
    const int64_t base = ((int64_t)r * H + h) * p.max_parts;
    float M = -INFINITY;
    for (int i = 0; i < pr.nparts; i++) M = fmaxf(M, p.part_ml[(base + i) * 2]);
    float den = 0.0f;
    for (int i = 0; i < pr.nparts; i++) den += exp2f(p.part_ml[(base + i) * 2] - M) * p.part_ml[(base + i) * 2 + 1];
    const float inv = 1.0f / den;
    QT *out = static_cast<QT *>(p.out);
    for (int d0 = threadIdx.x * 4; d0 < HD; d0 += 256) {
        float a[4] = {0.f, 0.f, 0.f, 0.f};
        for (int i = 0; i < pr.nparts; i++) {
            const float w = exp2f(p.part_ml[(base + i) * 2] - M);
            float v[4];
            load4<float>(p.part_o + (base + i) * HD + d0, v);
#pragma unroll
            for (int e = 0; e < 4; e++) a[e] += w * v[e];
        }
#pragma unroll
        for (int e = 0; e < 4; e++) a[e] *= inv;
        store4<QT>(out + (c.out_row * H + h) * (int64_t)HD + d0, a);
    }
}

// ------------------------------------------------------------------ launchers

bool mfma_supported(int32_t dtype, int32_t head_dim, int32_t group) {
    return (dtype == kF16 || dtype == kFP8) && (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
           group >= 1 && group <= 16;
}

template <typename KV, int HD>
static hipError_t launch_mfma_hd(const AttnParams &p, hipStream_t stream) {
    dim3 grid(p.max_parts, p.num_kv_heads, p.rows);
    if (p.block_size == 16)
        hipLaunchKernelGGL((attn_mfma_kernel<KV, HD, true>), grid, dim3(64), 0, stream, p);
    else
        hipLaunchKernelGGL((attn_mfma_kernel<KV, HD, false>), grid, dim3(64), 0, stream, p);
    return hipGetLastError();
}

template <typename KV>
static hipError_t launch_mfma(const AttnParams &p, hipStream_t stream) {
    switch (p.head_dim) {
        case 64: return launch_mfma_hd<KV, 64>(p, stream);
        case 128: return launch_mfma_hd<KV, 128>(p, stream);
        case 256: return launch_mfma_hd<KV, 256>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <typename KV, typename QT>
static hipError_t launch_valu(const AttnParams &p, hipStream_t stream) {
    int lpr = 1;
    while (lpr * 4 < p.head_dim) lpr <<= 1;
    if (lpr > 64 || p.head_dim % 4 != 0) return hipErrorInvalidValue;
    const int nh = p.heads_per_wave;
    dim3 grid(p.max_parts, p.num_heads / nh, p.rows);
    switch (nh) {
        case 1: hipLaunchKernelGGL((attn_valu_kernel<KV, QT, 1>), grid, dim3(64), 0, stream, p, lpr); break;
        case 2: hipLaunchKernelGGL((attn_valu_kernel<KV, QT, 2>), grid, dim3(64), 0, stream, p, lpr); break;
        case 4: hipLaunchKernelGGL((attn_valu_kernel<KV, QT, 4>), grid, dim3(64), 0, stream, p, lpr); break;
        case 8: hipLaunchKernelGGL((attn_valu_kernel<KV, QT, 8>), grid, dim3(64), 0, stream, p, lpr); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_attention(const AttnParams &p, int32_t dtype, bool use_mfma, hipStream_t stream,
                            hipEvent_t after_main) {
    if (p.rows <= 0) return hipSuccess;
    hipError_t e;
    if (use_mfma) {
        e = dtype == kF16 ? launch_mfma<f16>(p, stream) : launch_mfma<uint8_t>(p, stream);
    } else {
        switch (dtype) {
            case kF32: e = launch_valu<float, float>(p, stream); break;
            case kF16: e = launch_valu<f16, f16>(p, stream); break;
            case kFP8: e = launch_valu<uint8_t, f16>(p, stream); break;
            default: return hipErrorInvalidValue;
        }
    }
    if (e != hipSuccess) return e;
    if (after_main) (void)hipEventRecord(after_main, stream);
    if (p.max_parts <= 1) return e;
    dim3 grid(p.num_heads, p.rows);
    if (dtype == kF32)
        hipLaunchKernelGGL((attn_reduce_kernel<float>), grid, dim3(64), 0, stream, p);
    else
        hipLaunchKernelGGL((attn_reduce_kernel<f16>), grid, dim3(64), 0, stream, p);
    return hipGetLastError();
}

}  // namespace pam
