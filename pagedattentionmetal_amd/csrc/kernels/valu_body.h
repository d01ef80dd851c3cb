// valu_body.h - device bodies of the VALU row kernel and the split-context
// reduce (gfx950).  Included by attention.hip (the library's kernels) and by
// the code-object entries (module_entry.hip), which wrap the same bodies.
#pragma once
#include "attention_body.h"

namespace pam {

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

constexpr int kValuBatch = 8;  // steps of the VALU kernel whose loads are in flight together
// LDS of the workgroup form: every partition's (O, m, l) for NH heads at the
// largest head size the VALU kernel takes (256: 64 lanes of 4 dims)
template <int NH>
constexpr int kValuWgLds = kValuWgMaxParts * NH * (256 + 2);

// lanes_per_row: power of two >= head_dim / 4 (<= 64); heads NH share one kv head.
// WG: the workgroup is one (row, head group) and wave w its partition w; the
// partitions merge in wg_lds (kValuWgLds<NH> floats: max_parts * NH *
// (head_dim + 2) of them are used).
template <typename KV, typename QT, int NH, bool WG = false>
__device__ __forceinline__ void valu_body(const AttnParams &p, int lanes_per_row, float *wg_lds = nullptr) {
    const int lane = WG ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
    const int part = WG ? (int)(threadIdx.x >> 6) : (int)blockIdx.x, hg = blockIdx.y, r = blockIdx.z;
    const int HD = p.head_dim, H = p.num_heads;
    const int G = H / p.num_kv_heads;
    const int h0 = hg * NH;
    const int kvh = h0 / G;
    const int LPR = lanes_per_row, TPI = 64 / lanes_per_row;
    const int sub = lane / LPR;
    constexpr int UB = kValuBatch;
    // A decode row without a window starts its keys at token 0, so the first
    // batch's block-table entries are known before the row's length: they are
    // requested beside it.  The index is clamped into the row's max_num_blocks
    // entries; only entries of tokens below the length are used, and those lie
    // below the clamp.
    const bool early_bt = p.mode == kRowDecode && p.window <= 0 && p.max_num_blocks > 0;
    int32_t bt_first[UB];
    if (early_bt) {
        const int32_t *bt_row = p.block_tables + (int64_t)r * p.bt_stride;
#pragma unroll
        for (int u = 0; u < UB; u++) {
            const int idx = (part * p.part_tokens + u * TPI + sub) / p.block_size;
            bt_first[u] = bt_row[idx < p.max_num_blocks ? idx : p.max_num_blocks - 1];
        }
    }
    const RowCtx c = row_ctx(p, r);
    const PartRange pr = part_range(c, part, p.part_tokens);
    // a wave past the row's partitions has no tiles; in a workgroup it stays
    // for the merge's barrier when there is one
    if (part >= (pr.nparts > 1 ? pr.nparts : 1) && (!WG || pr.nparts <= 1)) return;

    const int d0 = (lane % LPR) * 4;
    const bool dim_ok = d0 < HD;
    QT *out = static_cast<QT *>(p.out);
    if (pr.nparts == 0) {
        if (sub == 0 && dim_ok && (!WG || part == 0)) {
            float nanv[4] = {__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
            for (int hh = 0; hh < NH; hh++) store4<QT>(out + (c.out_row * H + h0 + hh) * (int64_t)HD + d0, nanv);
        }
        return;
    }

    float q[NH][4];
#pragma unroll
    for (int hh = 0; hh < NH; hh++) {
        if (dim_ok)
            load4<QT>(static_cast<const QT *>(p.q) + ((int64_t)c.out_row * H + h0 + hh) * HD + d0, q[hh]);
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

    // Tokens go in batches of kValuBatch steps of TPI tokens: the block-table
    // entries of a batch are requested together, then its K/V slices, so a batch
    // waits on two memory latencies; one online-softmax update covers the batch.
    // one batch at token j0; bte: the block-table entries of its steps
    auto batch = [&](const int j0, const int32_t (&bte)[UB]) {
        bool ok[UB];
        int64_t phys[UB];
#pragma unroll
        for (int u = 0; u < UB; u++) {
            const int j = j0 + u * TPI + sub;
            ok[u] = j >= c.k_lo && j < c.k_hi && j < pr.t_end * 16;
            phys[u] = ok[u] ? (int64_t)bte[u] : 0;
        }
        float kv[UB][4], vv[UB][4];
#pragma unroll
        for (int u = 0; u < UB; u++) {
#pragma unroll
            for (int e = 0; e < 4; e++) kv[u][e] = vv[u][e] = 0.0f;
            if (ok[u] && dim_ok) {
                const int j = j0 + u * TPI + sub;
                const int64_t off = (phys[u] * bs + j % bs) * row_stride + (int64_t)kvh * HD + d0;
                f16 ks = (f16)1.0f, vs = (f16)1.0f;
                if constexpr (sizeof(KV) == 1) {
                    ks = bits_to_f16(p.k_scale[phys[u]]);
                    vs = bits_to_f16(p.v_scale[phys[u]]);
                }
                load_kv4<KV>(kpool + off, ks, kv[u]);
                load_kv4<KV>(vpool + off, vs, vv[u]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            float sv[UB];
            float mt = -INFINITY;
#pragma unroll
            for (int u = 0; u < UB; u++) {
                float sd = q[hh][0] * kv[u][0] + q[hh][1] * kv[u][1] + q[hh][2] * kv[u][2] + q[hh][3] * kv[u][3];
                sd = wave_sum_xor(sd, 1, LPR);
                sv[u] = ok[u] ? sd * p.scale_log2 : -INFINITY;
                mt = fmaxf(mt, sv[u]);
            }
            mt = wave_max_xor(mt, LPR, 64);
            const float m_new = fmaxf(m[hh], mt);
            // a batch whose tokens all fall outside the key range keeps the state
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float corr = exp2f(m[hh] - m_use);
            float ls = l[hh] * corr;
            float a4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) a4[e] = acc[hh][e] * corr;
#pragma unroll
            for (int u = 0; u < UB; u++) {
                const float pj = exp2f(sv[u] - m_use);
                ls += pj;
#pragma unroll
                for (int e = 0; e < 4; e++) a4[e] += pj * vv[u][e];
            }
            l[hh] = ls;
            m[hh] = m_new;
#pragma unroll
            for (int e = 0; e < 4; e++) acc[hh][e] = a4[e];
        }
    };
    int j0 = pr.t_begin * 16;
    if (early_bt && j0 < pr.t_end * 16) {
        batch(j0, bt_first);
        j0 += UB * TPI;
    }
    for (; j0 < pr.t_end * 16; j0 += UB * TPI) {
        int32_t bte[UB];
#pragma unroll
        for (int u = 0; u < UB; u++) {
            const int j = j0 + u * TPI + sub;
            bte[u] = j >= c.k_lo && j < c.k_hi && j < pr.t_end * 16 ? c.bt[j / bs] : 0;
        }
        batch(j0, bte);
    }

#pragma unroll
    for (int hh = 0; hh < NH; hh++) {
        l[hh] = wave_sum_xor(l[hh], LPR, 64);
#pragma unroll
        for (int e = 0; e < 4; e++) acc[hh][e] = wave_sum_xor(acc[hh][e], LPR, 64);
    }
    if constexpr (WG) {
        if (pr.nparts > 1) {
            // each wave's partial into LDS, then wave 0 folds the partitions in
            // order, as the global merge below does (the same bits)
            const int stride = NH * (HD + 2);
            float *mine = wg_lds + part * stride;
            if (part < pr.nparts && sub == 0 && dim_ok) {
#pragma unroll
                for (int hh = 0; hh < NH; hh++) {
                    *reinterpret_cast<float4 *>(mine + hh * HD + d0) = make_float4(acc[hh][0], acc[hh][1], acc[hh][2], acc[hh][3]);
                    if (d0 == 0) {
                        mine[NH * HD + 2 * hh] = m[hh];
                        mine[NH * HD + 2 * hh + 1] = l[hh];
                    }
                }
            }
            __syncthreads();
            if (part == 0 && sub == 0 && dim_ok) {
#pragma unroll
                for (int hh = 0; hh < NH; hh++) {
                    float M = -INFINITY;
                    for (int pt = 0; pt < pr.nparts; pt++) M = fmaxf(M, wg_lds[pt * stride + NH * HD + 2 * hh]);
                    float den = 0.0f, a[4] = {0.f, 0.f, 0.f, 0.f};
                    for (int pt = 0; pt < pr.nparts; pt++) {
                        const float *src = wg_lds + pt * stride;
                        const float mp = src[NH * HD + 2 * hh], lp = src[NH * HD + 2 * hh + 1];
                        const float4 v = *reinterpret_cast<const float4 *>(src + hh * HD + d0);
                        const float w = mp == -INFINITY ? 0.0f : exp2f(mp - M);
                        den += w * lp;
                        a[0] += w * v.x, a[1] += w * v.y, a[2] += w * v.z, a[3] += w * v.w;
                    }
                    const float inv = 1.0f / den;
#pragma unroll
                    for (int e = 0; e < 4; e++) a[e] *= inv;
                    store4<QT>(out + (c.out_row * H + h0 + hh) * (int64_t)HD + d0, a);
                }
            }
            return;
        }
    }
    if (sub != 0 || !dim_ok) return;
    if (pr.nparts == 1) {
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            const float inv = 1.0f / l[hh];
            float v[4] = {acc[hh][0] * inv, acc[hh][1] * inv, acc[hh][2] * inv, acc[hh][3] * inv};
            store4<QT>(out + (c.out_row * H + h0 + hh) * (int64_t)HD + d0, v);
        }
    } else if (p.seg_count == nullptr) {  // partials for attn_reduce_kernel
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            const int64_t slot = ((int64_t)r * H + h0 + hh) * p.max_parts + part;
            store4<float>(p.part_o + slot * HD + d0, acc[hh]);
            if (d0 == 0) {
                p.part_ml[slot * 2 + 0] = m[hh];
                p.part_ml[slot * 2 + 1] = l[hh];
            }
        }
    } else {
        // Merged in the kernel (no reduce launch): the partial is published with
        // write-through stores and counted on the (row, head group) counter; the
        // wave that completes the count folds all partitions in order, as
        // attn_reduce_kernel does, and writes the rows.  Offsets are bytes from
        // part_o (< 2 GiB).
        const __amdgpu_buffer_rsrc_t prs = part_rsrc(p);
        const int ml_off = (int)((const char *)p.part_ml - (const char *)p.part_o);
        auto slot_of = [&](int hh, int pt) { return ((int64_t)r * H + h0 + hh) * p.max_parts + pt; };
#pragma unroll
        for (int hh = 0; hh < NH; hh++) {
            const int64_t slot = slot_of(hh, part);
            const f32x4 v = {acc[hh][0], acc[hh][1], acc[hh][2], acc[hh][3]};
            __builtin_amdgcn_raw_buffer_store_b128(v, prs, (int)((slot * HD + d0) * 4), 0, kSc1);
            if (d0 == 0) {
                const f32x2 ml = {m[hh], l[hh]};
                __builtin_amdgcn_raw_buffer_store_b64(ml, prs, ml_off + (int)(slot * 8), 0, kSc1);
            }
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        uint32_t before = 0;
        if (lane == 0)  // lane 0 has sub 0 and d0 0: it is active here
            before = arrive_count(p.seg_count + (int64_t)r * (H / NH) + hg, p.epoch);
        before = __builtin_amdgcn_readfirstlane(before);
        if (before != (uint32_t)(pr.nparts - 1)) return;
        // the first kMergeCache partitions' partials are loaded with the maxima,
        // so a short row's merge waits on one memory latency, not two
        constexpr int kMergeCache = 16;
        for (int hh = 0; hh < NH; hh++) {
            float M = -INFINITY;
            f32x2 mlc[kMergeCache];
            f32x4 vc[kMergeCache];
#pragma unroll
            for (int pt = 0; pt < kMergeCache; pt++) {
                if (pt < pr.nparts) {
                    const int64_t slot = slot_of(hh, pt);
                    mlc[pt] = __builtin_amdgcn_raw_buffer_load_b64(prs, ml_off + (int)(slot * 8), 0, kSc1);
                    vc[pt] = __builtin_amdgcn_raw_buffer_load_b128(prs, (int)((slot * HD + d0) * 4), 0, kSc1);
                }
            }
#pragma unroll
            for (int pt = 0; pt < kMergeCache; pt++)
                if (pt < pr.nparts) M = fmaxf(M, mlc[pt][0]);
            for (int pt = kMergeCache; pt < pr.nparts; pt++) {
                const f32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(prs, ml_off + (int)(slot_of(hh, pt) * 8), 0, kSc1);
                M = fmaxf(M, ml[0]);
            }
            float den = 0.0f, a[4] = {0.f, 0.f, 0.f, 0.f};
            auto fold = [&](const f32x2 ml, const f32x4 v) {
                const float w = ml[0] == -INFINITY ? 0.0f : exp2f(ml[0] - M);
                den += w * ml[1];
#pragma unroll
                for (int e = 0; e < 4; e++) a[e] += w * v[e];
            };
#pragma unroll
            for (int pt = 0; pt < kMergeCache; pt++)
                if (pt < pr.nparts) fold(mlc[pt], vc[pt]);
            for (int pt = kMergeCache; pt < pr.nparts; pt++) {
                const int64_t slot = slot_of(hh, pt);
                fold(__builtin_amdgcn_raw_buffer_load_b64(prs, ml_off + (int)(slot * 8), 0, kSc1),
                     __builtin_amdgcn_raw_buffer_load_b128(prs, (int)((slot * HD + d0) * 4), 0, kSc1));
            }
            const float inv = 1.0f / den;
#pragma unroll
            for (int e = 0; e < 4; e++) a[e] *= inv;
            store4<QT>(out + (c.out_row * H + h0 + hh) * (int64_t)HD + d0, a);
        }
    }
}

// ------------------------------------------------------------------ split-context reduce
// O = sum_p 2^{m_p - M} O_p / sum_p 2^{m_p - M} l_p over the row's partitions.
// Split-context reduce: one wave per (row, head), four per workgroup.  The
// partials' maxima and sums are reduced across lanes (one partition per lane),
// then lane groups of HD/4 lanes each accumulate a share of the partitions'
// weighted outputs and the groups are summed with shuffles.
template <typename QT>
__device__ __forceinline__ void reduce_body(const AttnParams &p) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.y, h = blockIdx.x * 4 + wave;
    if (h >= p.num_heads) return;
    const RowCtx c = row_ctx(p, r);
    const PartRange pr = part_range(c, 0, p.part_tokens);
    const int np = pr.nparts;
    if (np <= 1) return;
    const int HD = p.head_dim, H = p.num_heads;
    const int64_t base = ((int64_t)r * H + h) * p.max_parts;
    // one pass over (m, l): each lane folds its partitions, then the lanes merge
    float Ml = -INFINITY, dl = 0.0f;
    for (int i = lane; i < np; i += 64) {
        const float mi = p.part_ml[(base + i) * 2], li = p.part_ml[(base + i) * 2 + 1];
        const float Mn = fmaxf(Ml, mi);
        if (Mn != -INFINITY) dl = dl * exp2f(Ml - Mn) + li * exp2f(mi - Mn);
        Ml = Mn;
    }
    const float M = wave_max_xor(Ml, 1, 64);
    float den = Ml == -INFINITY ? 0.0f : dl * exp2f(Ml - M);
    den = wave_sum_xor(den, 1, 64);
    // lanes per group: HD/4 rounded up to a power of two (<= 64)
    int lpg = 1;
    while (lpg * 4 < HD) lpg <<= 1;
    const int ng = 64 / lpg, g = lane / lpg, d0 = (lane % lpg) * 4;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    if (d0 < HD) {
#pragma unroll 4
        for (int i = g; i < np; i += ng) {
            const float w = exp2f(p.part_ml[(base + i) * 2] - M);
            float v[4];
            load4<float>(p.part_o + (base + i) * HD + d0, v);
#pragma unroll
            for (int e = 0; e < 4; e++) a[e] += w * v[e];
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) a[e] = wave_sum_xor(a[e], lpg, 64);
    if (g == 0 && d0 < HD) {
        const float inv = 1.0f / den;
#pragma unroll
        for (int e = 0; e < 4; e++) a[e] *= inv;
        store4<QT>(static_cast<QT *>(p.out) + (c.out_row * H + h) * (int64_t)HD + d0, a);
    }
}

}  // namespace pam
