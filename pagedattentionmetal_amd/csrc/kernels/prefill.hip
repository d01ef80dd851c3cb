// prefill.hip - dense chunked prefill on MFMA for gfx950.
//
// Computes rows [q_offset, q_offset + len) of causal (or full) attention for one
// or more sequence chunks whose first q_offset tokens are already in the paged
// pool (kernels.metal:693-917 semantics: scale 1/sqrt(d), GQA head h reads kv
// head h / G, a fixed window start max(0, kv_len - W) for every row).
//
// A workgroup (4 waves) owns 64*NB query rows of one kv head: the (token, head)
// pairs of 64*NB / G consecutive tokens, so the G query heads sharing a kv head
// share every K/V tile.  Each wave owns NB blocks of 16 rows.  Per 32-key tile:
//   * all 256 threads stage K (row-major) and V (transposed, [dim][key]) into
//     LDS; the next tile is fetched into registers while this one is computed;
//   * S^T = K Q^T per 16-row block with v_mfma_f32_16x16x32_f16: K from LDS is
//     the A operand, Q^T stays in registers as B.  The A rows are ordered so that
//     the two 16-key halves leave lane group g holding keys 8g .. 8g+7, which is
//     exactly the B-operand layout of O^T += V^T P^T (16x16x32 again, V^T read
//     from the transposed LDS tile with one 16-byte load per lane);
//   * softmax keeps a per-row reference max that is only raised (and O rescaled)
//     when a tile's max exceeds it by more than 2^8, so most tiles skip the
//     rescale; P is bounded by 2^8 and goes to the MFMA in f16.
#include "kernels.h"
#include "pam_device.h"

namespace pam {

constexpr int kPrefillWaves = 4;
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)

template <int HD, int NB>
__global__ __launch_bounds__(64 * kPrefillWaves, NB >= 4 ? 1 : 2) void prefill_mfma_kernel(AttnParams p) {
    constexpr int KT = 32;            // keys per tile
    constexpr int NC = HD / 32;       // 16x16x32 chunks over d (S)
    constexpr int NO = HD / 16;       // 16-dim output chunks (PV)
    constexpr int KL = HD + 8;        // K row in LDS (halves)
    constexpr int VS = KT + 8;        // V^T row in LDS (halves): 80 bytes, 16-byte aligned
    constexpr int PIECES = HD / 8;    // 16-byte pieces per token row
    constexpr int THREADS = 64 * kPrefillWaves;
    constexpr int PER_THREAD = KT * PIECES / THREADS;
    static_assert(KT * PIECES % THREADS == 0, "tile must split evenly over the threads");
    constexpr int ROWS = 16 * NB * kPrefillWaves;
    __shared__ __attribute__((aligned(16))) f16 k_lds[2][KT * KL];
    __shared__ __attribute__((aligned(16))) f16 v_lds[2][HD * VS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, grp = lane >> 4;
    const int4 ch = p.chunks[blockIdx.z];  // {bt_row, q_offset, len, row_base}
    const int G = p.num_heads / p.num_kv_heads, H = p.num_heads, kvh = blockIdx.y;
    const int tok_per_wg = ROWS / G;
    // heaviest (latest) token blocks first
    const int tok0 = (gridDim.x - 1 - blockIdx.x) * tok_per_wg;
    if (tok0 >= ch.z) return;
    const int32_t *bt = p.block_tables + (int64_t)ch.x * p.bt_stride;
    const int kv_len = ch.y + ch.z;
    const int ws = p.window > 0 ? (kv_len > p.window ? kv_len - p.window : 0) : 0;
    const int tok_end = tok0 + tok_per_wg < ch.z ? tok0 + tok_per_wg : ch.z;
    const int key_end = p.causal ? ch.y + tok_end : kv_len;  // exclusive
    const int t_lo = ws / KT, t_hi = (key_end + KT - 1) / KT;

    // row of lane column n in block b: wave*16*NB + b*16 + n
    int qpos[NB];
    bool row_ok[NB];
    f16x8 qv[NB][NC];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int rr = wave * 16 * NB + b * 16 + n;
        const int tok = tok0 + rr / G, head = rr % G;
        row_ok[b] = tok < tok_end;
        qpos[b] = ch.y + tok;
        const f16 *qp = static_cast<const f16 *>(p.q) +
                        ((int64_t)(ch.w + (row_ok[b] ? tok : tok0)) * H + kvh * G + head) * HD + grp * 8;
#pragma unroll
        for (int c = 0; c < NC; c++) qv[b][c] = *reinterpret_cast<const f16x8 *>(qp + 32 * c);
    }

    // staging map: element e = tid + i*THREADS -> key e % KT, piece e / KT
    const int64_t row_stride = (int64_t)p.num_kv_heads * HD;
    const f16 *kpool = static_cast<const f16 *>(p.k_pool) + (int64_t)kvh * HD;
    const f16 *vpool = static_cast<const f16 *>(p.v_pool) + (int64_t)kvh * HD;
    f16x8 kreg[PER_THREAD], vreg[PER_THREAD];
    auto fetch = [&](int tile) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            const int e = tid + i * THREADS;
            const int key = e % KT, piece = e / KT;
            int j = tile * KT + key;
            // keys outside [ws, kv_len) read key ws instead: finite data whose
            // probability is zero after masking
            j = (j >= ws && j < kv_len) ? j : ws;
            const int64_t off = ((int64_t)bt[j / p.block_size] * p.block_size + j % p.block_size) * row_stride + piece * 8;
            kreg[i] = *reinterpret_cast<const f16x8 *>(kpool + off);
            vreg[i] = *reinterpret_cast<const f16x8 *>(vpool + off);
        }
    };
    auto stage = [&](int s) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            const int e = tid + i * THREADS;
            const int key = e % KT, piece = e / KT;
            *reinterpret_cast<f16x8 *>(&k_lds[s][key * KL + piece * 8]) = kreg[i];
            const f16x8 v = vreg[i];
#pragma unroll
            for (int q = 0; q < 8; q++) v_lds[s][(piece * 8 + q) * VS + key] = v[q];
        }
    };

    float m_use[NB], l_run[NB];
    f32x4 o[NB][NO];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        m_use[b] = -INFINITY;
        l_run[b] = 0.0f;
#pragma unroll
        for (int i = 0; i < NO; i++) o[b][i] = (f32x4)0.0f;
    }

    // A-operand row n of key half h holds key 8*(n/4) + 4h + n%4, so the S^T
    // accumulator of half h leaves lane group g with keys 8g + 4h + r
    const int krow0 = 8 * (n >> 2) + (n & 3);
    if (t_lo < t_hi) {
        fetch(t_lo);
        stage(0);
        __syncthreads();
    }
    for (int tile = t_lo; tile < t_hi; tile++) {
        const int s = (tile - t_lo) & 1;
        // the last tile re-fetches itself: keeps the loads unconditional
        fetch(tile + 1 < t_hi ? tile + 1 : tile);
        const f16 *kt = k_lds[s];
        const f16 *vt = v_lds[s];

        f32x4 sacc[NB][2];
#pragma unroll
        for (int b = 0; b < NB; b++) sacc[b][0] = sacc[b][1] = (f32x4)0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const f16x8 ka = *reinterpret_cast<const f16x8 *>(&kt[(krow0 + 4 * h) * KL + 32 * c + 8 * grp]);
#pragma unroll
                for (int b = 0; b < NB; b++)
                    sacc[b][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qv[b][c], sacc[b][h], 0, 0, 0);
            }

        const int kbase = tile * KT + 8 * grp;  // key of slot 0 of this lane group
        // tiles that need a mask: they start before the window, run past the keys,
        // or reach past the earliest query position of the workgroup
        const bool edge = tile * KT < ws || tile * KT + KT > kv_len || (p.causal && tile * KT + KT - 1 > ch.y + tok0);
        f16x8 pb[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float sv[8];
            float mt = -INFINITY;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int j = kbase + q;
                bool ok = true;
                if (edge) ok = j >= ws && j < kv_len && (!p.causal || j <= qpos[b]);
                sv[q] = ok ? sacc[b][q >> 2][q & 3] * p.scale_log2 : -INFINITY;
                mt = fmaxf(mt, sv[q]);
            }
            mt = fmaxf(mt, shfl_xor(mt, 16));
            mt = fmaxf(mt, shfl_xor(mt, 32));
            const bool need = mt > -INFINITY && (m_use[b] == -INFINITY || mt > m_use[b] + kRescaleLog2);
            if (__any(need)) {  // raise the reference max (uniform branch)
                const float m_new = fmaxf(m_use[b], mt);
                const float corr = m_use[b] == -INFINITY ? 0.0f : exp2f(m_use[b] - m_new);
                l_run[b] *= corr;
#pragma unroll
                for (int i = 0; i < NO; i++) o[b][i] *= corr;
                m_use[b] = m_new;
            }
            const float mref = m_use[b] == -INFINITY ? 0.0f : m_use[b];
            float psum = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float pq = exp2f(sv[q] - mref);
                psum += pq;
                pb[b][q] = (f16)pq;
            }
            l_run[b] += psum;
        }
#pragma unroll
        for (int i = 0; i < NO; i++) {
            const f16x8 va = *reinterpret_cast<const f16x8 *>(&vt[(16 * i + n) * VS + 8 * grp]);
#pragma unroll
            for (int b = 0; b < NB; b++) o[b][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[b], o[b][i], 0, 0, 0);
        }
        stage(s ^ 1);
        __syncthreads();
    }

    // finish: l summed over the lane groups, O / l, rows in range only
    f16 *out = static_cast<f16 *>(p.out);
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float l = l_run[b] + shfl_xor(l_run[b], 16);
        l += shfl_xor(l, 32);
        if (!row_ok[b]) continue;
        const int rr = wave * 16 * NB + b * 16 + n;
        const int tok = tok0 + rr / G, head = rr % G;
        // no key in range (window past the row): 0/0, as the reference's m/l bookkeeping gives
        const float inv = 1.0f / l;
        f16 *op = out + ((int64_t)(ch.w + tok) * H + kvh * G + head) * HD + 4 * grp;
#pragma unroll
        for (int i = 0; i < NO; i++) {
            f16x4 v;
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = (f16)(o[b][i][q] * inv);
            *reinterpret_cast<f16x4 *>(op + 16 * i) = v;
        }
    }
}

constexpr int kPrefillNB = 2;

bool prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group) {
    return dtype == kF16 && head_dim == 128 && group >= 1 && group <= 16 && (16 % group) == 0;
}

hipError_t launch_prefill_mfma(const AttnParams &p, hipStream_t stream) {
    if (p.chunks == nullptr || p.num_chunks <= 0 || p.max_chunk_len <= 0) return hipErrorInvalidValue;
    const int G = p.num_heads / p.num_kv_heads;
    if (!prefill_mfma_supported(kF16, p.head_dim, G)) return hipErrorInvalidValue;
    const int tok_per_wg = 16 * kPrefillNB * kPrefillWaves / G;
    dim3 grid((p.max_chunk_len + tok_per_wg - 1) / tok_per_wg, p.num_kv_heads, p.num_chunks);
    hipLaunchKernelGGL((prefill_mfma_kernel<128, kPrefillNB>), grid, dim3(64 * kPrefillWaves), 0, stream, p);
    return hipGetLastError();
}

}  // namespace pam
