// prefill.hip - dense chunked prefill on MFMA for gfx950.
//
// Computes rows [q_offset, q_offset + len) of causal (or full) attention for one
// or more sequence chunks whose first q_offset tokens are already in the paged
// pool (kernels.metal:693-917 semantics: scale 1/sqrt(d), GQA head h reads kv
// head h / G, a fixed window start max(0, kv_len - W) for every row).
//
// A workgroup (4 waves) owns 64*NB query rows of one kv head: the (token, head)
// pairs of 64*NB / G consecutive tokens, so the G query heads sharing a kv head
// share every K/V tile.  Each wave owns NB blocks of 16 rows.  Per KT-key tile:
//   * all 256 threads stage K (row-major, 16-byte pieces XOR-swizzled) and V
//     (transposed, [dim][key]) into LDS; the next tile is fetched into
//     registers while this one is computed;
//   * S^T = K Q^T per 16-row block and 16-key quarter with
//     v_mfma_f32_16x16x32_f16: K from LDS is the A operand, Q^T stays in
//     registers as B.  The A rows are ordered so that, within every 32 keys, lane
//     group g ends up holding keys 8g .. 8g+7, which is exactly the B-operand
//     layout of O^T += V^T P^T (16x16x32 again, V^T read from the transposed LDS
//     tile with one 16-byte load per lane);
//   * softmax keeps a per-row reference max that is only raised (and O rescaled)
//     when some score exceeds it by more than 2^8, so P is bounded by 2^8 and
//     goes to the MFMA in f16; the common case needs no cross-lane reduction;
//   * tiles wholly inside [window start, causal limit) run a mask-free body.
#include "kernels.h"
#include "pam_device.h"

namespace pam {

constexpr int kPrefillWaves = 4;
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)
constexpr int kBtCache = 2048;        // block-table entries a workgroup keeps in LDS

template <int HD, int NB, int KT>
__global__ __launch_bounds__(64 * kPrefillWaves, NB >= 4 ? 1 : 2) void prefill_mfma_kernel(AttnParams p) {
    constexpr int NC = HD / 32;       // 16x16x32 chunks over d (S)
    constexpr int NO = HD / 16;       // 16-dim output chunks (PV)
    constexpr int SQ = KT / 16;       // 16-key quarters per tile (S)
    constexpr int PH = KT / 32;       // 32-key halves per tile (PV)
    constexpr int KL = HD + 8;        // K row in LDS (halves): 17 16-byte units for d = 128
    constexpr int VS = KT + 8;        // V^T row in LDS (halves): an odd number of 16-byte units
    constexpr int PIECES = HD / 8;    // 16-byte pieces per token row
    constexpr int THREADS = 64 * kPrefillWaves;
    constexpr int PER_THREAD = KT * PIECES / THREADS;
    static_assert(KT * PIECES % THREADS == 0, "tile must split evenly over the threads");
    static_assert(KT == 32 || KT == 64, "tile of 32 or 64 keys");
    constexpr int ROWS = 16 * NB * kPrefillWaves;
    __shared__ __attribute__((aligned(16))) f16 k_lds[2][KT * KL];
    __shared__ __attribute__((aligned(16))) f16 v_lds[2][HD * VS];
    __shared__ int32_t bt_lds[kBtCache];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, grp = lane >> 4;
    const int4 ch = p.chunks[blockIdx.z];  // {bt_row, q_offset, len, row_base}
    const int G = p.num_heads / p.num_kv_heads, H = p.num_heads, kvh = blockIdx.y;
    const int tok_per_wg = ROWS / G;
    // heaviest (latest) token blocks first
    const int tok0 = (gridDim.x - 1 - blockIdx.x) * tok_per_wg;
    if (tok0 >= ch.z) return;
    const int32_t *bt = p.block_tables + (int64_t)ch.x * p.bt_stride;
    const int bsh = __builtin_ctz(p.block_size), bsm = p.block_size - 1;  // block_size is a power of two
    const int kv_len = ch.y + ch.z;
    const int ws = p.window > 0 ? (kv_len > p.window ? kv_len - p.window : 0) : 0;
    const int tok_end = tok0 + tok_per_wg < ch.z ? tok0 + tok_per_wg : ch.z;
    const int key_end = p.causal ? ch.y + tok_end : kv_len;  // exclusive
    const int t_lo = ws / KT, t_hi = (key_end + KT - 1) / KT;
    // tiles [full_lo, full_hi) need no mask for any row of the workgroup
    const int full_lo = (ws + KT - 1) / KT;
    int full_hi = kv_len / KT;
    if (p.causal) full_hi = min(full_hi, (ch.y + tok0 + 1) / KT);

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
    // K piece swizzle: rows 16..31 of every 32 use piece ^ 4, which spreads the
    // 16 rows one S operand load touches over all 64 banks
    auto kswz = [](int row, int piece) { return piece ^ (((row >> 4) & 1) << 2); };
    f16x8 kreg[PER_THREAD], vreg[PER_THREAD];
    // the thread's key within a tile is the same for all its pieces (THREADS % KT == 0)
    static_assert(THREADS % KT == 0, "one key per thread per tile");
    const int my_key = tid % KT, my_piece = tid / KT;
    int blk0 = 0;  // first block of the block-table segment held in bt_lds
    auto fetch = [&](int tile) {
        int j = tile * KT + my_key;
        // keys outside [ws, kv_len) read the nearest key inside instead: finite
        // data whose probability is zero after masking (and a block-table entry
        // of the current segment)
        j = j < ws ? ws : (j >= kv_len ? kv_len - 1 : j);
        const uint32_t slot = ((uint32_t)bt_lds[(j >> bsh) - blk0] << bsh) | (uint32_t)(j & bsm);
        const int64_t off = (int64_t)slot * row_stride + my_piece * 8;
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            kreg[i] = *reinterpret_cast<const f16x8 *>(kpool + off + i * (THREADS / KT) * 8);
            vreg[i] = *reinterpret_cast<const f16x8 *>(vpool + off + i * (THREADS / KT) * 8);
        }
    };
    auto stage = [&](int s) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            const int e = tid + i * THREADS;
            const int key = e % KT, piece = e / KT;
            *reinterpret_cast<f16x8 *>(&k_lds[s][key * KL + kswz(key, piece) * 8]) = kreg[i];
#pragma unroll
            for (int q = 0; q < 8; q++) v_lds[s][(piece * 8 + q) * VS + key] = vreg[i][q];
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

    // A-operand row n of quarter (32-key half hh, sub-half h) holds key
    // 32hh + 8*(n/4) + 4h + n%4, so lane group g of that accumulator holds keys
    // 32hh + 8g + 4h + r: P slot 4h + r of half hh
    const int krow0 = 8 * (n >> 2) + (n & 3);
    const float sl2 = p.scale_log2;

    auto body = [&](int tile, int s, auto masked) {
        constexpr bool MASK = decltype(masked)::value;
        const f16 *kt = k_lds[s];
        const f16 *vt = v_lds[s];
        f32x4 sacc[NB][SQ];
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int q4 = 0; q4 < SQ; q4++) sacc[b][q4] = (f32x4)0.0f;
#pragma unroll
        for (int q4 = 0; q4 < SQ; q4++) {
            const int row = 32 * (q4 >> 1) + 4 * (q4 & 1) + krow0;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const f16x8 ka = *reinterpret_cast<const f16x8 *>(&kt[row * KL + kswz(row, 4 * c + grp) * 8]);
#pragma unroll
                for (int b = 0; b < NB; b++)
                    sacc[b][q4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qv[b][c], sacc[b][q4], 0, 0, 0);
            }
        }

        f16x8 pb[NB][PH];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if constexpr (MASK) {
#pragma unroll
                for (int q4 = 0; q4 < SQ; q4++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int j = tile * KT + 32 * (q4 >> 1) + 8 * grp + 4 * (q4 & 1) + r;
                        const bool ok = j >= ws && j < kv_len && (!p.causal || j <= qpos[b]);
                        sacc[b][q4][r] = ok ? sacc[b][q4][r] : -INFINITY;
                    }
            }
            float lmax = sacc[b][0][0];
#pragma unroll
            for (int q4 = 0; q4 < SQ; q4++)
#pragma unroll
                for (int r = 0; r < 4; r++) lmax = fmaxf(lmax, sacc[b][q4][r]);
            // only when a score passes the reference by 2^8 (or there is none yet)
            // is the row max formed and the reference raised
            if (__any(lmax * sl2 > m_use[b] + kRescaleLog2)) {
                float mt = lmax * sl2;
                mt = fmaxf(mt, shfl_xor(mt, 16));
                mt = fmaxf(mt, shfl_xor(mt, 32));
                const float m_new = fmaxf(m_use[b], mt);
                const float corr = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_use[b] - m_new);
                l_run[b] *= corr;
#pragma unroll
                for (int i = 0; i < NO; i++) o[b][i] *= corr;
                m_use[b] = m_new;
            }
            const float mref = MASK ? (m_use[b] == -INFINITY ? 0.0f : m_use[b]) : m_use[b];
            float psum = 0.0f;
#pragma unroll
            for (int q4 = 0; q4 < SQ; q4++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float pq = __builtin_amdgcn_exp2f(fmaf(sacc[b][q4][r], sl2, -mref));
                    psum += pq;
                    pb[b][q4 >> 1][4 * (q4 & 1) + r] = (f16)pq;
                }
            l_run[b] += psum;
        }
#pragma unroll
        for (int i = 0; i < NO; i++)
#pragma unroll
            for (int hh = 0; hh < PH; hh++) {
                const f16x8 va = *reinterpret_cast<const f16x8 *>(&vt[(16 * i + n) * VS + 32 * hh + 8 * grp]);
#pragma unroll
                for (int b = 0; b < NB; b++)
                    o[b][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[b][hh], o[b][i], 0, 0, 0);
            }
    };

    // tiles run in segments whose block-table entries fit in bt_lds (one segment
    // covers kBtCache * block_size keys, so long contexts only)
    const int seg_tiles = ((kBtCache - 1) << bsh) / KT;
    for (int seg = t_lo; seg < t_hi; seg += seg_tiles) {
        const int seg_end = min(t_hi, seg + seg_tiles);
        blk0 = (seg * KT) >> bsh;
        const int nblk = (((min(seg_end * KT, kv_len) - 1) >> bsh) - blk0) + 1;
        __syncthreads();  // previous segment done with bt_lds and the stages
        for (int i = tid; i < nblk; i += THREADS) bt_lds[i] = bt[blk0 + i];
        __syncthreads();
        fetch(seg);
        stage(0);
        __syncthreads();
        for (int tile = seg; tile < seg_end; tile++) {
            const int s = (tile - seg) & 1;
            // the last tile re-fetches itself: keeps the loads unconditional
            fetch(tile + 1 < seg_end ? tile + 1 : tile);
            if (tile >= full_lo && tile < full_hi)
                body(tile, s, std::false_type{});
            else
                body(tile, s, std::true_type{});
            stage(s ^ 1);
            __syncthreads();
        }
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
constexpr int kPrefillKT = 32;

bool prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size) {
    return dtype == kF16 && head_dim == 128 && group >= 1 && group <= 16 && (16 % group) == 0 && block_size > 0 &&
           (block_size & (block_size - 1)) == 0;
}

hipError_t launch_prefill_mfma(const AttnParams &p, hipStream_t stream) {
    if (p.chunks == nullptr || p.num_chunks <= 0 || p.max_chunk_len <= 0) return hipErrorInvalidValue;
    const int G = p.num_heads / p.num_kv_heads;
    if (!prefill_mfma_supported(kF16, p.head_dim, G, p.block_size)) return hipErrorInvalidValue;
    const int tok_per_wg = 16 * kPrefillNB * kPrefillWaves / G;
    dim3 grid((p.max_chunk_len + tok_per_wg - 1) / tok_per_wg, p.num_kv_heads, p.num_chunks);
    hipLaunchKernelGGL((prefill_mfma_kernel<128, kPrefillNB, kPrefillKT>), grid, dim3(64 * kPrefillWaves), 0, stream,
                       p);
    return hipGetLastError();
}

}  // namespace pam
