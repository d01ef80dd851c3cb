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
constexpr int kPrefillKT = 32;        // keys per tile
constexpr int kPrefillBufs = 3;       // LDS ring: tile t computed, t+1 scored, t+2 being written
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)
constexpr int kBtCache = 2048;        // block-table entries a workgroup keeps in LDS

typedef __fp16 fp16x4_raw __attribute__((__vector_size__(4 * sizeof(__fp16))));

// ds_read_b64_tr_b16: the 16 lanes of a group each address 4 consecutive halves
// a[i][0..3]; lane o receives a[4j + o/4][o%4] for j = 0..3.
__device__ __forceinline__ f16x4 lds_read_tr16(const f16 *p) {
    const fp16x4_raw v =
        __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) fp16x4_raw *)(p));
    return __builtin_bit_cast(f16x4, v);
}

// LDS tiles (layouts chosen by measuring SQ_LDS_BANK_CONFLICT on gfx950).
// K: unpadded rows of 128 halves, 16-byte piece p of row r stored at
// p ^ (r%4 + 4*((r/8)%4)); the S operand loads (rows 4h + n%4 + 8*(n/4)) are
// then conflict free, and each lane reads chunk c at one of four bases.
// V: rows of VL = HD + 16 halves, piece p of row r at p ^ 8*bit3(r), which
// keeps the transposed loads (rows 8g + 4r' + i/4) conflict free with two bases.
constexpr int kPrefillKL = 128;
constexpr int kPrefillVL = 128 + 16;
__device__ __forceinline__ int k_lds_at(int key, int piece) {
    return key * kPrefillKL + ((piece ^ ((key & 3) + 4 * ((key >> 3) & 3))) << 3);
}
__device__ __forceinline__ int v_lds_at(int key, int piece) {
    return key * kPrefillVL + ((piece ^ (((key >> 3) & 1) << 3)) << 3);
}

// three-way maximum (v_maximum3_f32); scores are never NaN
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

template <int HD, int NB>
__global__ __launch_bounds__(64 * kPrefillWaves, 2) void prefill_mfma_kernel(AttnParams p) {
    static_assert(HD == 128, "the LDS swizzle assumes 16 pieces per row");
    constexpr int KT = kPrefillKT;
    constexpr int NC = HD / 32;       // 16x16x32 chunks over d (S)
    constexpr int NO = HD / 16;       // 16-dim output chunks (PV)
    constexpr int SQ = KT / 16;       // 16-key quarters per tile (S)
    constexpr int PIECES = HD / 8;    // 16-byte pieces per token row
    constexpr int THREADS = 64 * kPrefillWaves;
    constexpr int PER_THREAD = KT * PIECES / THREADS;  // 16-byte pieces per thread per pool
    constexpr int ROWS = 16 * NB * kPrefillWaves;
    static_assert(KT == 32 && THREADS % PIECES == 0 && KT * PIECES % THREADS == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) f16 k_lds[kPrefillBufs][KT * kPrefillKL];
    __shared__ __attribute__((aligned(16))) f16 v_lds[kPrefillBufs][KT * kPrefillVL];
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

    // staging map: 8 threads per key, thread piece p and p + 8 of it; the two
    // keys of every 16-lane group are 8 apart, which keeps the LDS writes of a
    // group on distinct bank groups
    static_assert(PER_THREAD == 2 && THREADS / 8 == KT, "8 threads per key, two pieces each");
    const int kk = tid >> 3, my_piece = tid & 7;
    const int my_key = (kk & 16) | ((kk & 1) << 3) | ((kk >> 1) & 7);
    const uint32_t row_stride = (uint32_t)(p.num_kv_heads * HD);  // halves per pool row (< 2^32)
    const f16 *kpool = static_cast<const f16 *>(p.k_pool) + (int64_t)kvh * HD + my_piece * 8;
    const f16 *vpool = static_cast<const f16 *>(p.v_pool) + (int64_t)kvh * HD + my_piece * 8;
    f16x8 kreg[2], vreg[2];
    int blk0 = 0;  // first block of the block-table segment held in bt_lds
    auto fetch = [&](int tile) {
        int j = tile * KT + my_key;
        // keys outside [ws, kv_len) read the nearest key inside instead: finite
        // data whose probability is zero after masking (and a block-table entry
        // of the current segment)
        j = j < ws ? ws : (j >= kv_len ? kv_len - 1 : j);
        const uint32_t slot = ((uint32_t)bt_lds[(j >> bsh) - blk0] << bsh) | (uint32_t)(j & bsm);
        const uint64_t off = (uint64_t)slot * row_stride;
        kreg[0] = *reinterpret_cast<const f16x8 *>(kpool + off);
        kreg[1] = *reinterpret_cast<const f16x8 *>(kpool + off + 64);
        vreg[0] = *reinterpret_cast<const f16x8 *>(vpool + off);
        vreg[1] = *reinterpret_cast<const f16x8 *>(vpool + off + 64);
    };
    const int k_st0 = k_lds_at(my_key, my_piece), k_st1 = k_lds_at(my_key, my_piece + 8);
    const int v_st0 = v_lds_at(my_key, my_piece), v_st1 = v_lds_at(my_key, my_piece + 8);
    auto stage = [&](int buf) {
        *reinterpret_cast<f16x8 *>(&k_lds[buf][k_st0]) = kreg[0];
        *reinterpret_cast<f16x8 *>(&k_lds[buf][k_st1]) = kreg[1];
        *reinterpret_cast<f16x8 *>(&v_lds[buf][v_st0]) = vreg[0];
        *reinterpret_cast<f16x8 *>(&v_lds[buf][v_st1]) = vreg[1];
    };

    // S^T for one tile: A-operand row n of quarter h holds key 8*(n/4) + 4h + n%4,
    // so lane group g of that accumulator holds keys 8g + 4h + r: P slot 4h + r
    const int krow0 = 8 * (n >> 2) + (n & 3);
    // piece 4c + g of row krow0 + 4h sits at k_base[c] + 4h rows
    int k_base[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) k_base[c] = k_lds_at(krow0, 4 * c + grp);
    auto score = [&](int buf, f32x4 (&sacc)[NB][SQ]) {
        const f16 *kt = k_lds[buf];
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int q4 = 0; q4 < SQ; q4++) sacc[b][q4] = (f32x4)0.0f;
#pragma unroll
        for (int q4 = 0; q4 < SQ; q4++) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int at = k_base[c] + 4 * q4 * kPrefillKL;
                const f16x8 ka = *reinterpret_cast<const f16x8 *>(&kt[at]);
#pragma unroll
                for (int b = 0; b < NB; b++)
                    sacc[b][q4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qv[b][c], sacc[b][q4], 0, 0, 0);
            }
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
    const float sl2 = p.scale_log2;
    // transposed V loads: lane (n, g) addresses row 8g + 4r + n/4, dims
    // 16i + 4*(n%4), i.e. piece 2i + (n%4)/2 at half offset 4*(n%2); pieces of
    // i < 4 sit at v_base_lo + 16i, the others at v_base_hi + 16i (+ 4r rows)
    const int vb3 = grp & 1;
    const int v_row0 = (8 * grp + (n >> 2)) * kPrefillVL + 8 * ((n & 3) >> 1) + 4 * (n & 1);
    const int v_base_lo = v_row0 + 64 * vb3;
    const int v_base_hi = v_row0 - 64 * vb3;
    const f16x2 ones = {(f16)1.0f, (f16)1.0f};

    f32x4 sacc[NB][SQ], snext[NB][SQ];
    // tiles run in segments whose block-table entries fit in bt_lds (one segment
    // covers kBtCache * block_size keys, so long contexts only)
    const int seg_tiles = ((kBtCache - 1) << bsh) / KT;
    for (int seg = t_lo; seg < t_hi; seg += seg_tiles) {
        const int seg_end = min(t_hi, seg + seg_tiles);
        blk0 = (seg * KT) >> bsh;
        const int nblk = (((min(seg_end * KT, kv_len) - 1) >> bsh) - blk0) + 1;
        __syncthreads();  // previous segment done with bt_lds and the ring
        for (int i = tid; i < nblk; i += THREADS) bt_lds[i] = bt[blk0 + i];
        __syncthreads();
        fetch(seg);
        stage(0);
        fetch(min(seg + 1, seg_end - 1));
        stage(1);
        fetch(min(seg + 2, seg_end - 1));
        __syncthreads();
        score(0, sacc);
        int buf = 0;
        for (int tile = seg; tile < seg_end; tile++) {
            const int b1 = buf == kPrefillBufs - 1 ? 0 : buf + 1;
            const int b2 = b1 == kPrefillBufs - 1 ? 0 : b1 + 1;
            // masks of edge tiles (window start, causal diagonal, end of keys)
            if (!(tile >= full_lo && tile < full_hi)) {
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int q4 = 0; q4 < SQ; q4++)
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int j = tile * KT + 8 * grp + 4 * q4 + r;
                            const bool ok = j >= ws && j < kv_len && (!p.causal || j <= qpos[b]);
                            sacc[b][q4][r] = ok ? sacc[b][q4][r] : -INFINITY;
                        }
            }
            // raise the reference max only when a score passes it by 2^8 (or
            // there is none yet); the row max is formed only then
            float lmax[NB];
            bool need = false;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                static_assert(SQ == 2, "eight scores per lane");
                const float mx = vmax3(vmax3(sacc[b][0][0], sacc[b][0][1], sacc[b][0][2]),
                                       vmax3(sacc[b][0][3], sacc[b][1][0], sacc[b][1][1]),
                                       __builtin_elementwise_maximum(sacc[b][1][2], sacc[b][1][3]));
                lmax[b] = mx * sl2;
                need |= lmax[b] > m_use[b] + kRescaleLog2;
            }
            if (__any(need)) {
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    float mt = lmax[b];
                    mt = fmaxf(mt, shfl_xor(mt, 16));
                    mt = fmaxf(mt, shfl_xor(mt, 32));
                    const float m_new = fmaxf(m_use[b], mt);
                    const float corr = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_use[b] - m_new);
                    l_run[b] *= corr;
#pragma unroll
                    for (int i = 0; i < NO; i++) o[b][i] *= corr;
                    m_use[b] = m_new;
                }
            }
            // scores of the next tile (overlaps the exponentials below)
            score(b1, snext);
            f16x8 pb[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const float mref = m_use[b] == -INFINITY ? 0.0f : m_use[b];
#pragma unroll
                for (int q4 = 0; q4 < SQ; q4++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        pb[b][4 * q4 + r] = (f16)__builtin_amdgcn_exp2f(fmaf(sacc[b][q4][r], sl2, -mref));
                // row sum of the f16 probabilities the MFMA consumes
                float ps = l_run[b];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const f16x2 pr = {pb[b][2 * k], pb[b][2 * k + 1]};
                    ps = __builtin_amdgcn_fdot2(pr, ones, ps, false);
                }
                l_run[b] = ps;
            }
            // O^T += V^T P^T
            const f16 *vt = v_lds[buf];
#pragma unroll
            for (int i = 0; i < NO; i++) {
                const int vb = (i < 4 ? v_base_lo : v_base_hi) + 16 * i;
                const f16x4 lo = lds_read_tr16(vt + vb);
                const f16x4 hi = lds_read_tr16(vt + vb + 4 * kPrefillVL);
                const f16x8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
                for (int b = 0; b < NB; b++) o[b][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[b], o[b][i], 0, 0, 0);
            }
            stage(b2);
            fetch(min(tile + 3, seg_end - 1));
            __syncthreads();
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int q4 = 0; q4 < SQ; q4++) sacc[b][q4] = snext[b][q4];
            buf = b1;
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
    hipLaunchKernelGGL((prefill_mfma_kernel<128, kPrefillNB>), grid, dim3(64 * kPrefillWaves), 0, stream,
                       p);
    return hipGetLastError();
}

}  // namespace pam
