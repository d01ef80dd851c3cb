// prefill.hip - dense chunked prefill on MFMA for gfx950.
//
// Computes rows [q_offset, q_offset + len) of causal (or full) attention for one
// or more sequence chunks whose first q_offset tokens are already in the paged
// pool (kernels.metal:693-917 semantics: scale 1/sqrt(d), GQA head h reads kv
// head h / G, a fixed window start max(0, kv_len - W) for every row).
//
// Matrix work runs on v_mfma_f32_32x32x16_f16, which on gfx950 retires twice
// the flops per cycle of the 16x16 shapes.  A workgroup (8 waves, two per SIMD)
// owns 256 query rows of one kv head: the (token, head) pairs of 256 / G
// consecutive tokens, so the G query heads sharing a kv head share every K/V
// tile.  Each wave owns RB blocks of 32 rows (RB = 2 would halve the LDS
// traffic but needs AGPR accumulators and one wave per SIMD, measured slower).
// Per 32-key tile t a wave runs two phases separated by workgroup barriers:
//   * matrix phase M_t: S^T(t+1) = K Q^T (32 keys x 32 rows, 8 MFMAs over d; K
//     from LDS is the A operand, Q^T stays in registers as B) and
//     O^T += V^T(t) P^T(t) (8 MFMAs; V^T read with the transposing
//     ds_read_b64_tr_b16), then the global loads of tile t + 4;
//   * vector phase V_t: mask and reference max of S(t), exponentials to P(t) in
//     f16, row sums, the K operands of M_t and the LDS staging of tile t + 2.
//   The S^T accumulator leaves lane (n, h) holding keys 8q + 4h + r (q, r < 4) of
//   row n, and the 8 of them with q in {2c, 2c+1} are exactly the B operand of
//   O^T += V^T P^T over key chunk c (16 keys), so P never leaves registers.
//   Waves 4-7 run one phase behind waves 0-3; waves w and w + 4 share a SIMD,
//   so its MFMA pipe works on one wave's matrix phase while the other wave's
//   vector phase runs.
// Softmax keeps a per-row reference max that is only raised (and O rescaled)
// when some score exceeds it by more than 2^8, so P is bounded by 2^8 and goes
// to the MFMA in f16; the common case needs no cross-lane reduction.
#include "kernels.h"
#include "pam_device.h"

namespace pam {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPrefillWaves = 8;                               // one workgroup per CU
constexpr int kPrefillRB = 1;                                  // 32-row blocks per wave
constexpr int kPrefillRows = 32 * kPrefillRB * kPrefillWaves;  // query rows per workgroup
constexpr int kPrefillKT = 32;                                 // keys per tile
constexpr int kPrefillBufs = 4;                // LDS ring of K/V tiles
constexpr float kRescaleLog2 = 8.0f;           // lazy-rescale threshold (log2 units)
constexpr int kBtCache = 2048;                 // block-table entries a workgroup keeps in LDS
constexpr int kXcds = 8;                       // accelerator dies (each with its own L2)

typedef __fp16 fp16x4_raw __attribute__((__vector_size__(4 * sizeof(__fp16))));

// ds_read_b64_tr_b16: the 16 lanes of a group each address 4 consecutive halves
// a[i][0..3]; lane o receives a[4j + o/4][o%4] for j = 0..3.
__device__ __forceinline__ f16x4 lds_read_tr16(const f16 *p) {
    const fp16x4_raw v =
        __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) fp16x4_raw *)(p));
    return __builtin_bit_cast(f16x4, v);
}

// LDS tiles (layouts checked against SQ_LDS_BANK_CONFLICT on gfx950).
// K: rows of 128 + 8 halves, so the 16 consecutive rows one 16-lane pass of an
// operand load touches fall on 16 distinct 16-byte bank groups.
// V: rows of 128 halves, 16-byte piece p of row r stored at p ^ 4*(r%4): the 4
// rows x 64 bytes of each 32-lane pass of a transposed load cover all banks once.
constexpr int kPrefillKL = 128 + 8;
constexpr int kPrefillVL = 128;
__device__ __forceinline__ int k_lds_at(int key, int piece) { return key * kPrefillKL + (piece << 3); }
__device__ __forceinline__ int v_lds_at(int key, int piece) {
    return key * kPrefillVL + ((piece ^ ((key & 3) << 2)) << 3);
}

// three-way maximum (v_maximum3_f32); scores are never NaN
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

template <int HD, int RB>
__global__ __launch_bounds__(64 * kPrefillWaves, 1) void prefill_mfma_kernel(AttnParams p) {
    static_assert(HD == 128, "layouts assume d = 128");
    constexpr int KT = kPrefillKT;
    constexpr int KH = KT / 32;       // 32-key score blocks per tile
    constexpr int DC = HD / 16;       // 16-wide d chunks (S operands)
    constexpr int DT = HD / 32;       // 32-wide output dim tiles
    constexpr int PIECES = HD / 8;    // 16-byte pieces per token row
    constexpr int THREADS = 64 * kPrefillWaves;
    constexpr int KEYS_PER_PASS = THREADS / PIECES;  // 16 lanes per key row
    constexpr int KPT = KT / KEYS_PER_PASS;          // keys per thread per tile
    constexpr int ROWS = 32 * RB * kPrefillWaves;
    static_assert(KT % KEYS_PER_PASS == 0 && KPT <= 2, "whole keys per thread");
    __shared__ __attribute__((aligned(16))) f16 k_lds[kPrefillBufs][KT * kPrefillKL];
    __shared__ __attribute__((aligned(16))) f16 v_lds[kPrefillBufs][KT * kPrefillVL];
    __shared__ int32_t bt_lds[kBtCache];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
    const int G = p.num_heads / p.num_kv_heads, H = p.num_heads;
    const int tok_per_wg = ROWS / G;
    // Workgroup -> (chunk, kv head, token block).  Workgroups are dispatched to
    // the 8 XCDs round-robin by id, and each XCD has its own L2: all token
    // blocks of one (chunk, kv head) get ids of one residue mod 8, so the K/V
    // rows they share are fetched from HBM into one L2 only.  Chunks arrive
    // longest first; within a group the latest (heaviest) token blocks go first.
    const int nx = (p.max_chunk_len + tok_per_wg - 1) / tok_per_wg;
    const int xcd = blockIdx.x & (kXcds - 1), r = blockIdx.x / kXcds;
    const int grp = xcd + kXcds * (r / nx);
    if (grp >= p.num_chunks * p.num_kv_heads) return;
    const int4 ch = p.chunks[grp / p.num_kv_heads];  // {bt_row, q_offset, len, row_base}
    const int kvh = grp % p.num_kv_heads;
    const int tok0 = (nx - 1 - r % nx) * tok_per_wg;
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

    // this lane's query rows: column n of each of the wave's 32-row blocks
    int my_tok[RB], my_head[RB], qpos[RB];
    bool row_ok[RB];
    f16x8 qv[RB][DC];
#pragma unroll
    for (int b = 0; b < RB; b++) {
        const int rr = (wave * RB + b) * 32 + n;
        my_tok[b] = tok0 + rr / G;
        my_head[b] = rr % G;
        row_ok[b] = my_tok[b] < tok_end;
        qpos[b] = ch.y + my_tok[b];
        const f16 *qp = static_cast<const f16 *>(p.q) +
                        ((int64_t)(ch.w + (row_ok[b] ? my_tok[b] : tok0)) * H + kvh * G + my_head[b]) * HD + 8 * h;
#pragma unroll
        for (int c = 0; c < DC; c++) qv[b][c] = *reinterpret_cast<const f16x8 *>(qp + 16 * c);
    }

    // staging map: thread -> piece tid % 16 of keys tid / 16 (+ THREADS / 16)
    // (16 lanes read one key row's 256 contiguous bytes)
    const int my_piece = tid % PIECES, my_key = tid / PIECES;
    const uint32_t row_stride = (uint32_t)(p.num_kv_heads * HD);  // halves per pool row (< 2^32)
    const f16 *kpool = static_cast<const f16 *>(p.k_pool) + (int64_t)kvh * HD + my_piece * 8;
    const f16 *vpool = static_cast<const f16 *>(p.v_pool) + (int64_t)kvh * HD + my_piece * 8;
    // two register sets in flight: a tile's rows are loaded two iterations
    // before they are written to LDS
    f16x8 kra[KPT], vra[KPT], krb[KPT], vrb[KPT];
    int blk0 = 0;  // first block of the block-table segment held in bt_lds
    // pool row of this thread's key(s) of a tile, then the loads from it
    auto lookup = [&](int tile, uint32_t(&slot)[KPT]) {
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            int j = tile * KT + my_key + i * KEYS_PER_PASS;
            // keys outside [ws, kv_len) read the nearest key inside instead: finite
            // data whose probability is zero after masking (and a block-table entry
            // of the current segment)
            j = j < ws ? ws : (j >= kv_len ? kv_len - 1 : j);
            slot[i] = ((uint32_t)bt_lds[(j >> bsh) - blk0] << bsh) | (uint32_t)(j & bsm);
        }
    };
    auto load = [&](const uint32_t(&slot)[KPT], f16x8(&kreg)[KPT], f16x8(&vreg)[KPT]) {
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            const uint64_t off = (uint64_t)slot[i] * row_stride;
            kreg[i] = *reinterpret_cast<const f16x8 *>(kpool + off);
            vreg[i] = *reinterpret_cast<const f16x8 *>(vpool + off);
        }
    };
    auto fetch = [&](int tile, f16x8(&kreg)[KPT], f16x8(&vreg)[KPT]) {
        uint32_t slot[KPT];
        lookup(tile, slot);
        load(slot, kreg, vreg);
    };
    int k_st[KPT], v_st[KPT];
#pragma unroll
    for (int i = 0; i < KPT; i++) {
        k_st[i] = k_lds_at(my_key + i * KEYS_PER_PASS, my_piece);
        v_st[i] = v_lds_at(my_key + i * KEYS_PER_PASS, my_piece);
    }
    auto stage = [&](int buf, const f16x8(&kreg)[KPT], const f16x8(&vreg)[KPT]) {
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            *reinterpret_cast<f16x8 *>(&k_lds[buf][k_st[i]]) = kreg[i];
            *reinterpret_cast<f16x8 *>(&v_lds[buf][v_st[i]]) = vreg[i];
        }
    };

    // S^T: A operand of chunk c = K[key n][16c + 8h .. +7], shared by the row blocks
    const int k_rd = k_lds_at(n, h);
    auto score = [&](int buf, f32x16(&sc)[RB][KH]) {
        const f16 *kt = k_lds[buf];
#pragma unroll
        for (int e = 0; e < KH; e++) {
#pragma unroll
            for (int b = 0; b < RB; b++) sc[b][e] = (f32x16)0.0f;
#pragma unroll
            for (int c = 0; c < DC; c++) {
                const f16x8 ka = *reinterpret_cast<const f16x8 *>(&kt[k_rd + 32 * e * kPrefillKL + 16 * c]);
#pragma unroll
                for (int b = 0; b < RB; b++)
                    sc[b][e] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qv[b][c], sc[b][e], 0, 0, 0);
            }
        }
    };
    // V^T operand of dim tile dt, key chunk c: lane (o = lane % 16 of its 16-lane
    // group, half hh = (lane / 16) % 2, h) reads row 16c + 4h + 8jj + o/4
    // (jj = 0, 1) at dims 32dt + 16hh + 4(o%4): two transposed loads give keys
    // 16c + 4h + {0..3, 8..11} of dim 32dt + 16hh + o, the P slot order
    int v_rd[DT];
    {
        const int o = lane & 15, hh = (lane >> 4) & 1;
        const int row = 4 * h + (o >> 2);
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
            v_rd[dt] = v_lds_at(row, 4 * dt + 2 * hh + ((o & 3) >> 1)) + 4 * (o & 1);
    }

    float m_use[RB], l_run[RB], lmax[RB];
    f32x16 o[RB][DT];
#pragma unroll
    for (int b = 0; b < RB; b++) {
        m_use[b] = -INFINITY;
        l_run[b] = 0.0f;
        lmax[b] = -INFINITY;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[b][dt] = (f32x16)0.0f;
    }
    const float sl2 = p.scale_log2;
    const f16x2 ones = {(f16)1.0f, (f16)1.0f};

    // accumulator register r of block e holds key 32e + 8(r/4) + 4h + r%4 of the tile
    auto prepare = [&](int tile, f32x16(&sc)[RB][KH]) -> bool {
        bool need = false;
#pragma unroll
        for (int b = 0; b < RB; b++) {
            if (!(tile >= full_lo && tile < full_hi)) {
#pragma unroll
                for (int e = 0; e < KH; e++)
#pragma unroll
                    for (int r2 = 0; r2 < 16; r2++) {
                        const int j = tile * KT + 32 * e + 8 * (r2 >> 2) + 4 * h + (r2 & 3);
                        const bool ok = j >= ws && j < kv_len && (!p.causal || j <= qpos[b]);
                        sc[b][e][r2] = ok ? sc[b][e][r2] : -INFINITY;
                    }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int e = 0; e < KH; e++) {
                mx = vmax3(mx, sc[b][e][0], sc[b][e][1]);
#pragma unroll
                for (int r2 = 2; r2 < 16; r2 += 2) mx = vmax3(mx, sc[b][e][r2], sc[b][e][r2 + 1]);
            }
            lmax[b] = mx * sl2;
            need |= lmax[b] > m_use[b] + kRescaleLog2;
        }
        return need;
    };
    // raise the reference max to the row max (rare: wave-uniform branch)
    auto rescale = [&]() {
#pragma unroll
        for (int b = 0; b < RB; b++) {
            const float mt = fmaxf(lmax[b], shfl_xor(lmax[b], 32));
            const float m_new = fmaxf(m_use[b], mt);
            const float corr = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_use[b] - m_new);
            l_run[b] *= corr;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[b][dt] *= corr;
            m_use[b] = m_new;
        }
    };

    // Ping-pong schedule.  A tile's work splits into a matrix phase M_t (scores
    // S(t+1) = K(t+1) Q^T and O += V(t) P(t), with the loads of tile t + 4) and a
    // vector phase V_t (mask, reference max and exponentials of S(t), row sums,
    // and the LDS staging of tile t + 2).  Each wave runs
    // M_-1 V_0 M_0 V_1 M_1 ... with a workgroup barrier after every phase; waves
    // 4-7 start one barrier late, so each SIMD (waves w and w + 4) has one wave in
    // a matrix phase while the other is in a vector phase, and the MFMA and VALU
    // pipes overlap.  LDS ring of 4 tiles: tile t + 2 is written (half by each
    // wave group) at V_t, K(t) is read at M_t-1 and V(t) at M_t, so a buffer is
    // rewritten only after both groups have left the phases that read it.
    constexpr int NBUF = kPrefillBufs;
    static_assert(NBUF == 4, "the ring schedule above needs 4 tiles");
    const bool lag = wave >= kPrefillWaves / 2;
    f32x16 sacc[RB][KH];
    f16x8 pb[RB][2 * KH];
    // tiles run in segments whose block-table entries fit in bt_lds (one segment
    // covers kBtCache * block_size keys, so long contexts only)
    // (an even number of tiles: the loop below runs tiles in pairs, and a segment
    // of odd length gets one extra tile past the keys, fully masked)
    const int seg_tiles = (((kBtCache - 1) << bsh) / KT) & ~1;
    for (int seg = t_lo; seg < t_hi; seg += seg_tiles) {
        const int seg_end = min(t_hi, seg + seg_tiles);
        const int T = (seg_end - seg + 1) & ~1;
        blk0 = (seg * KT) >> bsh;
        const int nblk = (((min(seg_end * KT, kv_len) - 1) >> bsh) - blk0) + 1;
        __syncthreads();  // previous segment done with bt_lds and the ring
        for (int i = tid; i < nblk; i += THREADS) bt_lds[i] = bt[blk0 + i];
        __syncthreads();
        fetch(seg, kra, vra);
        stage(0, kra, vra);
        fetch(min(seg + 1, seg_end - 1), kra, vra);
        stage(1, kra, vra);
        fetch(min(seg + 2, seg_end - 1), kra, vra);
        fetch(min(seg + 3, seg_end - 1), krb, vrb);
        __syncthreads();
        if (lag) __syncthreads();
        score(0, sacc);  // M_-1
        __syncthreads();

        // The vector phase requests the K operands of the next matrix phase (its
        // tile is staged by then) and looks up the rows the matrix phase will
        // load; the matrix phase requests its V operands first and runs the score
        // MFMAs while they arrive.
        f16x8 ka[KH][DC];
        uint32_t nslot[KPT];
        auto vphase = [&](int t, f16x8(&kreg)[KPT], f16x8(&vreg)[KPT]) {
            if (t + 1 < T) {
                const f16 *kt = k_lds[(t + 1) % NBUF];
#pragma unroll
                for (int e = 0; e < KH; e++)
#pragma unroll
                    for (int c = 0; c < DC; c++)
                        ka[e][c] = *reinterpret_cast<const f16x8 *>(&kt[k_rd + 32 * e * kPrefillKL + 16 * c]);
            }
            lookup(min(seg + t + 4, seg_end - 1), nslot);
            if (__any(prepare(seg + t, sacc))) rescale();
#pragma unroll
            for (int b = 0; b < RB; b++) {
                const float mref = m_use[b] == -INFINITY ? 0.0f : m_use[b];
#pragma unroll
                for (int e = 0; e < KH; e++)
#pragma unroll
                    for (int r2 = 0; r2 < 16; r2++)
                        pb[b][2 * e + (r2 >> 3)][r2 & 7] =
                            (f16)__builtin_amdgcn_exp2f(fmaf(sacc[b][e][r2], sl2, -mref));
                // row sum of the f16 probabilities the MFMA consumes
                float ps = l_run[b];
#pragma unroll
                for (int k = 0; k < 8 * KH; k++) {
                    const f16x2 pr = {pb[b][k >> 2][2 * (k & 3)], pb[b][k >> 2][2 * (k & 3) + 1]};
                    ps = __builtin_amdgcn_fdot2(pr, ones, ps, false);
                }
                l_run[b] = ps;
            }
            // P and the row sums are complete here: without this the compiler
            // sinks the exponentials past the barrier into the matrix phase
#pragma unroll
            for (int b = 0; b < RB; b++) {
#pragma unroll
                for (int c = 0; c < 2 * KH; c++) asm volatile("" : "+v"(pb[b][c]));
                asm volatile("" : "+v"(l_run[b]));
            }
            stage((t + 2) % NBUF, kreg, vreg);  // tile t + 2, fetched at M_t-2
        };
        auto mphase = [&](int t, f16x8(&kreg)[KPT], f16x8(&vreg)[KPT]) {
            const f16 *vt = v_lds[t % NBUF];
            f16x8 va[2 * KH][DT];
#pragma unroll
            for (int c = 0; c < 2 * KH; c++)
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const f16x4 lo = lds_read_tr16(vt + v_rd[dt] + 16 * c * kPrefillVL);
                    const f16x4 hi = lds_read_tr16(vt + v_rd[dt] + (16 * c + 8) * kPrefillVL);
                    va[c][dt] = (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
            if (t + 1 < T) {
#pragma unroll
                for (int e = 0; e < KH; e++) {
#pragma unroll
                    for (int b = 0; b < RB; b++) sacc[b][e] = (f32x16)0.0f;
#pragma unroll
                    for (int c = 0; c < DC; c++)
#pragma unroll
                        for (int b = 0; b < RB; b++)
                            sacc[b][e] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[e][c], qv[b][c], sacc[b][e], 0, 0, 0);
                }
            }
            // O^T += V^T P^T, each V^T operand shared by the row blocks
#pragma unroll
            for (int c = 0; c < 2 * KH; c++)
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int b = 0; b < RB; b++)
                        o[b][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[c][dt], pb[b][c], o[b][dt], 0, 0, 0);
            // the matrix work stays in this phase (the compiler would otherwise move
            // the last MFMAs past the barrier)
#pragma unroll
            for (int b = 0; b < RB; b++) {
#pragma unroll
                for (int dt = 0; dt < DT; dt++) asm volatile("" : "+v"(o[b][dt]));
#pragma unroll
                for (int e = 0; e < KH; e++) asm volatile("" : "+v"(sacc[b][e]));
            }
            load(nslot, kreg, vreg);  // tile t + 4
        };
        for (int t = 0; t < T; t += 2) {
            vphase(t, kra, vra);
            __syncthreads();
            mphase(t, kra, vra);
            __syncthreads();
            vphase(t + 1, krb, vrb);
            __syncthreads();
            mphase(t + 1, krb, vrb);
            __syncthreads();
        }
        if (!lag) __syncthreads();
    }

    // finish: l summed over the two lane halves, O / l, rows in range only
#pragma unroll
    for (int b = 0; b < RB; b++) {
        const float l = l_run[b] + shfl_xor(l_run[b], 32);
        if (!row_ok[b]) continue;
        // no key in range (window past the row): 0/0, as the reference's m/l bookkeeping gives
        const float inv = 1.0f / l;
        f16 *op = static_cast<f16 *>(p.out) + ((int64_t)(ch.w + my_tok[b]) * H + kvh * G + my_head[b]) * HD + 4 * h;
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                f16x4 v;
#pragma unroll
                for (int r2 = 0; r2 < 4; r2++) v[r2] = (f16)(o[b][dt][4 * q + r2] * inv);
                *reinterpret_cast<f16x4 *>(op + 32 * dt + 8 * q) = v;
            }
    }
}

bool prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size) {
    return dtype == kF16 && head_dim == 128 && group >= 1 && group <= 32 && (kPrefillRows % group) == 0 &&
           block_size > 0 && (block_size & (block_size - 1)) == 0;
}

hipError_t launch_prefill_mfma(const AttnParams &p, hipStream_t stream) {
    if (p.chunks == nullptr || p.num_chunks <= 0 || p.max_chunk_len <= 0) return hipErrorInvalidValue;
    const int G = p.num_heads / p.num_kv_heads;
    if (!prefill_mfma_supported(kF16, p.head_dim, G, p.block_size)) return hipErrorInvalidValue;
    const int tok_per_wg = kPrefillRows / G;
    const int nx = (p.max_chunk_len + tok_per_wg - 1) / tok_per_wg;
    const int groups = p.num_chunks * p.num_kv_heads;
    dim3 grid(kXcds * nx * ((groups + kXcds - 1) / kXcds));
    hipLaunchKernelGGL((prefill_mfma_kernel<128, kPrefillRB>), grid, dim3(64 * kPrefillWaves), 0, stream, p);
    return hipGetLastError();
}

}  // namespace pam
