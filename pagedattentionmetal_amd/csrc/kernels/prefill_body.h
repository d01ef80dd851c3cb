// prefill_body.h - device body of the dense chunked prefill (gfx950); the
// schedule and layouts are described in prefill.hip.  Included by prefill.hip,
// mixed.hip and the code-object entries.
#pragma once
#include <type_traits>

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


// LDS tiles for head size HD (layouts checked against SQ_LDS_BANK_CONFLICT on
// gfx950 at d = 128).
// K: rows of HD + 8 halves (an odd number of 16-byte units), so the 16
// consecutive rows one 16-lane pass of an operand load touches fall on 16
// distinct 16-byte bank groups.
// V: rows of HD halves with 16-byte piece p of row r stored at p ^ s(r), so the
// 4 rows x 64 bytes of each 32-lane pass of a transposed load cover all banks
// once: s(r) = 4 (r % 4) for 256-byte rows (d = 128); for 128-byte rows
// (d = 64), rows r and r + 1 already fall on opposite bank halves and
// s(r) = 4 ((r / 2) % 2) separates r from r + 2.
template <int HD>
constexpr int pf_kl() { return HD + 8; }
template <int HD>
__device__ __forceinline__ int k_lds_at(int key, int piece) { return key * pf_kl<HD>() + (piece << 3); }
template <int HD>
__device__ __forceinline__ int v_lds_at(int key, int piece) {
    const int sw = HD == 128 ? (key & 3) << 2 : ((key >> 1) & 1) << 2;
    return key * HD + ((piece ^ sw) << 3);
}

// three-way maximum (v_maximum3_f32); scores are never NaN
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

template <int HD, int RB, bool FUSED, typename KV>
__device__ __forceinline__ void prefill_body(const AttnParams &p) {
    // KV: f16 pools, or e4m3 codes (uint8_t) with a half scale per physical block
    constexpr bool FP8 = sizeof(KV) == 1;
    static_assert(!(FUSED && FP8), "the fused append is f16 only");
    static_assert(HD == 128 || HD == 64, "layouts for d = 64 and 128");
    constexpr int KL = pf_kl<HD>(), VL = HD;
    constexpr int KT = kPrefillKT;
    constexpr int KH = KT / 32;       // 32-key score blocks per tile
    constexpr int DC = HD / 16;       // 16-wide d chunks (S operands)
    constexpr int DT = HD / 32;       // 32-wide output dim tiles
    constexpr int PIECES = HD / 8;    // 16-byte pieces per token row
    constexpr int THREADS = 64 * kPrefillWaves;
    // staging: a thread loads one 16-byte piece of K and of V for each of its
    // keys (d = 128: 16 lanes per key row); at d = 64 the threads outnumber a
    // tile's K pieces twice, so the first half stages K and the second V
    constexpr bool SPLIT = THREADS / PIECES >= 2 * KT;
    constexpr int KEYS_PER_PASS = SPLIT ? KT : THREADS / PIECES;
    constexpr int KPT = KT / KEYS_PER_PASS;          // keys per thread per tile
    constexpr int ROWS = 32 * RB * kPrefillWaves;
    static_assert(KT % KEYS_PER_PASS == 0 && KPT <= 2 && (!SPLIT || THREADS / PIECES == 2 * KT), "whole keys per thread");
    // the K and V rings in one array: after a segment's tile loop the whole of
    // it holds the waves' output rows on their way to memory (finish, below)
    constexpr int kRingK = kPrefillBufs * KT * KL, kRingV = kPrefillBufs * KT * VL;
    __shared__ __attribute__((aligned(16))) f16 ring_lds[kRingK + kRingV];
    f16(*k_lds)[KT * KL] = reinterpret_cast<f16(*)[KT * KL]>(ring_lds);
    f16(*v_lds)[KT * VL] = reinterpret_cast<f16(*)[KT * VL]>(ring_lds + kRingK);
    static_assert(RB == 1 && kPrefillWaves * 32 * HD <= kRingK + kRingV, "one 32-row output tile per wave in the ring");
    __shared__ int32_t bt_lds[kBtCache];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
    const int G = p.num_heads / p.num_kv_heads, H = p.num_heads;
    const int tok_per_wg = ROWS / G;
    // This workgroup's segments of the work list (prefill_split_plan): each is
    // an item (chunk, kv head, block of 256 / G tokens) over key tiles
    // [t_lo, t_hi), either all the item's tiles or one piece of them.
    const int2 rg = p.pf_range[blockIdx.x];
    __shared__ int32_t merge_flag;
    const int bsh = __builtin_ctz(p.block_size), bsm = p.block_size - 1;  // block_size is a power of two
    // descriptors of the next segment are requested while this one runs.  They
    // are uniform, but loaded through an offset the compiler cannot see is zero
    // so that they stay in vector registers until the next segment reads them
    // into scalars: loaded as uniform values they would be moved to scalar
    // registers, and waited for, right after the load.
    int vzero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
    const int4 *work = p.pf_work + vzero;
    int4 nx_ch = make_int4(0, 0, 0, 0), nx_wa = nx_ch, nx_wb = nx_ch;
    if (rg.x < rg.y) {
        nx_ch = work[3 * rg.x];
        nx_wa = work[3 * rg.x + 1];
        nx_wb = work[3 * rg.x + 2];
    }
    auto uniform4 = [](const int4 v) {
        return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                         __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
    };
    int32_t pre_bt = 0;    // a block-table entry of the next segment, loaded ahead
    int pre_nb = 0;        // how many of them the next segment's first block-table part holds
    bool pre_ok = false;
    // Workgroup barrier for LDS only: this wave's LDS accesses are complete, then
    // every wave arrives.  A __syncthreads at an item's start would also wait for
    // the wave's outstanding global accesses (the item's Q loads, the last item's
    // output stores), which the LDS it protects does not depend on.
    auto lds_barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    for (int sgi = rg.x; sgi < rg.y; sgi++) {
        const bool use_pre = pre_ok;
        pre_ok = false;
        const int4 ch = uniform4(nx_ch);  // {bt_row, q_offset, len, row_base}
        const int4 wa = uniform4(nx_wa);  // {kv head, first token, t_lo, t_hi}
        const int4 wb = uniform4(nx_wb);  // {slot0, piece, pieces, 0}
        if (sgi + 1 < rg.y) {
            nx_ch = work[3 * sgi + 3];
            nx_wa = work[3 * sgi + 4];
            nx_wb = work[3 * sgi + 5];
        }
        const int kvh = wa.x, tok0 = wa.y;
        const int32_t *bt = p.block_tables + (int64_t)ch.x * p.bt_stride;
        const int kv_len = ch.y + ch.z;
        const int ws = p.window > 0 ? (kv_len > p.window ? kv_len - p.window : 0) : 0;
        const int tok_end = tok0 + tok_per_wg < ch.z ? tok0 + tok_per_wg : ch.z;
        const int t_lo = wa.z, t_hi = wa.w;
        // keys at or past key_hi belong to later pieces (or do not exist)
        const int key_hi = min(kv_len, t_hi * KT);
        // tiles [full_lo, full_hi) need no mask for any row of the workgroup
        const int full_lo = (ws + KT - 1) / KT;
        int full_hi = min(kv_len / KT, t_hi);
        if (p.causal) full_hi = min(full_hi, (ch.y + tok0 + 1) / KT);

        // Fused append: the first piece of an item writes its tokens' rows of kv
        // head kvh into the pools (readers of these keys use the inputs).
        if constexpr (FUSED) {
            if (wb.y == 0) {
                const int64_t rs = (int64_t)p.num_kv_heads * HD;
                for (int idx = tid; idx < (tok_end - tok0) * (HD / 8); idx += 64 * kPrefillWaves) {
                    const int tk = tok0 + idx / (HD / 8), pc = idx % (HD / 8);
                    const int pos = ch.y + tk;
                    const int64_t slot = ((int64_t)bt[pos >> bsh] << bsh) | (pos & bsm);
                    const int64_t src = (int64_t)(ch.w + tk) * rs + kvh * HD + 8 * pc;
                    const int64_t dst = slot * rs + kvh * HD + 8 * pc;
                    *reinterpret_cast<f16x8 *>(static_cast<f16 *>(const_cast<void *>(p.k_pool)) + dst) =
                        *reinterpret_cast<const f16x8 *>(static_cast<const f16 *>(p.fuse_k) + src);
                    *reinterpret_cast<f16x8 *>(static_cast<f16 *>(const_cast<void *>(p.v_pool)) + dst) =
                        *reinterpret_cast<const f16x8 *>(static_cast<const f16 *>(p.fuse_v) + src);
                }
            }
        }

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

        // staging map: thread -> piece tid % PIECES of keys tid / PIECES (+
        // THREADS / PIECES) (PIECES lanes read one key row's contiguous bytes);
        // SPLIT: key (tid / PIECES) % KT of K (first half) or V (second half)
        const bool vhalf = SPLIT && tid >= THREADS / 2;
        const int my_piece = tid % PIECES, my_key = (tid / PIECES) % (SPLIT ? KT : THREADS);
        const uint32_t row_stride = (uint32_t)(p.num_kv_heads * HD);  // halves per pool row (< 2^32)
        const KV *kpool = static_cast<const KV *>(vhalf ? p.v_pool : p.k_pool) + (int64_t)kvh * HD + my_piece * 8;
        const KV *vpool = static_cast<const KV *>(p.v_pool) + (int64_t)kvh * HD + my_piece * 8;
        // fused append: rows of the chunk's new tokens have the pools' row stride;
        // a load of one adds the (uniform) distance from the pool to the input
        // (in halves; both buffers hold f16, so the byte distance is even)
        const int64_t vin_d = FUSED ? (int64_t)((uintptr_t)p.fuse_v - (uintptr_t)p.v_pool) / 2 : 0;
        const int64_t kin_d = FUSED ? (vhalf ? vin_d : (int64_t)((uintptr_t)p.fuse_k - (uintptr_t)p.k_pool) / 2) : 0;
        const uint16_t *kscale = FP8 ? (vhalf ? p.v_scale : p.k_scale) : nullptr;
        // two register sets in flight: a tile's rows are loaded two iterations
        // before they are written to LDS.  A thread's piece of a row is 8
        // elements: 16 bytes of f16, or 8 e4m3 codes plus the block's scales.
        using Raw = typename std::conditional<FP8, uint2, f16x8>::type;
        struct Regs {
            Raw k[KPT], v[KPT];
            uint32_t ks[KPT], vs[KPT];  // e4m3: half scale bits of the row's block
        };
        Regs ra, rb;
        int blk0 = 0;  // first block of the block-table segment held in bt_lds
        const int32_t *bt_seg = bt_lds;  // bt_lds - blk0: indexed by logical block
        // pool row of this thread's key(s) of a tile, then the loads from it
        // (SPLIT: the thread's one piece, of K or of V, goes to r.k)
        auto lookup = [&](int tile, uint32_t(&slot)[KPT]) {
#pragma unroll
            for (int i = 0; i < KPT; i++) {
                int j = tile * KT + my_key + i * KEYS_PER_PASS;
                // keys outside [ws, kv_len) read the nearest key inside instead: finite
                // data whose probability is zero after masking (and a block-table entry
                // of the current segment); ws < kv_len
                j = min(max(j, ws), kv_len - 1);
                slot[i] = ((uint32_t)bt_seg[(uint32_t)j >> bsh] << bsh) | ((uint32_t)j & bsm);
                // fused append: a new token's row of the inputs (top bit set)
                if (FUSED && j >= ch.y) slot[i] = 0x80000000u | (uint32_t)(ch.w + j - ch.y);
            }
        };
        // the V pool's distance from the K pool (bytes): one multiply-add gives a
        // row's K address, one add its V address
        const int64_t kv_gap = (const char *)vpool - (const char *)kpool;
        const uint64_t row_bytes = (uint64_t)row_stride * sizeof(KV);
        auto load = [&](const uint32_t(&slot)[KPT], Regs &r) {
#pragma unroll
            for (int i = 0; i < KPT; i++) {
                const uint32_t row = slot[i] & 0x7FFFFFFFu;
                if constexpr (SPLIT) {
                    const uint64_t off = (uint64_t)row * row_stride;
                    if constexpr (FP8) {
                        r.k[i] = *reinterpret_cast<const uint2 *>(kpool + off);
                        r.ks[i] = kscale[row >> bsh];
                    } else {
                        const bool in = FUSED && (slot[i] >> 31);
                        r.k[i] = *reinterpret_cast<const f16x8 *>(kpool + off + (in ? kin_d : 0));
                    }
                    continue;
                }
                if constexpr (!FP8 && !FUSED) {
                    const char *ka = (const char *)kpool + (uint64_t)row * row_bytes;
                    r.k[i] = *reinterpret_cast<const f16x8 *>(ka);
                    r.v[i] = *reinterpret_cast<const f16x8 *>(ka + kv_gap);
                    continue;
                }
                const uint64_t off = (uint64_t)row * row_stride;
                if constexpr (FP8) {
                    r.k[i] = *reinterpret_cast<const uint2 *>(kpool + off);
                    r.v[i] = *reinterpret_cast<const uint2 *>(vpool + off);
                    r.ks[i] = p.k_scale[row >> bsh];
                    r.vs[i] = p.v_scale[row >> bsh];
                } else {
                    const bool in = FUSED && (slot[i] >> 31);
                    r.k[i] = *reinterpret_cast<const f16x8 *>(kpool + off + (in ? kin_d : 0));
                    r.v[i] = *reinterpret_cast<const f16x8 *>(vpool + off + (in ? vin_d : 0));
                }
            }
        };
        auto fetch = [&](int tile, Regs &r) {
            uint32_t slot[KPT];
            lookup(tile, slot);
            load(slot, r);
        };
        int k_st[KPT], v_st[KPT];
#pragma unroll
        for (int i = 0; i < KPT; i++) {
            k_st[i] = k_lds_at<HD>(my_key + i * KEYS_PER_PASS, my_piece);
            v_st[i] = v_lds_at<HD>(my_key + i * KEYS_PER_PASS, my_piece);
        }
        auto stage = [&](int buf, const Regs &r) {
#pragma unroll
            for (int i = 0; i < KPT; i++) {
                if constexpr (SPLIT) {
                    f16 *dst = ring_lds + (vhalf ? kRingK + buf * KT * VL + v_st[i] : buf * KT * KL + k_st[i]);
                    if constexpr (FP8)
                        *reinterpret_cast<f16x8 *>(dst) =
                            e4m3x8_to_f16x8(r.k[i].x, r.k[i].y) * (f16x8)bits_to_f16((uint16_t)r.ks[i]);
                    else
                        *reinterpret_cast<f16x8 *>(dst) = r.k[i];
                    continue;
                }
                if constexpr (FP8) {
                    // exact code values times the block scale in one binary16
                    // multiply: the reference's half dequantisation, as in decode
                    const f16x8 ks8 = (f16x8)bits_to_f16((uint16_t)r.ks[i]);
                    const f16x8 vs8 = (f16x8)bits_to_f16((uint16_t)r.vs[i]);
                    *reinterpret_cast<f16x8 *>(&k_lds[buf][k_st[i]]) = e4m3x8_to_f16x8(r.k[i].x, r.k[i].y) * ks8;
                    *reinterpret_cast<f16x8 *>(&v_lds[buf][v_st[i]]) = e4m3x8_to_f16x8(r.v[i].x, r.v[i].y) * vs8;
                } else {
                    *reinterpret_cast<f16x8 *>(&k_lds[buf][k_st[i]]) = r.k[i];
                    *reinterpret_cast<f16x8 *>(&v_lds[buf][v_st[i]]) = r.v[i];
                }
            }
        };

        // S^T: A operand of chunk c = K[key n][16c + 8h .. +7], shared by the row blocks
        const int k_rd = k_lds_at<HD>(n, h);
        auto score = [&](int buf, f32x16(&sc)[RB][KH]) {
            const f16 *kt = k_lds[buf];
#pragma unroll
            for (int e = 0; e < KH; e++) {
#pragma unroll
                for (int b = 0; b < RB; b++) sc[b][e] = (f32x16)0.0f;
#pragma unroll
                for (int c = 0; c < DC; c++) {
                    const f16x8 ka = *reinterpret_cast<const f16x8 *>(&kt[k_rd + 32 * e * KL + 16 * c]);
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
                v_rd[dt] = v_lds_at<HD>(row, 4 * dt + 2 * hh + ((o & 3) >> 1)) + 4 * (o & 1);
        }

        // lmax: the tile's raw row max (score units); m_thr: the score above which
        // the reference max must move, (m_use + kRescaleLog2) / scale_log2
        float m_use[RB], l_run[RB], lmax[RB], m_thr[RB];
        f32x16 o[RB][DT];
#pragma unroll
        for (int b = 0; b < RB; b++) {
            m_use[b] = -INFINITY;
            m_thr[b] = -INFINITY;
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
                            const bool ok = j >= ws && j < key_hi && (!p.causal || j <= qpos[b]);
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
                lmax[b] = mx;
                need |= mx > m_thr[b];
            }
            return need;
        };
        // raise the reference max to the row max (rare: wave-uniform branch)
        auto rescale = [&]() {
#pragma unroll
            for (int b = 0; b < RB; b++) {
                const float mt = fmaxf(lmax[b], shfl_xor(lmax[b], 32)) * sl2;
                const float m_new = fmaxf(m_use[b], mt);
                const float corr = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_use[b] - m_new);
                l_run[b] *= corr;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) o[b][dt] *= corr;
                m_use[b] = m_new;
                m_thr[b] = (m_new + kRescaleLog2) / sl2;
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
            bt_seg = bt_lds - blk0;
            const int nblk = (((min(seg_end * KT, kv_len) - 1) >> bsh) - blk0) + 1;
            lds_barrier();  // previous segment done with bt_lds and the ring
            // entries loaded during the previous item are in bt_lds already
            const int i0 = tid + (seg == t_lo && use_pre ? THREADS : 0);
            for (int i = i0; i < nblk; i += THREADS) bt_lds[i] = bt[blk0 + i];
            lds_barrier();
            // the first four tiles are requested together
            {
                Regs rc, rd;
                fetch(seg, ra);
                fetch(min(seg + 1, seg_end - 1), rb);
                fetch(min(seg + 2, seg_end - 1), rc);
                fetch(min(seg + 3, seg_end - 1), rd);
                stage(0, ra);
                stage(1, rb);
                ra = rc;
                rb = rd;
            }
            lds_barrier();
            if (lag) lds_barrier();
            score(0, sacc);  // M_-1
            lds_barrier();
            // request the first block-table entries of the workgroup's next segment
            // (its descriptors arrived long ago); they are stored at its start
            if (seg == t_lo && sgi + 1 < rg.y) {
                const int4 nch = uniform4(nx_ch), nwa = uniform4(nx_wa);
                const int kvn = nch.y + nch.z, tlo_n = nwa.z;
                const int send = min(nwa.w, tlo_n + seg_tiles);
                const int b0 = (tlo_n * KT) >> bsh;
                const int nb = send > tlo_n ? (((min(send * KT, kvn) - 1) >> bsh) - b0) + 1 : 0;
                if (tid < nb) pre_bt = p.block_tables[(int64_t)nch.x * p.bt_stride + b0 + tid];
                pre_nb = nb;
                pre_ok = true;
            }

            // The vector phase requests the K operands of the next matrix phase (its
            // tile is staged by then) and looks up the rows the matrix phase will
            // load; the matrix phase requests its V operands first and runs the score
            // MFMAs while they arrive.
            f16x8 ka[KH][DC];
            uint32_t nslot[KPT];
            // `slot` = t % NBUF as a compile-time constant (std::integral_constant):
            // the ring buffers' LDS offsets then need no per-phase arithmetic
            auto vphase = [&](int t, auto slot, Regs &r) {
                constexpr int S = decltype(slot)::value;
                // the LDS staging of tile t + 2 (fetched at M_t-2) goes first: its
                // writes then overlap the rest of the phase (measured 2% faster
                // than staging last)
                stage((S + 2) % NBUF, r);
                __builtin_amdgcn_sched_barrier(0);
                if (t + 1 < T) {
                    const f16 *kt = k_lds[(S + 1) % NBUF];
#pragma unroll
                    for (int e = 0; e < KH; e++)
#pragma unroll
                        for (int c = 0; c < DC; c++)
                            ka[e][c] = *reinterpret_cast<const f16x8 *>(&kt[k_rd + 32 * e * KL + 16 * c]);
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
            };
            auto mphase = [&](int t, auto slot, Regs &r) {
                constexpr int S = decltype(slot)::value;
                // the matrix phase runs at raised wave priority: its V operand
                // reads then issue ahead of the other wave's vector work on the
                // SIMD (measured 2% faster; the same from the MFMAs on only:
                // no gain; the vector phase raised instead: 2% slower)
                __builtin_amdgcn_s_setprio(1);
                const f16 *vt = v_lds[S];
                f16x8 va[2 * KH][DT];
#pragma unroll
                for (int c = 0; c < 2 * KH; c++)
#pragma unroll
                    for (int dt = 0; dt < DT; dt++) {
                        const f16x4 lo = lds_read_tr16(vt + v_rd[dt] + 16 * c * VL);
                        const f16x4 hi = lds_read_tr16(vt + v_rd[dt] + (16 * c + 8) * VL);
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
                load(nslot, r);  // tile t + 4
                __builtin_amdgcn_s_setprio(0);
            };
            using S0 = std::integral_constant<int, 0>;
            using S1 = std::integral_constant<int, 1>;
            using S2 = std::integral_constant<int, 2>;
            using S3 = std::integral_constant<int, 3>;
            int t = 0;
            for (; t + 4 <= T; t += 4) {  // four tiles: one turn of the ring
                vphase(t, S0{}, ra);
                __syncthreads();
                mphase(t, S0{}, ra);
                __syncthreads();
                vphase(t + 1, S1{}, rb);
                __syncthreads();
                mphase(t + 1, S1{}, rb);
                __syncthreads();
                vphase(t + 2, S2{}, ra);
                __syncthreads();
                mphase(t + 2, S2{}, ra);
                __syncthreads();
                vphase(t + 3, S3{}, rb);
                __syncthreads();
                mphase(t + 3, S3{}, rb);
                __syncthreads();
            }
            if (t < T) {  // T is even: two tiles left, starting at slot 0
                vphase(t, S0{}, ra);
                __syncthreads();
                mphase(t, S0{}, ra);
                __syncthreads();
                vphase(t + 1, S1{}, rb);
                __syncthreads();
                mphase(t + 1, S1{}, rb);
                __syncthreads();
            }
            if (!lag) lds_barrier();
        }
        // every wave has left the item's tile loop: the next item's first
        // block-table entries go into bt_lds now, with nothing of the next item
        // in flight yet
        if (pre_ok && tid < pre_nb) bt_lds[tid] = pre_bt;

        // A piece of a split item publishes its state (O^T, reference max and row
        // sums, per lane) in its slot with write-through stores and counts it;
        // the workgroup that brings the count to the number of pieces merges all
        // of them in piece order (the same result whichever workgroup merges)
        // and writes the rows.  The counter carries the launch's epoch
        // (arrive_count), so it is never reset.
        if (wb.z > 1) {
            static_assert(kPrefillSlotBytes >= (int64_t)kPrefillWaves * 64 * RB * (16 * DT + 2) * 4, "slot size");
            const __amdgpu_buffer_rsrc_t prs =
                __builtin_amdgcn_make_buffer_rsrc(p.pf_part, 0, (int)p.pf_part_bytes, 0x00020000);
            constexpr int NQ = RB * DT * 4;  // 16-byte pieces of O^T per lane
            auto o_at = [&](int slot, int q) { return (int)(slot * kPrefillSlotBytes) + ((wave * NQ + q) * 64 + lane) * 16; };
            auto ml_at = [&](int slot, int b) {
                return (int)(slot * kPrefillSlotBytes) + kPrefillWaves * 64 * NQ * 16 + ((wave * RB + b) * 64 + lane) * 8;
            };
            const int mine = wb.x + wb.y;
#pragma unroll
            for (int b = 0; b < RB; b++) {
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int qq = 0; qq < 4; qq++) {
                        const f32x4 v = {o[b][dt][4 * qq], o[b][dt][4 * qq + 1], o[b][dt][4 * qq + 2], o[b][dt][4 * qq + 3]};
                        __builtin_amdgcn_raw_buffer_store_b128(v, prs, o_at(mine, (b * DT + dt) * 4 + qq), 0, kSc1);
                    }
                // P was taken against 0 while the reference max is still unset
                const f32x2 ml = {m_use[b] == -INFINITY ? 0.0f : m_use[b], l_run[b]};
                __builtin_amdgcn_raw_buffer_store_b64(ml, prs, ml_at(mine, b), 0, kSc1);
            }
            // the stores have completed (written through) before the count
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __syncthreads();
            if (tid == 0) merge_flag = arrive_count(p.pf_count + wb.x, p.epoch) == (uint32_t)(wb.z - 1);
            __syncthreads();
            if (!merge_flag) continue;
#pragma unroll
            for (int b = 0; b < RB; b++) {
                float M = -INFINITY, den = 0.0f;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) o[b][dt] = (f32x16)0.0f;
                for (int k = 0; k < wb.z; k++) {
                    const f32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(prs, ml_at(wb.x + k, b), 0, kSc1);
                    f32x4 v[DT * 4];
#pragma unroll
                    for (int q = 0; q < DT * 4; q++)
                        v[q] = __builtin_amdgcn_raw_buffer_load_b128(prs, o_at(wb.x + k, b * DT * 4 + q), 0, kSc1);
                    const float Mn = fmaxf(M, ml[0]);
                    const float ca = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
                    const float cb = __builtin_amdgcn_exp2f(ml[0] - Mn);
                    den = den * ca + ml[1] * cb;
#pragma unroll
                    for (int dt = 0; dt < DT; dt++)
#pragma unroll
                        for (int qq = 0; qq < 4; qq++)
#pragma unroll
                            for (int r2 = 0; r2 < 4; r2++)
                                o[b][dt][4 * qq + r2] = o[b][dt][4 * qq + r2] * ca + v[dt * 4 + qq][r2] * cb;
                    M = Mn;
                }
                l_run[b] = den;
            }
        }

        // finish: O / l (l summed over the two lane halves) into the wave's
        // 32-row slice of the ring, idle since every wave left the tile loop
        // (the barrier after it), then out as whole rows: PIECES lanes store one
        // row with 16-byte stores, where the accumulator layout would have each
        // store instruction touch 32 rows.  Row r's 16-byte piece p sits at
        // p ^ (r % PIECES), so neither side's LDS accesses conflict.
        // A row with no key in range (window past the row) is 0/0, as the
        // reference's m/l bookkeeping gives.
        {
            // the lane's row and piece indices pass through an empty asm so the
            // compiler cannot compute this block's addresses ahead of the tile
            // loop (they would hold registers through it)
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int on = ln & 31, oh = ln >> 5;
            f16 *ot = ring_lds + wave * 32 * HD;
            const float l = l_run[0] + shfl_xor(l_run[0], 32);
            const float inv = 1.0f / l;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    f16x4 v;
#pragma unroll
                    for (int r2 = 0; r2 < 4; r2++) v[r2] = (f16)(o[0][dt][4 * q + r2] * inv);
                    *reinterpret_cast<f16x4 *>(ot + on * HD + (((4 * dt + q) ^ (on & (PIECES - 1))) << 3) + 4 * oh) = v;
                }
            constexpr int RPP = 64 / PIECES;  // rows per 64-lane pass
#pragma unroll
            for (int i = 0; i < 32 / RPP; i++) {
                const int rl = RPP * i + ln / PIECES, pc = ln % PIECES;
                const f16x8 v = *reinterpret_cast<const f16x8 *>(ot + rl * HD + ((pc ^ (rl & (PIECES - 1))) << 3));
                const int rr = wave * 32 + rl, tk = tok0 + rr / G;
                if (tk < tok_end)
                    *reinterpret_cast<f16x8 *>(static_cast<f16 *>(p.out) +
                                               ((int64_t)(ch.w + tk) * H + kvh * G + rr % G) * HD + 8 * pc) = v;
            }
        }
    }
}

}  // namespace pam
