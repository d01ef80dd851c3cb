// attention_body.h - device bodies of the paged-attention kernels (gfx950):
// row contexts, the MFMA tile loop (mfma_core), the workgroup-form item and
// the stream-K body.  Included by attention.hip (the library's kernels), by
// mixed.hip (one launch for a mixed step) and by the code-object entries.
#pragma once
#include "kernels.h"
#include "pam_device.h"

namespace pam {


// Token positions fit in 32 bits (sequence lengths are int32 at the boundary).
struct RowCtx {
    const int32_t *bt;
    int k_lo, k_hi;
    int out_row;
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
        c.k_lo = (int)ws;
        c.k_hi = (int)(L < cap ? L : cap);
        c.out_row = r;
    } else if (p.mode == kRowPrefill) {
        // one fixed window start for every row (PagedAttentionEngine.swift:802)
        const int64_t kv_len = (int64_t)p.q_offset + p.rows;
        c.bt = p.block_tables;
        c.k_lo = (int)(p.window > 0 ? (kv_len > p.window ? kv_len - p.window : 0) : 0);
        c.k_hi = (int)(p.causal ? (int64_t)p.q_offset + r + 1 : kv_len);
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
    int t_begin, t_end;  // 16-token tiles
    int nparts;
};

__device__ __forceinline__ PartRange part_range(const RowCtx &c, int part, int part_tokens) {
    PartRange pr;
    const int tile0 = c.k_lo / 16;
    const int tile_end = (c.k_hi + 15) / 16;
    const int ntiles = c.k_hi > c.k_lo ? tile_end - tile0 : 0;
    const int tpp = part_tokens / 16;
    pr.nparts = (ntiles + tpp - 1) / tpp;
    pr.t_begin = tile0 + part * tpp;
    pr.t_end = pr.t_begin + tpp < tile_end ? pr.t_begin + tpp : tile_end;
    return pr;
}

// Query-head slot v of kv head kvh in row out_row.  One layer (FL false): head
// kvh * G + v of p.q / p.out.  Fused layers (FL, decodeLayers): slots run over
// G * fused_layers heads, slot v being head kvh * G + v % G of layer v / G.
__device__ __forceinline__ int64_t head_elem(const AttnParams &p, int out_row, int kvh, int g) {
    return ((int64_t)out_row * p.num_heads + kvh * (p.num_heads / p.num_kv_heads) + g) * p.head_dim;
}
template <bool FL, typename T>
__device__ __forceinline__ const T *q_head(const AttnParams &p, int out_row, int kvh, int v) {
    if constexpr (!FL) {
        return static_cast<const T *>(p.q) + head_elem(p, out_row, kvh, v);
    } else {
        const int G = p.num_heads / p.num_kv_heads, layer = v / G;
        return static_cast<const T *>(p.layer_q[layer]) + head_elem(p, out_row, kvh, v - layer * G);
    }
}
template <bool FL, typename T>
__device__ __forceinline__ T *out_head(const AttnParams &p, int out_row, int kvh, int v) {
    if constexpr (!FL) {
        return static_cast<T *>(p.out) + head_elem(p, out_row, kvh, v);
    } else {
        const int G = p.num_heads / p.num_kv_heads, layer = v / G;
        return static_cast<T *>(p.layer_out[layer]) + head_elem(p, out_row, kvh, v - layer * G);
    }
}
// query-head slots per kv head
template <bool FL>
__device__ __forceinline__ int slot_group(const AttnParams &p) {
    return (p.num_heads / p.num_kv_heads) * (FL ? p.fused_layers : 1);
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

// ------------------------------------------------------------------ MFMA body


// Waves per workgroup of the MFMA kernels: in the workgroup form they split one
// partition's tiles and merge in LDS; in the stream-K form they read up to four
// kv heads of the same tiles side by side.
constexpr int kMfmaWaves = 4;
// lazy online softmax: the reference max moves only when a score passes it by
// this many log2 units, which bounds P by 2^8
constexpr float kLazyRescaleLog2 = 8.0f;
// Rows the stream-K form can index from LDS (its row prefix table).
constexpr int kStreamKMaxRows = 2048;
// Decode rows whose key ranges the stream-K form keeps in LDS (8 KiB: three
// workgroups of the e4m3 kernel still fit a CU).
constexpr int kStreamKRangeCache = 1024;
// Rounds of 64 pieces (256 floats) of a (row, kv head)'s partials that the
// stream-K merge folds together (its loads in flight per batch: 4 units x this).
// Measured on gfx950 against 1 and 4: 2 is best on c2, c4 and c5 (4 raises the
// kernel's registers to 254 and slows c2; d = 64, three workgroups per CU,
// spills at 4).
constexpr int kMergeRounds = 2;
// Fewest tiles per stream-K unit: shorter units would only add partials for
// the merge.  Measured on a batch-1 decode of 4096 tokens (32/8 heads): 8 tiles
// 26.4 us per adapter step, 16 tiles 23.6, 32 tiles 28.5; c2 and c4 unchanged.
constexpr int kStreamKMinTiles = 16;

// How a 16-token tile finds its physical blocks.
enum BlockMode : int {
    kBlkTile = 0,   // block_size a power of two >= 16: the whole tile lies in one block
    kBlkSmall = 1,  // block_size 8: two blocks per tile
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename KV, int HD>
struct MfmaShape {
    static constexpr int NC = HD / 32;                        // 16x16x32 chunks per S tile
    static constexpr int NO = HD / 16;                        // 16-dim output chunks
    static constexpr int EPL = 16 / KvTraits<KV>::kBytes;     // elements per 16-byte load
    static constexpr int LPR = HD / EPL;                      // lanes per token row (one 16-byte load each)
    static constexpr int RPI = 64 / LPR;                      // token rows per load instruction
    static constexpr int NI = 16 / RPI;                       // load instructions per 16-token tile
    static constexpr int KL = HD + 8;                         // K row in LDS (halves): odd 16-byte units
    static constexpr int VL = HD + 16;                        // V row in LDS (halves)
    static constexpr int NW = kMfmaWaves;
    // register tiles in flight per wave, and resident workgroups per CU the
    // registers allow (measured on gfx950: d = 128 runs best at two workgroups
    // per CU for both f16 and e4m3; a third e4m3 workgroup forces spills)
    static constexpr int DEPTH = (sizeof(KV) == 2 && HD <= 128) ? 3 : 2;
    static constexpr int OCC = HD >= 256 ? 1 : (HD == 128 ? 2 : 3);
    // stream-K workgroups launched per CU: f16 with d = 128 streams fastest with
    // one (four waves per CU: c2 and c5 8-9% faster than with two, e4m3, whose
    // dequantisation needs the second workgroup, 40% slower with one)
    static constexpr int GRID_PER_CU = (sizeof(KV) == 2 && HD == 128) ? 1 : OCC;
    static constexpr int WT = 16 * (KL + VL);                 // halves of one wave's K and V tiles
    static constexpr int kSmemBytes = NW * WT * 2 > NW * 16 * HD * 4 ? NW * WT * 2 : NW * 16 * HD * 4;
    static_assert(64 % LPR == 0 && 16 % RPI == 0, "token rows must tile the wave");
};

// The tile loop shared by both work forms: tiles [t_begin, t_end) of row
// context c for kv head kvh, on the calling wave alone, using its LDS tiles kt
// (K) and kt + 16 * KL (V).  Leaves the wave's online-softmax state: m_run (the
// reference max in log2 units, per head; l and O are relative to it, and it is
// -inf only while no key was seen), l_run (this lane's share of the row sum) and o[i], lane
// (head `lane % 16`, quad `lane / 16`) holding dims 16i + 4 quad .. +4.
//
// Loads: 16 lanes (8 for e4m3) cover one token row's HD elements with 16-byte
// loads, so each load instruction reads whole 256-byte rows (measured on
// gfx950: ~6.4 TB/s for this pattern against ~4.8 TB/s when one instruction
// gathers 64-byte slices of 16 rows).  The rows then pass through LDS: K is read
// back as the A operand of S^T = K Q^T (v_mfma_f32_16x16x32_f16, query heads on
// the N side) and V with the transposing ds_read_b64_tr_b16 as the A operand of
// O^T = V^T P^T (v_mfma_f32_16x16x16_f16), whose B operand is the S^T
// accumulator layout itself (lane%16 = head, lane/16 = token quad).
template <typename KV, int HD, int BLK, bool FL>
__device__ __forceinline__ void mfma_core(const AttnParams &p, const RowCtx &c, int kvh, const PartRange pr, f16 *kt,
                                          float &m_run, float &l_run, f32x4 (&o)[MfmaShape<KV, HD>::NO]) {
    using S = MfmaShape<KV, HD>;
    constexpr int NC = S::NC, NO = S::NO, EPL = S::EPL, LPR = S::LPR, RPI = S::RPI, NI = S::NI, KL = S::KL,
                  VL = S::VL;
    constexpr bool kFp8 = sizeof(KV) == 1;
    constexpr bool kTileScale = kFp8 && BLK == kBlkTile;  // one block (one scale pair) per tile
    const int lane = threadIdx.x & 63, row = lane & 15, grp = lane >> 4;
    // this lane's query-head slot (N column): a head of kv head kvh, of one of
    // the fused layers
    const bool head_ok = row < slot_group<FL>(p);
    f16 *vt = kt + 16 * KL;

    // Q^T B operand: lane holds Q[h][32c + 8g .. +8] for chunk c
    f16x8 qv[NC];
    {
        const f16 *qp = q_head<FL, f16>(p, c.out_row, kvh, head_ok ? row : 0) + 8 * grp;
#pragma unroll
        for (int i = 0; i < NC; i++) {
            f16x8 v = *reinterpret_cast<const f16x8 *>(qp + 32 * i);
            qv[i] = head_ok ? v : (f16x8)(f16)0.0f;
        }
    }

    const int64_t row_stride = (int64_t)p.num_kv_heads * HD;  // elements per token
    const char *kbase = static_cast<const char *>(p.k_pool);
    const char *vbase = static_cast<const char *>(p.v_pool);
    const int bs = p.block_size;
    const int bsh = __builtin_ctz(bs);  // block_size is a power of two
    const int lrow = lane / LPR, piece = lane % LPR;  // row within an instruction, 16-byte piece of the row

    // Raw loads stay untouched until they are consumed: any arithmetic on them
    // right after the load would make the wave wait for it there.  Lanes whose
    // token lies outside the key range read a zero page instead of the pool, so
    // no masking of loaded data is needed (their S entries become -inf anyway).
    struct Tile {
        u32x4 k[NI], v[NI];
        uint16_t ksb[kTileScale ? 1 : NI], vsb[kTileScale ? 1 : NI];
    };

    // Block-table entries of 64 consecutive blocks from window_blk sit in one
    // VGPR (lane i = block window_blk + i), refreshed once per 16-tile chunk, so
    // a tile's address never waits on a table load.  The window covers the
    // chunk's tiles and the tiles loaded ahead of its end.
    const int nlb = (c.k_hi + bs - 1) >> bsh;  // blocks holding keys of this row
    int window_blk = 0;
    int32_t bt_window = 0;
    auto refresh_window = [&](int tile) {
        window_blk = (tile * 16) >> bsh;
        const int idx = window_blk + lane < nlb ? window_blk + lane : nlb - 1;
        bt_window = c.bt[idx];
    };
    if (pr.t_begin < pr.t_end) refresh_window(pr.t_begin);

    // Tokens this wave may use: [k_lo, k_hi) cut to the partition.  Tiles past the
    // partition end are still "loaded" (from its last tile, a cache hit) so that
    // every step issues the same loads: with no load under a branch the compiler
    // can wait for exactly the tile it needs instead of draining all of them.
    const int j_hi = c.k_hi < pr.t_end * 16 ? c.k_hi : pr.t_end * 16;
    const uint32_t row_bytes = (uint32_t)(row_stride * KvTraits<KV>::kBytes);  // bytes per token row (< 2^32)
    const uint32_t lane_const = (uint32_t)(kvh * HD * KvTraits<KV>::kBytes + piece * 16);
    auto load_tile = [&](int tile, Tile &t) {
        const int lt = tile < pr.t_end ? tile : pr.t_end - 1;
        if constexpr (BLK == kBlkTile) {
            // One block holds the tile: a uniform base plus a per-lane 32-bit
            // offset.  Rows outside [k_lo, j_hi) read the nearest row inside
            // instead (finite data; their scores are masked to -inf, so their
            // probabilities are 0).
            const int phys = __builtin_amdgcn_readlane(bt_window, ((lt * 16) >> bsh) - window_blk);
            const uint64_t tile_off =
                (uint64_t)(((uint32_t)phys << bsh) + (uint32_t)((lt * 16) & (bs - 1))) * row_bytes;
            const int r_lo = c.k_lo - lt * 16 > 0 ? c.k_lo - lt * 16 : 0;
            const int r_hi = j_hi - lt * 16 < 16 ? j_hi - lt * 16 : 16;
            const char *kb = kbase + tile_off, *vb = vbase + tile_off;
#pragma unroll
            for (int u = 0; u < NI; u++) {
                int trow = u * RPI + lrow;
                trow = trow < r_lo ? r_lo : (trow >= r_hi ? r_hi - 1 : trow);
                const uint32_t off = (uint32_t)trow * row_bytes + lane_const;
                // K/V rows are read once per step (streaming): non-temporal loads
                // measured 2-7% faster on the e4m3 and long-window workloads
                t.k[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kb + off));
                t.v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vb + off));
            }
            if constexpr (kTileScale) {
                t.ksb[0] = p.k_scale[phys];
                t.vsb[0] = p.v_scale[phys];
            }
        } else {
            const char *zp = static_cast<const char *>(p.zero_page) + piece * 16;
#pragma unroll
            for (int u = 0; u < NI; u++) {
                const int trow = u * RPI + lrow;
                const int j = tile * 16 + trow;
                const bool valid = j >= c.k_lo && j < j_hi;
                const int jt = lt * 16 + trow;  // inside the window
                const int phys = __shfl(bt_window, (jt >> bsh) - window_blk, 64);
                const uint64_t off =
                    (uint64_t)(((uint32_t)phys << bsh) + (uint32_t)(jt & (bs - 1))) * row_bytes + lane_const;
                // Every lane loads unconditionally (loads under a branch would make
                // the compiler drain every outstanding load before each use):
                // masked lanes select the zero page.
                const uint64_t ka = valid ? (uint64_t)kbase + off : (uint64_t)zp;
                const uint64_t va = valid ? (uint64_t)vbase + off : (uint64_t)zp;
                t.k[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(ka));
                t.v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(va));
                if constexpr (kFp8) {
                    t.ksb[u] = p.k_scale[phys];
                    t.vsb[u] = p.v_scale[phys];
                }
            }
        }
    };
    // raw 16-byte pieces -> LDS rows (e4m3: widened to halves)
    auto stage_rows = [&](const u32x4 *raw, const uint16_t *sb, f16 tile_scale, f16 *dst, int ld) {
#pragma unroll
        for (int u = 0; u < NI; u++) {
            f16 *d = dst + (u * RPI + lrow) * ld + piece * EPL;
            if constexpr (!kFp8) {
                *reinterpret_cast<u32x4 *>(d) = raw[u];
            } else if constexpr (kTileScale) {
                // exact code value times the block scale in one binary16 multiply:
                // the reference's half dequantisation (two half products, the second
                // a power of two) up to results below the normal range
                const f16x8 s8 = (f16x8)tile_scale;
                *reinterpret_cast<f16x8 *>(d) = e4m3x8_to_f16x8(raw[u][0], raw[u][1]) * s8;
                *reinterpret_cast<f16x8 *>(d + 8) = e4m3x8_to_f16x8(raw[u][2], raw[u][3]) * s8;
            } else {
                const f16 sc = bits_to_f16(sb[u]);
                const uint32_t w[4] = {raw[u][0], raw[u][1], raw[u][2], raw[u][3]};
                f16x8 lo, hi;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    lo[i] = fp8_dequant((w[i >> 2] >> (8 * (i & 3))) & 0xFFu, sc);
                    hi[i] = fp8_dequant((w[2 + (i >> 2)] >> (8 * (i & 3))) & 0xFFu, sc);
                }
                *reinterpret_cast<f16x8 *>(d) = lo;
                *reinterpret_cast<f16x8 *>(d + 8) = hi;
            }
        }
    };

    m_run = -INFINITY;
    l_run = 0.0f;
#pragma unroll
    for (int i = 0; i < NO; i++) o[i] = (f32x4)0.0f;

    // DEPTH register tiles in flight per wave.  As soon as a tile's rows sit in
    // LDS, its registers are refilled with the tile DEPTH ahead, so the next
    // tiles are always loading while this one's scores, softmax and PV run.
    auto step = [&](int tile, Tile &t) {
        // keep the scheduler from hoisting the next tile's work (and with it the
        // wait for its loads) into this one
        __builtin_amdgcn_sched_barrier(0);
        // per-tile scales (a tile inside one block has one scale pair); otherwise
        // each row is dequantised on staging
        f16 ks = (f16)1.0f, vs = (f16)1.0f;
        if constexpr (kTileScale) {
            ks = bits_to_f16(t.ksb[0]);
            vs = bits_to_f16(t.vsb[0]);
        }
        stage_rows(t.k, t.ksb, ks, kt, KL);
        stage_rows(t.v, t.vsb, vs, vt, VL);
        // LDS ops of one wave execute in order; the wave barrier pins the compiler's
        __builtin_amdgcn_wave_barrier();
        load_tile(tile + S::DEPTH, t);
        // e4m3: the scores, softmax and PV run at raised wave priority, ahead
        // of the other waves' dequantising (c4 1% faster; f16 measured 0.9%
        // slower with it)
        if constexpr (kFp8) __builtin_amdgcn_s_setprio(1);

        // S^T[token][head] over HD dims: K row `row`, dims 32i + 8g .. +8
        f32x4 s = (f32x4)0.0f;
#pragma unroll
        for (int i = 0; i < NC; i++)
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const f16x8 *>(&kt[row * KL + 32 * i + 8 * grp]),
                                                       qv[i], s, 0, 0, 0);
        const float sc = p.scale_log2;

        // online softmax on this lane's 4 tokens of head `row`.  The reference
        // max m_run is raised (and l, O rescaled) only when a score passes it by
        // 2^8, so P <= 2^8 fits the f16 operand and most tiles skip the rescale.
        float sv[4];
        float mt = -INFINITY;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int j = tile * 16 + 4 * grp + q;
            sv[q] = (j >= c.k_lo && j < j_hi) ? s[q] * sc : -INFINITY;
            mt = fmaxf(mt, sv[q]);
        }
        if (__any(mt > m_run + kLazyRescaleLog2)) {  // wave-uniform, rare after the first tile
            mt = fmaxf(mt, shfl_xor(mt, 16));
            mt = fmaxf(mt, shfl_xor(mt, 32));
            const float m_new = mt > m_run + kLazyRescaleLog2 ? mt : m_run;
            // 1 for heads that keep their reference; 0 while m_run is unset (l, O are 0)
            const float corr = m_new == m_run ? 1.0f : exp2f(m_run - m_new);
            l_run *= corr;
#pragma unroll
            for (int i = 0; i < NO; i++) o[i] *= corr;
            m_run = m_new;
        }
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        f16x4 pb;
        float psum = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float pq = exp2f(sv[q] - m_use);
            psum += pq;
            pb[q] = (f16)pq;
        }
        l_run += psum;

        // V^T operand of dims 16i..: lane (o, g) addresses row 4g + o/4, dims
        // 16i + 4(o%4); the transposed load hands it tokens 4g..4g+3 of dim 16i + o
        const f16 *vrow = vt + (4 * grp + (row >> 2)) * VL + 4 * (row & 3);
#pragma unroll
        for (int i = 0; i < NO; i++)
            o[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(lds_read_tr16(vrow + 16 * i), pb, o[i], 0, 0, 0);
        if constexpr (kFp8) __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_wave_barrier();
    };

    // 15- or 16-tile chunks run as straight-line code: inside a chunk the compiler can
    // count outstanding loads exactly and waits only for the tile it consumes (a
    // loop back edge makes it drain everything).  Exits are uniform branches.
    if (pr.t_begin < pr.t_end) {
    constexpr int CH = S::DEPTH * (16 / S::DEPTH);  // tiles per straight-line chunk
    Tile ta, tb, tc;
    load_tile(pr.t_begin, ta);
    load_tile(pr.t_begin + 1, tb);
    if constexpr (S::DEPTH == 3) load_tile(pr.t_begin + 2, tc);
    for (int chunk = pr.t_begin; chunk < pr.t_end; chunk += CH) {
        // the window holds 64 blocks: refresh it only when this chunk's loads
        // (tiles up to chunk + CH - 1 + DEPTH) would leave it
        if (chunk != pr.t_begin) {
            const int far = chunk + CH - 1 + S::DEPTH < pr.t_end - 1 ? chunk + CH - 1 + S::DEPTH : pr.t_end - 1;
            if (((far * 16 + 15) >> bsh) - window_blk >= 64) refresh_window(chunk);
        }
#pragma unroll
        for (int k = 0; k < CH; k += S::DEPTH) {
            const int tile = chunk + k;
            if (k > 0 && tile >= pr.t_end) break;
            step(tile, ta);
            step(tile + 1, tb);  // tiles past the partition end are fully masked
            if constexpr (S::DEPTH == 3) step(tile + 2, tc);
        }
    }
    }
}

// One work item of the workgroup form: (row r, split-context partition `part`,
// kv head kvh) shared by the whole workgroup.  Each wave takes a contiguous
// share of the partition's tiles; the waves merge their softmax states in LDS
// and write the output (one partition) or the partial for the reduce kernel.
// Returns uniformly across the workgroup.
template <typename KV, int HD, int BLK>
__device__ __forceinline__ void mfma_item(const AttnParams &p, int r, int part, int kvh, char *smem,
                                          float (*sm_ml)[16][2]) {
    using S = MfmaShape<KV, HD>;
    constexpr int NO = S::NO, NW = S::NW, WT = S::WT;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63, row = lane & 15, grp = lane >> 4;
    const int H = p.num_heads;
    const int G = H / p.num_kv_heads;
    const RowCtx c = row_ctx(p, r);
    const PartRange wg = part_range(c, part, p.part_tokens);
    if (part >= (wg.nparts > 1 ? wg.nparts : 1)) return;
    const bool head_ok = row < G;
    f16 *out = static_cast<f16 *>(p.out);
    if (wg.nparts == 0) {
        // no keys: 0/0 as in the reference's m/l bookkeeping
        for (int idx = threadIdx.x; idx < G * HD; idx += 64 * NW)
            out[(c.out_row * H + kvh * G) * (int64_t)HD + idx] = (f16)__builtin_nanf("");
        return;
    }
    // this wave's contiguous share of the workgroup's tiles (possibly empty)
    PartRange pr = wg;
    {
        const int per = (wg.t_end - wg.t_begin + NW - 1) / NW;
        pr.t_begin = wg.t_begin + wave * per;
        pr.t_end = pr.t_begin + per < wg.t_end ? pr.t_begin + per : wg.t_end;
    }
    float m_run, l_run;
    f32x4 o[NO];
    mfma_core<KV, HD, BLK, false>(p, c, kvh, pr, reinterpret_cast<f16 *>(smem) + wave * WT, m_run, l_run, o);
    float l_tot = l_run + shfl_xor(l_run, 16);
    l_tot += shfl_xor(l_tot, 32);


    // Merge the waves' states.  The merge area overlays the K/V tiles, so every
    // wave must be done with its tiles first.
    __syncthreads();
    float *mo = reinterpret_cast<float *>(smem);  // [NW][16][HD]
    if (head_ok) {
        float *dst = mo + (wave * 16 + row) * HD + 4 * grp;
#pragma unroll
        for (int i = 0; i < NO; i++) *reinterpret_cast<f32x4 *>(dst + 16 * i) = o[i];
        if (grp == 0) {
            sm_ml[wave][row][0] = m_run;
            sm_ml[wave][row][1] = l_tot;
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x * 4; idx < G * HD; idx += 64 * NW * 4) {
        const int hh = idx / HD, d = idx % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, sm_ml[w][hh][0]);
        float den = 0.0f, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float mw = sm_ml[w][hh][0];
            const float wt = mw == -INFINITY ? 0.0f : exp2f(mw - M);
            den += wt * sm_ml[w][hh][1];
            const f32x4 v = *reinterpret_cast<const f32x4 *>(mo + (w * 16 + hh) * HD + d);
#pragma unroll
            for (int q = 0; q < 4; q++) acc[q] += wt * v[q];
        }
        const int hq = kvh * G + hh;
        if (wg.nparts == 1) {
            const float inv = 1.0f / den;
            f16x4 v;
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = (f16)(acc[q] * inv);
            *reinterpret_cast<f16x4 *>(out + (c.out_row * H + hq) * (int64_t)HD + d) = v;
        } else {
            const int64_t slot = ((int64_t)r * H + hq) * p.max_parts + part;
            *reinterpret_cast<f32x4 *>(p.part_o + slot * HD + d) = (f32x4){acc[0], acc[1], acc[2], acc[3]};
            if (d == 0) {
                p.part_ml[slot * 2 + 0] = M;
                p.part_ml[slot * 2 + 1] = den;
            }
        }
    }
}


// Stream-K partials are accessed with kSc1 (agent scope); offsets are bytes
// from the partial area's base (< 2 GiB).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const AttnParams &p) {
    return __builtin_amdgcn_make_buffer_rsrc(p.part_o, 0, (int)p.part_bytes, 0x00020000);
}

// Stream-K form (rows <= kStreamKMaxRows).  The key tiles of all rows are laid
// end to end on one line, row after row.  The workgroups are taken in runs of
// NHG = Hkv / NH (NH = 4, 2 or 1 kv heads, the largest dividing Hkv, read side by
// side by the NH waves of a workgroup): the run of unit u covers tiles
// [u T / U, (u + 1) T / U) of the line, one workgroup per head group, so all
// heads of a tile are read at about the same time.  Every wave streams the same
// number of tiles (+-1) whatever the row lengths, and no wave waits on another.
//
// A unit that covers part of a row leaves a partial softmax state per head.
// It is written with write-through stores, then the (row, kv head) counter is
// incremented; the wave that brings it to the number of units covering the row
// merges all partials with the whole wave (write-through loads) and writes the
// output.  Counters carry the launch's epoch (arrive_count), so none is ever
// reset.  A row inside one unit is finished in registers.  No reduce kernel runs.  The partials of (unit u, row r) sit in slot
// block u + r, unique because a row's units start where the previous row's end:
// floats [((u + r) * Hkv + kvh) * G + g] * d for query head g of kv head kvh.
//
// NW waves per workgroup and room for MAXR rows in LDS; the workgroup is number
// `bid` of the `nblk` that share the rows (the whole grid, or the decode part of
// a mixed-step launch).
template <typename KV, int HD, int BLK, bool FL, int NW = kMfmaWaves, int MAXR = kStreamKMaxRows>
__device__ __forceinline__ void streamk_body(const AttnParams &p, const int bid, const int nblk) {
    using S = MfmaShape<KV, HD>;
    constexpr int NO = S::NO, WT = S::WT;
    __shared__ __attribute__((aligned(16))) f16 tiles[NW * WT];
    __shared__ int32_t prefix[MAXR + 1];
    constexpr int RC = MAXR < kStreamKRangeCache ? MAXR : kStreamKRangeCache;
    __shared__ int2 key_range[RC];  // decode rows: {k_lo, k_hi}
    __shared__ int32_t wave_sum[NW];
    constexpr int NT = 64 * NW;
    const int tid = threadIdx.x;
    const int rows = p.rows;
    const bool cached = p.mode == kRowDecode && rows <= RC;
    // tiles per row (0 for a row without keys), prefix-summed in LDS: each
    // thread counts a contiguous run of rows, a wave scan plus the totals of
    // the waves before it place the runs
    const int per = (rows + NT - 1) / NT;
    const int r0 = tid * per, r1 = r0 + per < rows ? r0 + per : rows;
    int32_t run = 0;
    for (int rr = r0; rr < r1; rr++) {
        const RowCtx c = row_ctx(p, rr);
        const PartRange whole = part_range(c, 0, 1 << 30);
        if (cached) key_range[rr] = make_int2(c.k_lo, c.k_hi);
        prefix[rr] = run;
        run += whole.nparts > 0 ? whole.t_end - whole.t_begin : 0;
    }
    int32_t incl = run;  // inclusive scan over the wave's lanes
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int32_t v = __shfl_up(incl, off, 64);
        if ((tid & 63) >= off) incl += v;
    }
    if ((tid & 63) == 63) wave_sum[tid >> 6] = incl;
    __syncthreads();
    int32_t base = incl - run;
    for (int w = 0; w < (tid >> 6); w++) base += wave_sum[w];
    for (int rr = r0; rr < r1; rr++) prefix[rr] += base;
    if (tid == NT - 1) prefix[rows] = base + run;
    __syncthreads();
    // row context from the LDS copy where there is one (no global load)
    auto ctx_of = [&](int r) -> RowCtx {
        if (!cached) return row_ctx(p, r);
        RowCtx c;
        c.bt = p.block_tables + (int64_t)r * p.bt_stride;
        c.k_lo = key_range[r].x;
        c.k_hi = key_range[r].y;
        c.out_row = r;
        return c;
    };

    const int H = p.num_heads, Hkv = p.num_kv_heads;
    const int G = slot_group<FL>(p);  // query-head slots per kv head (all fused layers)
    const int nl = FL ? p.fused_layers : 1;
    // rows without keys: 0/0 as in the reference's m/l bookkeeping
    for (int rr = bid; rr < rows; rr += nblk)
        if (prefix[rr + 1] == prefix[rr]) {
            const int orow = ctx_of(rr).out_row;
            for (int l = 0; l < nl; l++) {
                f16 *ob = out_head<FL, f16>(p, orow, 0, l * (H / Hkv));
                for (int idx = tid; idx < H * HD; idx += NT) ob[idx] = (f16)__builtin_nanf("");
            }
        }

    const int NH = Hkv % 4 == 0 ? 4 : (Hkv % 2 == 0 ? 2 : 1);
    const int WPH = NW / NH, NHG = Hkv / NH;
    // wave-uniform values read from LDS are moved to scalar registers
    const int64_t T = __builtin_amdgcn_readfirstlane(prefix[rows]);
    int64_t U = (int64_t)nblk * WPH / NHG;
    const int64_t u_cap = (T + kStreamKMinTiles - 1) / kStreamKMinTiles;
    if (U > u_cap) U = u_cap;
    const int wave = tid >> 6, lane = tid & 63, row = lane & 15, grp = lane >> 4;
    const int64_t wu = (int64_t)bid * WPH + wave / NH;  // workgroup unit
    const int64_t u = wu / NHG;
    const int kvh = (int)(wu % NHG) * NH + wave % NH;
    if (u >= U) return;  // no workgroup barrier follows
    const bool head_ok = row < G;
    f16 *kt = tiles + wave * WT;
    const __amdgpu_buffer_rsrc_t prs = part_rsrc(p);
    const int ml_off = (int)((const char *)p.part_ml - (const char *)p.part_o);  // bytes

    const int64_t x1 = (u + 1) * T / U;
    for (int64_t x = u * T / U; x < x1;) {
        // the row holding line position x: last r with prefix[r] <= x
        int lo = 0, hi = rows;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (prefix[mid] <= x) lo = mid;
            else hi = mid;
        }
        lo = __builtin_amdgcn_readfirstlane(lo);
        const int64_t P = __builtin_amdgcn_readfirstlane(prefix[lo]);
        const int nt = __builtin_amdgcn_readfirstlane(prefix[lo + 1]) - (int)P;  // > 0: x lies inside this row
        const int64_t e = x1 < P + nt ? x1 : P + nt;
        const RowCtx c = ctx_of(lo);
        const int tile0 = c.k_lo / 16;
        PartRange pr;
        pr.t_begin = tile0 + (int)(x - P);
        pr.t_end = tile0 + (int)(e - P);
        pr.nparts = 1;
        const int64_t first = ((P + 1) * U - 1) / T, last = ((P + nt) * U - 1) / T;
        const int nseg = (int)(last - first + 1);
        x = e;

        float m_run, l_run;
        f32x4 o[NO];
        mfma_core<KV, HD, BLK, FL>(p, c, kvh, pr, kt, m_run, l_run, o);
        float l_tot = l_run + shfl_xor(l_run, 16);
        l_tot += shfl_xor(l_tot, 32);
        if (nseg == 1) {
            if (head_ok) {
                f16 *oh = out_head<FL, f16>(p, c.out_row, kvh, row);
                const float inv = 1.0f / l_tot;
#pragma unroll
                for (int i = 0; i < NO; i++) {
                    f16x4 v;
#pragma unroll
                    for (int q = 0; q < 4; q++) v[q] = (f16)(o[i][q] * inv);
                    *reinterpret_cast<f16x4 *>(oh + 16 * i + 4 * grp) = v;
                }
            }
            continue;
        }
        // publish this unit's partial and count it
        auto slot0 = [&](int64_t uu) { return ((uu + lo) * Hkv + kvh) * (int64_t)G; };  // head g: + g
        if (head_ok) {
            const int ob = (int)((slot0(u) + row) * HD * 4) + 16 * grp;
#pragma unroll
            for (int i = 0; i < NO; i++) __builtin_amdgcn_raw_buffer_store_b128(o[i], prs, ob + 64 * i, 0, kSc1);
            if (grp == 0) {
                const f32x2 ml = {m_run, l_tot};
                __builtin_amdgcn_raw_buffer_store_b64(ml, prs, ml_off + (int)((slot0(u) + row) * 8), 0, kSc1);
            }
        }
        // the stores have completed (written through) before the count
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        uint32_t before = 0;
        if (lane == 0) before = arrive_count(p.seg_count + (int64_t)lo * Hkv + kvh, p.epoch);
        before = __builtin_amdgcn_readfirstlane(before);
        if (before != (uint32_t)(nseg - 1)) continue;

        // Last unit of this (row, kv head): merge all partials, the whole wave at
        // once.  The G * HD floats of one unit are contiguous; the lane owns the
        // 4-float pieces v = lane + 64 k (head 4v / HD).  Up to kMergeRounds
        // rounds k are merged together, four units at a time, so every batch of
        // loads covers 4 * kMergeRounds partials (the merge's dependent load
        // batches, not its arithmetic, set its time).  Each piece folds the
        // units in ascending order: the result does not depend on the batching.
        constexpr int R = kMergeRounds;
        const int nv = G * HD / 4, rounds = (nv + 63) / 64;
        for (int k0 = 0; k0 < rounds; k0 += R) {
            int v[R], g[R];
            float M[R], den[R];
            f32x4 acc[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int kv = lane + 64 * (k0 + r);
                v[r] = kv < nv ? kv : lane;  // inactive lanes (and rounds) re-read piece `lane`
                g[r] = (4 * v[r]) / HD;
                M[r] = -INFINITY;
                den[r] = 0.0f;
                acc[r] = (f32x4)0.0f;
            }
            auto fold = [&](int r, const f32x2 ml, const f32x4 ov) {
                const float Mn = fmaxf(M[r], ml[0]);
                const float a = M[r] == -INFINITY ? 0.0f : exp2f(M[r] - Mn);
                const float b = ml[0] == -INFINITY ? 0.0f : exp2f(ml[0] - Mn);
                den[r] = den[r] * a + ml[1] * b;
                acc[r] = acc[r] * a + ov * b;
                M[r] = Mn;
            };
            auto ld_ml = [&](int64_t uu, int r) {
                return __builtin_amdgcn_raw_buffer_load_b64(prs, ml_off + (int)((slot0(uu) + g[r]) * 8), 0, kSc1);
            };
            auto ld_o = [&](int64_t uu, int r) {
                return __builtin_amdgcn_raw_buffer_load_b128(prs, (int)(slot0(uu) * HD * 4) + 16 * v[r], 0, kSc1);
            };
            int64_t uu = first;
            for (; uu + 3 <= last; uu += 4) {
                f32x2 m[4][R];
                f32x4 o[4][R];
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        m[j][r] = ld_ml(uu + j, r);
                        o[j][r] = ld_o(uu + j, r);
                    }
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int r = 0; r < R; r++) fold(r, m[j][r], o[j][r]);
            }
            for (; uu <= last; uu++) {
                f32x2 m[R];
                f32x4 o[R];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    m[r] = ld_ml(uu, r);
                    o[r] = ld_o(uu, r);
                }
#pragma unroll
                for (int r = 0; r < R; r++) fold(r, m[r], o[r]);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                if (lane + 64 * (k0 + r) < nv) {
                    const float inv = 1.0f / den[r];
                    f16x4 h;
#pragma unroll
                    for (int q = 0; q < 4; q++) h[q] = (f16)(acc[r][q] * inv);
                    *reinterpret_cast<f16x4 *>(out_head<FL, f16>(p, c.out_row, kvh, g[r]) + (4 * v[r] - g[r] * HD)) = h;
                }
            }
        }
    }
}

}  // namespace pam
