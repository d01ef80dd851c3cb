// backward.hip - gradients of paged attention for gfx950 (training path).
//
// Semantics of paged_attention_backward{,_f16} (kernels.metal:1217-1415): rows
// i < seq_len of one sequence attend, without a causal mask, over keys
// j in [window_start, seq_len) of the block table (window_start =
// max(0, seq_len - W)); the forward's row max m and sum l (natural-log units,
// scores scaled by 1/sqrt(d)) are inputs.  With P_ij = exp(s_ij - m_i) / l_i,
// dP_ij = dO_i . v_j and D_i = sum_j P_ij dP_ij:
//   dQ_i = scale sum_j P_ij (dP_ij - D_i) k_j               (written)
//   dK_j += scale sum_{i, heads of kv group} dS_ij q_i        (accumulated in the pool)
//   dV_j += sum_{i, heads of kv group} P_ij dO_i
//
// The reference adds every (i, j) contribution to dK/dV with an atomic (for f16
// a half add, rounding each term).  Here two kernels need no atomics:
//   * bwd_rows_kernel: one wave per (row, head) computes D and dQ;
//   * bwd_keys_kernel: one wave per (key, kv head) recomputes P and dS over the
//     rows of its head group and adds its dK/dV row to the pool once, summed in
//     f32.
// Lanes hold dims lane + 64 t of the head (t < 4, d <= 256); dot products are
// wave reductions, loads of a key or query row are 64 lanes over contiguous dims.
#include <type_traits>

#include "kernels.h"
#include "pam_device.h"

namespace pam {

constexpr int kBwdMaxDims = 4;  // dims per lane: head_dim <= 256

template <typename T>
__device__ __forceinline__ float ld(const T *p) { return (float)*p; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// pool row of token j of kv head g
template <typename T>
__device__ __forceinline__ const T *pool_row(const T *pool, const BackwardParams &p, int j, int g) {
    const int64_t phys = p.block_table[j / p.block_size];
    return pool + ((phys * p.block_size + j % p.block_size) * p.num_kv_heads + g) * (int64_t)p.head_dim;
}

template <typename T>
__global__ __launch_bounds__(64) void bwd_rows_kernel(BackwardParams p) {
    const int i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int d = p.head_dim, g = h / (p.num_heads / p.num_kv_heads);
    const T *Q = static_cast<const T *>(p.q), *dO = static_cast<const T *>(p.d_out);
    const T *K = static_cast<const T *>(p.k_pool), *V = static_cast<const T *>(p.v_pool);
    const int64_t qo = ((int64_t)i * p.num_heads + h) * d;
    float q[kBwdMaxDims], go[kBwdMaxDims], dq[kBwdMaxDims];
#pragma unroll
    for (int t = 0; t < kBwdMaxDims; t++) {
        const int e = lane + 64 * t;
        q[t] = e < d ? ld(Q + qo + e) : 0.0f;
        go[t] = e < d ? ld(dO + qo + e) : 0.0f;
        dq[t] = 0.0f;
    }
    const float m = p.m[(int64_t)i * p.num_heads + h], l = p.l[(int64_t)i * p.num_heads + h];
    const float scale = p.scale;
    // pass 1: D = sum_j P dP
    float D = 0.0f;
    for (int j = p.window_start; j < p.seq_len; j++) {
        const T *kr = pool_row(K, p, j, g), *vr = pool_row(V, p, j, g);
        float s = 0.0f, dp = 0.0f;
#pragma unroll
        for (int t = 0; t < kBwdMaxDims; t++) {
            const int e = lane + 64 * t;
            if (e < d) {
                s += q[t] * ld(kr + e);
                dp += go[t] * ld(vr + e);
            }
        }
        s = wave_sum(s);
        dp = wave_sum(dp);
        D += __expf(s * scale - m) / l * dp;
    }
    // pass 2: dQ = scale sum_j dS k
    for (int j = p.window_start; j < p.seq_len; j++) {
        const T *kr = pool_row(K, p, j, g), *vr = pool_row(V, p, j, g);
        float kv[kBwdMaxDims], s = 0.0f, dp = 0.0f;
#pragma unroll
        for (int t = 0; t < kBwdMaxDims; t++) {
            const int e = lane + 64 * t;
            kv[t] = e < d ? ld(kr + e) : 0.0f;
            s += q[t] * kv[t];
            dp += e < d ? go[t] * ld(vr + e) : 0.0f;
        }
        s = wave_sum(s);
        dp = wave_sum(dp);
        const float P = __expf(s * scale - m) / l;
        const float dS = P * (dp - D);
#pragma unroll
        for (int t = 0; t < kBwdMaxDims; t++) dq[t] += dS * kv[t];
    }
    T *dQ = static_cast<T *>(p.d_q);
#pragma unroll
    for (int t = 0; t < kBwdMaxDims; t++) {
        const int e = lane + 64 * t;
        if (e < d) dQ[qo + e] = (T)(dq[t] * scale);
    }
    if (lane == 0) p.row_d[(int64_t)i * p.num_heads + h] = D;
}

template <typename T>
__global__ __launch_bounds__(64) void bwd_keys_kernel(BackwardParams p) {
    const int j = p.window_start + blockIdx.x, g = blockIdx.y, lane = threadIdx.x;
    const int d = p.head_dim, G = p.num_heads / p.num_kv_heads;
    const T *Q = static_cast<const T *>(p.q), *dO = static_cast<const T *>(p.d_out);
    const T *kr = pool_row(static_cast<const T *>(p.k_pool), p, j, g);
    const T *vr = pool_row(static_cast<const T *>(p.v_pool), p, j, g);
    float k[kBwdMaxDims], v[kBwdMaxDims], dk[kBwdMaxDims], dv[kBwdMaxDims];
#pragma unroll
    for (int t = 0; t < kBwdMaxDims; t++) {
        const int e = lane + 64 * t;
        k[t] = e < d ? ld(kr + e) : 0.0f;
        v[t] = e < d ? ld(vr + e) : 0.0f;
        dk[t] = dv[t] = 0.0f;
    }
    const float scale = p.scale;
    for (int i = 0; i < p.seq_len; i++) {
        for (int h = g * G; h < (g + 1) * G; h++) {
            const int64_t qo = ((int64_t)i * p.num_heads + h) * d;
            float q[kBwdMaxDims], go[kBwdMaxDims], s = 0.0f, dp = 0.0f;
#pragma unroll
            for (int t = 0; t < kBwdMaxDims; t++) {
                const int e = lane + 64 * t;
                q[t] = e < d ? ld(Q + qo + e) : 0.0f;
                go[t] = e < d ? ld(dO + qo + e) : 0.0f;
                s += q[t] * k[t];
                dp += go[t] * v[t];
            }
            s = wave_sum(s);
            dp = wave_sum(dp);
            const int64_t r = (int64_t)i * p.num_heads + h;
            const float P = __expf(s * scale - p.m[r]) / p.l[r];
            const float dS = P * (dp - p.row_d[r]);
#pragma unroll
            for (int t = 0; t < kBwdMaxDims; t++) {
                dk[t] += dS * q[t];
                dv[t] += P * go[t];
            }
        }
    }
    // this wave alone owns the (key, kv head) row of the gradient pools
    T *dkr = const_cast<T *>(pool_row(static_cast<const T *>(p.d_k_pool), p, j, g));
    T *dvr = const_cast<T *>(pool_row(static_cast<const T *>(p.d_v_pool), p, j, g));
#pragma unroll
    for (int t = 0; t < kBwdMaxDims; t++) {
        const int e = lane + 64 * t;
        if (e < d) {
            dkr[e] = (T)((float)dkr[e] + dk[t] * scale);
            dvr[e] = (T)((float)dvr[e] + dv[t]);
        }
    }
}

// ---------------------------------------------------------------- MFMA path
// f16 caches with d = 128 run on v_mfma_f32_32x32x16_f16 in two kernels, the
// same split of the work as above (no atomics):
//   * bwd_dq_mfma: a wave owns 32 query rows (token, head) of one kv head and
//     walks the key tiles twice: pass 1 sums D_i = sum_j P_ij dP_ij, pass 2 adds
//     dQ^T += K^T dS^T.  Per 32-key tile S^T = K Q^T and dP^T = V dO^T (K and V
//     tiles in LDS as A operands, Q^T and dO^T in registers as B operands); the
//     S^T accumulator layout is the B-operand layout of the dS^T chunk, so dS
//     never leaves registers (the forward prefill's P^T arrangement).  It writes
//     D and c_i = m_i log2(e) + log2(l_i) for the second kernel.
//   * bwd_dkv_mfma: a wave owns 32 keys of one kv head, keeps K^T and V^T in
//     registers as B operands and walks the 32-row tiles of all the group's
//     query rows: S = Q K^T, dP = dO V^T (Q and dO tiles in LDS), then
//     dV^T += dO^T P and dK^T += Q^T dS with dO^T and Q^T read transposed
//     (ds_read_b64_tr_b16), software-pipelined across row tiles.  It adds its
//     rows to the gradient pools once.
// P and dS enter the MFMA as binary16 scaled by 2^8 (P <= 1; the scale keeps
// small probabilities of long rows out of the subnormal range) and the
// accumulators are scaled back at the end.
typedef float bw_f32x16 __attribute__((ext_vector_type(16)));
constexpr int kBwdWaves = 4;             // waves per workgroup, 32 rows / keys each
constexpr float kBwdPScale = 256.0f;
constexpr float kPScaleLog2 = 8.0f;  // log2(kBwdPScale)
constexpr int kBwdRing = 4;                // LDS tiles per operand (kBwdRing - 1 loads in flight)
constexpr int kBwdBtCache = 8192;          // block-table entries the dQ kernel can keep in LDS
constexpr int kBwdBtCacheSmall = 2048;     // ... in its two-workgroups-per-CU form

// LDS tile of 32 rows x 128 halves; 16-byte piece p of row r sits at
// p ^ (4 (r % 4) + (r / 4) % 4): 16 consecutive rows reading one piece
// (operand rows, ds_read_b128) hit 16 different bank groups, and the 4 rows x
// 64 bytes of a 32-lane transposed read cover all banks once.
__device__ __forceinline__ int bw_at(int row, int piece) {
    const int swz = ((row & 3) << 2) | ((row >> 2) & 3);
    return row * 128 + ((piece ^ swz) << 3);
}

__device__ __forceinline__ bw_f32x16 bw_mfma(const f16x8 a, const f16x8 b, const bw_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Transposed operand (32 dims of dim tile dt x 16 rows of row chunk c) of a
// tile: lane (o = lane % 16, hh = (lane / 16) % 2, h = lane / 32) reads rows
// 16c + 4h + o/4 (+ 8) at dims 32dt + 16hh + 4(o % 4), the k order of the
// accumulator-as-B-operand chunks.
struct TrAddr {
    int lo[4], hi[4];
};
__device__ __forceinline__ TrAddr tr_addr(int lane) {
    TrAddr a;
    const int o = lane & 15, hh = (lane >> 4) & 1, h = lane >> 5;
    const int row = 4 * h + (o >> 2);
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
        const int piece = 4 * dt + 2 * hh + ((o & 3) >> 1);
        a.lo[dt] = bw_at(row, piece) + 4 * (o & 1);
        a.hi[dt] = bw_at(row + 8, piece) + 4 * (o & 1);
    }
    return a;
}
__device__ __forceinline__ f16x8 tr_operand(const f16 *tile, const TrAddr &a, int dt, int c) {
    const f16x4 lo = lds_read_tr16(tile + a.lo[dt] + 16 * c * 128);
    const f16x4 hi = lds_read_tr16(tile + a.hi[dt] + 16 * c * 128);
    return (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// accumulator register r of a 32x32 tile holds row 8 (r / 4) + 4 h + r % 4 of
// the lane's column; the 8 registers of chunk c as a B operand (binary16)
__device__ __forceinline__ void to_chunks(const bw_f32x16 &v, f16x8 (&out)[2]) {
#pragma unroll
    for (int r = 0; r < 16; r++) out[r >> 3][r & 7] = (f16)v[r];
}

// Workgroup barrier for the LDS rings: this wave's LDS reads and all but its
// last `N` loads are complete, then every wave arrives.  A __syncthreads would
// not do: the compiler does not count the inline-assembly loads, so it emits
// no wait for them.
template <int N>
__device__ __forceinline__ void ring_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Loads of one 32-row tile (8 KB) of a [row][128] f16 operand into `tile`, two
// instructions per wave: instruction i of wave w fills rows 4 (2w + i) .. +3,
// lane L the 16-byte slot L % 16 of row 4 (2w + i) + L / 16, which holds
// logical piece (L % 16) ^ swz(row) (bw_at's layout).  `row_ptr(r)` gives the
// global address of tile row r.
template <typename F>
__device__ __forceinline__ void tile_dma(f16 *tile, int wave, int lane, F row_ptr) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int blk = 2 * wave + i, R = 4 * blk + (lane >> 4), S = lane & 15;
        const int piece = S ^ (((R & 3) << 2) | ((R >> 2) & 3));
        lds_dma16(row_ptr(R) + 8 * piece, tile + 512 * blk);
    }
}

// BT block-table entries in LDS: with kBwdBtCacheSmall two workgroups fit a CU
// (registers and LDS), which measured 12% faster at T = 4096; longer tables take
// the one-workgroup form.
template <int NB, int BT>
__global__ __launch_bounds__(64 * kBwdWaves, BT == kBwdBtCacheSmall ? 2 : 1) void bwd_dq_mfma(BackwardParams p,
                                                                                              int group_shift) {
    __shared__ __attribute__((aligned(16))) f16 k_lds[kBwdRing][32 * 128];
    __shared__ __attribute__((aligned(16))) f16 v_lds[kBwdRing][32 * 128];
    __shared__ int32_t bt_lds[BT];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
    const int H = p.num_heads, G = 1 << group_shift, kvh = blockIdx.y;
    const int T = p.seq_len, ws = p.window_start, bs = p.block_size;
    const int rows = T * G;
    const f16 *Q = static_cast<const f16 *>(p.q), *dO = static_cast<const f16 *>(p.d_out);
    const f16 *K = static_cast<const f16 *>(p.k_pool), *V = static_cast<const f16 *>(p.v_pool);
    // the sequence's block-table entries from the window start on
    const int blk0 = ws / bs, nblk = (T - 1) / bs - blk0 + 1;
    for (int i = tid; i < nblk; i += 64 * kBwdWaves) bt_lds[i] = p.block_table[blk0 + i];
    // the wave's NB blocks of 32 rows; lane n's row of block b: token r / G, head r % G
    bool row_ok[NB];
    int64_t qo[NB], so[NB];
    f16x8 qv[NB][8], gv[NB][8];
    float crow[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int r = ((blockIdx.x * kBwdWaves + wave) * NB + b) * 32 + n;
        row_ok[b] = r < rows;
        const int tok = row_ok[b] ? r >> group_shift : 0, hq = kvh * G + (row_ok[b] ? r & (G - 1) : 0);
        so[b] = (int64_t)tok * H + hq;
        qo[b] = so[b] * 128;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            qv[b][c] = row_ok[b] ? *reinterpret_cast<const f16x8 *>(Q + qo[b] + 16 * c + 8 * h) : (f16x8)(f16)0.0f;
            gv[b][c] = row_ok[b] ? *reinterpret_cast<const f16x8 *>(dO + qo[b] + 16 * c + 8 * h) : (f16x8)(f16)0.0f;
        }
        crow[b] = row_ok[b] ? p.m[so[b]] * kLog2e + __builtin_log2f(p.l[so[b]]) : INFINITY;
    }
    const float sl2 = p.scale * kLog2e;
    __syncthreads();  // bt_lds
    const int t0 = ws / 32, t1 = (T + 31) / 32, NT = t1 - t0, NI = 2 * NT;
    // iteration it reads key tile t0 + it % NT (both passes) from ring slot it % kBwdRing
    // The lane's two tile rows (tile_dma's map) and 16-byte pieces, fixed for the
    // kernel; per tile only the key, its block-table entry and one multiply-add
    // remain.  Blocks are a power of two in tokens.
    const int bsh = __builtin_ctz((unsigned)bs);
    const int64_t row_stride = (int64_t)p.num_kv_heads * 128;  // halves per pool row
    int dma_row[2], dma_off[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int blk = 2 * wave + i, R = 4 * blk + (lane >> 4);
        dma_row[i] = R;
        dma_off[i] = kvh * 128 + 8 * ((lane & 15) ^ (((R & 3) << 2) | ((R >> 2) & 3)));
    }
    auto issue = [&](int it) {
        const int t = t0 + (it < NI ? it : NI - 1) % NT, slot = it % kBwdRing;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int j = t * 32 + dma_row[i];
            j = j < ws ? ws : (j >= T ? T - 1 : j);  // finite rows outside the keys (masked)
            const int64_t row = ((int64_t)bt_lds[(j >> bsh) - blk0] << bsh) | (j & (bs - 1));
            const int64_t o = row * row_stride + dma_off[i];
            lds_dma16(K + o, k_lds[slot] + 512 * (2 * wave + i));
            lds_dma16(V + o, v_lds[slot] + 512 * (2 * wave + i));
        }
    };
    const TrAddr ta = tr_addr(lane);
    bw_f32x16 dq[NB][4];
    float dsum[NB], D[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        dsum[b] = D[b] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) dq[b][dt] = (bw_f32x16)0.0f;
    }
    // the operand loads are complete before the ring starts (as in bwd_dkv_mfma)
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
        for (int c = 0; c < 8; c++) asm volatile("" ::"v"(qv[b][c]), "v"(gv[b][c]));
        asm volatile("" ::"v"(crow[b]));
    }
#pragma unroll
    for (int u = 0; u < kBwdRing - 1; u++) issue(u);
    // scores and 2^8 P of iteration it's tile (P straight from the exponential, c - 8)
    auto tile_probs = [&](int it, bw_f32x16 (&s)[NB], bw_f32x16 (&dp)[NB]) {
        const int t = t0 + it % NT, slot = it % kBwdRing;
        const f16 *kt = k_lds[slot], *vt = v_lds[slot];
#pragma unroll
        for (int b = 0; b < NB; b++) s[b] = dp[b] = (bw_f32x16)0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const f16x8 ka = *reinterpret_cast<const f16x8 *>(&kt[bw_at(n, 2 * c + h)]);
            const f16x8 va = *reinterpret_cast<const f16x8 *>(&vt[bw_at(n, 2 * c + h)]);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                s[b] = bw_mfma(ka, qv[b][c], s[b]);
                dp[b] = bw_mfma(va, gv[b][c], dp[b]);
            }
        }
        auto probs = [&](auto edge) {
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int r2 = 0; r2 < 16; r2++) {
                    float pr = __builtin_amdgcn_exp2f(fmaf(s[b][r2], sl2, kPScaleLog2 - crow[b]));
                    if (decltype(edge)::value) {
                        const int j = t * 32 + 8 * (r2 >> 2) + 4 * h + (r2 & 3);
                        pr = (j >= ws && j < T) ? pr : 0.0f;
                    }
                    s[b][r2] = pr;
                }
        };
        if (t * 32 < ws || t * 32 + 32 > T)
            probs(std::true_type{});
        else
            probs(std::false_type{});
    };
    // The two passes are two loops over the same ring (iterations 0 .. NT - 1,
    // then NT .. 2 NT - 1): at each barrier this wave's loads of the iteration's
    // tile are done (4 loads per tile), then every wave's, and every wave has
    // finished the iteration before, whose slot then takes a new tile.
    for (int it = 0; it < NT; it++) {  // pass 1: D
        ring_barrier<4 * (kBwdRing - 2)>();
        issue(it + kBwdRing - 1);
        bw_f32x16 s[NB], dp[NB];
        tile_probs(it, s, dp);
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int r2 = 0; r2 < 16; r2++) dsum[b] = fmaf(s[b][r2], dp[b][r2], dsum[b]);
    }
    // each row's D: the two lane halves hold different keys
#pragma unroll
    for (int b = 0; b < NB; b++) D[b] = (dsum[b] + __shfl_xor(dsum[b], 32, 64)) * (1.0f / kBwdPScale);
    for (int it = NT; it < NI; it++) {  // pass 2: dQ^T += K^T dS^T
        ring_barrier<4 * (kBwdRing - 2)>();
        issue(it + kBwdRing - 1);
        bw_f32x16 s[NB], dp[NB];
        tile_probs(it, s, dp);
        const f16 *kt = k_lds[it % kBwdRing];
        f16x8 db[NB][2];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            bw_f32x16 ds;
#pragma unroll
            for (int r2 = 0; r2 < 16; r2++) ds[r2] = s[b][r2] * (dp[b][r2] - D[b]);
            to_chunks(ds, db[b]);
        }
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const f16x8 kT = tr_operand(kt, ta, dt, c);
#pragma unroll
                for (int b = 0; b < NB; b++) dq[b][dt] = bw_mfma(kT, db[b][c], dq[b][dt]);
            }
    }
    ring_barrier<0>();  // the loads issued past the last tile
    const float f = p.scale / kBwdPScale;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if (!row_ok[b]) continue;
        if (h == 0) {
            p.row_d[so[b]] = NT > 0 ? D[b] : 0.0f;
            p.row_c[so[b]] = crow[b];
        }
        // dQ^T accumulator: lane (row n, h) holds dims 32 dt + 8 q + 4 h + (0..3)
        f16 *dQ = static_cast<f16 *>(p.d_q) + qo[b] + 4 * h;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                f16x4 v;
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = (f16)(dq[b][dt][4 * q + e] * f);
                *reinterpret_cast<f16x4 *>(dQ + 32 * dt + 8 * q) = v;
            }
    }
}


// acc += a b on v_mfma_f32_32x32x16_f16 with the accumulator in AGPRs (the
// compiler keeps MFMA results in VGPRs in this file).  As inline assembly the
// MFMA is invisible to the compiler's hazard checks: the leading s_nop covers a
// VALU write of a or b just before it, and readers of acc wait on their own
// (see bwd_dkv_mfma's end).
__device__ __forceinline__ void mfma_agpr(bw_f32x16 &acc, const f16x8 a, const f16x8 b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// dK/dV: a wave owns 32 keys of one kv head (K^T and V^T in registers as B
// operands, dK^T and dV^T accumulated in AGPRs) and walks the 32-row tiles of
// the group's query rows, streamed through a 4-slot LDS ring.  It runs alone on
// its SIMD (the registers allow no second wave), so its own vector work has to
// overlap its MFMAs: the loop is software-pipelined, each row tile t issuing the
// S/dP MFMAs of tile t + 1 beside tile t's exponentials, dS and conversions
// (independent of them), then tile t's dV/dK MFMAs.  Measured on gfx950 at
// T = 4096 (32/8 heads): 18% fewer cycles than the same kernel without the
// pipelining (MFMA busy 0.42 against 0.345 of the SIMD cycles).  Rows past the
// end of the last tile get c = +inf in LDS, so their P and dS are 0 without a
// per-element mask.
template <int NB>
__global__ __launch_bounds__(64 * kBwdWaves, 1) void bwd_dkv_mfma(BackwardParams p, int group_shift) {
    static_assert(NB == 1, "one block of 32 keys per wave");
    constexpr int R = kBwdRing;
    __shared__ __attribute__((aligned(16))) f16 q_lds[R][32 * 128];
    __shared__ __attribute__((aligned(16))) f16 g_lds[R][32 * 128];
    __shared__ __attribute__((aligned(16))) float c_lds[R][32];
    __shared__ __attribute__((aligned(16))) float d_lds[R][32];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
    const int H = p.num_heads, G = 1 << group_shift, kvh = blockIdx.y;
    const int T = p.seq_len, ws = p.window_start;
    const int rows = T * G;
    const f16 *Q = static_cast<const f16 *>(p.q), *dO = static_cast<const f16 *>(p.d_out);
    const f16 *K = static_cast<const f16 *>(p.k_pool), *V = static_cast<const f16 *>(p.v_pool);
    // the wave's 32 keys; K^T and V^T as B operands: lane (key n, h) holds
    // dims 16c + 8h .. +7
    const int key = ws + (blockIdx.x * kBwdWaves + wave) * 32 + n;
    f16x8 kb[8], vb[8];
    {
        const int kj = key < T ? key : T - 1;
        const f16 *kr = pool_row(K, p, kj, kvh), *vr = pool_row(V, p, kj, kvh);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            kb[c] = *reinterpret_cast<const f16x8 *>(kr + 16 * c + 8 * h);
            vb[c] = *reinterpret_cast<const f16x8 *>(vr + 16 * c + 8 * h);
        }
    }
    const float sl2 = p.scale * kLog2e;
    const int NT = (rows + 31) / 32;
    auto head_row = [&](int r) -> int64_t {
        r = r < rows ? r : rows - 1;
        return (int64_t)(r >> group_shift) * H + kvh * G + (r & (G - 1));
    };
    auto issue = [&](int t) {
        const int w = t % R;
        t = t < NT ? t : NT - 1;
        tile_dma(q_lds[w], wave, lane, [&](int Rw) { return Q + head_row(t * 32 + Rw) * 128; });
        tile_dma(g_lds[w], wave, lane, [&](int Rw) { return dO + head_row(t * 32 + Rw) * 128; });
        const float *src = (wave & 1) ? p.row_d : p.row_c;
        float *dst = (wave & 1) ? d_lds[w] : c_lds[w];
        if (lane < 32) lds_dma4(src + head_row(t * 32 + lane), dst);
    };
    // rows of the last tile past the end: c = +inf (P = 0); its loads are done
    const int tail = rows - 32 * (NT - 1);
    auto patch_tail = [&](int t) {
        if (t == NT - 1 && tail < 32 && tid >= tail && tid < 32) c_lds[t % R][tid] = INFINITY;
    };
    const TrAddr ta = tr_addr(lane);
    bw_f32x16 dk[4], dv[4];  // in AGPRs (mfma_agpr)
#pragma unroll
    for (int dt = 0; dt < 4; dt++) dk[dt] = dv[dt] = (bw_f32x16)0.0f;
    // S = Q K^T and dP = dO V^T of the tile in slot w (the first tile only)
    auto scores = [&](int w, bw_f32x16 &s, bw_f32x16 &dp) {
        const f16 *qt = q_lds[w], *gt = g_lds[w];
        s = dp = (bw_f32x16)0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            s = bw_mfma(*reinterpret_cast<const f16x8 *>(&qt[bw_at(n, 2 * c + h)]), kb[c], s);
            dp = bw_mfma(*reinterpret_cast<const f16x8 *>(&gt[bw_at(n, 2 * c + h)]), vb[c], dp);
        }
    };
#pragma unroll
    for (int c = 0; c < 8; c++) asm volatile("" ::"v"(kb[c]), "v"(vb[c]));
#pragma unroll
    for (int u = 0; u < R - 1; u++) issue(u);
    ring_barrier<5 * (R - 2)>();  // tile 0
    patch_tail(0);
    bw_f32x16 s0, dp0, s1, dp1;
    scores(0, s0, dp0);
    // Iteration t: at its barrier tile t + 1 is loaded (tile t + 2 may still be
    // in flight) and every wave has left iteration t - 1, whose slot then
    // receives tile t + 3.  The block is laid out by hand (sched_barrier
    // fences): eight steps of the two score MFMAs of tile t + 1 over a 16-dim
    // chunk, each beside tile t's vector work on two accumulator registers, then
    // eight steps of two gradient MFMAs; LDS operands are read two (scores) or
    // one (gradients) steps ahead.
    auto body = [&](int t, const bw_f32x16 &sc, const bw_f32x16 &dc, bw_f32x16 &sn, bw_f32x16 &dn) {
        ring_barrier<5 * (R - 3)>();
        issue(t + R - 1);
        patch_tail(t + 1);
        const int w = t % R, wn = (t + 1) % R;
        const f16 *qn = q_lds[wn], *gn = g_lds[wn], *qc = q_lds[w], *gc = g_lds[w];
        // c and D of the lane's 16 rows of tile t: rows 8 q + 4 h + e
        float4 cq[4], dq4[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            cq[q] = *reinterpret_cast<const float4 *>(&c_lds[w][8 * q + 4 * h]);
            dq4[q] = *reinterpret_cast<const float4 *>(&d_lds[w][8 * q + 4 * h]);
        }
        f16x8 qa[8], ga[8];
#pragma unroll
        for (int c = 0; c < 2; c++) {
            qa[c] = *reinterpret_cast<const f16x8 *>(&qn[bw_at(n, 2 * c + h)]);
            ga[c] = *reinterpret_cast<const f16x8 *>(&gn[bw_at(n, 2 * c + h)]);
        }
        sn = dn = (bw_f32x16)0.0f;
        f16x8 pb[2], db[2];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            if (c + 2 < 8) {
                qa[c + 2] = *reinterpret_cast<const f16x8 *>(&qn[bw_at(n, 2 * (c + 2) + h)]);
                ga[c + 2] = *reinterpret_cast<const f16x8 *>(&gn[bw_at(n, 2 * (c + 2) + h)]);
            }
            sn = bw_mfma(qa[c], kb[c], sn);
            dn = bw_mfma(ga[c], vb[c], dn);
            // registers 2c, 2c + 1: rows 8 (c / 2) + 4 h + 2 (c % 2) + {0, 1}
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int r2 = 2 * c + u, q = r2 >> 2, e = r2 & 3;
                const float cv = e == 0 ? cq[q].x : e == 1 ? cq[q].y : e == 2 ? cq[q].z : cq[q].w;
                const float dd = e == 0 ? dq4[q].x : e == 1 ? dq4[q].y : e == 2 ? dq4[q].z : dq4[q].w;
                const float P = __builtin_amdgcn_exp2f(fmaf(sc[r2], sl2, kPScaleLog2 - cv));
                pb[r2 >> 3][r2 & 7] = (f16)P;
                db[r2 >> 3][r2 & 7] = (f16)(P * (dc[r2] - dd));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // dV^T += dO^T P and dK^T += Q^T dS: step k covers dim tile k % 4 of
        // row chunk k / 4
        f16x8 gT[8], qT[8];
        gT[0] = tr_operand(gc, ta, 0, 0);
        qT[0] = tr_operand(qc, ta, 0, 0);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (k + 1 < 8) {
                gT[k + 1] = tr_operand(gc, ta, (k + 1) & 3, (k + 1) >> 2);
                qT[k + 1] = tr_operand(qc, ta, (k + 1) & 3, (k + 1) >> 2);
            }
            mfma_agpr(dv[k & 3], gT[k], pb[k >> 2]);
            mfma_agpr(dk[k & 3], qT[k], db[k >> 2]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    int t = 0;
    for (; t + 2 <= NT; t += 2) {
        body(t, s0, dp0, s1, dp1);
        body(t + 1, s1, dp1, s0, dp0);
    }
    if (t < NT) body(t, s0, dp0, s1, dp1);
    // the last gradient MFMAs have written their AGPRs before they are read
    asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");
#pragma unroll
    for (int dt = 0; dt < 4; dt++) asm volatile("" : "+a"(dk[dt]), "+a"(dv[dt]));
    ring_barrier<0>();  // the loads issued past the last tile
    const float fk = p.scale / kBwdPScale, fv = 1.0f / kBwdPScale;
    if (key < T) {
        f16 *dkr = const_cast<f16 *>(pool_row(static_cast<const f16 *>(p.d_k_pool), p, key, kvh)) + 4 * h;
        f16 *dvr = const_cast<f16 *>(pool_row(static_cast<const f16 *>(p.d_v_pool), p, key, kvh)) + 4 * h;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                f16x4 a = *reinterpret_cast<const f16x4 *>(dkr + 32 * dt + 8 * q);
                f16x4 c = *reinterpret_cast<const f16x4 *>(dvr + 32 * dt + 8 * q);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    a[e] = (f16)((float)a[e] + dk[dt][4 * q + e] * fk);
                    c[e] = (f16)((float)c[e] + dv[dt][4 * q + e] * fv);
                }
                *reinterpret_cast<f16x4 *>(dkr + 32 * dt + 8 * q) = a;
                *reinterpret_cast<f16x4 *>(dvr + 32 * dt + 8 * q) = c;
            }
    }
}

constexpr int kBwdNB = 1;  // 32-row / 32-key blocks per wave (2 needs more than 512 registers)

hipError_t launch_backward(const BackwardParams &p, int32_t dtype, hipStream_t stream) {
    if (p.seq_len <= 0) return hipSuccess;
    if (p.head_dim > 64 * kBwdMaxDims || p.row_d == nullptr) return hipErrorInvalidValue;
    const dim3 rows(p.seq_len, p.num_heads), keys(p.seq_len - p.window_start, p.num_kv_heads);
    const int G = p.num_heads / p.num_kv_heads;
    const int64_t nblk = p.block_size > 0 ? (int64_t)(p.seq_len - 1) / p.block_size - p.window_start / p.block_size + 1 : 0;
    if (dtype == kF16 && p.head_dim == 128 && p.row_c != nullptr && (G & (G - 1)) == 0 && nblk <= kBwdBtCache) {
        const int64_t qrows = (int64_t)p.seq_len * G;
        const int64_t nkeys = p.seq_len - p.window_start;
        const int per = 32 * kBwdWaves * kBwdNB, gs = __builtin_ctz((unsigned)G);
        const dim3 dq_grid((unsigned)((qrows + per - 1) / per), p.num_kv_heads);
        if (nblk <= kBwdBtCacheSmall)
            hipLaunchKernelGGL((bwd_dq_mfma<kBwdNB, kBwdBtCacheSmall>), dq_grid, dim3(64 * kBwdWaves), 0, stream, p, gs);
        else
            hipLaunchKernelGGL((bwd_dq_mfma<kBwdNB, kBwdBtCache>), dq_grid, dim3(64 * kBwdWaves), 0, stream, p, gs);
        if (nkeys > 0)
            hipLaunchKernelGGL(bwd_dkv_mfma<kBwdNB>, dim3((unsigned)((nkeys + per - 1) / per), p.num_kv_heads),
                               dim3(64 * kBwdWaves), 0, stream, p, gs);
        return hipGetLastError();
    }
    if (dtype == kF32) {
        hipLaunchKernelGGL((bwd_rows_kernel<float>), rows, dim3(64), 0, stream, p);
        if (keys.x > 0) hipLaunchKernelGGL((bwd_keys_kernel<float>), keys, dim3(64), 0, stream, p);
    } else if (dtype == kF16) {
        hipLaunchKernelGGL((bwd_rows_kernel<f16>), rows, dim3(64), 0, stream, p);
        if (keys.x > 0) hipLaunchKernelGGL((bwd_keys_kernel<f16>), keys, dim3(64), 0, stream, p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace pam
