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
//     (ds_read_b64_tr_b16).  It adds its rows to the gradient pools once.
// P and dS enter the MFMA as binary16 scaled by 2^8 (P <= 1; the scale keeps
// small probabilities of long rows out of the subnormal range) and the
// accumulators are scaled back at the end.
typedef float bw_f32x16 __attribute__((ext_vector_type(16)));
constexpr int kBwdWaves = 4;             // waves per workgroup, 32 rows / keys each
constexpr float kBwdPScale = 256.0f;

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

__global__ __launch_bounds__(64 * kBwdWaves, 1) void bwd_dq_mfma(BackwardParams p) {
    __shared__ __attribute__((aligned(16))) f16 k_lds[2][32 * 128];
    __shared__ __attribute__((aligned(16))) f16 v_lds[2][32 * 128];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
    const int H = p.num_heads, G = H / p.num_kv_heads, kvh = blockIdx.y;
    const int T = p.seq_len, ws = p.window_start;
    const int rows = T * G;
    const int r = (blockIdx.x * kBwdWaves + wave) * 32 + n;  // this lane's row: token r / G, head r % G
    const bool row_ok = r < rows;
    const int tok = row_ok ? r / G : 0, hq = kvh * G + (row_ok ? r % G : 0);
    const int64_t qo = ((int64_t)tok * H + hq) * 128;
    const f16 *Q = static_cast<const f16 *>(p.q), *dO = static_cast<const f16 *>(p.d_out);
    const f16 *K = static_cast<const f16 *>(p.k_pool), *V = static_cast<const f16 *>(p.v_pool);
    f16x8 qv[8], gv[8];
#pragma unroll
    for (int c = 0; c < 8; c++) {
        qv[c] = row_ok ? *reinterpret_cast<const f16x8 *>(Q + qo + 16 * c + 8 * h) : (f16x8)(f16)0.0f;
        gv[c] = row_ok ? *reinterpret_cast<const f16x8 *>(dO + qo + 16 * c + 8 * h) : (f16x8)(f16)0.0f;
    }
    const float m = row_ok ? p.m[(int64_t)tok * H + hq] : 0.0f, l = row_ok ? p.l[(int64_t)tok * H + hq] : 1.0f;
    const float crow = row_ok ? m * kLog2e + __builtin_log2f(l) : INFINITY;
    const float sl2 = p.scale * kLog2e;

    // staging: thread -> piece tid % 16 of tile rows tid / 16 and tid / 16 + 16
    const int sp = tid & 15, sr = tid >> 4;
    const int t0 = ws / 32, t1 = (T + 31) / 32, NT = t1 - t0;
    auto fetch = [&](int t, f16x8 (&kr)[2], f16x8 (&vr)[2]) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int j = t * 32 + sr + 16 * i;
            j = j < ws ? ws : (j >= T ? T - 1 : j);  // finite rows outside the keys (masked)
            kr[i] = *reinterpret_cast<const f16x8 *>(pool_row(K, p, j, kvh) + 8 * sp);
            vr[i] = *reinterpret_cast<const f16x8 *>(pool_row(V, p, j, kvh) + 8 * sp);
        }
    };
    auto stage = [&](int buf, const f16x8 (&kr)[2], const f16x8 (&vr)[2]) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            *reinterpret_cast<f16x8 *>(&k_lds[buf][bw_at(sr + 16 * i, sp)]) = kr[i];
            *reinterpret_cast<f16x8 *>(&v_lds[buf][bw_at(sr + 16 * i, sp)]) = vr[i];
        }
    };
    const TrAddr ta = tr_addr(lane);
    bw_f32x16 dq[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) dq[dt] = (bw_f32x16)0.0f;
    float dsum = 0.0f, D = 0.0f;
    f16x8 kr[2], vr[2];
    fetch(t0, kr, vr);
    stage(0, kr, vr);
    __syncthreads();
    for (int it = 0; it < 2 * NT; it++) {
        const int t = t0 + it % NT, buf = it & 1;
        const bool second = it >= NT;
        if (it + 1 < 2 * NT) fetch(t0 + (it + 1) % NT, kr, vr);
        if (it == NT) {  // pass 1 done: the row's D (the two lane halves hold different keys)
            D = dsum + __shfl_xor(dsum, 32, 64);
        }
        const f16 *kt = k_lds[buf], *vt = v_lds[buf];
        bw_f32x16 s = (bw_f32x16)0.0f, dp = (bw_f32x16)0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const f16x8 ka = *reinterpret_cast<const f16x8 *>(&kt[bw_at(n, 2 * c + h)]);
            const f16x8 va = *reinterpret_cast<const f16x8 *>(&vt[bw_at(n, 2 * c + h)]);
            s = bw_mfma(ka, qv[c], s);
            dp = bw_mfma(va, gv[c], dp);
        }
        const bool edge = t * 32 < ws || t * 32 + 32 > T;
#pragma unroll
        for (int r2 = 0; r2 < 16; r2++) {
            float pr = __builtin_amdgcn_exp2f(s[r2] * sl2 - crow);
            if (edge) {
                const int j = t * 32 + 8 * (r2 >> 2) + 4 * h + (r2 & 3);
                pr = (j >= ws && j < T) ? pr : 0.0f;
            }
            s[r2] = pr;
        }
        if (!second) {
#pragma unroll
            for (int r2 = 0; r2 < 16; r2++) dsum = fmaf(s[r2], dp[r2], dsum);
        } else {
            bw_f32x16 ds;
#pragma unroll
            for (int r2 = 0; r2 < 16; r2++) ds[r2] = s[r2] * (dp[r2] - D) * kBwdPScale;
            f16x8 db[2];
            to_chunks(ds, db);
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int dt = 0; dt < 4; dt++) dq[dt] = bw_mfma(tr_operand(kt, ta, dt, c), db[c], dq[dt]);
        }
        __syncthreads();  // every wave is done with buffer buf ^ 1 (read two iterations ago)
        if (it + 1 < 2 * NT) stage(buf ^ 1, kr, vr);
        __syncthreads();
    }
    if (NT == 0) D = 0.0f;
    if (!row_ok) return;
    if (h == 0) {
        p.row_d[(int64_t)tok * H + hq] = D;
        p.row_c[(int64_t)tok * H + hq] = crow;
    }
    // dQ^T accumulator: lane (row n, h) holds dims 32 dt + 8 q + 4 h + (0..3)
    f16 *dQ = static_cast<f16 *>(p.d_q) + qo + 4 * h;
    const float f = p.scale / kBwdPScale;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            f16x4 v;
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = (f16)(dq[dt][4 * q + e] * f);
            *reinterpret_cast<f16x4 *>(dQ + 32 * dt + 8 * q) = v;
        }
}

__global__ __launch_bounds__(64 * kBwdWaves, 1) void bwd_dkv_mfma(BackwardParams p) {
    __shared__ __attribute__((aligned(16))) f16 q_lds[2][32 * 128];
    __shared__ __attribute__((aligned(16))) f16 g_lds[2][32 * 128];
    __shared__ __attribute__((aligned(16))) float c_lds[2][32];
    __shared__ __attribute__((aligned(16))) float d_lds[2][32];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
    const int H = p.num_heads, G = H / p.num_kv_heads, kvh = blockIdx.y;
    const int T = p.seq_len, ws = p.window_start;
    const int rows = T * G;
    const int key = ws + (blockIdx.x * kBwdWaves + wave) * 32 + n;  // this lane's key
    const bool key_ok = key < T;
    const int kj = key_ok ? key : T - 1;
    const f16 *Q = static_cast<const f16 *>(p.q), *dO = static_cast<const f16 *>(p.d_out);
    const f16 *K = static_cast<const f16 *>(p.k_pool), *V = static_cast<const f16 *>(p.v_pool);
    // K^T and V^T as B operands: lane (key n, h) holds dims 16c + 8h .. +7
    f16x8 kb[8], vb[8];
    {
        const f16 *kr = pool_row(K, p, kj, kvh), *vr = pool_row(V, p, kj, kvh);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            kb[c] = *reinterpret_cast<const f16x8 *>(kr + 16 * c + 8 * h);
            vb[c] = *reinterpret_cast<const f16x8 *>(vr + 16 * c + 8 * h);
        }
    }
    const float sl2 = p.scale * kLog2e;
    const int sp = tid & 15, sr = tid >> 4;
    const int NT = (rows + 31) / 32;
    // row tile t: rows 32t .. 32t + 31 (token r / G, head kvh G + r % G)
    auto fetch = [&](int t, f16x8 (&qr)[2], f16x8 (&gr)[2], float &cr, float &dr) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int r = t * 32 + sr + 16 * i;
            if (r < rows) {
                const int64_t o = ((int64_t)(r / G) * H + kvh * G + r % G) * 128 + 8 * sp;
                qr[i] = *reinterpret_cast<const f16x8 *>(Q + o);
                gr[i] = *reinterpret_cast<const f16x8 *>(dO + o);
            } else {
                qr[i] = gr[i] = (f16x8)(f16)0.0f;
            }
        }
        if (tid < 32) {
            const int r = t * 32 + tid;
            const int64_t o = (int64_t)(r / G) * H + kvh * G + r % G;
            cr = r < rows ? p.row_c[o] : INFINITY;  // rows past the end: P = 0
            dr = r < rows ? p.row_d[o] : 0.0f;
        }
    };
    auto stage = [&](int buf, const f16x8 (&qr)[2], const f16x8 (&gr)[2], float cr, float dr) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            *reinterpret_cast<f16x8 *>(&q_lds[buf][bw_at(sr + 16 * i, sp)]) = qr[i];
            *reinterpret_cast<f16x8 *>(&g_lds[buf][bw_at(sr + 16 * i, sp)]) = gr[i];
        }
        if (tid < 32) {
            c_lds[buf][tid] = cr;
            d_lds[buf][tid] = dr;
        }
    };
    const TrAddr ta = tr_addr(lane);
    bw_f32x16 dk[4], dv[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) dk[dt] = dv[dt] = (bw_f32x16)0.0f;
    f16x8 qr[2], gr[2];
    float cr = 0.0f, dr = 0.0f;
    fetch(0, qr, gr, cr, dr);
    stage(0, qr, gr, cr, dr);
    __syncthreads();
    for (int t = 0; t < NT; t++) {
        const int buf = t & 1;
        if (t + 1 < NT) fetch(t + 1, qr, gr, cr, dr);
        const f16 *qt = q_lds[buf], *gt = g_lds[buf];
        bw_f32x16 s = (bw_f32x16)0.0f, dp = (bw_f32x16)0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const f16x8 qa = *reinterpret_cast<const f16x8 *>(&qt[bw_at(n, 2 * c + h)]);
            const f16x8 ga = *reinterpret_cast<const f16x8 *>(&gt[bw_at(n, 2 * c + h)]);
            s = bw_mfma(qa, kb[c], s);
            dp = bw_mfma(ga, vb[c], dp);
        }
        // registers r hold rows 8 (r / 4) + 4 h + r % 4 of the tile
        bw_f32x16 pr, ds;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 cq = *reinterpret_cast<const float4 *>(&c_lds[buf][8 * q + 4 * h]);
            const float4 dq = *reinterpret_cast<const float4 *>(&d_lds[buf][8 * q + 4 * h]);
            const float cv[4] = {cq.x, cq.y, cq.z, cq.w}, dv4[4] = {dq.x, dq.y, dq.z, dq.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float P = __builtin_amdgcn_exp2f(s[4 * q + e] * sl2 - cv[e]);
                pr[4 * q + e] = P * kBwdPScale;
                ds[4 * q + e] = P * (dp[4 * q + e] - dv4[e]) * kBwdPScale;
            }
        }
        f16x8 pb[2], db[2];
        to_chunks(pr, pb);
        to_chunks(ds, db);
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                dv[dt] = bw_mfma(tr_operand(gt, ta, dt, c), pb[c], dv[dt]);
                dk[dt] = bw_mfma(tr_operand(qt, ta, dt, c), db[c], dk[dt]);
            }
        __syncthreads();
        if (t + 1 < NT) stage(buf ^ 1, qr, gr, cr, dr);
        __syncthreads();
    }
    if (!key_ok) return;
    // accumulators: lane (key n, h) holds dims 32 dt + 8 q + 4 h + (0..3); this
    // wave alone owns the key's rows of the gradient pools
    f16 *dkr = const_cast<f16 *>(pool_row(static_cast<const f16 *>(p.d_k_pool), p, key, kvh)) + 4 * h;
    f16 *dvr = const_cast<f16 *>(pool_row(static_cast<const f16 *>(p.d_v_pool), p, key, kvh)) + 4 * h;
    const float fk = p.scale / kBwdPScale, fv = 1.0f / kBwdPScale;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            f16x4 a = *reinterpret_cast<const f16x4 *>(dkr + 32 * dt + 8 * q);
            f16x4 b = *reinterpret_cast<const f16x4 *>(dvr + 32 * dt + 8 * q);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                a[e] = (f16)((float)a[e] + dk[dt][4 * q + e] * fk);
                b[e] = (f16)((float)b[e] + dv[dt][4 * q + e] * fv);
            }
            *reinterpret_cast<f16x4 *>(dkr + 32 * dt + 8 * q) = a;
            *reinterpret_cast<f16x4 *>(dvr + 32 * dt + 8 * q) = b;
        }
}

hipError_t launch_backward(const BackwardParams &p, int32_t dtype, hipStream_t stream) {
    if (p.seq_len <= 0) return hipSuccess;
    if (p.head_dim > 64 * kBwdMaxDims || p.row_d == nullptr) return hipErrorInvalidValue;
    const dim3 rows(p.seq_len, p.num_heads), keys(p.seq_len - p.window_start, p.num_kv_heads);
    if (dtype == kF16 && p.head_dim == 128 && p.row_c != nullptr) {
        const int64_t qrows = (int64_t)p.seq_len * (p.num_heads / p.num_kv_heads);
        const int64_t nkeys = p.seq_len - p.window_start;
        const int per = 32 * kBwdWaves;
        hipLaunchKernelGGL(bwd_dq_mfma, dim3((unsigned)((qrows + per - 1) / per), p.num_kv_heads), dim3(64 * kBwdWaves),
                           0, stream, p);
        if (nkeys > 0)
            hipLaunchKernelGGL(bwd_dkv_mfma, dim3((unsigned)((nkeys + per - 1) / per), p.num_kv_heads),
                               dim3(64 * kBwdWaves), 0, stream, p);
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
