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

hipError_t launch_backward(const BackwardParams &p, int32_t dtype, hipStream_t stream) {
    if (p.seq_len <= 0) return hipSuccess;
    if (p.head_dim > 64 * kBwdMaxDims || p.row_d == nullptr) return hipErrorInvalidValue;
    const dim3 rows(p.seq_len, p.num_heads), keys(p.seq_len - p.window_start, p.num_kv_heads);
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
