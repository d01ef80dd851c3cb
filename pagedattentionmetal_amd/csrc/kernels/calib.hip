// calib.hip - reference streams of known size for bandwidth calibration.
//
// stream_read: every byte of a buffer read once with 16-byte loads (eight in
// flight per lane), one word per workgroup written back so the loads cannot be
// dropped.  stream_copy: a plain 16-byte copy.  Their HIP-event times give the
// achievable HBM rates of the box, and the FETCH_SIZE / WRITE_SIZE counters read
// on them give the scale factor between those counters and true bytes.
// mfma_loop: every wave of 8-wave workgroups issues v_mfma_f32_32x32x16_f16 on
// four independent accumulators, nothing else: the dense f16 MFMA rate the part
// sustains at its power-limited clock, the ceiling the prefill is set against.
#include "kernels.h"

namespace pam {

__global__ __launch_bounds__(256) void stream_read_kernel(const uint4 *src, int64_t n16, uint32_t *sink) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 7 * stride < n16; i += 8 * stride) {
        uint4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = src[i + k * stride];
#pragma unroll
        for (int k = 0; k < 8; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < n16; i += stride) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    // fold the lanes so the loads stay live; one word per workgroup
    for (int m = 32; m > 0; m >>= 1) acc ^= __shfl_xor(acc, m, 64);
    if ((threadIdx.x & 63) == 0 && acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

__global__ __launch_bounds__(256) void stream_copy_kernel(const uint4 *src, uint4 *dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

typedef _Float16 cal_f16x8 __attribute__((ext_vector_type(8)));
typedef float cal_f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(512, 1) void mfma_loop_kernel(int iters, float seed, float *sink) {
    const int lane = threadIdx.x & 63;
    cal_f16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (_Float16)(seed * (float)(lane + i));
        b[i] = (_Float16)(seed * (float)(i - lane));
    }
    cal_f32x16 c0 = (cal_f32x16)0.0f, c1 = c0, c2 = c0, c3 = c0;
    for (int it = 0; it < iters; it++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
    }
    float r = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) r += c0[i] + c1[i] + c2[i] + c3[i];
    if (r == 1234.5f) sink[blockIdx.x] = r;  // keeps the MFMAs live; never true for these inputs
}

hipError_t launch_mfma_loop(int blocks, int iters, float *sink, hipStream_t stream) {
    if (blocks <= 0 || iters <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mfma_loop_kernel, dim3(blocks), dim3(512), 0, stream, iters, 1e-3f, sink);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void *src, size_t bytes, uint32_t *sink, int blocks, hipStream_t stream) {
    if (bytes % 16 != 0 || blocks <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<const uint4 *>(src),
                       (int64_t)(bytes / 16), sink);
    return hipGetLastError();
}

hipError_t launch_stream_copy(const void *src, void *dst, size_t bytes, int blocks, hipStream_t stream) {
    if (bytes % 16 != 0 || blocks <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_copy_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<const uint4 *>(src),
                       static_cast<uint4 *>(dst), (int64_t)(bytes / 16));
    return hipGetLastError();
}

}  // namespace pam
