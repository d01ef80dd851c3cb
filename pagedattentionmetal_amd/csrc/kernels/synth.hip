// synth.hip - counter-based synthetic data for the measured workloads.
//
// Element i of stream s under seed S is built from SplitMix64 outputs taken at
// sequence positions (s << 40) + 2i and (s << 40) + 2i + 1 of the generator
// started at S (output k = mix(S + (k + 1) * 0x9E3779B97F4A7C15)).  Any element
// can be computed on its own, so a multi-GiB pool is filled in parallel, and
// the host restates the same values with integer arithmetic plus binary64
// log / cos / sqrt.  Each output's top 53 bits give a uniform u in [0, 1); a
// pair gives one standard normal by the Box-Muller cosine branch,
// sqrt(-2 ln(1 - u0)) cos(2 pi u1), computed in binary64, scaled, rounded to
// binary32 and then (f16 output) to binary16.  An optional outlier stream
// multiplies an element by 8 when its own uniform is below `outlier_frac`.
#include "kernels.h"
#include "pam_device.h"

namespace pam {

__device__ __forceinline__ uint64_t splitmix_at(uint64_t seed, uint64_t k) {
    uint64_t z = seed + (k + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ double unit_of(uint64_t z) { return (double)(z >> 11) * 0x1.0p-53; }

template <typename T>
__global__ __launch_bounds__(256) void synth_normal_kernel(T *dst, uint64_t n, uint64_t seed, uint64_t stream,
                                                           float stddev, int64_t outlier_stream, float outlier_frac) {
    const uint64_t base = stream << 40;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        const double u0 = unit_of(splitmix_at(seed, base + 2 * i));
        const double u1 = unit_of(splitmix_at(seed, base + 2 * i + 1));
        double x = sqrt(-2.0 * log(1.0 - u0)) * cos(6.283185307179586 * u1) * (double)stddev;
        if (outlier_stream >= 0 && unit_of(splitmix_at(seed, ((uint64_t)outlier_stream << 40) + i)) < (double)outlier_frac)
            x *= 8.0;
        // binary64 -> binary32 -> output type, two roundings as the host does them
        // (the barrier keeps the compiler from fusing them into one conversion)
        float xf = (float)x;
        asm volatile("" : "+v"(xf));
        dst[i] = (T)xf;
    }
}

hipError_t launch_synth_normal(void *dst, int32_t dtype, uint64_t n, uint64_t seed, uint64_t stream, float stddev,
                               int64_t outlier_stream, float outlier_frac, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (stream >= ((uint64_t)1 << 23) || outlier_stream >= ((int64_t)1 << 23) || n >= ((uint64_t)1 << 39))
        return hipErrorInvalidValue;
    const uint64_t blocks64 = (n + 255) / 256;
    const unsigned blocks = (unsigned)(blocks64 < 8192 ? blocks64 : 8192);
    if (dtype == kF32)
        hipLaunchKernelGGL(synth_normal_kernel<float>, dim3(blocks), dim3(256), 0, s, static_cast<float *>(dst), n, seed,
                           stream, stddev, outlier_stream, outlier_frac);
    else if (dtype == kF16)
        hipLaunchKernelGGL(synth_normal_kernel<f16>, dim3(blocks), dim3(256), 0, s, static_cast<f16 *>(dst), n, seed,
                           stream, stddev, outlier_stream, outlier_frac);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace pam
