// stage.hip - host-to-device staging on the compute queue.
//
// Per-call metadata (block-table slabs, row and chunk descriptors, token
// positions: a few KB) is written to pinned host memory and copied to the
// device by this kernel, on the stream that consumes it.  A DMA-engine copy in
// the same stream costs tens of microseconds of hand-off between the compute
// and copy engines around every call; a kernel reading the mapped host memory
// over the bus does not.
#include "kernels.h"
#include "pam_device.h"

namespace pam {

__global__ __launch_bounds__(256) void stage_copy_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                          size_t n16, const uint8_t *__restrict__ src_tail,
                                                          uint8_t *__restrict__ dst_tail, int tail) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) dst[i] = src[i];
    if (i < (size_t)tail) dst_tail[i] = src_tail[i];
}

hipError_t launch_stage_copy(const void *host_mapped, void *dst, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    if (((uintptr_t)host_mapped | (uintptr_t)dst) & 15) return hipErrorInvalidValue;
    const size_t n16 = bytes / 16;
    const int tail = (int)(bytes % 16);
    const size_t threads = n16 > (size_t)tail ? n16 : (size_t)tail;
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(stage_copy_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<const uint4 *>(host_mapped),
                       static_cast<uint4 *>(dst), n16, static_cast<const uint8_t *>(host_mapped) + n16 * 16,
                       static_cast<uint8_t *>(dst) + n16 * 16, tail);
    return hipGetLastError();
}

}  // namespace pam
