// stage.hip - host-to-device staging on the compute queue.
//
// Per-call metadata (block-table slabs, row and chunk descriptors, token
// positions: a few KB) is written to pinned host memory and copied to the
// device by this kernel, on the stream that consumes it.  A DMA-engine copy in
// the same stream costs tens of microseconds of hand-off between the compute
// and copy engines around every call; a kernel reading the mapped host memory
// over the bus does not.
#include "stage_body.h"

namespace pam {

// the kernel (the fat binary's entry); stage_body also backs the code object's
__global__ __launch_bounds__(256) void stage_copy_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                          size_t n16, const uint8_t *__restrict__ src_tail,
                                                          uint8_t *__restrict__ dst_tail, int tail) {
    stage_body(src, dst, n16, src_tail, dst_tail, tail);
}

hipError_t launch_stage_copy(const void *host_mapped, void *dst, size_t bytes, hipStream_t stream,
                             const KernelTable *kt) {
    if (bytes == 0) return hipSuccess;
    if (((uintptr_t)host_mapped | (uintptr_t)dst) & 15) return hipErrorInvalidValue;
    const size_t n16 = bytes / 16;
    const int tail = (int)(bytes % 16);
    const size_t threads = n16 > (size_t)tail ? n16 : (size_t)tail;
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    const uint4 *src16 = static_cast<const uint4 *>(host_mapped);
    uint4 *dst16 = static_cast<uint4 *>(dst);
    const uint8_t *src_tail = static_cast<const uint8_t *>(host_mapped) + n16 * 16;
    uint8_t *dst_tail = static_cast<uint8_t *>(dst) + n16 * 16;
    hipError_t e;
    if (via_module(kt, kt ? kt->stage : nullptr, &e, dim3(blocks), dim3(256), stream, src16, dst16, n16, src_tail,
                   dst_tail, tail))
        return e;
    hipLaunchKernelGGL(stage_copy_kernel, dim3(blocks), dim3(256), 0, stream, src16, dst16, n16, src_tail, dst_tail,
                       tail);
    return hipGetLastError();
}

}  // namespace pam
