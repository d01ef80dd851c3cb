// stage_body.h - device body of the staging copy (mapped pinned host memory to
// the device on the compute queue).  Included by stage.hip and by the
// code-object entries (module_entry.hip).
#pragma once
#include "kernels.h"
#include "pam_device.h"

namespace pam {

// 16-byte pieces, then a byte tail of fewer than 16 bytes
__device__ __forceinline__ void stage_body(const uint4 *__restrict__ src, uint4 *__restrict__ dst, size_t n16,
                                           const uint8_t *__restrict__ src_tail, uint8_t *__restrict__ dst_tail,
                                           int tail) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) dst[i] = src[i];
    if (i < (size_t)tail) dst_tail[i] = src_tail[i];
}

}  // namespace pam
