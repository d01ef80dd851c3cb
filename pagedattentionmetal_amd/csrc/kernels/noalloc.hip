// noalloc.hip - the device scratch of the allocation-free decode entry point.
//
// pam_engine_decode_noalloc runs the decode kernels with their split-context
// workspace (partial outputs, merge counters) and the zero page of masked
// lanes in this fixed array instead of buffers the context allocates, so it
// never calls hipMalloc.  Each GPU the library runs on holds its own copy of
// the array until the process ends.  Host code reaches it only through the
// address hipGetSymbolAddress gives for the current device (the array's name
// is a host-side stand-in, not a device address).
#include <mutex>

#include "kernels.h"

namespace pam {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};
}  // namespace

__global__ void zero_bytes_kernel(uint4 *p, size_t n16) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) p[i] = make_uint4(0, 0, 0, 0);
}

hipError_t noalloc_scratch_setup(int device, hipStream_t stream, void **out) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(g_mu);
    if (g_ptr[device] == nullptr) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (ptr == nullptr) return hipErrorInvalidSymbol;
        // the zero page must read as zeros: cleared once, no kernel writes it
        hipLaunchKernelGGL(zero_bytes_kernel, dim3((unsigned)(kNoAllocZeroBytes / 16 + 255) / 256), dim3(256), 0,
                           stream, static_cast<uint4 *>(ptr), kNoAllocZeroBytes / 16);
        const hipError_t le = hipGetLastError();
        if (le != hipSuccess) return le;
        const hipError_t se = hipStreamSynchronize(stream);
        if (se != hipSuccess) return se;
        g_ptr[device] = ptr;
    }
    *out = g_ptr[device];
    return hipSuccess;
}

void *noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> g(g_mu);
    return g_ptr[device];
}

}  // namespace pam
