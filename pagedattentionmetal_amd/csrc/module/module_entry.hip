// module_entry.hip - the kernels as a loadable code object (libpam_kernels.hsaco).
//
// The reference builds its compute pipelines at run time from a shader library
// (PagedAttentionEngine.swift:151-198, 248-333).  Here the equivalent is a gfx950
// code object with named (extern "C") entry points, loaded with hipModuleLoad
// and launched with hipModuleLaunchKernel (pam_module_load / pam_module_launch).
// Each entry runs the same body as the library's own kernel of that
// configuration, with the same launch bounds, so a context bound to the module
// gives the same results bit for bit.  Built by build.py with hipcc --genco; it
// is not part of libpam.so.
#include "../kernels/attention_body.h"
#include "../kernels/prefill_body.h"

namespace pam {

#define PAM_STREAMK_ENTRY(NAME, KV, HD, BLK, FL)                                                      \
    extern "C" __global__ __launch_bounds__(64 * kMfmaWaves, (MfmaShape<KV, HD>::OCC)) void NAME( \
        AttnParams p) {                                                                                \
        streamk_body<KV, HD, BLK, FL>(p, blockIdx.x, gridDim.x);                                     \
    }
#define PAM_PREFILL_ENTRY(NAME, FUSED, KV)                                                   \
    extern "C" __global__ __launch_bounds__(64 * kPrefillWaves, 1) void NAME(AttnParams p) { \
        prefill_body<128, kPrefillRB, FUSED, KV>(p);                                          \
    }

// decode, stream-K form, d = 128, blocks of 16 tokens or more
PAM_STREAMK_ENTRY(pam_decode_streamk_f16_d128, f16, 128, kBlkTile, false)
PAM_STREAMK_ENTRY(pam_decode_streamk_e4m3_d128, uint8_t, 128, kBlkTile, false)
// decodeLayers: the heads of several layers per K/V tile
PAM_STREAMK_ENTRY(pam_decode_layers_streamk_f16_d128, f16, 128, kBlkTile, true)
PAM_STREAMK_ENTRY(pam_decode_layers_streamk_e4m3_d128, uint8_t, 128, kBlkTile, true)
// dense chunked prefill, d = 128
PAM_PREFILL_ENTRY(pam_prefill_f16_d128, false, f16)
PAM_PREFILL_ENTRY(pam_prefill_fused_f16_d128, true, f16)
PAM_PREFILL_ENTRY(pam_prefill_e4m3_d128, false, uint8_t)

// A plain entry for callers that drive pam_module_launch themselves: n words of
// dst set to value.
extern "C" __global__ __launch_bounds__(256) void pam_fill_u32(uint32_t *dst, uint32_t value, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = value;
}

}  // namespace pam
