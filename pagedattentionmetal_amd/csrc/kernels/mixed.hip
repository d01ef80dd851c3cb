// mixed.hip - a continuous-batching step's attention in one launch.
//
// The reference runs a step's prefill chunks and decode rows as separate
// engine calls (PagedAttentionInference.swift:138-144, 221-278).  Here one grid
// holds both: workgroups [0, pf_groups) run the dense prefill's work list
// (prefill_body, MFMA-bound) and the workgroups after them run the stream-K
// decode over the single-token rows (streamk_body with eight waves, HBM-bound).
// The hardware dispatches workgroups in id order, so the prefill's workgroups
// take their CUs first (one workgroup fills a CU: eight waves at two per SIMD
// and most of the LDS) and the decode runs on the CUs left over and on those
// the prefill frees, instead of after the prefill's last workgroup.
//
// Neither part waits on the other: both merge their split work with their own
// epoch-tagged counters (pf_count, seg_count), and the K/V they read was
// written by an earlier launch (the step's append).
#include "mixed_body.h"

namespace pam {


// the kernel (the fat binary's entry); mixed_body also backs the code object's
template <typename KV>
__global__ __launch_bounds__(64 * kPrefillWaves, 1) void mixed_step_kernel(AttnParams p) {
    mixed_body<KV>(p);
}

bool mixed_launch_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size, int32_t rows) {
    return prefill_mfma_supported(dtype, head_dim, group, block_size) &&
           mfma_supported(dtype, head_dim, group, block_size) && group >= 4 && head_dim == 128 &&
           block_size % 16 == 0 && rows > 0 && rows <= kMixedMaxRows;
}

void mixed_decode_slots(const AttnParams &p, int32_t decode_groups, int64_t *part_slots, int64_t *counters) {
    const int64_t Hkv = p.num_kv_heads, G = p.num_heads / p.num_kv_heads;
    const int64_t NH = Hkv % 4 == 0 ? 4 : (Hkv % 2 == 0 ? 2 : 1);
    const int64_t units = (int64_t)decode_groups * (kPrefillWaves / NH) / (Hkv / NH);
    *part_slots = (units + (int64_t)p.rows) * Hkv * G;
    *counters = (int64_t)p.rows * Hkv;
}

hipError_t launch_mixed_step(const AttnParams &p_in, int32_t dtype, int32_t decode_groups, hipStream_t stream,
                             const KernelTable *kt) {
    AttnParams p = p_in;
    p.epoch = next_launch_epoch();
    const int G = p.num_heads / p.num_kv_heads;
    if (!mixed_launch_supported(dtype, p.head_dim, G, p.block_size, p.rows)) return hipErrorInvalidValue;
    if (p.pf_work == nullptr || p.pf_range == nullptr || p.pf_groups <= 0 || decode_groups <= 0) return hipErrorInvalidValue;
    if (p.seg_count == nullptr || p.part_o == nullptr || p.zero_page == nullptr) return hipErrorInvalidValue;
    if ((int64_t)p.pf_groups + decode_groups > INT32_MAX) return hipErrorInvalidValue;
    const dim3 grid(p.pf_groups + decode_groups), block(64 * kPrefillWaves);
    hipError_t e;
    if (via_module(kt, kt ? kt->mixed[dtype == kFP8] : nullptr, &e, grid, block, stream, p)) return e;
    if (dtype == kFP8)
        hipLaunchKernelGGL((mixed_step_kernel<uint8_t>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((mixed_step_kernel<f16>), grid, block, 0, stream, p);
    return hipGetLastError();
}

}  // namespace pam
