// module_entry.hip - the kernels as a loadable code object (libpam_kernels.hsaco).
//
// The reference builds its compute pipelines at run time from a shader library
// (PagedAttentionEngine.swift:151-198, 248-333).  Here the equivalent is a gfx950
// code object with named (extern "C") entry points, loaded with hipModuleLoad
// and launched with hipModuleLaunchKernel (pam_module_load / pam_module_launch).
// Each entry runs the same body as the library's own kernel of that
// configuration, with the same launch bounds and parameters, so a context bound
// to the module gives the same results bit for bit.  Built by build.py with
// hipcc --cuda-device-only; it is not part of libpam.so.
#include "../kernels/append_body.h"
#include "../kernels/attention_body.h"
#include "../kernels/mixed_body.h"
#include "../kernels/prefill_body.h"
#include "../kernels/stage_body.h"
#include "../kernels/valu_body.h"

namespace pam {

#define PAM_STREAMK_ENTRY(NAME, KV, HD, BLK, FL)                                                      \
    extern "C" __global__ __launch_bounds__(64 * kMfmaWaves, (MfmaShape<KV, HD>::OCC)) void NAME( \
        AttnParams p) {                                                                                \
        streamk_body<KV, HD, BLK, FL>(p, blockIdx.x, gridDim.x);                                     \
    }
#define PAM_WG_ENTRY(NAME, KV)                                                                        \
    extern "C" __global__ __launch_bounds__(64 * kMfmaWaves, (MfmaShape<KV, 128>::OCC)) void NAME( \
        AttnParams p) {                                                                                \
        __shared__ __attribute__((aligned(16))) char smem[MfmaShape<KV, 128>::kSmemBytes];           \
        __shared__ float sm_ml[kMfmaWaves][16][2];                                                    \
        mfma_item<KV, 128, kBlkTile>(p, blockIdx.z, blockIdx.x, blockIdx.y, smem, sm_ml);             \
    }
#define PAM_PREFILL_ENTRY(NAME, HD, FUSED, KV)                                               \
    extern "C" __global__ __launch_bounds__(64 * kPrefillWaves, 1) void NAME(AttnParams p) { \
        prefill_body<HD, kPrefillRB, FUSED, KV>(p);                                           \
    }
#define PAM_MIXED_ENTRY(NAME, KV)                                                            \
    extern "C" __global__ __launch_bounds__(64 * kPrefillWaves, 1) void NAME(AttnParams p) { \
        mixed_body<KV>(p);                                                                    \
    }
#define PAM_VALU_ENTRY(NAME, KV, QT, NH)                                                          \
    extern "C" __global__ __launch_bounds__(64) void NAME(AttnParams p, int lanes_per_row) {    \
        valu_body<KV, QT, NH>(p, lanes_per_row);                                                 \
    }
#define PAM_VALU_WG_ENTRY(NAME, KV, QT, NH)                                                                  \
    extern "C" __global__ __launch_bounds__(64 * kValuWgMaxParts) void NAME(AttnParams p, int lanes_per_row) { \
        __shared__ float wg_lds[kValuWgLds<NH>];                                                             \
        valu_body<KV, QT, NH, true>(p, lanes_per_row, wg_lds);                                              \
    }
#define PAM_APPEND_ENTRY(NAME, CH)                                                                          \
    extern "C" __global__ __launch_bounds__(256) void NAME(AppendParams p, int64_t chunks_per_row,        \
                                                           int64_t total) {                               \
        append_body<CH>(p, chunks_per_row, total);                                                         \
    }
#define PAM_APPEND_BATCH_ENTRY(NAME, CH)                                                                    \
    extern "C" __global__ __launch_bounds__(256) void NAME(AppendBatchParams p, int64_t chunks_per_row,   \
                                                           int64_t total) {                               \
        append_batch_body<CH>(p, chunks_per_row, total);                                                   \
    }

// decode, stream-K form, d = 128, blocks of 16 tokens or more
PAM_STREAMK_ENTRY(pam_decode_streamk_f16_d128, f16, 128, kBlkTile, false)
PAM_STREAMK_ENTRY(pam_decode_streamk_e4m3_d128, uint8_t, 128, kBlkTile, false)
// decodeLayers: the heads of several layers per K/V tile
PAM_STREAMK_ENTRY(pam_decode_layers_streamk_f16_d128, f16, 128, kBlkTile, true)
PAM_STREAMK_ENTRY(pam_decode_layers_streamk_e4m3_d128, uint8_t, 128, kBlkTile, true)
// decode, workgroup form (more rows than the stream-K form takes)
PAM_WG_ENTRY(pam_decode_wg_f16_d128, f16)
PAM_WG_ENTRY(pam_decode_wg_e4m3_d128, uint8_t)
// VALU rows (f32 KV, groups below 4): KV type and query heads per wave
PAM_VALU_ENTRY(pam_decode_valu_f32_h1, float, float, 1)
PAM_VALU_ENTRY(pam_decode_valu_f32_h2, float, float, 2)
PAM_VALU_ENTRY(pam_decode_valu_f32_h4, float, float, 4)
PAM_VALU_ENTRY(pam_decode_valu_f32_h8, float, float, 8)
PAM_VALU_ENTRY(pam_decode_valu_f16_h1, f16, f16, 1)
PAM_VALU_ENTRY(pam_decode_valu_f16_h2, f16, f16, 2)
PAM_VALU_ENTRY(pam_decode_valu_f16_h4, f16, f16, 4)
PAM_VALU_ENTRY(pam_decode_valu_f16_h8, f16, f16, 8)
PAM_VALU_ENTRY(pam_decode_valu_e4m3_h1, uint8_t, f16, 1)
PAM_VALU_ENTRY(pam_decode_valu_e4m3_h2, uint8_t, f16, 2)
PAM_VALU_ENTRY(pam_decode_valu_e4m3_h4, uint8_t, f16, 4)
PAM_VALU_ENTRY(pam_decode_valu_e4m3_h8, uint8_t, f16, 8)
// their workgroup form: a (row, head group)'s partitions as the waves of one
// workgroup, merged in LDS
PAM_VALU_WG_ENTRY(pam_decode_valu_wg_f32_h1, float, float, 1)
PAM_VALU_WG_ENTRY(pam_decode_valu_wg_f32_h2, float, float, 2)
PAM_VALU_WG_ENTRY(pam_decode_valu_wg_f16_h1, f16, f16, 1)
PAM_VALU_WG_ENTRY(pam_decode_valu_wg_f16_h2, f16, f16, 2)
PAM_VALU_WG_ENTRY(pam_decode_valu_wg_e4m3_h1, uint8_t, f16, 1)
PAM_VALU_WG_ENTRY(pam_decode_valu_wg_e4m3_h2, uint8_t, f16, 2)
// split-context reduce, by output type
extern "C" __global__ __launch_bounds__(256) void pam_reduce_f32(AttnParams p) { reduce_body<float>(p); }
extern "C" __global__ __launch_bounds__(256) void pam_reduce_f16(AttnParams p) { reduce_body<f16>(p); }
// dense chunked prefill, d = 128 and d = 64
PAM_PREFILL_ENTRY(pam_prefill_f16_d128, 128, false, f16)
PAM_PREFILL_ENTRY(pam_prefill_fused_f16_d128, 128, true, f16)
PAM_PREFILL_ENTRY(pam_prefill_e4m3_d128, 128, false, uint8_t)
PAM_PREFILL_ENTRY(pam_prefill_f16_d64, 64, false, f16)
PAM_PREFILL_ENTRY(pam_prefill_fused_f16_d64, 64, true, f16)
PAM_PREFILL_ENTRY(pam_prefill_e4m3_d64, 64, false, uint8_t)
// one-launch mixed step
PAM_MIXED_ENTRY(pam_mixed_step_f16_d128, f16)
PAM_MIXED_ENTRY(pam_mixed_step_e4m3_d128, uint8_t)
// KV append: token rows moved in 16-, 4- or 2-byte pieces
PAM_APPEND_ENTRY(pam_append_b16, uint4)
PAM_APPEND_ENTRY(pam_append_b4, uint32_t)
PAM_APPEND_ENTRY(pam_append_b2, uint16_t)
PAM_APPEND_BATCH_ENTRY(pam_append_batch_b16, uint4)
PAM_APPEND_BATCH_ENTRY(pam_append_batch_b4, uint32_t)
PAM_APPEND_BATCH_ENTRY(pam_append_batch_b2, uint16_t)
// FP8 quantize-on-append, one workgroup per touched block
extern "C" __global__ __launch_bounds__(256) void pam_append_fp8(AppendBatchParams p, int32_t first_lb,
                                                                 int32_t single_offset) {
    append_fp8_body(p, first_lb, single_offset);
}
// copy-on-write of one block
extern "C" __global__ __launch_bounds__(256) void pam_block_copy(uint4 *k_pool, uint4 *v_pool, uint16_t *k_scale,
                                                                 uint16_t *v_scale, int64_t n16, int32_t src,
                                                                 int32_t dst) {
    block_copy_body(k_pool, v_pool, k_scale, v_scale, n16, src, dst);
}
// staging copy of per-call metadata from mapped pinned host memory
extern "C" __global__ __launch_bounds__(256) void pam_stage_copy(const uint4 *__restrict__ src,
                                                                 uint4 *__restrict__ dst, size_t n16,
                                                                 const uint8_t *__restrict__ src_tail,
                                                                 uint8_t *__restrict__ dst_tail, int tail) {
    stage_body(src, dst, n16, src_tail, dst_tail, tail);
}

// A plain entry for callers that drive pam_module_launch themselves: n words of
// dst set to value.
extern "C" __global__ __launch_bounds__(256) void pam_fill_u32(uint32_t *dst, uint32_t value, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = value;
}

}  // namespace pam
