// attention.hip - paged attention over query rows for gfx950.
//
// A row is a decode query (kernels.metal:1417-1802 semantics), a prefill query
// position (kernels.metal:693-917 semantics with an explicit query offset) or a
// ragged row of a mixed continuous-batching step.  Keys are walked in 16-token
// tiles of the logical sequence; the block table maps each token to its
// physical block, so blocks may sit anywhere in the pool.
//
// Bodies:
//  * the MFMA tile loop (mfma_core) - GQA groups >= 4, f16 or e4m3 KV: token
//    rows are loaded whole (16 lanes per 256-byte row), staged through LDS, and
//    S^T = K Q^T (v_mfma_f32_16x16x32_f16, query heads on the N side) and
//    O^T = V^T P^T (v_mfma_f32_16x16x16_f16, V^T read with the transposing
//    ds_read_b64_tr_b16) run on them; the S^T accumulator layout is P^T's
//    B-operand layout, so softmax needs no data movement.  Two work forms:
//      - attn_mfma_streamk (up to kStreamKMaxRows rows): the resident grid
//        splits all rows' tiles into equal units and merges split rows itself;
//      - attn_mfma_kernel: one workgroup per (row, partition, kv head), its
//        waves merged in LDS, partitions merged by attn_reduce_kernel;
//  * attn_valu_kernel - any group and f32 KV: lanes split a token row into
//    4-element slices, dot products reduce across the row's lanes.
// All keep the online-softmax state of Reference/paged_attention_sim.py:94-123
// (in log2 units).
#include "attention_body.h"
#include "valu_body.h"

namespace pam {

template <typename KV, int HD, int BLK>
__global__ __launch_bounds__(64 * kMfmaWaves, (MfmaShape<KV, HD>::OCC)) void attn_mfma_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) char smem[MfmaShape<KV, HD>::kSmemBytes];
    __shared__ float sm_ml[kMfmaWaves][16][2];
    mfma_item<KV, HD, BLK>(p, blockIdx.z, blockIdx.x, blockIdx.y, smem, sm_ml);
}

// The kernel (the fat binary's entry); streamk_body also backs the named
// entries of the code object (module_entry.hip).
template <typename KV, int HD, int BLK, bool FL>
__global__ __launch_bounds__(64 * kMfmaWaves, (MfmaShape<KV, HD>::OCC)) void attn_mfma_streamk(AttnParams p) {
    streamk_body<KV, HD, BLK, FL>(p, blockIdx.x, gridDim.x);
}

// The kernels (the fat binary's entries); valu_body and reduce_body also back
// the named entries of the code object (module_entry.hip).
template <typename KV, typename QT, int NH>
__global__ __launch_bounds__(64) void attn_valu_kernel(AttnParams p, int lanes_per_row) {
    valu_body<KV, QT, NH>(p, lanes_per_row);
}

// One workgroup per (row, head group): wave w runs partition w, the waves merge
// in LDS (AttnParams::valu_wg).
template <typename KV, typename QT, int NH>
__global__ __launch_bounds__(64 * kValuWgMaxParts) void attn_valu_wg_kernel(AttnParams p, int lanes_per_row) {
    __shared__ float wg_lds[kValuWgLds<NH>];
    valu_body<KV, QT, NH, true>(p, lanes_per_row, wg_lds);
}

template <typename QT>
__global__ __launch_bounds__(256) void attn_reduce_kernel(AttnParams p) {
    reduce_body<QT>(p);
}

// ------------------------------------------------------------------ launchers

bool mfma_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size) {
    return (dtype == kF16 || dtype == kFP8) && (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
           group >= 1 && group <= 16 && block_size >= 8 && (block_size & (block_size - 1)) == 0;
}

// Resident workgroups of the stream-K kernel on this device (its grid), queried
// once per instantiation.
template <typename KV, int HD, int BLK>
static hipError_t streamk_grid(int *grid) {
    static int resident = 0;
    if (resident == 0) {
        int dev = 0, cus = 0, per_cu = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e == hipSuccess)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_mfma_streamk<KV, HD, BLK, false>,
                                                             64 * kMfmaWaves, 0);
        if (e != hipSuccess) return e;
        if (per_cu > MfmaShape<KV, HD>::GRID_PER_CU) per_cu = MfmaShape<KV, HD>::GRID_PER_CU;
        resident = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    }
    *grid = resident;
    return hipSuccess;
}

hipError_t streamk_occupancy(int32_t dtype, bool fused_layers, int *per_cu) {
    const int t = 64 * kMfmaWaves;
    if (dtype == kF16)
        return fused_layers
                   ? hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, attn_mfma_streamk<f16, 128, kBlkTile, true>, t, 0)
                   : hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, attn_mfma_streamk<f16, 128, kBlkTile, false>, t, 0);
    if (dtype == kFP8)
        return fused_layers
                   ? hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, attn_mfma_streamk<uint8_t, 128, kBlkTile, true>, t, 0)
                   : hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, attn_mfma_streamk<uint8_t, 128, kBlkTile, false>, t, 0);
    return hipErrorInvalidValue;
}

template <typename KV, int HD, int BLK>
static hipError_t launch_mfma_blk(const AttnParams &p, hipStream_t stream, const KernelTable *kt) {
    const dim3 block(64 * kMfmaWaves);
    if (p.seg_count != nullptr) {
        if (p.rows > kStreamKMaxRows) return hipErrorInvalidValue;
        int grid = 0;
        const hipError_t e = streamk_grid<KV, HD, BLK>(&grid);
        if (e != hipSuccess) return e;
        hipError_t me;
        if (via_module(kt, kt && HD == 128 && BLK == kBlkTile ? kt->streamk[sizeof(KV) == 1][p.fused_layers > 1] : nullptr,
                       &me, dim3(grid), block, stream, p))
            return me;
        // fused layers run on the same grid (the partial slots are planned for it;
        // no wave waits on another, so residency is a matter of speed only)
        if (p.fused_layers > 1)
            hipLaunchKernelGGL((attn_mfma_streamk<KV, HD, BLK, true>), dim3(grid), block, 0, stream, p);
        else
            hipLaunchKernelGGL((attn_mfma_streamk<KV, HD, BLK, false>), dim3(grid), block, 0, stream, p);
        return hipGetLastError();
    }
    const dim3 grid(p.max_parts, p.num_kv_heads, p.rows);
    hipError_t me;
    if (via_module(kt, kt && HD == 128 && BLK == kBlkTile ? kt->mfma_wg[sizeof(KV) == 1] : nullptr, &me, grid, block,
                   stream, p))
        return me;
    hipLaunchKernelGGL((attn_mfma_kernel<KV, HD, BLK>), grid, block, 0, stream, p);
    return hipGetLastError();
}

template <typename KV, int HD>
static hipError_t launch_mfma_hd(const AttnParams &p, hipStream_t stream, const KernelTable *kt) {
    if (p.block_size % 16 == 0) return launch_mfma_blk<KV, HD, kBlkTile>(p, stream, kt);
    if (p.block_size == 8) return launch_mfma_blk<KV, HD, kBlkSmall>(p, stream, kt);
    return hipErrorInvalidValue;
}

template <typename KV>
static hipError_t launch_mfma(const AttnParams &p, hipStream_t stream, const KernelTable *kt) {
    switch (p.head_dim) {
        case 64: return launch_mfma_hd<KV, 64>(p, stream, kt);
        case 128: return launch_mfma_hd<KV, 128>(p, stream, kt);
        case 256: return launch_mfma_hd<KV, 256>(p, stream, kt);
        default: return hipErrorInvalidValue;
    }
}

template <typename KV, int HD>
static hipError_t streamk_grid_hd(int block_size, int *grid) {
    if (block_size % 16 == 0) return streamk_grid<KV, HD, kBlkTile>(grid);
    if (block_size == 8) return streamk_grid<KV, HD, kBlkSmall>(grid);
    return hipErrorInvalidValue;
}

template <typename KV>
static hipError_t streamk_grid_kv(int head_dim, int block_size, int *grid) {
    switch (head_dim) {
        case 64: return streamk_grid_hd<KV, 64>(block_size, grid);
        case 128: return streamk_grid_hd<KV, 128>(block_size, grid);
        case 256: return streamk_grid_hd<KV, 256>(block_size, grid);
        default: return hipErrorInvalidValue;
    }
}

bool mfma_streamk_plan(const AttnParams &p, int32_t dtype, int64_t *part_slots, int64_t *counters) {
    if (p.rows <= 0 || p.rows > kStreamKMaxRows) return false;
    if (!mfma_supported(dtype, p.head_dim, p.num_heads / p.num_kv_heads, p.block_size)) return false;
    int grid = 0;
    const hipError_t e = dtype == kF16 ? streamk_grid_kv<f16>(p.head_dim, p.block_size, &grid)
                                       : streamk_grid_kv<uint8_t>(p.head_dim, p.block_size, &grid);
    if (e != hipSuccess) return false;
    const int64_t Hkv = p.num_kv_heads;
    const int64_t G = (int64_t)(p.num_heads / p.num_kv_heads) * (p.fused_layers > 1 ? p.fused_layers : 1);
    const int64_t NH = Hkv % 4 == 0 ? 4 : (Hkv % 2 == 0 ? 2 : 1);
    const int64_t units = (int64_t)grid * (kMfmaWaves / NH) / (Hkv / NH);
    *part_slots = (units + (int64_t)p.rows) * Hkv * G;
    *counters = (int64_t)p.rows * Hkv;
    return true;
}

template <typename KV, typename QT>
static hipError_t launch_valu(const AttnParams &p, hipStream_t stream, const KernelTable *kt) {
    int lpr = 1;
    while (lpr * 4 < p.head_dim) lpr <<= 1;
    if (lpr > 64 || p.head_dim % 4 != 0) return hipErrorInvalidValue;
    const int nh = p.heads_per_wave;
    if (p.valu_wg) {
        if ((nh != 1 && nh != 2) || p.max_parts < 2 || p.max_parts > kValuWgMaxParts) return hipErrorInvalidValue;
        const dim3 wgrid(1, p.num_heads / nh, p.rows), wblock(64 * p.max_parts);
        const int kvi = sizeof(KV) == 4 ? 0 : (sizeof(KV) == 2 ? 1 : 2);
        hipError_t me;
        if (via_module(kt, kt ? kt->valu_wg[kvi][nh - 1] : nullptr, &me, wgrid, wblock, stream, p, lpr)) return me;
        if (nh == 1)
            hipLaunchKernelGGL((attn_valu_wg_kernel<KV, QT, 1>), wgrid, wblock, 0, stream, p, lpr);
        else
            hipLaunchKernelGGL((attn_valu_wg_kernel<KV, QT, 2>), wgrid, wblock, 0, stream, p, lpr);
        return hipGetLastError();
    }
    dim3 grid(p.max_parts, p.num_heads / nh, p.rows);
    const int slot = nh == 1 ? 0 : (nh == 2 ? 1 : (nh == 4 ? 2 : (nh == 8 ? 3 : -1)));
    if (slot < 0) return hipErrorInvalidValue;
    const int kvi = sizeof(KV) == 4 ? 0 : (sizeof(KV) == 2 ? 1 : 2);
    hipError_t me;
    if (via_module(kt, kt ? kt->valu[kvi][slot] : nullptr, &me, grid, dim3(64), stream, p, lpr)) return me;
    switch (nh) {
        case 1: hipLaunchKernelGGL((attn_valu_kernel<KV, QT, 1>), grid, dim3(64), 0, stream, p, lpr); break;
        case 2: hipLaunchKernelGGL((attn_valu_kernel<KV, QT, 2>), grid, dim3(64), 0, stream, p, lpr); break;
        case 4: hipLaunchKernelGGL((attn_valu_kernel<KV, QT, 4>), grid, dim3(64), 0, stream, p, lpr); break;
        case 8: hipLaunchKernelGGL((attn_valu_kernel<KV, QT, 8>), grid, dim3(64), 0, stream, p, lpr); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_attention(const AttnParams &p_in, int32_t dtype, bool use_mfma, hipStream_t stream,
                            hipEvent_t after_main, const KernelTable *kt) {
    if (p_in.rows <= 0) return hipSuccess;
    AttnParams p = p_in;
    p.epoch = next_launch_epoch();
    // masked lanes of the MFMA kernel read a lane-group slice of one token row
    // from the zero page: it must exist and cover head_dim elements
    if (p.zero_page == nullptr || (size_t)p.head_dim * 4 > kZeroPageBytes) return hipErrorInvalidValue;
    hipError_t e;
    if (use_mfma) {
        e = dtype == kF16 ? launch_mfma<f16>(p, stream, kt) : launch_mfma<uint8_t>(p, stream, kt);
    } else {
        switch (dtype) {
            case kF32: e = launch_valu<float, float>(p, stream, kt); break;
            case kF16: e = launch_valu<f16, f16>(p, stream, kt); break;
            case kFP8: e = launch_valu<uint8_t, f16>(p, stream, kt); break;
            default: return hipErrorInvalidValue;
        }
    }
    if (e != hipSuccess) return e;
    if (after_main) (void)hipEventRecord(after_main, stream);
    // stream-K (MFMA) and the VALU kernel with counters merge in the kernel
    if (p.max_parts <= 1 || p.seg_count != nullptr || p.valu_wg) return e;
    dim3 grid((p.num_heads + 3) / 4, p.rows);
    if (via_module(kt, kt ? kt->reduce[dtype != kF32] : nullptr, &e, grid, dim3(256), stream, p)) return e;
    if (dtype == kF32)
        hipLaunchKernelGGL((attn_reduce_kernel<float>), grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((attn_reduce_kernel<f16>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace pam
