// kernels.h - launch interface of the gfx950 kernels (host side).
//
// The runtime (engine.cpp) fills these parameter blocks and calls the launchers;
// every launcher enqueues on the given HIP stream and returns the launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <vector>

namespace pam {

enum DType : int32_t { kF32 = 0, kF16 = 1, kFP8 = 2 };

constexpr float kLog2eHost = 1.4426950408889634f;
// size of the all-zero device page the attention kernels read for masked lanes
constexpr size_t kZeroPageBytes = 4096;

// How a work row (one query token) finds its keys.
enum RowMode : int32_t {
    kRowDecode = 0,   // row r = sequence r of a batch; keys [L - W, L) of seq_lengths[r]
    kRowPrefill = 1,  // row r = query position q_offset + r of one sequence (causal / fixed window)
    kRowRagged = 2,   // row r described by row_info[r] = {bt_row, k_lo, k_hi, q/out row}
};

// Layers whose query heads one decode launch can serve from each K/V tile (the
// MFMA decode holds up to 16 query heads per kv head; G >= 4).
constexpr int kMaxFusedLayers = 4;

// most partitions of the VALU kernel's workgroup form (one wave each)
constexpr int kValuWgMaxParts = 16;

struct AttnParams {
    const void *q;             // [rows][H][d] (f32 for f32 caches, f16 otherwise)
    void *out;                 // [rows][H][d] same type as q
    const void *k_pool;        // [nb][bs][Hkv][d]
    const void *v_pool;
    const uint16_t *k_scale;   // fp8 only: half per physical block
    const uint16_t *v_scale;
    const int32_t *block_tables;   // [bt_rows][bt_stride]
    const uint32_t *seq_lengths;   // decode mode
    const int4 *row_info;          // ragged mode
    float *part_o;             // [rows][H][max_parts][d] split-context partial outputs
    float *part_ml;            // [rows][H][max_parts][2] (max in log2 units, sum)
                               // (stream-K: [part_slots][d] and [part_slots][2])
    uint64_t *seg_count;       // stream-K MFMA form: [rows][Hkv] merge counters (epoch-tagged)
    uint32_t part_bytes;       // stream-K: bytes of part_o + part_ml (< 2^31)
    const void *zero_page;     // >= 1 KiB of zeros: the source of masked lanes' loads
    int32_t rows;
    int32_t bt_stride;
    int32_t max_num_blocks;    // decode: logical blocks readable per row
    int32_t num_heads, num_kv_heads, head_dim, block_size, window;
    int32_t q_offset, causal, mode;
    int32_t part_tokens;       // tokens per split-context partition (multiple of 16)
    int32_t max_parts;
    int32_t heads_per_wave;    // VALU kernel: query heads handled by one wave
    float scale_log2;          // log2(e) / sqrt(d)
    // dense prefill work list (prefill_split_plan): three int4 per segment
    //   {bt_row, q_offset, len, row_base} of its chunk, {kv head, first token,
    //   t_lo, t_hi} (key tiles), {slot0, piece, pieces, 0},
    // a [first, last) segment range per workgroup, and the partial slots and
    // counters of items split over several workgroups
    const int4 *pf_work;
    const int2 *pf_range;
    float *pf_part;
    uint64_t *pf_count;        // one merge counter per slot (epoch-tagged)
    uint32_t pf_part_bytes;
    int32_t pf_groups;         // workgroups of the launch
    // dense prefill, fused append (f16): the chunks' new keys and values
    // [rows][Hkv][d] (row = the chunk's row_base + token).  Keys at or past a
    // chunk's q_offset are read from here, and the kernel writes them into the
    // pools.  Null: all keys come from the pools.
    const void *fuse_k, *fuse_v;
    // decode over layers sharing one pool (decodeLayers): the heads of
    // fused_layers layers share every K/V tile, so query-head slot v of a kv
    // head is head v % G of layer v / G, read from layer_q[v / G] and written to
    // layer_out[v / G].  fused_layers <= 1: p.q / p.out only.  Stream-K MFMA
    // decode only (G * fused_layers <= 16).
    int32_t fused_layers;
    const void *layer_q[kMaxFusedLayers];
    void *layer_out[kMaxFusedLayers];
    // tag of this launch for the merge counters: a counter holding another epoch
    // counts as zero arrivals, so counters need no reset.  The launchers set a
    // fresh nonzero epoch for every launch (a retried launch gets a new one).
    uint32_t epoch;
    // VALU kernel: 1 runs a (row, head group)'s partitions as the waves of one
    // workgroup (attn_valu_wg_kernel), merged in LDS
    int32_t valu_wg;
};

// Entry points of a loaded code object (libpam_kernels.hsaco, module_entry.hip).
// A launcher given a table launches a configuration the table holds through
// hipModuleLaunchKernel, and any other through the library's own kernel (or
// refuses it with hipErrorNotFound when the table is strict); both run the same
// kernel body.
struct KernelTable {
    hipFunction_t streamk[2][2];  // decode stream-K, d = 128, blocks >= 16: [f16, e4m3][one layer, fused layers]
    hipFunction_t mfma_wg[2];     // decode, workgroup form (rows > 2048), d = 128, blocks >= 16: f16, e4m3
    hipFunction_t prefill[2][3];  // dense prefill, [d = 128, d = 64][f16, f16 with fused append, e4m3]
    hipFunction_t mixed[2];       // one-launch mixed step: f16, e4m3
    hipFunction_t valu[3][4];     // VALU rows: [f32, f16, e4m3 KV][1, 2, 4, 8 heads per wave]
    hipFunction_t valu_wg[3][2];  // their workgroup form: [KV][1, 2 heads per wave]
    hipFunction_t reduce[2];      // split-context reduce: f32, f16 outputs
    hipFunction_t append[3];      // append copy in 16-, 4- or 2-byte pieces
    hipFunction_t append_batch[3];
    hipFunction_t append_fp8;     // FP8 quantize-on-append (single sequence and batched)
    hipFunction_t stage;          // staging copy
    hipFunction_t block_copy;     // copy-on-write of one block
    bool strict;                  // refuse configurations the table lacks
};
// hipModuleLaunchKernel of `f` with the kernel arguments `a...` (each passed by
// address, as the kernel declares them).
template <class... A>
inline hipError_t module_launch(hipFunction_t f, dim3 grid, dim3 block, hipStream_t stream, A... a) {
    void *args[] = {static_cast<void *>(&a)...};
    return hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0, stream, args, nullptr);
}
// The code-object side of a launcher: with a table, launches its entry `f`
// (or, strict and without one, refuses) and returns true with the status in
// *e; false: launch the library's kernel.
template <class... A>
inline bool via_module(const KernelTable *kt, hipFunction_t f, hipError_t *e, dim3 grid, dim3 block,
                       hipStream_t stream, A... a) {
    if (!kt) return false;
    if (f) {
        *e = module_launch(f, grid, block, stream, a...);
        return true;
    }
    if (kt->strict) {
        *e = hipErrorNotFound;
        return true;
    }
    return false;
}
// Resident workgroups per CU of the library's stream-K kernel (dtype f16 / fp8,
// d = 128, blocks >= 16, one layer or fused layers), for checking a code
// object's entry against it.
hipError_t streamk_occupancy(int32_t dtype, bool fused_layers, int *per_cu);

// Paged attention over rows (decode / prefill-as-rows / ragged).  Chooses the
// MFMA kernel for 4 <= H/Hkv <= 16 with f16/fp8 KV and d in {64,128,256},
// otherwise the VALU kernel.  Launches the split-context reduce when max_parts > 1.
hipError_t launch_attention(const AttnParams &p, int32_t dtype, bool use_mfma, hipStream_t stream,
                            hipEvent_t after_main = nullptr, const KernelTable *kt = nullptr);
bool mfma_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size);
// A fresh launch epoch for the merge counters: process-wide (one counter for the
// whole library, an inline function's static), so launches of any context that
// share counters never repeat one; 0 (zeroed memory) is skipped.
inline uint32_t next_launch_epoch() {
    static std::atomic<uint32_t> epoch{0};
    uint32_t e;
    do e = epoch.fetch_add(1, std::memory_order_relaxed) + 1;
    while (e == 0);
    return e;
}
// Stream-K form of the MFMA kernel (rows <= 2048): one launch, no reduce kernel.
// Gives the partial slots (floats per slot: d + 2) and the 64-bit merge counters
// it needs.  Counters start as any value an earlier launch left (or zero) and
// are never reset; launches that share counters must not overlap.  False: not
// applicable.
bool mfma_streamk_plan(const AttnParams &p, int32_t dtype, int64_t *part_slots, int64_t *counters);

// Allocation-free decode: a fixed device array per GPU (noalloc.hip) laid out as
// [zero page | merge counters | split-context partials].
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
constexpr size_t kNoAllocZeroBytes = 4096;
constexpr size_t kNoAllocCounterBytes = (size_t)1 << 20;
// Looks up (once per device, with `device` current) the array's device address,
// clears its zero page on `stream` and returns the address.
hipError_t noalloc_scratch_setup(int device, hipStream_t stream, void **out);
// The address set up for `device`, or null before noalloc_scratch_setup.
void *noalloc_scratch(int device);

// KV append into the paged pools.
struct AppendParams {
    const void *keys;          // [n][Hkv][d] (f32 for f32 caches, f16 for f16 and fp8)
    const void *values;
    void *k_pool;
    void *v_pool;
    uint16_t *k_scale;         // fp8: per-block half scales (read-modify-write)
    uint16_t *v_scale;
    const int32_t *block_table;   // one sequence's table (token_offset mode)
    const int64_t *slot_mapping;  // optional: explicit slot per token (overrides the table)
    int32_t token_offset;
    int32_t num_tokens;
    int32_t num_kv_heads, head_dim, block_size;
    // one-token appends of a sequence whose table lives on the device (the
    // decode step): fixed_slot >= 0 is token 0's pool slot, computed by the
    // host, and the kernel also writes table_patch[patch_index] = patch_block
    // (when table_patch is set) and *length_patch = length_value, the table
    // and length the decode launched after it reads
    int64_t fixed_slot = -1;
    int32_t *table_patch = nullptr;
    uint32_t *length_patch = nullptr;
    int32_t patch_index = 0, patch_block = 0;
    uint32_t length_value = 0;
};
hipError_t launch_append(const AppendParams &p, int32_t dtype, hipStream_t stream, const KernelTable *kt = nullptr);

// Batched append for a mixed step.  f32/f16: token t goes to position
// token_pos[t].y of sequence token_pos[t].x through that sequence's block-table
// row.  fp8: one workgroup per work entry (sequence, logical block); the
// sequence's tokens are keys[cu_tokens[s] .. cu_tokens[s+1]) at positions
// token_offsets[s] + i.
struct AppendBatchParams {
    const void *keys;
    const void *values;
    void *k_pool;
    void *v_pool;
    uint16_t *k_scale;
    uint16_t *v_scale;
    const int32_t *block_tables;  // [seqs][bt_stride]
    const int32_t *cu_tokens;     // [seqs + 1] prefix sums of tokens per sequence
    const int32_t *token_offsets; // [seqs]
    const int4 *work;             // fp8: one entry per touched block {seq, logical block, 0, 0}
    int32_t num_work;
    const int2 *token_pos;        // f32/f16: per input token {sequence, position}
    int32_t seqs, bt_stride, total_tokens;
    int32_t num_kv_heads, head_dim, block_size;
};
// Copy-on-write of one block (block_bytes per pool, a multiple of 16): K and V
// bytes and, when the scale pointers are set, the FP8 scales, src -> dst.
// hipErrorInvalidValue for sizes or pools it cannot copy in 16-byte pieces.
hipError_t launch_block_copy(void *k_pool, void *v_pool, uint16_t *k_scale, uint16_t *v_scale, size_t block_bytes,
                             int32_t src, int32_t dst, hipStream_t stream, const KernelTable *kt = nullptr);
hipError_t launch_append_batch(const AppendBatchParams &p, int32_t dtype, hipStream_t stream,
                               const KernelTable *kt = nullptr);

// Attention gradients of one sequence (training path): non-causal rows
// 0 .. seq_len-1 over keys [window_start, seq_len); m, l are the forward's row max
// and sum (natural-log units), row_d is a [seq_len][H] float workspace.
struct BackwardParams {
    const void *q, *k_pool, *v_pool, *d_out;  // f32 or f16 (the cache type)
    const int32_t *block_table;
    const float *m, *l;
    void *d_q, *d_k_pool, *d_v_pool;
    float *row_d;  // [seq_len][num_heads]: D_i = sum_j P_ij dP_ij
    float *row_c;  // [seq_len][num_heads]: m_i log2(e) + log2(l_i) (MFMA path)
    int32_t seq_len, window_start;
    int32_t num_heads, num_kv_heads, head_dim, block_size;
    float scale;  // 1 / sqrt(head_dim)
};
hipError_t launch_backward(const BackwardParams &p, int32_t dtype, hipStream_t stream);

// Exhaustive codec entry points (used by the codec tests through the C ABI).
hipError_t launch_fp8_quantize(const uint16_t *values, const uint16_t *scales, uint8_t *out, int64_t n,
                               hipStream_t stream);
hipError_t launch_fp8_dequant(const uint8_t *codes, const uint16_t *scales, uint16_t *out, int64_t n,
                              hipStream_t stream);

// Copy `bytes` from mapped pinned host memory to the device, as a kernel on
// `stream` (both pointers 16-byte aligned).
hipError_t launch_stage_copy(const void *host_mapped, void *dst, size_t bytes, hipStream_t stream,
                             const KernelTable *kt = nullptr);

// Calibration streams of known size (achievable HBM rates, counter scaling).
hipError_t launch_stream_read(const void *src, size_t bytes, uint32_t *sink, int blocks, hipStream_t stream);
hipError_t launch_stream_copy(const void *src, void *dst, size_t bytes, int blocks, hipStream_t stream);
// Dense f16 MFMA loop: `blocks` workgroups of 8 waves, each wave `iters` x 4
// v_mfma_f32_32x32x16_f16 (32768 flops each); sink never written in practice.
hipError_t launch_mfma_loop(int blocks, int iters, float *sink, hipStream_t stream);
// Counter-based synthetic normals (synth.hip).
hipError_t launch_synth_normal(void *dst, int32_t dtype, uint64_t n, uint64_t seed, uint64_t stream, float stddev,
                               int64_t outlier_stream, float outlier_frac, hipStream_t s);

// Dense chunked-prefill (MFMA, f16): rows [q_offset, q_offset + T) of one sequence.
// Dense prefill (MFMA): f16 or e4m3 KV, d = 128; Q and O f16.
hipError_t launch_prefill_mfma(const AttnParams &p, int32_t dtype, hipStream_t stream,
                              const KernelTable *kt = nullptr);
// Work list of the dense prefill kernel for chunks {bt_row, q_offset, len,
// row_base} (host memory).  An item is (chunk, kv head, block of 256 / G query rows)
// over its key tiles; items are cut into segments so that the `groups`
// workgroups get about the same number of tiles.  Fills p.pf_groups; the caller
// stages `work` and `range` to the device and provides `slots` partial slots of
// kPrefillSlotBytes and as many 64-bit merge counters (epoch-tagged: any
// starting value).
struct PrefillSplit {
    std::vector<int4> work;
    std::vector<int2> range;
    int64_t slots = 0;
};
constexpr int64_t kPrefillSlotBytes = 8 * 64 * (64 + 2) * 4;  // one workgroup's O^T, m, l
// allow_split false: grid order only (no item is cut into pieces).
void prefill_split_plan(const int4 *chunks, int32_t n, AttnParams &p, int32_t groups, PrefillSplit &out,
                        bool allow_split = true);
bool prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size);

// One launch for a mixed step (mixed.hip): the dense prefill's work list (p.pf_*,
// p.pf_groups workgroups first) and the stream-K decode of p.rows single-token
// rows on `decode_groups` workgroups of 8 waves after them.
constexpr int kMixedMaxRows = 1024;  // decode rows one mixed launch takes
bool mixed_launch_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size, int32_t rows);
// partial slots (d + 2 floats each) and merge counters of the decode part
void mixed_decode_slots(const AttnParams &p, int32_t decode_groups, int64_t *part_slots, int64_t *counters);
hipError_t launch_mixed_step(const AttnParams &p, int32_t dtype, int32_t decode_groups, hipStream_t stream,
                             const KernelTable *kt = nullptr);

}  // namespace pam
