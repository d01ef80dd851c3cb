// pam_device.h - device-side helpers shared by the gfx950 kernels.
//
// Vector types for MFMA operands, the e4m3 KV codec (bit-exact with the
// reference's kernels.metal:553-601 quantize_fp8 / dequant_fp8) and wave64
// shuffles.  Compiled only for gfx950.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pam {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// Cache-policy bits of an agent-scope buffer access on gfx950 (sc1): stores
// write through the XCD's L2 and loads do not hit a stale line there, so data
// written on one XCD can be read on another within a launch without a
// whole-L2 writeback.
constexpr int kSc1 = 16;

typedef __fp16 fp16x4_raw __attribute__((__vector_size__(4 * sizeof(__fp16))));
// ds_read_b64_tr_b16: the 16 lanes of a group each address 4 consecutive halves
// a[i][0..3]; lane o receives a[4j + o/4][o%4] for j = 0..3.
__device__ __forceinline__ f16x4 lds_read_tr16(const f16 *p) {
    const fp16x4_raw v =
        __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) fp16x4_raw *)(p));
    return __builtin_bit_cast(f16x4, v);
}

// 16 bytes per lane from global memory straight into LDS: lane L of the wave
// writes lds_base + 16 L (global_load_lds_dwordx4, counted by vmcnt).  With 4
// bytes, lane L writes lds_base + 4 L; inactive lanes write nothing.  Issued
// as inline assembly so that the compiler, which does not see these LDS writes,
// adds no wait for them before unrelated LDS reads: their users order them with
// explicit vmcnt waits and barriers.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p);
}
__device__ __forceinline__ void lds_dma16(const void *g, const void *lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr(lds_base)), "v"(g)
                 : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void *g, const void *lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds_addr(lds_base)), "v"(g)
                 : "memory", "m0");
}

__device__ __forceinline__ f16 bits_to_f16(uint16_t b) { return __builtin_bit_cast(f16, b); }
__device__ __forceinline__ uint16_t f16_to_bits(f16 h) { return __builtin_bit_cast(uint16_t, h); }

// ---------------------------------------------------------------- e4m3 codec
// dequant_fp8 (kernels.metal:553-562) evaluated in half, left to right:
//   e == 0: (+-scale * (m/8)) * 2^-6 ;  else (+-scale * (1 + m/8)) * 2^(e-7).
// Both products are single IEEE binary16 multiplies (round to nearest even),
// matching the reference's half arithmetic bit for bit.
__device__ __forceinline__ f16 fp8_dequant(uint32_t code, f16 scale) {
    const uint32_t e = (code >> 3) & 0xFu, m = code & 7u;
    if ((code & 0x7Fu) == 0u) return (f16)0.0f;
    f16 s = (code & 0x80u) ? -scale : scale;
    // mantissa factor as an exact half: 1 + m/8 (bits 0x3C00 | m<<7) or m/8
    f16 mx = e ? bits_to_f16((uint16_t)(0x3C00u | (m << 7))) : (f16)((float)m * 0.125f);
    // power of two 2^(max(e,1)-7): half exponent field max(e,1) + 8
    f16 p2 = bits_to_f16((uint16_t)(((e ? e : 1u) + 8u) << 10));
    f16 t = s * mx;
    return t * p2;
}

// quantize_fp8 (kernels.metal:564-601): value/scale in float (IEEE division),
// clamp to +-448, subnormal codes below 2^-6 from round(v*512) clamped to 7,
// otherwise a 3-bit mantissa rounded half away from zero; saturates at 0x7E.
__device__ __forceinline__ uint32_t fp8_quantize(f16 value, f16 scale) {
    float v = (float)value / (float)scale;
    v = fminf(fmaxf(v, -448.0f), 448.0f);
    const uint32_t sign = v < 0.0f ? 0x80u : 0u;
    v = fabsf(v);
    if (v == 0.0f) return 0u;
    if (v < 0x1p-6f) {
        int mi = (int)roundf(v * 512.0f);
        mi = mi > 7 ? 7 : (mi < 0 ? 0 : mi);
        return sign | (uint32_t)mi;
    }
    int ex;
    float mant = frexpf(v, &ex);
    mant *= 2.0f;
    ex -= 1;
    if (ex > 8) return sign | 0x7Eu;
    int eb = ex + 7;
    int mi = (int)roundf((mant - 1.0f) * 8.0f);
    if (mi > 7) {
        mi = 0;
        eb++;
    }
    if (eb > 0xF) return sign | 0x7Eu;
    if (eb == 0xF && mi > 6) mi = 6;
    return sign | ((uint32_t)eb << 3) | (uint32_t)mi;
}

// per-block scale rule (kernels.metal:1944-1957)
__device__ __forceinline__ f16 fp8_scale_rule(float new_max_abs, f16 old_scale) {
    float mk = fmaxf(new_max_abs, (float)old_scale * 448.0f);
    return mk > 0.0f ? (f16)(mk / 448.0f) : (f16)1.0f;
}

// ---------------------------------------------------------------- wave64 shuffles
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// v moved across lanes by a DPP pattern (row_mask, bank_mask all lanes)
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Reduction of v over the lane distances lo, 2 lo, .., hi / 2 (powers of two):
// lane i combines the lanes i ^ m for m in that range.  A reduction from lo = 1
// runs its stages below 16 as DPP moves (quad_perm [1,0,3,2] and [2,3,0,1], then
// the half-row and row mirrors, which pair the already reduced quads and
// octets); other stages are ds_bpermute shuffles.
template <bool MAX>
__device__ __forceinline__ float wave_reduce_xor(float v, int lo, int hi) {
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    int m = lo;
    if (lo == 1) {
        if (hi > 1) v = op(v, dpp_mov<0xB1>(v));
        if (hi > 2) v = op(v, dpp_mov<0x4E>(v));
        if (hi > 4) v = op(v, dpp_mov<0x141>(v));
        if (hi > 8) v = op(v, dpp_mov<0x140>(v));
        m = 16;
    }
    for (; m < hi; m <<= 1) v = op(v, shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ float wave_max_xor(float v, int lo, int hi) { return wave_reduce_xor<true>(v, lo, hi); }
__device__ __forceinline__ float wave_sum_xor(float v, int lo, int hi) { return wave_reduce_xor<false>(v, lo, hi); }

// e4m3 bytes -> their exact binary16 values, two bytes per
// v_cvt_scalef32_pk_f16_fp8 (scale 1.0; word_sel picks bytes 0-1 or 2-3).  The
// hardware's OCP e4m3 decoding equals the reference's dequant_fp8 table
// (kernels.metal:553-562) for every code except 0x7F / 0xFF, which the
// reference's quantiser never writes (it saturates at 0x7E).
__device__ __forceinline__ f16x8 e4m3x8_to_f16x8(uint32_t w0, uint32_t w1) {
    const auto a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
    const auto b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
    const auto c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
    const auto d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
    return (f16x8){(f16)a[0], (f16)a[1], (f16)b[0], (f16)b[1], (f16)c[0], (f16)c[1], (f16)d[0], (f16)d[1]};
}

// Cross-workgroup merge counters.  A counter is 64 bits: the launch's epoch in
// the high word, the arrivals of that launch in the low word.  Every launch
// carries a fresh nonzero epoch, so a counter left behind by an earlier launch
// (one abandoned part-way, or zeroed memory: epoch 0) reads as zero arrivals and
// nothing ever resets a counter.  Launches that share counters never overlap,
// so a counter's epoch never exceeds the running launch's.
//
// arrive_count returns how many arrivals of this launch came before the
// caller's.  The caller must have completed (s_waitcnt vmcnt(0)) the sc1
// (agent-scope, L2 write-through) stores of whatever it publishes; the one
// that sees count - 1 reads the published data with sc1 loads issued after this
// returns.  Called by one lane.
__device__ __forceinline__ uint32_t arrive_count(uint64_t *counter, uint32_t epoch) {
    using g64 = __attribute__((address_space(1))) uint64_t;
    g64 *c = (g64 *)counter;
    const uint64_t tag = (uint64_t)epoch << 32;
    // raise a stale counter to (epoch, 0); a current one is already above tag.
    // The add is issued without waiting for the maximum: two atomics of one
    // thread on one location are applied in program order (same-location
    // coherence; a wave's requests to one address share one L2 channel queue).
    (void)__hip_atomic_fetch_max(c, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t old = __hip_atomic_fetch_add(c, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // no load of the published data may be moved above the count
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return (uint32_t)old;
}

}  // namespace pam
