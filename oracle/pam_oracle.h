/*
 * pam_oracle.h - CPU restatement of PagedAttentionMetal's ragged paged-attention
 * path.  TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg are the only callers.  The product (libpam) never links it.
 *
 * Every routine cites the reference file:line it restates.  Paths are relative
 * to the reference checkout (abderahmane-ai/PagedAttentionMetal).
 *
 * Conventions shared with the reference (kernels.metal:1829-1832):
 *   pool element (block p, slot s, kv head h, dim i) = ((p*bs + s)*Hkv + h)*d + i
 *   Q / O are [rows][H][d]; kv head of query head h is h / (H / Hkv).
 * dtype codes follow PagedAttentionDataType (PagedAttentionTypes.swift:67-73):
 *   0 = f32 pools and f32 Q/O, 1 = f16 pools and f16 Q/O,
 *   2 = e4m3 byte pools with per-block half scales and f16 Q/O.
 * Half values are passed as raw IEEE binary16 bit patterns (uint16_t).
 */
#ifndef PAM_ORACLE_H
#define PAM_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- binary16 helpers (IEEE 754, round-to-nearest-even) ---- */
uint16_t pamo_f32_to_f16(float x);
float pamo_f16_to_f32(uint16_t h);

/* ---- FP8 codec: kernels.metal:553-601 and the scale rule :1944-1957 ---- */
uint8_t pamo_quantize_fp8(uint16_t value_h, uint16_t scale_h);
uint16_t pamo_dequant_fp8(uint8_t code, uint16_t scale_h);
/* elementwise forms over n values (per-element scales) */
void pamo_quantize_fp8_n(const uint16_t *values, const uint16_t *scales, uint8_t *out, int64_t n);
void pamo_dequant_fp8_n(const uint8_t *codes, const uint16_t *scales, uint16_t *out, int64_t n);
/* new per-block scale from this append's max |x| and the old scale */
uint16_t pamo_fp8_scale(float new_max_abs, uint16_t old_scale_h);

/* ---- slot mapping: kernels.metal:1823-1832 ---- */
int64_t pamo_slot(const int32_t *block_table, int64_t pos, int32_t block_size);

/* ---- KV append (kernels.metal:1804-1874, 1876-1961) ----
 * keys/values: [n_new][Hkv][d] in the pool's element type (f16 for dtype 2).
 * dtype 2 updates k_scale/v_scale (half bits, one per physical block).
 * Returns 0, or -1 if a block-table lookup is out of range (n_bt entries). */
int pamo_append(int dtype, const void *keys, const void *values, void *k_pool, void *v_pool,
                uint16_t *k_scale, uint16_t *v_scale, const int32_t *block_table, int32_t n_bt,
                int32_t token_offset, int32_t n_new, int32_t num_kv_heads, int32_t head_dim,
                int32_t block_size);

/* ---- Reference/paged_attention_sim.py:12-138 (batch 1, one head, fp64) ----
 * q: [S][d] f32, pools: [nb][bs][d] f32, block_table: [nlb].
 * out: [S][d]; m_hist, l_hist: [nlb][S] (may be NULL). Unscaled scores, no mask,
 * key count tied to the query count exactly as in the sim. */
void pamo_sim_forward(const float *q, const float *k_pool, const float *v_pool,
                      const int32_t *block_table, int32_t nlb, int32_t S, int32_t block_size,
                      int32_t head_dim, double *out, double *m_hist, double *l_hist);

/* ---- batched paged decode (kernels.metal:1417-1620 semantics; sim algorithm) ----
 * One query row per sequence; keys [ws, L) with ws = (W > 0 && L > W) ? L - W : 0.
 * Scores scaled by 1/sqrt(d).  Accumulation per logical block in fp64 (sim :70-136).
 * out: [B][H][d] fp64.  n_threads > 1 parallelises over (b, h) with OpenMP.
 * Returns -1 if any block-table lookup would leave [0, max_num_blocks). */
int pamo_decode(int dtype, const void *q, const void *k_pool, const void *v_pool,
                const uint16_t *k_scale, const uint16_t *v_scale, const int32_t *block_tables,
                const uint32_t *seq_lengths, int32_t batch, int32_t max_num_blocks,
                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                int32_t window, double *out, int n_threads);

/* ---- prefill rows of one sequence (kernels.metal:693-917 semantics) ----
 * Query rows are logical positions [q_offset, q_offset + T); kv_len = q_offset + T.
 * Row i sees keys j in [ws, kv_len) with j <= q_offset + i when causal, where
 * ws = (W > 0) ? max(0, kv_len - W) : 0 (one fixed start, PagedAttentionEngine.swift:802).
 * q: [T][H][d]; out: [T][H][d] fp64. */
int pamo_prefill(int dtype, const void *q, const void *k_pool, const void *v_pool,
                 const uint16_t *k_scale, const uint16_t *v_scale, const int32_t *block_table,
                 int32_t n_bt, int32_t q_offset, int32_t T, int32_t num_heads,
                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t window,
                 int32_t causal, double *out, int n_threads);

/* ---- split-context merge of partial softmax states (no reference counterpart) ----
 * parts: P partial states for one row: m[P] (natural-log domain max), l[P], o[P][d]
 * (unnormalised).  out[d] = sum_p e^{m_p-M} o_p / sum_p e^{m_p-M} l_p. */
void pamo_merge(int32_t P, const double *m, const double *l, const double *o, int32_t d,
                double *out);

#ifdef __cplusplus
}
#endif
#endif
