/*
 * peregrine_oracle.h — TEST INFRASTRUCTURE, not product code.
 *
 * A scalar C restatement of the reference's Metal shader semantics for the
 * Qwen3.5-9B 4-bit decode path (XiaoConstantine/peregrine, shaders/ and
 * src/model/). It is the parity checker for the HIP kernels in
 * peregrine_amd/csrc and the CPU baseline timed by bench.py. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Every function cites the reference file:line it restates and reproduces
 * each bf16 rounding point written there (RNE f32 -> bf16). Reductions that
 * the reference leaves to hardware (Metal simd_sum over 32 lanes, threadgroup
 * trees) are restated as butterfly / strided trees in the order noted at each
 * function; the hardware's own order is not observable here, so last-ulp
 * agreement with Apple GPUs is "parity unpinned": no test can pin it without
 * the reference's Metal build, which needs macOS.
 *
 * Parallelism: only across independent output rows (pthreads), so results do
 * not depend on the thread count (orc_set_threads).
 *
 * Layouts match the reference: Q4 weight u32 [N, K/8] (nibble j of word c is
 * column 8c+j), scales/biases bf16 [N, K/64]; bf16 values are uint16_t bits.
 */
#ifndef PEREGRINE_ORACLE_H
#define PEREGRINE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void orc_set_threads(int n);
int orc_get_threads(void);

/* bf16 helpers */
float orc_bf2f(uint16_t b);
uint16_t orc_f2bf(float f);

/* A1: w = bf16(s*q + b). shaders/linear.metal:422-444 */
void orc_q4_dequantize_bf16(const uint32_t *w, const uint16_t *s, const uint16_t *b,
                            uint16_t *out, uint32_t N, uint32_t K);

/* A2: raw fp32 dot of M activation rows against every weight row, in the
 * reference's lane structure (shaders/linear_decode.metal:13-74 /
 * shaders/linear.metal:65-126): 32 lanes x 16 values per 512-wide K step,
 * per-lane s*sum(q*x) + b*sum(x) accumulation, then a 32-lane butterfly sum.
 * dots: f32 [M, N]. */
void orc_q4_dots(const uint16_t *x, uint32_t M, const uint32_t *w, const uint16_t *s,
                 const uint16_t *b, float *dots, uint32_t N, uint32_t K);

/* A3: y = bf16(dot).  shaders/linear.metal:128-193 */
void orc_q4_gemv_bf16(const uint16_t *x, const uint32_t *w, const uint16_t *s,
                      const uint16_t *b, uint16_t *y, uint32_t M, uint32_t N, uint32_t K);

/* A4/A6: out = bf16(float(bf16(dot)) + float(res)).
 * shaders/linear_decode.metal:161-192 (M=1), :233-271 (M=2) */
void orc_q4_gemv_residual_add_bf16(const uint16_t *x, const uint32_t *w, const uint16_t *s,
                                   const uint16_t *b, const uint16_t *res, uint16_t *out,
                                   uint32_t M, uint32_t N, uint32_t K);

/* A5/A6: out = bf16(silu(bf16(g)) * bf16(u)), silu(g) = g/(1+exp(-g)).
 * shaders/linear_decode.metal:311-356 (M=1), :484-541 (M=2) */
void orc_q4_gemv_silu_gate_bf16(const uint16_t *x, const uint32_t *gw, const uint16_t *gs,
                                const uint16_t *gb, const uint32_t *uw, const uint16_t *us,
                                const uint16_t *ub, uint16_t *out, uint32_t M, uint32_t N,
                                uint32_t K);

/* A7/A6: per 8 rows the first strict max of bf16-rounded logits.
 * shaders/linear.metal:195-255 (M=1), :342-420 (M=2). pval/pidx: [M, N/8] */
void orc_q4_gemv_argmax_partial_bf16(const uint16_t *x, const uint32_t *w, const uint16_t *s,
                                     const uint16_t *b, float *pval, uint32_t *pidx,
                                     uint32_t M, uint32_t N, uint32_t K);

/* A7: 256-thread strided scan + tree, exactly. shaders/argmax.metal:6-43 */
uint32_t orc_argmax_pairs_f32_u32(const float *values, const uint32_t *indices, uint32_t n);

/* A16: shaders/rmsnorm.metal:80-116 (512 threads, tree reduction) */
void orc_rmsnorm_bf16(const uint16_t *x, const uint16_t *w, uint16_t *out, uint32_t hidden,
                      uint32_t rows, float eps);
/* A17: shaders/rmsnorm.metal:178-220 */
void orc_add_rmsnorm_bf16(const uint16_t *lhs, const uint16_t *rhs, const uint16_t *w,
                          uint16_t *residual_out, uint16_t *norm_out, uint32_t hidden,
                          uint32_t rows, float eps);
/* A18: shaders/embedding.metal:55-71 */
void orc_q4_embedding_gather_bf16(const uint32_t *w, const uint16_t *s, const uint16_t *b,
                                  uint16_t *out, uint32_t token, uint32_t hidden);
/* A8: shaders/conv1d.metal:40-62 */
void orc_conv1d_silu_decode_bf16(float *state, const uint16_t *qkv, const uint16_t *w,
                                 uint16_t *out, uint32_t conv_dim, uint32_t kernel_size);
/* A9: shaders/gated_delta.metal:147-261 */
void orc_gated_delta_decode_bf16(float *state, const uint16_t *conv_out, const uint16_t *a,
                                 const uint16_t *b, const float *A_log, const uint16_t *dt_bias,
                                 uint16_t *y, uint32_t Hk, uint32_t Hv, uint32_t Dk, uint32_t Dv,
                                 uint32_t has_previous_state);
/* A10: shaders/gated_norm.metal:163-189 */
void orc_rmsnorm_gated_bf16(const uint16_t *x, const uint16_t *w, const uint16_t *gate,
                            uint16_t *out, uint32_t dim, float eps, uint32_t rows);
/* A12: shaders/attention.metal:327-421 */
void orc_attn_decode_prepare_bf16(const uint16_t *packed_q, const uint16_t *q_weight,
                                  uint16_t *q_out, uint16_t *gate, const uint16_t *k_in,
                                  const uint16_t *v_in, const uint16_t *k_weight,
                                  uint16_t *key_dst, uint16_t *value_dst, uint32_t num_heads,
                                  uint32_t num_kv_heads, uint32_t head_dim, uint32_t rotary_dim,
                                  uint32_t position_offset, float theta, uint32_t stride,
                                  uint32_t dst);
/* A13+A14: shaders/attention_decode.metal:24-243 */
void orc_attn_decode_bf16(const uint16_t *q, const uint16_t *K, const uint16_t *V,
                          const uint16_t *gate, uint16_t *out, uint32_t num_q_heads,
                          uint32_t num_kv_heads, uint32_t stride, uint32_t seq_len, float scale);

/* ---- prompt (prefill) path ---- */
/* A22: shaders/linear.metal:780-941 (QMM; residual may be NULL) */
void orc_q4_qmm_bf16(const uint16_t *x, uint32_t M, const uint32_t *w, const uint16_t *s,
                     const uint16_t *b, const uint16_t *residual, uint16_t *out, uint32_t N,
                     uint32_t K);
/* shaders/elementwise.metal:64-73, 88-99 */
void orc_silu_mul_pair_bf16(uint16_t *gate, const uint16_t *up, size_t n);
void orc_sigmoid_mul_pair_bf16(uint16_t *x, const uint16_t *gate, size_t n);
/* A18 many: shaders/embedding.metal:73-96 */
void orc_q4_embedding_gather_many_bf16(const uint32_t *w, const uint16_t *s, const uint16_t *b,
                                       const uint32_t *tokens, uint32_t T, uint16_t *out,
                                       uint32_t hidden);
/* A23: shaders/layout.metal:68-89; attention.metal:146-220; block_attn.zig:500-631 */
void orc_split_qg_many_bf16(const uint16_t *qp, uint16_t *q, uint16_t *gate, uint32_t head_dim,
                            uint32_t heads, uint32_t T);
void orc_qk_norm_rope_append_many_bf16(uint16_t *q, const uint16_t *q_weight, const uint16_t *k,
                                       const uint16_t *k_weight, const uint16_t *v,
                                       uint16_t *cache_k, uint16_t *cache_v, uint32_t start_rope,
                                       uint32_t T, uint32_t start_cache, uint32_t stride,
                                       uint32_t num_q, uint32_t num_kv, uint32_t head_dim,
                                       uint32_t rotary_dim, float theta);
void orc_attn_prefill_bf16(const uint16_t *q, const uint16_t *cache_k, const uint16_t *cache_v,
                           uint16_t *out, uint32_t T, uint32_t prefix, uint32_t stride,
                           uint32_t num_q, uint32_t num_kv, uint32_t head_dim, float scale);
/* A24: shaders/conv1d.metal:136-198; gated_norm.metal:191-268; gated_delta.metal:35-138 */
void orc_conv1d_silu_prefill_bf16(float *state, const uint16_t *qkv, const uint16_t *w,
                                  uint16_t *out, uint32_t T, uint32_t conv_dim,
                                  uint32_t kernel_size, uint32_t has_previous_state);
void orc_qk_l2norm_prefill_bf16(const uint16_t *conv_out, float *qn, float *kn, uint32_t T,
                                uint32_t Hk, uint32_t Dk, uint32_t conv_dim);
void orc_gating_many_bf16(const float *A_log, const uint16_t *a, const uint16_t *dt_bias,
                          const uint16_t *b, float *g, float *beta, uint32_t Hv, uint32_t T);
void orc_gated_delta_prefill_bf16(float *state, const float *q, const float *k,
                                  const uint16_t *conv_out, const float *g, const float *beta,
                                  uint16_t *y, uint32_t T, uint32_t Hk, uint32_t Hv, uint32_t Dk,
                                  uint32_t Dv, uint32_t conv_dim, uint32_t has_previous_state);

#ifdef __cplusplus
}
#endif

#endif
