/*
 * peregrine_hip.h — C ABI of libperegrine_hip.so, the MI355X (gfx950) decode
 * path for the Qwen3.5-9B-shaped 4-bit token loop.
 *
 * This header replaces the reference's Objective-C/Metal bridge
 * (reference: src/runtime/bridge.h:1-103, declared for Zig in
 * src/runtime/ffi.zig:1-74). The reference addresses kernels by string name
 * through prg_pipeline_create + prg_cmdbuf_encode; here every fused op is one
 * typed entry point.
 *
 * Conventions (all entry points):
 *   - bf16 values are passed as uint16_t bit patterns; Q4 weights as uint32_t
 *     words (8 nibbles, lowest nibble = lowest column); f32 as float.
 *   - Pointers passed to op entry points are DEVICE pointers owned by the
 *     caller. `stream` is a hipStream_t (NULL = the default stream).
 *   - Ops are asynchronous on `stream`; none synchronises the host.
 *   - Return value: 0 on success, a PRG_ERR_* code otherwise (never a silent
 *     drop — the reference's encoders silently ignore bad arguments,
 *     bridge.m:235-243; these do not). prg_last_error() describes the failure.
 *   - Thread safety: calls on one stream are serialised by the caller.
 */
#ifndef PEREGRINE_HIP_H
#define PEREGRINE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PRG_OK = 0,
  PRG_ERR_INVALID_ARG = 1,   /* shape / pointer contract violated          */
  PRG_ERR_HIP = 2,           /* HIP runtime error                          */
  PRG_ERR_NO_DEVICE = 3,     /* no GPU visible                             */
  PRG_ERR_OOM = 4,           /* allocation failed                          */
  PRG_ERR_SEQUENCE_TOO_LONG = 5, /* cache_pos >= cache capacity (model.zig:805) */
  PRG_ERR_INVALID_TOKEN = 6, /* token id >= vocab (model.zig:806)           */
  PRG_ERR_EMPTY_INPUT = 7,   /* zero token_count (linear_q4.zig:85)         */
  PRG_ERR_NOT_FOUND = 8,     /* FileNotFound / TensorNotFound               */
  PRG_ERR_MALFORMED = 9,     /* TruncatedHeader / MalformedHeader / MalformedIndex /
                                NoShardsFound / MissingField / InvalidTensorShape
                                (safetensors.zig, std.json)                  */
  PRG_ERR_UNSUPPORTED = 10,  /* UnsupportedArchitecture / UnsupportedQuantization /
                                InvalidConfig / NotQwen35_9B (config.zig:44-72) */
  PRG_ERR_IO = 11            /* read / write failure                         */
};

/* Last error message of the calling thread ("" if none). */
const char *prg_last_error(void);
/* Library version string. */
const char *prg_version(void);

/* ======================================================================
 * Runtime. Replaces bridge.h's device/queue/buffer/command-buffer calls:
 *   prg_device_create        (bridge.h:23)  -> prg_hip_device_init
 *   prg_queue_create         (bridge.h:26)  -> prg_hip_stream_create
 *   prg_buffer_create_private(bridge.h:32)  -> prg_hip_alloc_device
 *   prg_buffer_create_shared (bridge.h:30)  -> prg_hip_alloc_host
 *   prg_blit_copy_buffer     (bridge.h:35)  -> prg_hip_memcpy
 *   prg_cmdbuf_commit_wait   (bridge.h:95)  -> prg_hip_stream_synchronize
 *   prg_cmdbuf_wait_destroy_profile (bridge.h:93) -> prg_hip_event_elapsed_ms
 * ====================================================================== */
int prg_hip_device_count(int *count);
int prg_hip_device_init(int ordinal);
int prg_hip_device_name(char *buf, size_t len);
int prg_hip_alloc_device(void **ptr, size_t bytes);
int prg_hip_free_device(void *ptr);
int prg_hip_alloc_host(void **ptr, size_t bytes); /* pinned, device-visible */
int prg_hip_free_host(void *ptr);
/* kind: 0 = host->device, 1 = device->host, 2 = device->device. Synchronous
 * when stream == NULL and `sync` != 0, otherwise async on `stream`. */
int prg_hip_memcpy(void *dst, const void *src, size_t bytes, int kind, void *stream, int sync);
int prg_hip_memset_device(void *dst, int value, size_t bytes, void *stream);
int prg_hip_stream_create(void **stream);
int prg_hip_stream_destroy(void *stream);
int prg_hip_stream_synchronize(void *stream);
int prg_hip_device_synchronize(void);
int prg_hip_event_create(void **event);
int prg_hip_event_destroy(void *event);
int prg_hip_event_record(void *event, void *stream);
int prg_hip_event_elapsed_ms(void *start, void *stop, float *ms);
/* Recorded command sequences. The reference encodes kernels into a command
 * buffer and commits it once (prg_cmdbuf_create / _encode / _commit /
 * _commit_wait / _destroy, bridge.h:60-97); here the ops issued on `stream`
 * between begin and end are captured into a HIP graph that can be replayed
 * any number of times with one launch each.
 *   prg_hip_graph_begin   : start capturing `stream` (not the NULL stream)
 *   prg_hip_graph_end     : stop capturing; *graph receives an executable graph
 *   prg_hip_graph_launch  : replay it on `stream` (asynchronous)
 *   prg_hip_graph_destroy : free it */
int prg_hip_graph_begin(void *stream);
int prg_hip_graph_end(void *stream, void **graph);
int prg_hip_graph_launch(void *graph, void *stream);
int prg_hip_graph_destroy(void *graph);
/* Plain device-to-device copy kernel (bytes % 16 == 0); the reference dispatch
 * for calibrating HBM byte counters. */
int prg_hip_copy_kernel(void *dst, const void *src, size_t bytes, void *stream);
/* Streaming read of `bytes` (% 16 == 0) with non-temporal 16-byte loads, four
 * in flight per thread over a 4096-block grid; writes at most one word of
 * sink. The single-launch HBM read floor the GEMVs are compared with. No
 * counterpart in the reference (measurement only). */
int prg_hip_read_kernel(const void *src, size_t bytes, uint32_t *sink, void *stream);

/* ======================================================================
 * Q4 linear ops — MLX affine 4-bit, group 64, bf16 scale + bias.
 *   w      : uint32 [out_dim, in_dim/8], nibble j of word c = column 8c+j
 *   scales : bf16   [out_dim, in_dim/64]
 *   biases : bf16   [out_dim, in_dim/64]
 *   dequantised weight = scale * q + bias
 * Contract (as the reference's Q4Linear.encodeBf16Fast, linear_q4.zig:85-86):
 *   in_dim % 512 == 0, out_dim % 8 == 0, token_count > 0.
 * ====================================================================== */

/* y[t, n] = bf16(sum_k x[t, k] * (s*q + b)), t < token_count.
 * Replaces linear_q4_affine_group64_qmv_fast_bf16 (shaders/linear.metal:158-193),
 * host Q4Linear.encodeBf16Fast (src/model/linear_q4.zig:77-95). */
int prg_q4_gemv_bf16(void *stream, const uint16_t *x, const uint32_t *w,
                     const uint16_t *scales, const uint16_t *biases, uint16_t *y,
                     uint32_t token_count, uint32_t out_dim, uint32_t in_dim);

/* out[t, n] = bf16(float(bf16(dot)) + float(residual[t, n])).
 * Replaces linear_q4_affine_group64_qmv_fast_residual_add_bf16
 * (shaders/linear_decode.metal:194-231), host encodeBf16FastResidualAdd
 * (linear_q4.zig:149-168). */
int prg_q4_gemv_residual_add_bf16(void *stream, const uint16_t *x, const uint32_t *w,
                                  const uint16_t *scales, const uint16_t *biases,
                                  const uint16_t *residual, uint16_t *out,
                                  uint32_t token_count, uint32_t out_dim, uint32_t in_dim);

/* Two activation rows, one weight pass. Replaces
 * linear_q4_affine_group64_qmv2_fast_residual_add_bf16
 * (shaders/linear_decode.metal:273-309), host linear_q4.zig:170-194. */
int prg_q4_gemv2_residual_add_bf16(void *stream, const uint16_t *x0, const uint16_t *x1,
                                   const uint32_t *w, const uint16_t *scales,
                                   const uint16_t *biases, const uint16_t *residual0,
                                   const uint16_t *residual1, uint16_t *out0,
                                   uint16_t *out1, uint32_t out_dim, uint32_t in_dim);

/* out[n] = bf16(silu(bf16(gate_dot)) * bf16(up_dot)), silu(g) = g/(1+exp(-g)).
 * Replaces linear_vec_q4_affine_group64_multi2_silu_gate_bf16
 * (shaders/linear_decode.metal:311-356,449-482), host
 * MlpBlock.encodeGateUpSiluBf16 (src/model/block_mlp.zig:313-345). */
int prg_q4_gemv_silu_gate_bf16(void *stream, const uint16_t *x,
                               const uint32_t *gate_w, const uint16_t *gate_s,
                               const uint16_t *gate_b, const uint32_t *up_w,
                               const uint16_t *up_s, const uint16_t *up_b,
                               uint16_t *out, uint32_t out_dim, uint32_t in_dim);

/* Two-row variant. Replaces linear_vec_q4_affine_group64_multi2_silu_gate2_bf16
 * (shaders/linear_decode.metal:484-580), host block_mlp.zig:347-383. */
int prg_q4_gemv_silu_gate2_bf16(void *stream, const uint16_t *x0, const uint16_t *x1,
                                const uint32_t *gate_w, const uint16_t *gate_s,
                                const uint16_t *gate_b, const uint32_t *up_w,
                                const uint16_t *up_s, const uint16_t *up_b,
                                uint16_t *out0, uint16_t *out1, uint32_t out_dim,
                                uint32_t in_dim);

/* RMSNorm fused into the GEMV prologue: y = bf16(W . bf16(x * rsqrt(mean(x^2)
 * + eps) * norm_w)) for one activation row; several blocks' norms become one
 * dispatch with their projection (decoder_layer.zig:419-437 + linear_q4.zig:77-95). */
int prg_q4_gemv_norm_bf16(void *stream, const uint16_t *x, const uint16_t *norm_weight, float eps,
                          const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                          uint16_t *y, uint32_t out_dim, uint32_t in_dim);

/* post_attention_layernorm fused with the gate/up SiLU GEMV
 * (decoder_layer.zig:756-781 + block_mlp.zig:313-345). */
int prg_q4_gemv_silu_gate_norm_bf16(void *stream, const uint16_t *x, const uint16_t *norm_weight,
                                    float eps, const uint32_t *gate_w, const uint16_t *gate_s,
                                    const uint16_t *gate_b, const uint32_t *up_w,
                                    const uint16_t *up_s, const uint16_t *up_b, uint16_t *out,
                                    uint32_t out_dim, uint32_t in_dim);

/* lm_head partial argmax: logits are bf16-rounded dots; partial p covers rows
 * [8p, 8p+8) and holds the first strict maximum in row order.
 * partial_values f32 [out_dim/8], partial_indices u32 [out_dim/8].
 * Replaces linear_vec_q4_affine_group64_qmv_fast_argmax_partial_bf16
 * (shaders/linear.metal:195-255), host Q4Linear.encodeBf16ArgmaxPartial
 * (linear_q4.zig:97-118). */
int prg_q4_gemv_argmax_partial_bf16(void *stream, const uint16_t *x, const uint32_t *w,
                                    const uint16_t *scales, const uint16_t *biases,
                                    float *partial_values, uint32_t *partial_indices,
                                    uint32_t out_dim, uint32_t in_dim);

/* Two-row variant. Replaces ..._qmv_fast_argmax2_partial_bf16
 * (shaders/linear.metal:342-420), host linear_q4.zig:120-146. */
int prg_q4_gemv_argmax2_partial_bf16(void *stream, const uint16_t *x0, const uint16_t *x1,
                                     const uint32_t *w, const uint16_t *scales,
                                     const uint16_t *biases, float *partial_values0,
                                     uint32_t *partial_indices0, float *partial_values1,
                                     uint32_t *partial_indices1, uint32_t out_dim,
                                     uint32_t in_dim);

/* Final (value, index) reduction with the reference's tie order: among equal
 * maxima the winner minimises (bitreverse8(p mod 256), p div 256) — the order
 * the reference's 256-thread scan + halving tree produces; NaN partials never
 * win; all -inf -> index 0. Replaces argmax_pairs_f32_u32 (shaders/argmax.metal:6-43),
 * host argmax.encodePairsF32U32 (src/model/argmax.zig:14-35). */
int prg_argmax_pairs_f32_u32(void *stream, const float *values, const uint32_t *indices,
                             uint32_t *out_index, uint32_t pair_count);

/* out[n, k] = bf16(s*q + b). Replaces q4_affine_group64_dequantize_bf16
 * (shaders/linear.metal:422-444). */
int prg_q4_dequantize_bf16(void *stream, const uint32_t *w, const uint16_t *scales,
                           const uint16_t *biases, uint16_t *out, uint32_t out_dim,
                           uint32_t in_dim);

/* Decode layout: the same bytes as (w, scales, biases), permuted so that the
 * matrix-core GEMV reads 1 KiB of contiguous memory per wave load. Rows in
 * tiles of 16, K in windows of 256; tw holds, for tile t, window v, step s
 * (0, 1) and lane l = j + 16 c, the 16 bytes of row 16 t + j at words
 * 32 v + 16 s + 4 c .. +3 (unit 128 (t * in_dim / 256 + v) + 64 s + l); ts / tb
 * entry 64 (t * in_dim / 256 + v) + l is group 4 v + c of row 16 t + j.
 * Sizes equal the MLX arrays'. out_dim % 16 == 0, in_dim % 1024 == 0.
 * No counterpart in the reference: its Metal kernels read the MLX layout. */
int prg_q4_repack_t16(void *stream, const uint32_t *w, const uint16_t *scales,
                      const uint16_t *biases, uint32_t *tw, uint16_t *ts, uint16_t *tb,
                      uint32_t out_dim, uint32_t in_dim);

/* prg_q4_gemv_bf16 on the decode layout, on the matrix cores (the kernel the
 * model runs for its large decode GEMVs); in_dim 4096, 8192 or 12288.
 * Replaces linear_q4_affine_group64_qmv_fast_bf16 (shaders/linear.metal:158-193). */
int prg_q4_gemv_t16_bf16(void *stream, const uint16_t *x, const uint32_t *tw,
                         const uint16_t *ts, const uint16_t *tb, uint16_t *y,
                         uint32_t token_count, uint32_t out_dim, uint32_t in_dim);

/* prg_q4_gemv_silu_gate_norm_bf16 on the decode layout (in_dim 4096): the
 * model's post_attention_layernorm + gate/up SiLU launch
 * (decoder_layer.zig:756-781 + block_mlp.zig:313-345). */
int prg_q4_gemv_t16_silu_gate_norm_bf16(void *stream, const uint16_t *x, const uint16_t *norm_weight,
                                        float eps, const uint32_t *gate_tw, const uint16_t *gate_ts,
                                        const uint16_t *gate_tb, const uint32_t *up_tw,
                                        const uint16_t *up_ts, const uint16_t *up_tb, uint16_t *out,
                                        uint32_t out_dim, uint32_t in_dim);

/* Greedy argmax of the bf16 logits of token_count (1 or 2) rows on the decode
 * layout (in_dim 4096): out_index[t] under the order of prg_argmax_pairs_f32_u32
 * over 8-row partials. workspace: prg_q4_gemv_t16_argmax_workspace_bytes().
 * Replaces linear_vec_q4_affine_group64_qmv_fast_argmax_partial_bf16
 * (shaders/linear.metal:195-255) + argmax_pairs_f32_u32 (shaders/argmax.metal:6-43). */
int prg_q4_gemv_t16_argmax_bf16(void *stream, const uint16_t *x, const uint32_t *tw,
                                const uint16_t *ts, const uint16_t *tb, uint32_t *out_index,
                                uint32_t token_count, uint32_t out_dim, uint32_t in_dim,
                                void *workspace);
size_t prg_q4_gemv_t16_argmax_workspace_bytes(void);

/* ======================================================================
 * Norms and embedding
 * ====================================================================== */

/* y[i] = bf16(x[i]): round to nearest even, NaN -> quiet NaN with the input's
 * sign and top payload bits. The rounding every kernel applies where the
 * reference's shaders write bfloat(f) (e.g. shaders/attention.metal:210). */
int prg_f32_to_bf16(void *stream, const float *x, uint16_t *y, size_t n);

/* out = bf16(x * rsqrt(mean(x^2) + eps) * w) per row of `hidden` values.
 * Replaces rmsnorm_bf16 (shaders/rmsnorm.metal:80-116,222-245), host
 * DecoderLayer.encodeRmsNormBf16 (src/model/decoder_layer.zig:419-437). */
int prg_rmsnorm_bf16(void *stream, const uint16_t *x, const uint16_t *weight, uint16_t *out,
                     uint32_t hidden, uint32_t rows, float eps);

/* residual_out = bf16(lhs + rhs); norm_out = rmsnorm(residual_out) (the norm of
 * the ROUNDED sum). Replaces add_rmsnorm_bf16 (shaders/rmsnorm.metal:178-220,
 * 280-307), host encodeAddRmsNormBf16 (decoder_layer.zig:439-459). */
int prg_add_rmsnorm_bf16(void *stream, const uint16_t *lhs, const uint16_t *rhs,
                         const uint16_t *weight, uint16_t *residual_out, uint16_t *norm_out,
                         uint32_t hidden, uint32_t rows, float eps);

/* out[h] = bf16(s*q + b) for row `token` of the Q4 embedding table
 * [vocab, hidden/8]. token >= vocab -> PRG_ERR_INVALID_TOKEN (model.zig:806).
 * Replaces q4_embedding_gather_bf16 (shaders/embedding.metal:55-71). */
int prg_q4_embedding_gather_bf16(void *stream, const uint32_t *weight, const uint16_t *scales,
                                 const uint16_t *biases, uint16_t *out, uint32_t token,
                                 uint32_t hidden, uint32_t vocab);

/* Batched gather of `tokens` rows (token_ids: device u32 [tokens]).
 * Replaces q4_embedding_gather_many_bf16 (shaders/embedding.metal:73-96). */
int prg_q4_embedding_gather_many_bf16(void *stream, const uint32_t *weight, const uint16_t *scales,
                                      const uint16_t *biases, uint16_t *out,
                                      const uint32_t *token_ids, uint32_t tokens, uint32_t hidden);

/* ======================================================================
 * Gated DeltaNet (linear attention) decode. Shape fixed by the model:
 * Hk=16, Hv=32, Dk=Dv=128, conv_dim=8192, conv kernel 4
 * (src/model/block_linear.zig:19-30).
 * ====================================================================== */

/* Depthwise causal conv + SiLU for one token, rolling the f32 state
 * [3, conv_dim] in place. Replaces conv1d_silu_decode_bf16
 * (shaders/conv1d.metal:40-62), host block_linear.zig:236-240. */
int prg_conv1d_silu_decode_bf16(void *stream, float *state, const uint16_t *qkv,
                                const uint16_t *weight, uint16_t *out, uint32_t conv_dim,
                                uint32_t kernel_size);

/* Delta-rule recurrence with inline q/k L2 norms and gates; state f32
 * [Hv, Dv, Dk] updated in place; y bf16 [Hv*Dv]. has_previous_state == 0
 * treats the state as zero. Replaces gated_delta_decode_h128_fused_bf16
 * (shaders/gated_delta.metal:147-261), host block_linear.zig:242-258. */
int prg_gated_delta_decode_bf16(void *stream, float *state, const uint16_t *conv_out,
                                const uint16_t *a, const uint16_t *b, const float *A_log,
                                const uint16_t *dt_bias, uint16_t *y, uint32_t Hk, uint32_t Hv,
                                uint32_t Dk, uint32_t Dv, uint32_t conv_dim,
                                uint32_t has_previous_state);

/* The recurrence fused with the gated RMSNorm of each head:
 * out = bf16(y * rsqrt(mean(y^2)+eps) * norm_weight * silu(z)). One dispatch for
 * the reference's gated_delta_decode + rmsnorm_gated pair
 * (block_linear.zig:242-262). */
int prg_gated_delta_decode_norm_bf16(void *stream, float *state, const uint16_t *conv_out,
                                     const uint16_t *a, const uint16_t *b, const float *A_log,
                                     const uint16_t *dt_bias, const uint16_t *norm_weight,
                                     const uint16_t *z, uint16_t *out, float eps,
                                     uint32_t has_previous_state);

/* Gated RMSNorm per row of `dim` (<= 128) values. Replaces rmsnorm_gated_bf16
 * (shaders/gated_norm.metal:163-189), host block_linear.zig:471-489.
 * dim == 128 with x, weight, gate and out 16-byte aligned: 16 lanes per row,
 * the same bits as the out_proj GEMV's gated-norm prologue; any other dim or
 * alignment: one 128-thread block per row (a different summation order). */
int prg_rmsnorm_gated_bf16(void *stream, const uint16_t *x, const uint16_t *weight,
                           const uint16_t *gate, uint16_t *out, uint32_t dim, float eps,
                           uint32_t rows);

/* ======================================================================
 * GQA decode attention. Shape fixed by the model: 16 q heads, 4 kv heads,
 * head_dim 256, partial RoPE on 64 dims, theta 1e7 (block_attn.zig:21-28).
 * Caches: K bf16 [4, stride, 256], V bf16 [4, 256, stride] (value-dim-major,
 * src/model/state.zig:41-48); stride % 64 == 0.
 * ====================================================================== */

/* Split packed q [16, 512] into q and gate, RMSNorm q/k with q_weight/k_weight,
 * RoPE at position_offset, append k and v to the caches at dst_token_index.
 * Replaces qwen35_q_gate_prepare_kv_append_pair_head_major_value_dim_major_bf16
 * (shaders/attention.metal:327-421), host block_attn.zig:321-326. */
int prg_attn_decode_prepare_bf16(void *stream, const uint16_t *packed_q, const uint16_t *q_weight,
                                 uint16_t *q_output, uint16_t *gate, const uint16_t *k_input,
                                 const uint16_t *v_input, const uint16_t *k_weight,
                                 uint16_t *key_cache, uint16_t *value_cache,
                                 uint32_t cache_stride_tokens, uint32_t dst_token_index,
                                 uint32_t position_offset);

/* out = bf16(softmax(scale * q.K^T) V * sigmoid(gate)) over the first seq_len
 * cache slots, as split-context partials + merge. partials: device f32 of
 * prg_attn_decode_partials_bytes(stride) bytes. Replaces the pair
 * sdpa_decode_prefix_flash_partials_bf16 + ..._reduce_gated_bf16
 * (shaders/attention_decode.metal:24-243), host block_attn.zig:328-358. */
int prg_attn_decode_bf16(void *stream, const uint16_t *q, const uint16_t *key_cache,
                         const uint16_t *value_cache, const uint16_t *gate, uint16_t *out,
                         float *partials, uint32_t cache_stride_tokens, uint32_t seq_len,
                         float scale);
size_t prg_attn_decode_partials_bytes(uint32_t cache_stride_tokens);

/* One decode step of a full-attention layer from the raw projections of the
 * new token: packed_q [16, 512] (q | gate per head), k_input / v_input
 * [4, 256]. Attends over the cached slots [0, cache_pos) plus the new token
 * (its q and k RMSNormed with q_weight / k_weight, partial RoPE at rope_pos),
 * writes out = bf16(softmax(scale q.K^T) V * sigmoid(gate)) [16, 256] and
 * appends the new K / V at cache_pos. workspace: device memory of
 * prg_attn_decode_step_workspace_bytes(stride). Two launches: split partials
 * over the cache with q prepared in every block, the split holding the last
 * cached slot also taking the new token and appending its K / V; then the
 * gated merge. Replaces prepare + partials + merge of
 * FullAttentionBlock.decodeStepBf16 (block_attn.zig:321-358;
 * attention.metal:327-421, attention_decode.metal:24-243). */
int prg_attn_decode_step_bf16(void *stream, const uint16_t *packed_q, const uint16_t *q_weight,
                              const uint16_t *k_input, const uint16_t *v_input, const uint16_t *k_weight,
                              uint16_t *key_cache, uint16_t *value_cache, uint16_t *out, void *workspace,
                              uint32_t cache_stride_tokens, uint32_t cache_pos, uint32_t rope_pos, float scale);
size_t prg_attn_decode_step_workspace_bytes(uint32_t cache_stride_tokens);

/* prg_attn_decode_bf16 without the partials argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. It allocates nothing:
 * the partials live in a library-owned device array (one per GPU, 4,227,072
 * bytes, held until the process ends) whose address is looked up once per
 * device by prg_hip_device_init or the first call on a device. Holds caches of
 * up to 256 splits, i.e. cache_stride_tokens <= 262144 at the default 1024
 * tokens per split; larger caches are rejected with PRG_ERR_INVALID_ARG.
 * Calls that overlap on one GPU (different streams, or threads) share the
 * array and race: serialise them. Output is bit-identical to
 * prg_attn_decode_bf16 on the same inputs. */
int prg_attn_decode_noalloc_bf16(void *stream, const uint16_t *q, const uint16_t *key_cache,
                                 const uint16_t *value_cache, const uint16_t *gate, uint16_t *out,
                                 uint32_t cache_stride_tokens, uint32_t seq_len, float scale);

/* ======================================================================
 * Prompt (prefill) path: T tokens at once through MFMA GEMMs.
 * Row-major [T, dim] activations; the same shape rules as above.
 * ====================================================================== */

/* out[t, n] = bf16(sum_k x[t, k] * bf16(s*q + b)) on the matrix cores: weights
 * dequantised in-kernel and rounded to bf16 before the product, f32
 * accumulation. in_dim % 64 == 0. Replaces
 * linear_q4_affine_group64_prefill_qmm_m32n64_nt_bf16_tiles_bf16
 * (shaders/linear.metal:780-964), host Q4Linear.encodePrefillQmmM32N64NtBf16
 * (src/model/linear_q4.zig:197-214), and the prepared-dense route
 * (q4_dequantize + MLX NT GEMM, src/model/mlx_nt.zig:139-162). */
int prg_q4_qmm_bf16(void *stream, const uint16_t *x, const uint32_t *w, const uint16_t *scales,
                    const uint16_t *biases, uint16_t *out, uint32_t token_count, uint32_t out_dim,
                    uint32_t in_dim);

/* out = bf16(float(bf16(acc)) + residual). Replaces
 * ..._prefill_qmm_m32n64_nt_bf16_tiles_residual_add_bf16
 * (shaders/linear.metal:966-988), host linear_q4.zig:216-233. */
int prg_q4_qmm_residual_add_bf16(void *stream, const uint16_t *x, const uint32_t *w,
                                 const uint16_t *scales, const uint16_t *biases,
                                 const uint16_t *residual, uint16_t *out, uint32_t token_count,
                                 uint32_t out_dim, uint32_t in_dim);

/* out = bf16(silu(bf16(x.gate)) * bf16(x.up)) in one pass: the gate and up
 * QMMs plus silu_mul_pair_inplace_bf16 (shaders/elementwise.metal:64-73),
 * host MlpBlock.encodePrefillGateUpSilu* (src/model/block_mlp.zig:155-214). */
int prg_q4_qmm_silu_gate_bf16(void *stream, const uint16_t *x, const uint32_t *gate_w,
                              const uint16_t *gate_scales, const uint16_t *gate_biases,
                              const uint32_t *up_w, const uint16_t *up_scales,
                              const uint16_t *up_biases, uint16_t *out, uint32_t token_count,
                              uint32_t out_dim, uint32_t in_dim);

/* For T tokens: split packed q [T, 16, 512] into q_output/gate_output
 * [T, 16, 256]; RMSNorm + RoPE (positions start_rope_pos + t) of q and of
 * k_input [T, 4, 256] (normed value kept in f32 through RoPE); append K/V at
 * cache slots start_cache_pos + t. Replaces split_qg_many_bf16
 * (shaders/layout.metal:68-89) + qwen35_qk_norm_rope_append_many_bf16
 * (shaders/attention.metal:146-220), host block_attn.zig:409-442. */
int prg_attn_prefill_prepare_bf16(void *stream, const uint16_t *packed_q, const uint16_t *q_weight,
                                  const uint16_t *k_input, const uint16_t *k_weight,
                                  const uint16_t *v_input, uint16_t *q_output, uint16_t *gate_output,
                                  uint16_t *key_cache, uint16_t *value_cache, uint32_t token_count,
                                  uint32_t start_rope_pos, uint32_t start_cache_pos,
                                  uint32_t cache_stride_tokens);

/* Causal attention of token_count queries over cache slots
 * [0, prefix_len + token_count): scores = bf16(q.k), softmax of scale*score
 * with the mask col <= prefix_len + t, probabilities bf16, then
 * out = bf16(bf16(P.V) * sigmoid(gate)). q, gate, out [T, 16, 256]. scores: a
 * device workspace of prg_attn_prefill_scores_bytes(token_count, prefix_len).
 * Replaces encodeMaterializedPrefillBf16 (src/model/block_attn.zig:500-631:
 * score GEMM, prefill_softmax_scaled_masked_bf16 attention.metal:1463-1523,
 * value GEMM) and sigmoid_mul_pair_inplace_bf16 (elementwise.metal:88-99). */
int prg_attn_prefill_bf16(void *stream, const uint16_t *q, const uint16_t *key_cache,
                          const uint16_t *value_cache, const uint16_t *gate, uint16_t *out,
                          uint16_t *scores, uint32_t token_count, uint32_t prefix_len,
                          uint32_t cache_stride_tokens, float scale);
size_t prg_attn_prefill_scores_bytes(uint32_t token_count, uint32_t prefix_len);

/* Depthwise causal conv + SiLU over qkv [T, 8192], history from the f32 state
 * [3, 8192] when has_previous_state (else zeros); the state then holds the
 * last three inputs. Replaces conv1d_silu_prefill_vec4_bf16 +
 * conv1d_silu_prefill_state_bf16 (shaders/conv1d.metal:136-198), host
 * block_linear.zig:363-390. */
int prg_conv1d_silu_prefill_bf16(void *stream, float *state, const uint16_t *qkv, const uint16_t *weight,
                                 uint16_t *out, uint32_t token_count, uint32_t conv_dim,
                                 uint32_t kernel_size, uint32_t has_previous_state);

/* f32 q/k [T, 16, 128] (l2-normed; q also times rsqrt(128)) from conv_out
 * [T, 8192], and gates g/beta f32 [T, 32] from a, b [T, 32]. kq_out (may be
 * NULL) receives k.q per (token, k-head), f32 [T, 16]. Replaces
 * qk_l2norm_prefill_bf16 + gating_many_bf16 (shaders/gated_norm.metal:191-268),
 * host block_linear.zig:392-434. */
int prg_gated_delta_prefill_prepare_bf16(void *stream, const uint16_t *conv_out, const uint16_t *a,
                                         const uint16_t *b, const float *A_log, const uint16_t *dt_bias,
                                         float *q_out, float *k_out, float *g_out, float *beta_out,
                                         float *kq_out, uint32_t token_count);

/* Delta-rule recurrence over T tokens with prepared q/k/gates; state f32
 * [32, 128, 128] in place; y bf16 [T, 4096]. Replaces
 * gated_delta_prefill_h128_norm_prepared_value_major_r8_bf16
 * (shaders/gated_delta.metal:35-138), host block_linear.zig:436-469. */
int prg_gated_delta_prefill_bf16(void *stream, float *state, const float *q, const float *k,
                                 const uint16_t *conv_out, const float *g, const float *beta, uint16_t *y,
                                 uint32_t token_count, uint32_t has_previous_state);

#ifdef __cplusplus
}
#endif

#endif /* PEREGRINE_HIP_H */
