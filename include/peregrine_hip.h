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
  PRG_ERR_EMPTY_INPUT = 7    /* zero token_count (linear_q4.zig:85)         */
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

#ifdef __cplusplus
}
#endif

#endif /* PEREGRINE_HIP_H */
