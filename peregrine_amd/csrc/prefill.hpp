// Prompt-path (prefill) kernel launchers shared by the C ABI and the model.
#pragma once

#include "common.hpp"

namespace prg {

// Elements of the bf16 score workspace for T new tokens after `prefix` cached
// ones: [kv head 4][q head in group 4 x T][round_up(prefix + T, 64)].
size_t attn_prefill_scores_elems(uint32_t T, uint32_t prefix);

// qp [T, 16, 512] (q ‖ gate per head), k_in/v_in [T, 4, 256] ->
// q_out/gate_out [T, 16, 256], K/V cache slots [start_cache, start_cache + T).
int launch_attn_prefill_prepare(hipStream_t s, const uint16_t* qp, const uint16_t* q_w, const uint16_t* k_in,
                                const uint16_t* k_w, const uint16_t* v_in, uint16_t* q_out, uint16_t* gate_out,
                                uint16_t* cache_k, uint16_t* cache_v, uint32_t T, uint32_t start_rope,
                                uint32_t start_cache, uint32_t stride);

// Causal attention of T queries [T, 16, 256] over cache slots [0, prefix + T),
// gated: out = bf16(bf16(P V) * sigmoid(gate)).
int launch_attn_prefill(hipStream_t s, const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                        const uint16_t* gate, uint16_t* out, uint16_t* scores, size_t scores_cap, uint32_t T,
                        uint32_t prefix, uint32_t stride, float scale);

// conv1d + SiLU over T tokens [T, 8192], then the f32 state [3, 8192] takes the
// last three inputs.
int launch_conv1d_prefill(hipStream_t s, float* state, const uint16_t* qkv, const uint16_t* w, uint16_t* out,
                          uint32_t T, uint32_t has_state);

// f32 q/k [T, 16, 128] (l2-normed, q also x rsqrt(128)), gates g/beta [T, 32]
// and, when kq != nullptr, k.q per (token, k-head) [T, 16].
int launch_gdn_prefill_prepare(hipStream_t s, const uint16_t* conv_out, const uint16_t* a, const uint16_t* b,
                               const float* A_log, const uint16_t* dt_bias, float* qn, float* kn, float* g,
                               float* beta, float* kq, uint32_t T);

// The delta-rule recurrence over T tokens; y [T, 32 * 128] bf16. kq from the
// prepare step, or nullptr to form it in the recurrence.
int launch_gdn_prefill(hipStream_t s, float* state, const float* qn, const float* kn, const uint16_t* conv_out,
                       const float* g, const float* beta, const float* kq, uint16_t* y, uint32_t T,
                       uint32_t has_state);

// out[r] = a[r] ‖ b[r], rows of `width` bf16 (width % 8 == 0).
int launch_concat_rows(hipStream_t s, const uint16_t* a, const uint16_t* b, uint16_t* out, uint32_t rows,
                       uint32_t width);

}  // namespace prg
