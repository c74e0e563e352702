// Gated DeltaNet (linear attention) decode kernels — shared declarations.
#pragma once

#include "common.hpp"

namespace prg {

// Qwen3.5 GDN dims (reference src/model/block_linear.zig:19-30).
constexpr uint32_t kGdnHk = 16;
constexpr uint32_t kGdnHv = 32;
constexpr uint32_t kGdnDk = 128;
constexpr uint32_t kGdnDv = 128;
constexpr uint32_t kGdnKeyDim = kGdnHk * kGdnDk;           // 2048
constexpr uint32_t kGdnValDim = kGdnHv * kGdnDv;           // 4096
constexpr uint32_t kGdnConvDim = 2 * kGdnKeyDim + kGdnValDim;  // 8192
constexpr uint32_t kGdnConvK = 4;

// conv1d + SiLU decode for one channel, rolling the f32 state
// (reference shaders/conv1d.metal:40-62). Unfused multiply/add in the
// reference's order. The rolled state goes to state_out (== state for the
// in-place update). Returns the bf16 output.
__device__ inline uint16_t conv1d_silu_step(const float* state, float* state_out, const uint16_t* w,
                                            uint32_t conv_dim, uint32_t c, float xnew) {
  const float s0 = state[c], s1 = state[conv_dim + c], s2 = state[2 * conv_dim + c];
  const uint2 wv = *reinterpret_cast<const uint2*>(w + static_cast<size_t>(c) * kGdnConvK);
  float acc = 0.0f;
  acc = __fadd_rn(acc, __fmul_rn(bf_lo(wv.x), s0));
  acc = __fadd_rn(acc, __fmul_rn(bf_hi(wv.x), s1));
  acc = __fadd_rn(acc, __fmul_rn(bf_lo(wv.y), s2));
  acc = __fadd_rn(acc, __fmul_rn(bf_hi(wv.y), xnew));
  state_out[c] = s1;
  state_out[conv_dim + c] = s2;
  state_out[2 * conv_dim + c] = xnew;
  return f2bf(acc / (1.0f + expf(-acc)));
}

// Two consecutive tokens of one channel (the two-token verify): x0 then x1
// through the same arithmetic as two conv1d_silu_step calls. The state after
// x0 goes to snap, the state after x1 to state_out; state is read once.
__device__ inline void conv1d_silu_step2(const float* state, float* snap, float* state_out, const uint16_t* w,
                                         uint32_t conv_dim, uint32_t c, float x0, float x1, uint16_t& o0,
                                         uint16_t& o1) {
  const float s0 = state[c], s1 = state[conv_dim + c], s2 = state[2 * conv_dim + c];
  const uint2 wv = *reinterpret_cast<const uint2*>(w + static_cast<size_t>(c) * kGdnConvK);
  const float w0 = bf_lo(wv.x), w1 = bf_hi(wv.x), w2 = bf_lo(wv.y), w3 = bf_hi(wv.y);
  float a0 = 0.0f;
  a0 = __fadd_rn(a0, __fmul_rn(w0, s0));
  a0 = __fadd_rn(a0, __fmul_rn(w1, s1));
  a0 = __fadd_rn(a0, __fmul_rn(w2, s2));
  a0 = __fadd_rn(a0, __fmul_rn(w3, x0));
  float a1 = 0.0f;
  a1 = __fadd_rn(a1, __fmul_rn(w0, s1));
  a1 = __fadd_rn(a1, __fmul_rn(w1, s2));
  a1 = __fadd_rn(a1, __fmul_rn(w2, x0));
  a1 = __fadd_rn(a1, __fmul_rn(w3, x1));
  snap[c] = s1;
  snap[conv_dim + c] = s2;
  snap[2 * conv_dim + c] = x0;
  state_out[c] = s2;
  state_out[conv_dim + c] = x0;
  state_out[2 * conv_dim + c] = x1;
  o0 = f2bf(a0 / (1.0f + expf(-a0)));
  o1 = f2bf(a1 / (1.0f + expf(-a1)));
}

// The GDN gate projections a = in_proj_a(x) and b = in_proj_b(x) (bf16, [Hv]
// each) computed by the recurrence kernel itself instead of by the in_proj
// GEMV: from the GEMV's normalised activation image (GemvParams::x_image)
// and the two Q4 matrices [Hv, K], a quarter of a quantisation group per
// thread of a 256-thread block, so K <= kGdnGateProjMaxK. Taking the 64 rows
// out of the in_proj launch leaves it 12288 rows, four per wave of its grid.
struct GdnGateProj {
  const uint32_t* x_image;  // activation rows back to back, K / 2 dwords each
  const uint32_t* wa;
  const uint16_t* sa;
  const uint16_t* ba;
  const uint32_t* wb;
  const uint16_t* sb;
  const uint16_t* bb;
  uint32_t K;
};
constexpr uint32_t kGdnGateProjMaxK = 4096;

// One block per v-head. With norm_w != nullptr the gated RMSNorm is fused and
// y_out receives the normalised output. The state counts as present when
// step_dev->rope_pos != 0 (decoder_layer.zig:564), or per has_state_host when
// step_dev is null. The updated state is written to state_out (nullptr: in
// place). With `gates` (unfused form only; a / b then unused) the gate
// projections are computed in the kernel.
int launch_gdn_decode(hipStream_t s, float* state, const uint16_t* conv_out, const uint16_t* a,
                      const uint16_t* b, const float* A_log, const uint16_t* dt_bias,
                      uint16_t* y_out, const StepScalars* step_dev, uint32_t has_state_host,
                      const uint16_t* norm_w, const uint16_t* z, float eps, float* state_out = nullptr,
                      const GdnGateProj* gates = nullptr);

// Two consecutive tokens (the two-token verify): token 0 reads `state` and
// writes `snap`, token 1 continues and writes `state_out` (may equal state).
// conv_out, a, b and y_out hold the two tokens' rows back to back
// (8192 / 32 / 32 / 4096 values apart); step_dev[0..1] are their steps.
// With `gates` (a / b then unused) the gate projections are computed in the
// kernel from the two rows of gates->x_image.
int launch_gdn_decode2(hipStream_t s, const float* state, float* snap, float* state_out, const uint16_t* conv_out,
                       const uint16_t* a, const uint16_t* b, const float* A_log, const uint16_t* dt_bias,
                       uint16_t* y_out, const StepScalars* step_dev, const GdnGateProj* gates = nullptr);

}  // namespace prg
