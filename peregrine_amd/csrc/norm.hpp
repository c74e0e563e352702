// RMSNorm building blocks shared by the standalone norm kernels and the
// fused-norm GEMV prologue, so both produce identical bits.
#pragma once

#include "common.hpp"

namespace prg {

constexpr int kNormThreads = 256;

// 1 / sqrt(mean(x^2) + eps) over a bf16 row read as n8 uint4 (8 values each).
// Each thread sums its uint4s (stride kNormThreads) pair by pair, then the
// block reduces in a fixed order. Every thread receives the scale.
__device__ inline float rms_scale(const uint4* src, uint32_t n8, uint32_t hidden, float eps,
                                  float* red) {
  float ss = 0.0f;
  for (uint32_t g = threadIdx.x; g < n8; g += kNormThreads) {
    const uint4 v = src[g];
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf_lo(d[i]), b = bf_hi(d[i]);
      ss = __fmaf_rn(a, a, ss);
      ss = __fmaf_rn(b, b, ss);
    }
  }
  static_assert(kNormThreads == 256, "block_sum256_dpp reduces a 256-thread block");
  const float total = block_sum256_dpp(ss, red);
  return 1.0f / sqrtf(__fadd_rn(total / static_cast<float>(hidden), eps));
}

// bf16(x * scale * w) for 8 values (reference order: (x * scale) * w).
__device__ inline uint4 rms_apply(uint4 v, uint4 w, float scale) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
  const uint32_t e[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f2bf2(bf_lo(d[i]) * scale * bf_lo(e[i]), bf_hi(d[i]) * scale * bf_hi(e[i]));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// bf16(((y * scale) * w) * sz) for 8 values, sz = silu(z) in f32: the gated
// RMSNorm of one GDN head row (reference shaders/gated_norm.metal:163-189).
__device__ inline uint4 gated_rms_apply(uint4 v, uint4 w, float4 z0, float4 z1, float scale) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
  const uint32_t e[4] = {w.x, w.y, w.z, w.w};
  const float g[8] = {z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = f2bf2(bf_lo(d[i]) * scale * bf_lo(e[i]) * g[2 * i], bf_hi(d[i]) * scale * bf_hi(e[i]) * g[2 * i + 1]);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

int launch_rmsnorm(hipStream_t s, const uint16_t* x, const uint16_t* w, uint16_t* out,
                   uint32_t hidden, uint32_t rows, float eps);
// Row r embeds tokens_dev[r * token_stride] (or token_host without tokens_dev).
int launch_embedding(hipStream_t s, const uint32_t* w, const uint16_t* sc, const uint16_t* bi,
                     uint16_t* out, const uint32_t* tokens_dev, uint32_t token_host, uint32_t rows,
                     uint32_t hidden, uint32_t token_stride = 1);
// out[0, H) = rmsnorm(embedding(*token_dev), w0), out[H, 2H) = rmsnorm(x1, w1) in
// one launch, bit-identical to the separate launches.
int launch_embed_norm_pair(hipStream_t s, const uint32_t* ew, const uint16_t* es, const uint16_t* eb,
                           const uint32_t* token_dev, const uint16_t* w0, const uint16_t* x1, const uint16_t* w1,
                           uint16_t* out, uint32_t hidden, float eps);

}  // namespace prg
