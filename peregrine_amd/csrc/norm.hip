// RMSNorm, add+RMSNorm and the Q4 embedding gather.
//
//   rmsnorm      out = bf16(x * rsqrt(mean(x^2) + eps) * w)
//                reference shaders/rmsnorm.metal:80-116, :222-245
//   add_rmsnorm  r = bf16(a + b); out = rmsnorm(r)  (norm of the ROUNDED sum)
//                reference shaders/rmsnorm.metal:178-220, :280-307
//   embedding    h = bf16(s*q + b) for row `token` of the Q4 table
//                reference shaders/embedding.metal:55-96
//
// One 256-thread block per row; each thread handles 8 consecutive bf16 per
// step (one dwordx4), and the sum of squares uses the same per-thread order and
// block reduction as the fused-norm GEMV prologue (q4_gemv.hpp), so the
// standalone and fused norms produce identical bits.
#include <algorithm>
#include "norm.hpp"

namespace {

using namespace prg;

template <bool ADD>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ residual_out, uint16_t* __restrict__ out, uint32_t hidden, float eps) {
  __shared__ float red[kNormThreads / kWave];
  const size_t row_off = static_cast<size_t>(blockIdx.x) * hidden;
  const uint4* src = reinterpret_cast<const uint4*>(a + row_off);
  const uint32_t n8 = hidden / 8;
  if constexpr (ADD) {
    constexpr int kRegUnits = 4;  // rows up to 8192 wide keep the rounded sum in registers
    if (n8 <= kRegUnits * kNormThreads) {
      // Every load first; the sum is stored and normalised from registers
      // (no read-back of residual_out). The sum of squares visits the units
      // in rms_scale's order, so the bits are those of the read-back form.
      const uint4* srcb = reinterpret_cast<const uint4*>(b + row_off);
      const uint4* ws = reinterpret_cast<const uint4*>(w);
      uint4 xv[kRegUnits], yv[kRegUnits], wv[kRegUnits];
#pragma unroll
      for (int k = 0; k < kRegUnits; ++k) {
        const uint32_t g = threadIdx.x + k * kNormThreads;
        if (g < n8) {
          xv[k] = src[g];
          yv[k] = srcb[g];
          wv[k] = ws[g];
        }
      }
      uint4* r = reinterpret_cast<uint4*>(residual_out + row_off);
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < kRegUnits; ++k) {
        const uint32_t g = threadIdx.x + k * kNormThreads;
        if (g >= n8) continue;
        const uint32_t xd[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w}, yd[4] = {yv[k].x, yv[k].y, yv[k].z, yv[k].w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t lo = f2bf(bf_lo(xd[i]) + bf_lo(yd[i]));
          const uint32_t hi = f2bf(bf_hi(xd[i]) + bf_hi(yd[i]));
          o[i] = lo | (hi << 16);
          const float fa = bf_lo(o[i]), fb = bf_hi(o[i]);
          ss = __fmaf_rn(fa, fa, ss);
          ss = __fmaf_rn(fb, fb, ss);
        }
        xv[k] = make_uint4(o[0], o[1], o[2], o[3]);
        r[g] = xv[k];
      }
      const float total = block_sum256_dpp(ss, red);
      const float scale = 1.0f / sqrtf(__fadd_rn(total / static_cast<float>(hidden), eps));
      uint4* dst = reinterpret_cast<uint4*>(out + row_off);
#pragma unroll
      for (int k = 0; k < kRegUnits; ++k) {
        const uint32_t g = threadIdx.x + k * kNormThreads;
        if (g < n8) dst[g] = rms_apply(xv[k], wv[k], scale);
      }
      return;
    }
    // r = bf16(float(lhs) + float(rhs)), stored, then normalised.
    const uint4* srcb = reinterpret_cast<const uint4*>(b + row_off);
    uint4* r = reinterpret_cast<uint4*>(residual_out + row_off);
    for (uint32_t g = threadIdx.x; g < n8; g += kNormThreads) {
      const uint4 x = src[g], y = srcb[g];
      const uint32_t xd[4] = {x.x, x.y, x.z, x.w}, yd[4] = {y.x, y.y, y.z, y.w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = f2bf(bf_lo(xd[i]) + bf_lo(yd[i]));
        const uint32_t hi = f2bf(bf_hi(xd[i]) + bf_hi(yd[i]));
        o[i] = lo | (hi << 16);
      }
      r[g] = make_uint4(o[0], o[1], o[2], o[3]);
    }
    __syncthreads();
    src = reinterpret_cast<const uint4*>(residual_out + row_off);
  }
  const float scale = rms_scale(src, n8, hidden, eps, red);
  const uint4* ws = reinterpret_cast<const uint4*>(w);
  uint4* dst = reinterpret_cast<uint4*>(out + row_off);
  for (uint32_t g = threadIdx.x; g < n8; g += kNormThreads) dst[g] = rms_apply(src[g], ws[g], scale);
}

// The 8 bf16 of packed word i of row `token` of the Q4 table.
__device__ inline uint4 embed_unit(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                   const uint16_t* __restrict__ b, uint32_t token, uint32_t i, uint32_t hidden) {
  const size_t words = hidden / 8, groups = hidden / 64;
  const uint32_t word = w[static_cast<size_t>(token) * words + i];
  const size_t meta = static_cast<size_t>(token) * groups + i / 8;
  const float sc = bf2f(s[meta]), bi = bf2f(b[meta]);
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // s*q is exact in f32; one rounding in the add, then bf16.
    const float lo = __fadd_rn(sc * static_cast<float>((word >> (8 * j)) & 0xF), bi);
    const float hi = __fadd_rn(sc * static_cast<float>((word >> (8 * j + 4)) & 0xF), bi);
    o[j] = f2bf(lo) | (static_cast<uint32_t>(f2bf(hi)) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__global__ void embedding_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                 const uint16_t* __restrict__ b, uint16_t* __restrict__ out,
                                 const uint32_t* __restrict__ tokens, uint32_t token_stride, uint32_t token_host,
                                 uint32_t hidden) {
  // one thread per packed word (8 outputs); blockIdx.y = row r, token tokens[r * token_stride]
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= hidden / 8) return;
  const uint32_t token = tokens ? tokens[blockIdx.y * token_stride] : token_host;
  reinterpret_cast<uint4*>(out + static_cast<size_t>(blockIdx.y) * hidden)[i] = embed_unit(w, s, b, token, i, hidden);
}

// Two RMSNorms in one launch, block 0: out[0, H) = rmsnorm(embedding(token),
// w0); block 1: out[H, 2H) = rmsnorm(x1, w1). Same per-thread order and block
// reduction as rmsnorm_kernel (rms_scale), so the bits equal the three
// separate launches. The drafter's pre-fc rows (mtp.zig:200-212).
constexpr int kPairUnits = 4;  // hidden <= 8 * 256 * kPairUnits
__global__ __launch_bounds__(kNormThreads) void embed_norm_pair_kernel(
    const uint32_t* __restrict__ ew, const uint16_t* __restrict__ es, const uint16_t* __restrict__ eb,
    const uint32_t* __restrict__ token, const uint16_t* __restrict__ w0, const uint16_t* __restrict__ x1,
    const uint16_t* __restrict__ w1, uint16_t* __restrict__ out, uint32_t hidden, float eps) {
  __shared__ float red[kNormThreads / kWave];
  const uint32_t n8 = hidden / 8;
  const bool emb = blockIdx.x == 0;
  const uint32_t tok = emb ? *token : 0u;
  uint4 v[kPairUnits];
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < kPairUnits; ++u) {
    const uint32_t g = threadIdx.x + u * kNormThreads;
    v[u] = make_uint4(0, 0, 0, 0);
    if (g < n8) {
      v[u] = emb ? embed_unit(ew, es, eb, tok, g, hidden) : reinterpret_cast<const uint4*>(x1)[g];
      const uint32_t d[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = bf_lo(d[i]), b = bf_hi(d[i]);
        ss = __fmaf_rn(a, a, ss);
        ss = __fmaf_rn(b, b, ss);
      }
    }
  }
  const float total = block_sum256_dpp(ss, red);
  const float scale = 1.0f / sqrtf(__fadd_rn(total / static_cast<float>(hidden), eps));
  const uint4* ws = reinterpret_cast<const uint4*>(emb ? w0 : w1);
  uint4* dst = reinterpret_cast<uint4*>(out + (emb ? 0 : hidden));
#pragma unroll
  for (int u = 0; u < kPairUnits; ++u) {
    const uint32_t g = threadIdx.x + u * kNormThreads;
    if (g < n8) dst[g] = rms_apply(v[u], ws[g], scale);
  }
}

}  // namespace

namespace prg {

int launch_rmsnorm(hipStream_t s, const uint16_t* x, const uint16_t* w, uint16_t* out,
                   uint32_t hidden, uint32_t rows, float eps) {
  hipLaunchKernelGGL((rmsnorm_kernel<false>), dim3(rows), dim3(kNormThreads), 0, s, x, nullptr, w,
                     nullptr, out, hidden, eps);
  PRG_CHECK_LAUNCH("rmsnorm");
  return PRG_OK;
}

int launch_embedding(hipStream_t s, const uint32_t* w, const uint16_t* sc, const uint16_t* bi,
                     uint16_t* out, const uint32_t* tokens_dev, uint32_t token_host,
                     uint32_t rows, uint32_t hidden, uint32_t token_stride) {
  const uint32_t words = hidden / 8;
  hipLaunchKernelGGL(embedding_kernel, dim3((words + 255) / 256, rows), dim3(256), 0, s, w, sc, bi, out,
                     tokens_dev, token_stride, token_host, hidden);
  PRG_CHECK_LAUNCH("embedding");
  return PRG_OK;
}

int launch_embed_norm_pair(hipStream_t s, const uint32_t* ew, const uint16_t* es, const uint16_t* eb,
                           const uint32_t* token_dev, const uint16_t* w0, const uint16_t* x1, const uint16_t* w1,
                           uint16_t* out, uint32_t hidden, float eps) {
  if (hidden % 64 != 0 || hidden > 8u * kNormThreads * kPairUnits)
    return set_error(PRG_ERR_INVALID_ARG, "embed_norm_pair: hidden %u unsupported", hidden);
  hipLaunchKernelGGL(embed_norm_pair_kernel, dim3(2), dim3(kNormThreads), 0, s, ew, es, eb, token_dev, w0, x1, w1,
                     out, hidden, eps);
  PRG_CHECK_LAUNCH("embed_norm_pair");
  return PRG_OK;
}

}  // namespace prg

namespace {
__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                          size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    y[i] = prg::f2bf(x[i]);
}
}  // namespace

extern "C" {

int prg_f32_to_bf16(void* stream, const float* x, uint16_t* y, size_t n) {
  PRG_CHECK_ARG(x && y, "prg_f32_to_bf16: null pointer");
  if (n == 0) return PRG_OK;
  const uint32_t blocks = static_cast<uint32_t>(std::min<size_t>((n + 255) / 256, 4096));
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(blocks), dim3(256), 0, prg::as_stream(stream), x, y, n);
  PRG_CHECK_LAUNCH("prg_f32_to_bf16");
  return PRG_OK;
}

int prg_rmsnorm_bf16(void* stream, const uint16_t* x, const uint16_t* weight, uint16_t* out,
                     uint32_t hidden, uint32_t rows, float eps) {
  PRG_CHECK_ARG(x && weight && out, "prg_rmsnorm_bf16: null pointer");
  PRG_CHECK_ARG(hidden > 0 && hidden % 8 == 0, "prg_rmsnorm_bf16: hidden %u must be a multiple of 8", hidden);
  PRG_CHECK_ARG(rows > 0, "prg_rmsnorm_bf16: rows == 0");
  return prg::launch_rmsnorm(prg::as_stream(stream), x, weight, out, hidden, rows, eps);
}

int prg_add_rmsnorm_bf16(void* stream, const uint16_t* lhs, const uint16_t* rhs,
                         const uint16_t* weight, uint16_t* residual_out, uint16_t* norm_out,
                         uint32_t hidden, uint32_t rows, float eps) {
  PRG_CHECK_ARG(lhs && rhs && weight && residual_out && norm_out, "prg_add_rmsnorm_bf16: null pointer");
  PRG_CHECK_ARG(hidden > 0 && hidden % 8 == 0, "prg_add_rmsnorm_bf16: hidden %u must be a multiple of 8", hidden);
  PRG_CHECK_ARG(rows > 0, "prg_add_rmsnorm_bf16: rows == 0");
  hipLaunchKernelGGL((rmsnorm_kernel<true>), dim3(rows), dim3(prg::kNormThreads), 0, prg::as_stream(stream),
                     lhs, rhs, weight, residual_out, norm_out, hidden, eps);
  PRG_CHECK_LAUNCH("prg_add_rmsnorm_bf16");
  return PRG_OK;
}

int prg_q4_embedding_gather_bf16(void* stream, const uint32_t* weight, const uint16_t* scales,
                                 const uint16_t* biases, uint16_t* out, uint32_t token,
                                 uint32_t hidden, uint32_t vocab) {
  PRG_CHECK_ARG(weight && scales && biases && out, "prg_q4_embedding_gather_bf16: null pointer");
  PRG_CHECK_ARG(hidden > 0 && hidden % 64 == 0, "prg_q4_embedding_gather_bf16: hidden %u", hidden);
  if (token >= vocab)
    return prg::set_error(PRG_ERR_INVALID_TOKEN, "prg_q4_embedding_gather_bf16: token %u >= vocab %u", token, vocab);
  return prg::launch_embedding(prg::as_stream(stream), weight, scales, biases, out, nullptr, token, 1, hidden);
}

int prg_q4_embedding_gather_many_bf16(void* stream, const uint32_t* weight, const uint16_t* scales,
                                      const uint16_t* biases, uint16_t* out,
                                      const uint32_t* token_ids, uint32_t tokens, uint32_t hidden) {
  PRG_CHECK_ARG(weight && scales && biases && out && token_ids, "prg_q4_embedding_gather_many_bf16: null pointer");
  PRG_CHECK_ARG(hidden > 0 && hidden % 64 == 0, "prg_q4_embedding_gather_many_bf16: hidden %u", hidden);
  PRG_CHECK_ARG(tokens > 0 && tokens <= 65535, "prg_q4_embedding_gather_many_bf16: tokens %u", tokens);
  return prg::launch_embedding(prg::as_stream(stream), weight, scales, biases, out, token_ids, 0, tokens, hidden);
}

}  // extern "C"
