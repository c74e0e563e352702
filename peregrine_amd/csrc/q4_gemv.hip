// Q4 GEMV family: launch dispatch and the C-ABI entry points.
//
// Reference semantics followed (file:line in the reference tree):
//   plain          shaders/linear.metal:65-193        (qmv_fast_bf16)
//   residual add   shaders/linear_decode.metal:161-309 (M=1 and M=2)
//   silu gate      shaders/linear_decode.metal:311-580 (M=1 and M=2)
//   argmax partial shaders/linear.metal:195-420        (M=1 and M=2)
//   argmax pairs   shaders/argmax.metal:6-43
//   dequantize     shaders/linear.metal:422-444
#include <stdlib.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "q4_gemv.hpp"

namespace prg {

int gemv_rows_per_wave(uint32_t total_rows, uint32_t K, int epi, int M) {
  if (epi == kEpiArgmax) return 8;
  const int nmat = (epi == kEpiSiluGate) ? 2 : 1;
  const int iters = static_cast<int>((K + kGemvKStep - 1) / kGemvKStep);
  // One register buffer holds ROWS x NMAT x ITERS dwordx4 loads; keep it at
  // <= 4 (two buffers in flight) and keep >= 4096 groups so every wave of a
  // full grid has work.
  static const int forced = [] {
    const char* e = getenv("PEREGRINE_GEMV_ROWS");  // tuning override: 1, 2 or 4
    const int v = e ? atoi(e) : 0;
    return (v == 1 || v == 2 || v == 4) ? v : 0;
  }();
  if (forced) return forced;
  // Measured on MI355X (2048-wide K steps): one row per wave with a grid of
  // 3 blocks/CU is fastest for every decode shape; 2 rows only when K is a
  // single step (more work per wave to amortise the per-group epilogue).
  int rows = iters == 1 ? 2 : 1;
  (void)M;
  (void)nmat;
  (void)total_rows;
  return rows;
}

int launch_q4_gemv(hipStream_t stream, GemvParams& p, int M, int rows, int epi, int norm,
                   const char* name) {
  if (p.K == 0 || p.K % 512 != 0)
    return set_error(PRG_ERR_INVALID_ARG, "%s: in_dim %u must be a positive multiple of 512", name, p.K);
  // K-steps of 2048; unrolled kernels exist for 1,2,3,4,6,8 steps (the model
  // uses 4096 -> 2, 8192 -> 4, 12288 -> 6).
  const int iters = static_cast<int>((p.K + kGemvKStep - 1) / kGemvKStep);
  if (iters > kGemvMaxIters || iters == 5 || iters == 7)
    return set_error(PRG_ERR_INVALID_ARG, "%s: in_dim %u (%d K-steps) unsupported", name, p.K, iters);
  const uint32_t rem = p.K % kGemvKStep;
  p.tail_lanes = rem == 0 ? 64u : rem / 32u;
  if (M < 1 || M > 2) return set_error(PRG_ERR_INVALID_ARG, "%s: M=%d", name, M);
  if (p.nseg < 1 || p.nseg > kGemvMaxSegs) return set_error(PRG_ERR_INVALID_ARG, "%s: nseg", name);
  if (p.argmax_waves != nullptr && (epi != kEpiArgmax || p.nseg != 1))
    return set_error(PRG_ERR_INVALID_ARG, "%s: per-wave argmax needs the argmax epilogue and one segment", name);
  uint32_t groups = 0;
  for (uint32_t i = 0; i < p.nseg; ++i) {
    GemvSeg& sg = p.seg[i];
    if (sg.rows == 0 || sg.rows % 8 != 0)
      return set_error(PRG_ERR_INVALID_ARG, "%s: out_dim %u must be a positive multiple of 8", name, sg.rows);
    sg.block_begin = groups;
    groups += (sg.rows + static_cast<uint32_t>(rows) - 1) / static_cast<uint32_t>(rows);
  }
  p.total_groups = groups;
  const size_t lds = static_cast<size_t>(M) * p.K * sizeof(uint16_t);
  int rc;
  if (norm == kNormGated && (p.K % kGdnDv != 0 || p.norm_w == nullptr || p.gz[0] == nullptr ||
                             (M == 2 && p.gz[1] == nullptr)))
    return set_error(PRG_ERR_INVALID_ARG, "%s: gated norm needs K %% 128 == 0, norm_w and gz", name);
  if (epi == kEpiPlain)
    rc = norm == kNormRms    ? launch_m<kEpiPlain, kNormRms>(stream, p, M, rows, iters, lds)
         : norm == kNormNone ? launch_m<kEpiPlain, kNormNone>(stream, p, M, rows, iters, lds)
                             : -1;
  else if (epi == kEpiResidual)
    rc = norm == kNormGated  ? launch_m<kEpiResidual, kNormGated>(stream, p, M, rows, iters, lds)
         : norm == kNormNone ? launch_m<kEpiResidual, kNormNone>(stream, p, M, rows, iters, lds)
                             : -1;
  else if (epi == kEpiSiluGate)
    rc = norm == kNormRms    ? launch_m<kEpiSiluGate, kNormRms>(stream, p, M, rows, iters, lds)
         : norm == kNormNone ? launch_m<kEpiSiluGate, kNormNone>(stream, p, M, rows, iters, lds)
                             : -1;
  else
    rc = norm == kNormRms    ? launch_m<kEpiArgmax, kNormRms>(stream, p, M, rows, iters, lds)
         : norm == kNormNone ? launch_m<kEpiArgmax, kNormNone>(stream, p, M, rows, iters, lds)
                             : -1;
  if (rc != 0) return set_error(PRG_ERR_INVALID_ARG, "%s: no kernel for M=%d rows=%d iters=%d", name, M, rows, iters);
  PRG_CHECK_LAUNCH(name);
  return PRG_OK;
}

}  // namespace prg

// ================================================================ kernels ====
namespace prg {
int launch_advance_forced(hipStream_t s, DecodeCtl* ctl, const uint32_t* prompt);
}  // namespace prg

namespace {

// Final argmax over partials with the reference's effective tie order.
// argmax_pairs_f32_u32 (shaders/argmax.metal:6-43) runs 256 threads; thread t
// scans p = t, t+256, ... keeping the first strict maximum, then a tree over
// (tid, tid+stride), stride 128..1, keeps the lower position on ties. The last
// tree level therefore prefers even threads, the level before it threads
// = 0 mod 4, and so on: among equal maxima the winner minimises
// (bitreverse8(p mod 256), p div 256). NaN never compares greater, and if
// nothing beats -inf the answer is index 0. This kernel evaluates that order
// directly with 1024 threads and a total order on (value, key)
// (prg::argmax_better).
constexpr int kArgmaxThreads = 1024;
using prg::argmax_better;

// Advance the token loop by one step (see DecodeCtl). `pred` is ignored when
// the step has no argmax (prompt ingestion).
__device__ inline void advance_ctl(prg::DecodeCtl* ctl, const uint32_t* prompt, uint32_t* predictions,
                                   bool has_pred, uint32_t pred) {
  const uint32_t n = ctl->n;
  if (has_pred && predictions) predictions[n] = pred;
  const uint32_t n1 = n + 1;
  if (n1 >= ctl->capacity) {  // never step past the cache
    ctl->overflow = 1;
    return;
  }
  const uint32_t next = (n1 < ctl->prompt_len || !has_pred) ? prompt[n1] : pred;
  ctl->s.token = next;
  ctl->s.cache_pos = n1;
  ctl->s.rope_pos = n1 + ctl->rope_off;
  ctl->s.seq_len = n1 + 1;
  ctl->n = n1;
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_pairs_kernel(
    const float* __restrict__ values, const uint32_t* __restrict__ indices, uint32_t* __restrict__ out,
    uint32_t n) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ uint32_t sp[kArgmaxThreads / 64];
  float bv = -INFINITY;
  uint32_t bp = 0xffffffffu;
  // 32 independent loads per thread (clamped in bounds, masked after the
  // load, no branches): the lm_head's 31040 partials take one memory round
  // trip instead of one per batch.
  constexpr int kU = 32;
  for (uint32_t base = threadIdx.x; base < n; base += kArgmaxThreads * kU) {
    float v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint32_t p = base + u * kArgmaxThreads;
      v[u] = values[min(p, n - 1)];
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (base + u * kArgmaxThreads >= n) v[u] = -INFINITY;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint32_t p = base + u * kArgmaxThreads;
      if (argmax_better(v[u], p, bv, bp)) {
        bv = v[u];
        bp = p;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const uint32_t op = __shfl_xor(bp, o, 64);
    if (argmax_better(ov, op, bv, bp)) {
      bv = ov;
      bp = op;
    }
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wid] = bv;
    sp[wid] = bp;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kArgmaxThreads / 64; ++i)
      if (argmax_better(sv[i], sp[i], bv, bp)) {
        bv = sv[i];
        bp = sp[i];
      }
    out[0] = (bp == 0xffffffffu) ? 0u : indices[bp];
  }
}

// Final argmax over the per-wave entries of a GEMV launched with
// GemvParams::argmax_waves: entry e holds a wave's best (value, row) under the
// same order (its partial position is row / 8), so the winner equals the one
// argmax_pairs_kernel picks from the full partial list. The entries and the
// count are loaded together (every index < kArgmaxMaxWaves is in bounds) and
// entries at or past the count are masked afterwards: one memory round trip.
// Block b reduces activation row b's entries (values[b], rows[b] -> out[b]).
struct ArgmaxWavesArgs {
  const float* values[2];
  const uint32_t* rows[2];
  uint32_t* out[2];
};
template <bool ADVANCE>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_waves_kernel(
    ArgmaxWavesArgs a, const uint32_t* __restrict__ count, prg::DecodeCtl* ctl, const uint32_t* prompt,
    uint32_t* predictions) {
  const float* __restrict__ values = a.values[blockIdx.x];
  const uint32_t* __restrict__ rows = a.rows[blockIdx.x];
  uint32_t* out = a.out[blockIdx.x];
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ uint32_t sr[kArgmaxThreads / 64];
  constexpr int kU = prg::kArgmaxMaxWaves / kArgmaxThreads;
  static_assert(kU * kArgmaxThreads == prg::kArgmaxMaxWaves, "entries per thread");
  const uint32_t n = *count;
  float v[kU];
  uint32_t r[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    v[u] = values[threadIdx.x + u * kArgmaxThreads];
    r[u] = rows[threadIdx.x + u * kArgmaxThreads];
  }
  float bv = -INFINITY;
  uint32_t br = 0xffffffffu;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const bool live = threadIdx.x + u * kArgmaxThreads < n;
    const float vu = live ? v[u] : -INFINITY;
    if (argmax_better(vu, r[u] >> 3, bv, br >> 3)) {
      bv = vu;
      br = r[u];
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const uint32_t orow = __shfl_xor(br, o, 64);
    if (argmax_better(ov, orow >> 3, bv, br >> 3)) {
      bv = ov;
      br = orow;
    }
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wid] = bv;
    sr[wid] = br;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kArgmaxThreads / 64; ++i)
      if (argmax_better(sv[i], sr[i] >> 3, bv, br >> 3)) {
        bv = sv[i];
        br = sr[i];
      }
    const uint32_t winner = (br == 0xffffffffu) ? 0u : br;
    if (out) out[0] = winner;
    if constexpr (ADVANCE) advance_ctl(ctl, prompt, predictions, true, winner);
  }
}

__global__ void advance_forced_kernel(prg::DecodeCtl* ctl, const uint32_t* prompt) {
  if (threadIdx.x == 0) advance_ctl(ctl, prompt, nullptr, false, 0);
}

__global__ void q4_dequantize_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                     const uint16_t* __restrict__ b, uint16_t* __restrict__ out,
                                     uint32_t out_dim, uint32_t in_dim) {
  // One thread per packed word (8 outputs).
  const size_t words = static_cast<size_t>(out_dim) * (in_dim / 8);
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const size_t row = i / (in_dim / 8);
  const uint32_t col8 = static_cast<uint32_t>(i - row * (in_dim / 8));
  const size_t meta = row * (in_dim / 64) + col8 / 8;
  const float sc = prg::bf2f(s[meta]);
  const float bi = prg::bf2f(b[meta]);
  const uint32_t word = w[i];
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = sc * static_cast<float>((word >> (8 * j)) & 0xF);
    const float hi = sc * static_cast<float>((word >> (8 * j + 4)) & 0xF);
    // s*q + b as two roundings, as written in the reference (no FMA).
    o[j] = prg::f2bf(__fadd_rn(lo, bi)) | (static_cast<uint32_t>(prg::f2bf(__fadd_rn(hi, bi))) << 16);
  }
  reinterpret_cast<uint4*>(out)[i] = make_uint4(o[0], o[1], o[2], o[3]);
}

int check_q4(const char* name, const void* x, const void* w, const void* s, const void* b,
             uint32_t out_dim, uint32_t in_dim) {
  PRG_CHECK_ARG(x && w && s && b, "%s: null pointer", name);
  PRG_CHECK_ARG(in_dim > 0 && in_dim % 512 == 0, "%s: in_dim %u must be a positive multiple of 512", name, in_dim);
  PRG_CHECK_ARG(out_dim > 0 && out_dim % 8 == 0, "%s: out_dim %u must be a positive multiple of 8", name, out_dim);
  return PRG_OK;
}

prg::GemvParams one_seg(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint32_t rows,
                        uint32_t K) {
  prg::GemvParams p{};
  p.nseg = 1;
  p.K = K;
  p.seg[0].w[0] = w;
  p.seg[0].s[0] = s;
  p.seg[0].b[0] = b;
  p.seg[0].rows = rows;
  return p;
}

}  // namespace

using prg::launch_q4_gemv;

namespace prg {
int launch_argmax_waves_advance(hipStream_t s, const float* values, const uint32_t* rows, const uint32_t* count,
                                DecodeCtl* ctl, const uint32_t* prompt, uint32_t* predictions) {
  ArgmaxWavesArgs a{{values, values}, {rows, rows}, {nullptr, nullptr}};
  hipLaunchKernelGGL(argmax_waves_kernel<true>, dim3(1), dim3(kArgmaxThreads), 0, s, a, count, ctl, prompt,
                     predictions);
  PRG_CHECK_LAUNCH("argmax_waves_advance");
  return PRG_OK;
}
int launch_argmax_waves(hipStream_t s, int M, const float* const* values, const uint32_t* const* rows,
                        const uint32_t* count, uint32_t* const* out) {
  if (M < 1 || M > 2) return set_error(PRG_ERR_INVALID_ARG, "argmax_waves: M=%d", M);
  ArgmaxWavesArgs a{};
  for (int m = 0; m < M; ++m) {
    a.values[m] = values[m];
    a.rows[m] = rows[m];
    a.out[m] = out[m];
  }
  hipLaunchKernelGGL(argmax_waves_kernel<false>, dim3(M), dim3(kArgmaxThreads), 0, s, a, count, nullptr, nullptr,
                     nullptr);
  PRG_CHECK_LAUNCH("argmax_waves");
  return PRG_OK;
}
int launch_advance_forced(hipStream_t s, DecodeCtl* ctl, const uint32_t* prompt) {
  hipLaunchKernelGGL(advance_forced_kernel, dim3(1), dim3(64), 0, s, ctl, prompt);
  PRG_CHECK_LAUNCH("advance_forced");
  return PRG_OK;
}
}  // namespace prg

extern "C" {

int prg_q4_gemv_bf16(void* stream, const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                     const uint16_t* biases, uint16_t* y, uint32_t token_count, uint32_t out_dim,
                     uint32_t in_dim) {
  const char* name = "prg_q4_gemv_bf16";
  if (int rc = check_q4(name, x, w, scales, biases, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(y != nullptr, "%s: null output", name);
  if (token_count == 0) return prg::set_error(PRG_ERR_EMPTY_INPUT, "%s: token_count == 0", name);
  hipStream_t s = prg::as_stream(stream);
  // Rows of x are processed two at a time so each weight pass serves both.
  for (uint32_t t = 0; t < token_count; t += 2) {
    const int M = (token_count - t >= 2) ? 2 : 1;
    prg::GemvParams p = one_seg(w, scales, biases, out_dim, in_dim);
    for (int m = 0; m < M; ++m) {
      p.x[m] = x + static_cast<size_t>(t + m) * in_dim;
      p.seg[0].out[m] = y + static_cast<size_t>(t + m) * out_dim;
    }
    const int rows = prg::gemv_rows_per_wave(out_dim, in_dim, prg::kEpiPlain, M);
    if (int rc = launch_q4_gemv(s, p, M, rows, prg::kEpiPlain, prg::kNormNone, name)) return rc;
  }
  return PRG_OK;
}

int prg_q4_gemv_residual_add_bf16(void* stream, const uint16_t* x, const uint32_t* w,
                                  const uint16_t* scales, const uint16_t* biases,
                                  const uint16_t* residual, uint16_t* out, uint32_t token_count,
                                  uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv_residual_add_bf16";
  if (int rc = check_q4(name, x, w, scales, biases, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(residual && out, "%s: null residual/output", name);
  if (token_count == 0) return prg::set_error(PRG_ERR_EMPTY_INPUT, "%s: token_count == 0", name);
  hipStream_t s = prg::as_stream(stream);
  for (uint32_t t = 0; t < token_count; t += 2) {
    const int M = (token_count - t >= 2) ? 2 : 1;
    prg::GemvParams p = one_seg(w, scales, biases, out_dim, in_dim);
    for (int m = 0; m < M; ++m) {
      p.x[m] = x + static_cast<size_t>(t + m) * in_dim;
      p.seg[0].out[m] = out + static_cast<size_t>(t + m) * out_dim;
      p.seg[0].res[m] = residual + static_cast<size_t>(t + m) * out_dim;
    }
    const int rows = prg::gemv_rows_per_wave(out_dim, in_dim, prg::kEpiResidual, M);
    if (int rc = launch_q4_gemv(s, p, M, rows, prg::kEpiResidual, prg::kNormNone, name)) return rc;
  }
  return PRG_OK;
}

int prg_q4_gemv2_residual_add_bf16(void* stream, const uint16_t* x0, const uint16_t* x1,
                                   const uint32_t* w, const uint16_t* scales,
                                   const uint16_t* biases, const uint16_t* residual0,
                                   const uint16_t* residual1, uint16_t* out0, uint16_t* out1,
                                   uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv2_residual_add_bf16";
  if (int rc = check_q4(name, x0, w, scales, biases, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(x1 && residual0 && residual1 && out0 && out1, "%s: null pointer", name);
  prg::GemvParams p = one_seg(w, scales, biases, out_dim, in_dim);
  p.x[0] = x0;
  p.x[1] = x1;
  p.seg[0].out[0] = out0;
  p.seg[0].out[1] = out1;
  p.seg[0].res[0] = residual0;
  p.seg[0].res[1] = residual1;
  const int rows = prg::gemv_rows_per_wave(out_dim, in_dim, prg::kEpiResidual, 2);
  return launch_q4_gemv(prg::as_stream(stream), p, 2, rows, prg::kEpiResidual, prg::kNormNone, name);
}

int prg_q4_gemv_silu_gate_bf16(void* stream, const uint16_t* x, const uint32_t* gate_w,
                               const uint16_t* gate_s, const uint16_t* gate_b,
                               const uint32_t* up_w, const uint16_t* up_s, const uint16_t* up_b,
                               uint16_t* out, uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv_silu_gate_bf16";
  if (int rc = check_q4(name, x, gate_w, gate_s, gate_b, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(up_w && up_s && up_b && out, "%s: null pointer", name);
  prg::GemvParams p = one_seg(gate_w, gate_s, gate_b, out_dim, in_dim);
  p.seg[0].w[1] = up_w;
  p.seg[0].s[1] = up_s;
  p.seg[0].b[1] = up_b;
  p.x[0] = x;
  p.seg[0].out[0] = out;
  const int rows = prg::gemv_rows_per_wave(out_dim, in_dim, prg::kEpiSiluGate, 1);
  return launch_q4_gemv(prg::as_stream(stream), p, 1, rows, prg::kEpiSiluGate, prg::kNormNone, name);
}

int prg_q4_gemv_silu_gate2_bf16(void* stream, const uint16_t* x0, const uint16_t* x1,
                                const uint32_t* gate_w, const uint16_t* gate_s,
                                const uint16_t* gate_b, const uint32_t* up_w,
                                const uint16_t* up_s, const uint16_t* up_b, uint16_t* out0,
                                uint16_t* out1, uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv_silu_gate2_bf16";
  if (int rc = check_q4(name, x0, gate_w, gate_s, gate_b, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(x1 && up_w && up_s && up_b && out0 && out1, "%s: null pointer", name);
  prg::GemvParams p = one_seg(gate_w, gate_s, gate_b, out_dim, in_dim);
  p.seg[0].w[1] = up_w;
  p.seg[0].s[1] = up_s;
  p.seg[0].b[1] = up_b;
  p.x[0] = x0;
  p.x[1] = x1;
  p.seg[0].out[0] = out0;
  p.seg[0].out[1] = out1;
  const int rows = prg::gemv_rows_per_wave(out_dim, in_dim, prg::kEpiSiluGate, 2);
  return launch_q4_gemv(prg::as_stream(stream), p, 2, rows, prg::kEpiSiluGate, prg::kNormNone, name);
}

int prg_q4_gemv_norm_bf16(void* stream, const uint16_t* x, const uint16_t* norm_weight, float eps,
                          const uint32_t* w, const uint16_t* scales, const uint16_t* biases, uint16_t* y,
                          uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv_norm_bf16";
  if (int rc = check_q4(name, x, w, scales, biases, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(norm_weight && y, "%s: null pointer", name);
  prg::GemvParams p = one_seg(w, scales, biases, out_dim, in_dim);
  p.x[0] = x;
  p.norm_w = norm_weight;
  p.eps = eps;
  p.seg[0].out[0] = y;
  const int rows = prg::gemv_rows_per_wave(out_dim, in_dim, prg::kEpiPlain, 1);
  return launch_q4_gemv(prg::as_stream(stream), p, 1, rows, prg::kEpiPlain, prg::kNormRms, name);
}

int prg_q4_gemv_silu_gate_norm_bf16(void* stream, const uint16_t* x, const uint16_t* norm_weight, float eps,
                                    const uint32_t* gate_w, const uint16_t* gate_s, const uint16_t* gate_b,
                                    const uint32_t* up_w, const uint16_t* up_s, const uint16_t* up_b,
                                    uint16_t* out, uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv_silu_gate_norm_bf16";
  if (int rc = check_q4(name, x, gate_w, gate_s, gate_b, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(norm_weight && up_w && up_s && up_b && out, "%s: null pointer", name);
  prg::GemvParams p = one_seg(gate_w, gate_s, gate_b, out_dim, in_dim);
  p.seg[0].w[1] = up_w;
  p.seg[0].s[1] = up_s;
  p.seg[0].b[1] = up_b;
  p.x[0] = x;
  p.norm_w = norm_weight;
  p.eps = eps;
  p.seg[0].out[0] = out;
  const int rows = prg::gemv_rows_per_wave(out_dim, in_dim, prg::kEpiSiluGate, 1);
  return launch_q4_gemv(prg::as_stream(stream), p, 1, rows, prg::kEpiSiluGate, prg::kNormRms, name);
}

int prg_q4_gemv_argmax_partial_bf16(void* stream, const uint16_t* x, const uint32_t* w,
                                    const uint16_t* scales, const uint16_t* biases,
                                    float* partial_values, uint32_t* partial_indices,
                                    uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv_argmax_partial_bf16";
  if (int rc = check_q4(name, x, w, scales, biases, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(partial_values && partial_indices, "%s: null partial buffers", name);
  prg::GemvParams p = one_seg(w, scales, biases, out_dim, in_dim);
  p.x[0] = x;
  p.seg[0].pval[0] = partial_values;
  p.seg[0].pidx[0] = partial_indices;
  return launch_q4_gemv(prg::as_stream(stream), p, 1, 8, prg::kEpiArgmax, prg::kNormNone, name);
}

int prg_q4_gemv_argmax2_partial_bf16(void* stream, const uint16_t* x0, const uint16_t* x1,
                                     const uint32_t* w, const uint16_t* scales,
                                     const uint16_t* biases, float* partial_values0,
                                     uint32_t* partial_indices0, float* partial_values1,
                                     uint32_t* partial_indices1, uint32_t out_dim,
                                     uint32_t in_dim) {
  const char* name = "prg_q4_gemv_argmax2_partial_bf16";
  if (int rc = check_q4(name, x0, w, scales, biases, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(x1 && partial_values0 && partial_indices0 && partial_values1 && partial_indices1,
                "%s: null pointer", name);
  prg::GemvParams p = one_seg(w, scales, biases, out_dim, in_dim);
  p.x[0] = x0;
  p.x[1] = x1;
  p.seg[0].pval[0] = partial_values0;
  p.seg[0].pidx[0] = partial_indices0;
  p.seg[0].pval[1] = partial_values1;
  p.seg[0].pidx[1] = partial_indices1;
  return launch_q4_gemv(prg::as_stream(stream), p, 2, 8, prg::kEpiArgmax, prg::kNormNone, name);
}

int prg_argmax_pairs_f32_u32(void* stream, const float* values, const uint32_t* indices,
                             uint32_t* out_index, uint32_t pair_count) {
  const char* name = "prg_argmax_pairs_f32_u32";
  PRG_CHECK_ARG(values && indices && out_index, "%s: null pointer", name);
  PRG_CHECK_ARG(pair_count > 0, "%s: pair_count == 0", name);
  hipLaunchKernelGGL(argmax_pairs_kernel, dim3(1), dim3(kArgmaxThreads), 0, prg::as_stream(stream), values,
                     indices, out_index, pair_count);
  PRG_CHECK_LAUNCH(name);
  return PRG_OK;
}

int prg_q4_dequantize_bf16(void* stream, const uint32_t* w, const uint16_t* scales,
                           const uint16_t* biases, uint16_t* out, uint32_t out_dim,
                           uint32_t in_dim) {
  const char* name = "prg_q4_dequantize_bf16";
  PRG_CHECK_ARG(w && scales && biases && out, "%s: null pointer", name);
  PRG_CHECK_ARG(out_dim > 0 && in_dim > 0 && in_dim % 64 == 0, "%s: bad shape %ux%u", name, out_dim, in_dim);
  const size_t words = static_cast<size_t>(out_dim) * (in_dim / 8);
  const uint32_t blocks = static_cast<uint32_t>((words + 255) / 256);
  hipLaunchKernelGGL(q4_dequantize_kernel, dim3(blocks), dim3(256), 0, prg::as_stream(stream), w,
                     scales, biases, out, out_dim, in_dim);
  PRG_CHECK_LAUNCH(name);
  return PRG_OK;
}

}  // extern "C"
