// Prompt-path (prefill) kernels other than the GEMMs: attention prepare and
// softmax, the materialised causal attention driver, conv1d prefill with its
// state publish, and the Gated DeltaNet prefill (q/k norms + gates, then the
// token-sequential recurrence).
//
// Reference semantics (file:line in the reference tree):
//   split_qg_many_bf16                       shaders/layout.metal:68-89
//   qwen35_qk_norm_rope_append_many_bf16     shaders/attention.metal:146-220
//   encodeMaterializedPrefillBf16            src/model/block_attn.zig:500-631
//   prefill_softmax_scaled_masked_bf16       shaders/attention.metal:1463-1523
//   sigmoid_mul_pair_inplace_bf16            shaders/elementwise.metal:88-99
//   conv1d_silu_prefill_vec4_bf16 / _state   shaders/conv1d.metal:136-198
//   qk_l2norm_prefill_bf16, gating_many_bf16 shaders/gated_norm.metal:191-268
//   gated_delta_prefill_h128_norm_prepared_value_major_r8_bf16
//                                            shaders/gated_delta.metal:35-138
//   composition                              src/model/block_linear.zig:265-469,
//                                            src/model/block_attn.zig:361-500
#include "attention.hpp"
#include "gdn.hpp"
#include "gemm.hpp"
#include "prefill.hpp"

namespace {

using namespace prg;

constexpr int kPrepThreads = 256;     // QWEN35_QK_PREPARE_THREADS (attention.metal:9)
constexpr int kSoftmaxThreads = 256;  // PREFILL_SOFTMAX_THREADS (attention.metal:42)
constexpr float kLog2e = 1.4426950408889634f;

// Halving tree over blockDim.x == N threads in the reference's order
// (partial[t] = op(partial[t], partial[t + stride]), stride N/2 .. 1). Every
// thread gets the root. `sh` holds N floats. N == 256 combines the first two
// levels from LDS in wave 0 and the rest inside that wave (v_permlane32_swap,
// v_permlane16_swap, then DPP row shifts): the same pairs, so the same bits,
// with two barriers instead of nine.
template <bool MAX>
__device__ inline float tree_op(float a, float b) {
  return MAX ? fmaxf(a, b) : __fadd_rn(a, b);
}
template <bool MAX>
__device__ inline float wave_tree_tail(float s) {  // strides 32 .. 1 within one wave; lane 0 holds the root
  {
    float x = s, y = s;
    swap32(x, y);
    s = tree_op<MAX>(x, y);
  }
  {
    float x = s, y = s;
    swap16(x, y);
    s = tree_op<MAX>(x, y);
  }
  s = tree_op<MAX>(s, dpp_f<0x108>(s));  // row_shl:8 -- lane i with lane i + 8
  s = tree_op<MAX>(s, dpp_f<0x104>(s));
  s = tree_op<MAX>(s, dpp_f<0x102>(s));
  s = tree_op<MAX>(s, dpp_f<0x101>(s));
  return s;
}
template <int N, bool MAX>
__device__ inline float tree_reduce(float v, float* sh) {
  sh[threadIdx.x] = v;
  __syncthreads();
  if constexpr (N == 256) {
    if (threadIdx.x < kWave) {
      const int l = threadIdx.x;
      const float s = tree_op<MAX>(tree_op<MAX>(sh[l], sh[l + 128]), tree_op<MAX>(sh[l + 64], sh[l + 192]));
      const float r = wave_tree_tail<MAX>(s);
      if (l == 0) sh[N] = r;
    }
    __syncthreads();
    return sh[N];
  } else {
#pragma unroll
    for (int stride = N / 2; stride > 0; stride >>= 1) {
      if (static_cast<int>(threadIdx.x) < stride)
        sh[threadIdx.x] = tree_op<MAX>(sh[threadIdx.x], sh[threadIdx.x + stride]);
      __syncthreads();
    }
    const float r = sh[0];
    __syncthreads();
    return r;
  }
}
// `sh` holds N + 1 floats.
template <int N>
__device__ inline float tree_sum(float v, float* sh) {
  return tree_reduce<N, false>(v, sh);
}
template <int N>
__device__ inline float tree_max(float v, float* sh) {
  return tree_reduce<N, true>(v, sh);
}

// ------------------------------------------------------- attention ----------
// Rows [0, 16T) are query heads (t = row/16, h = row%16), rows [16T, 20T)
// key heads (t = r/4, h = r%4). Queries: split from the packed q ‖ gate
// projection, RMS-normed, partial NeoX RoPE on dims [0, 64), written to q_out;
// gate copied to gate_out. Keys: same norm/RoPE into cache_k[h, stride, 256]
// at start_cache + t; values copied to cache_v[h, 256, stride]. The normed
// value stays f32 through RoPE.
// One wave per row, four rows per block: lane l holds elements l, l + 64,
// l + 128 and l + 192. The sum of squares combines them in the 256-thread
// halving tree's pairs ((l, l + 128) and (l + 64, l + 192), then l with
// l + 64) and finishes inside the wave, so the bits are the tree's; RoPE pairs
// element d < 32 with d + 32, i.e. lane l with lane l ^ 32.
constexpr int kPrepRows = kPrepThreads / kWave;
__global__ __launch_bounds__(kPrepThreads) void attn_prefill_prepare_kernel(
    const uint16_t* __restrict__ qp, const uint16_t* __restrict__ q_w, const uint16_t* __restrict__ k_in,
    const uint16_t* __restrict__ k_w, const uint16_t* __restrict__ v_in, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ gate_out, uint16_t* __restrict__ cache_k, uint16_t* __restrict__ cache_v, uint32_t T,
    uint32_t start_rope, uint32_t start_cache, uint32_t stride) {
  static_assert(kAttnHeadDim == 4 * kWave && kAttnRotary == kWave, "lane layout");
  const uint32_t rg = blockIdx.x * kPrepRows + (threadIdx.x / kWave), l = threadIdx.x % kWave;
  const uint32_t q_rows = T * kAttnQHeads;
  if (rg >= T * (kAttnQHeads + kAttnKvHeads)) return;  // whole wave: no barrier below
  const bool is_q = rg < q_rows;
  const uint32_t lr = is_q ? rg : rg - q_rows;
  const uint32_t heads = is_q ? kAttnQHeads : kAttnKvHeads;
  const uint32_t t = lr / heads, h = lr - t * heads;
  const uint16_t* src = is_q ? qp + static_cast<size_t>(lr) * 2 * kAttnHeadDim : k_in + static_cast<size_t>(lr) * kAttnHeadDim;
  const uint16_t* w = is_q ? q_w : k_w;
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = bf2f(src[l + kWave * i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = l + kWave * i;
    if (is_q) gate_out[static_cast<size_t>(lr) * kAttnHeadDim + d] = src[kAttnHeadDim + d];
    else cache_v[(static_cast<size_t>(h) * kAttnHeadDim + d) * stride + start_cache + t] = v_in[static_cast<size_t>(lr) * kAttnHeadDim + d];
  }
  const float sq0 = __fmul_rn(x[0], x[0]), sq1 = __fmul_rn(x[1], x[1]);
  const float sq2 = __fmul_rn(x[2], x[2]), sq3 = __fmul_rn(x[3], x[3]);
  const float root = wave_tree_tail<false>(__fadd_rn(__fadd_rn(sq0, sq2), __fadd_rn(sq1, sq3)));
  const float ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, root), 0));
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(kAttnHeadDim) + kAttnEps);
  uint16_t* dst = is_q ? q_out + static_cast<size_t>(lr) * kAttnHeadDim
                       : cache_k + (static_cast<size_t>(h) * stride + start_cache + t) * kAttnHeadDim;
  // rotary dims: after the swap every lane holds a = element d and b = element d + 32 (d = l % 32)
  {
    constexpr uint32_t half = kAttnRotary / 2;
    const uint32_t d = l % half;
    float a = __fmul_rn(__fmul_rn(x[0], scale), bf2f(w[l])), b = a;
    swap32(a, b);
    const float inv_freq = powf(kAttnTheta, -(2.0f * static_cast<float>(d)) / static_cast<float>(kAttnRotary));
    const float th = static_cast<float>(start_rope + t) * inv_freq;
    const float c = cosf(th), sn = sinf(th);
    dst[l] = l < half ? f2bf(__fsub_rn(__fmul_rn(a, c), __fmul_rn(b, sn))) : f2bf(__fadd_rn(__fmul_rn(b, c), __fmul_rn(a, sn)));
  }
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    const uint32_t d = l + kWave * i;
    dst[d] = f2bf(__fmul_rn(__fmul_rn(x[i], scale), bf2f(w[d])));
  }
}

// Causal softmax over one row of bf16 scores, in place (reference order: row
// max of float(s)*scale over visible columns, then the sum of
// exp2((v - max) * log2e), each thread striding the row, each reduced by a
// halving tree). Row r of kv head z (rows z*4T .. ) is token r % T; column c is
// visible iff c <= prefix + t. Columns [L, ld) are zeroed for the P*V GEMM.
__global__ __launch_bounds__(kSoftmaxThreads) void attn_prefill_softmax_kernel(uint16_t* __restrict__ scores,
                                                                               uint32_t ld, uint32_t L, uint32_t T,
                                                                               uint32_t prefix, float scale) {
  __shared__ float sh[kSoftmaxThreads + 1];
  uint16_t* row = scores + static_cast<size_t>(blockIdx.x) * ld;
  const uint32_t t = (blockIdx.x % (kAttnGroup * T)) % T;
  const uint32_t vis = prefix + t;
  // the P.V GEMM reads this row up to wend (zeros between vis and wend)
  const uint32_t wend = causal_pv_columns(blockIdx.x % (kAttnGroup * T), T, prefix, L);
  // The thread's first kCache columns (c = tid + 256 i) stay in registers
  // across the three passes (one read of the row); later columns are read
  // again. The arithmetic and its order per thread are unchanged. Masked
  // columns (c > vis) are never read: the scores GEMM skips tiles that hold
  // only masked columns, so they may hold anything.
  constexpr int kCache = 8;
  float xs[kCache];
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    const uint32_t c = threadIdx.x + kSoftmaxThreads * i;
    xs[i] = c <= vis ? __fmul_rn(bf2f(row[c]), scale) : 0.0f;
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    const uint32_t c = threadIdx.x + kSoftmaxThreads * i;
    if (c < L) m = fmaxf(m, c > vis ? -INFINITY : xs[i]);
  }
  for (uint32_t c = threadIdx.x + kSoftmaxThreads * kCache; c <= vis; c += kSoftmaxThreads)
    m = fmaxf(m, __fmul_rn(bf2f(row[c]), scale));
  const float row_max = tree_max<kSoftmaxThreads>(m, sh);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    const uint32_t c = threadIdx.x + kSoftmaxThreads * i;
    xs[i] = exp2f(__fmul_rn(__fsub_rn(xs[i], row_max), kLog2e));
    if (c < L && c <= vis) sum += xs[i];
  }
  for (uint32_t c = threadIdx.x + kSoftmaxThreads * kCache; c <= vis; c += kSoftmaxThreads)
    sum += exp2f(__fmul_rn(__fsub_rn(__fmul_rn(bf2f(row[c]), scale), row_max), kLog2e));
  const float total = tree_sum<kSoftmaxThreads>(sum, sh);
  const float denom = total == 0.0f ? 1.0f : total;
#pragma unroll
  for (int i = 0; i < kCache; ++i) {
    const uint32_t c = threadIdx.x + kSoftmaxThreads * i;
    if (c < wend) row[c] = c <= vis ? f2bf(xs[i] / denom) : uint16_t{0};
  }
  for (uint32_t c = threadIdx.x + kSoftmaxThreads * kCache; c < wend; c += kSoftmaxThreads) {
    uint16_t p = 0;
    if (c <= vis) p = f2bf(exp2f(__fmul_rn(__fsub_rn(__fmul_rn(bf2f(row[c]), scale), row_max), kLog2e)) / denom);
    row[c] = p;
  }
}

// ------------------------------------------------------------- GDN ----------
constexpr uint32_t kConvChunk = 16;  // tokens per thread

// x(u) over the virtual sequence [state rows 0..2 ‖ inputs] for channels c, c+1.
__device__ inline float2 conv_src(const float* state, const uint16_t* qkv, uint32_t u, uint32_t c, bool has_state) {
  if (u < kGdnConvK - 1) {
    if (!has_state) return make_float2(0.0f, 0.0f);
    return make_float2(state[u * kGdnConvDim + c], state[u * kGdnConvDim + c + 1]);
  }
  const uint32_t p = *reinterpret_cast<const uint32_t*>(qkv + static_cast<size_t>(u - (kGdnConvK - 1)) * kGdnConvDim + c);
  return make_float2(bf_lo(p), bf_hi(p));
}

__device__ inline float conv_tap(float acc, float w, float x) { return __fadd_rn(acc, __fmul_rn(w, x)); }

// Thread = (channel pair, 16-token chunk): out[t, c] = bf16(silu(sum_j w[c, j] * x(t + j))).
__global__ __launch_bounds__(256) void conv1d_prefill_kernel(const float* __restrict__ state,
                                                             const uint16_t* __restrict__ qkv,
                                                             const uint16_t* __restrict__ w,
                                                             uint16_t* __restrict__ out, uint32_t T,
                                                             uint32_t has_state) {
  constexpr uint32_t pairs = kGdnConvDim / 2;
  const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t c = 2 * (idx % pairs), t0 = (idx / pairs) * kConvChunk;
  if (t0 >= T) return;
  const uint4 wv = *reinterpret_cast<const uint4*>(w + static_cast<size_t>(c) * kGdnConvK);
  const float w0[4] = {bf_lo(wv.x), bf_hi(wv.x), bf_lo(wv.y), bf_hi(wv.y)};
  const float w1[4] = {bf_lo(wv.z), bf_hi(wv.z), bf_lo(wv.w), bf_hi(wv.w)};
  const bool hs = has_state != 0;
  const uint32_t t1 = min(t0 + kConvChunk, T);
  if (t1 - t0 == kConvChunk) {
    // A full chunk issues all of its kConvChunk + 3 loads before the first
    // tap (the same arithmetic per output as the loop below).
    float2 h[kConvChunk + kGdnConvK - 1];
#pragma unroll
    for (uint32_t i = 0; i < kConvChunk + kGdnConvK - 1; ++i) h[i] = conv_src(state, qkv, t0 + i, c, hs);
#pragma unroll
    for (uint32_t i = 0; i < kConvChunk; ++i) {
      float a0 = 0.0f, a1 = 0.0f;
      a0 = conv_tap(a0, w0[0], h[i].x); a0 = conv_tap(a0, w0[1], h[i + 1].x); a0 = conv_tap(a0, w0[2], h[i + 2].x); a0 = conv_tap(a0, w0[3], h[i + 3].x);
      a1 = conv_tap(a1, w1[0], h[i].y); a1 = conv_tap(a1, w1[1], h[i + 1].y); a1 = conv_tap(a1, w1[2], h[i + 2].y); a1 = conv_tap(a1, w1[3], h[i + 3].y);
      const uint32_t o = static_cast<uint32_t>(f2bf(a0 / (1.0f + expf(-a0)))) |
                         (static_cast<uint32_t>(f2bf(a1 / (1.0f + expf(-a1)))) << 16);
      *reinterpret_cast<uint32_t*>(out + static_cast<size_t>(t0 + i) * kGdnConvDim + c) = o;
    }
    return;
  }
  float2 h0 = conv_src(state, qkv, t0, c, hs), h1 = conv_src(state, qkv, t0 + 1, c, hs),
         h2 = conv_src(state, qkv, t0 + 2, c, hs);
  for (uint32_t t = t0; t < t1; ++t) {
    const float2 h3 = conv_src(state, qkv, t + 3, c, hs);
    float a0 = 0.0f, a1 = 0.0f;
    a0 = conv_tap(a0, w0[0], h0.x); a0 = conv_tap(a0, w0[1], h1.x); a0 = conv_tap(a0, w0[2], h2.x); a0 = conv_tap(a0, w0[3], h3.x);
    a1 = conv_tap(a1, w1[0], h0.y); a1 = conv_tap(a1, w1[1], h1.y); a1 = conv_tap(a1, w1[2], h2.y); a1 = conv_tap(a1, w1[3], h3.y);
    const uint32_t o = static_cast<uint32_t>(f2bf(a0 / (1.0f + expf(-a0)))) |
                       (static_cast<uint32_t>(f2bf(a1 / (1.0f + expf(-a1)))) << 16);
    *reinterpret_cast<uint32_t*>(out + static_cast<size_t>(t) * kGdnConvDim + c) = o;
    h0 = h1;
    h1 = h2;
    h2 = h3;
  }
}

// state[j, c] = x(T + j): the last three entries of the virtual sequence.
// Runs after conv1d_prefill_kernel (which reads the old state).
__global__ void conv1d_prefill_state_kernel(float* __restrict__ state, const uint16_t* __restrict__ qkv, uint32_t T,
                                            uint32_t has_state) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= kGdnConvDim) return;
  for (uint32_t j = 0; j < kGdnConvK - 1; ++j) {
    const uint32_t u = T + j;  // u > j: state[u] is read before it is rewritten
    float x = 0.0f;
    if (u < kGdnConvK - 1) x = has_state ? state[u * kGdnConvDim + c] : 0.0f;
    else x = bf2f(qkv[static_cast<size_t>(u - (kGdnConvK - 1)) * kGdnConvDim + c]);
    state[j * kGdnConvDim + c] = x;
  }
}

// Sum of 128 values in tree_sum<128>'s order (entry i += entry i + stride
// for stride 64, 32, ..., 1) within one wave: lane i holds entries i and
// i + 64; the 32- and 16-lane steps pair lanes with v_permlane32_swap /
// v_permlane16_swap, the rest shift within a DPP row. Returns the total to
// every lane. Each step adds the same two values as the LDS tree, so the
// bits are the tree's.
__device__ inline float tree128_wave(float lo, float hi) {
  float s = __fadd_rn(lo, hi);
  {
    float x = s, y = s;
    swap32(x, y);  // own value and lane i ^ 32's
    s = __fadd_rn(x, y);
  }
  {
    float x = s, y = s;
    swap16(x, y);  // own value and the partner row's lane
    s = __fadd_rn(x, y);
  }
  s = __fadd_rn(s, dpp_f<0x108>(s));  // row_shl:8 -- lane i += lane i + 8
  s = __fadd_rn(s, dpp_f<0x104>(s));
  s = __fadd_rn(s, dpp_f<0x102>(s));
  s = __fadd_rn(s, dpp_f<0x101>(s));
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, s)));
}

// One wave per (t, hk): f32 l2-normed q (x rsqrt(Dk)) and k of k-head hk and
// their dot product kq, with the 128-thread tree's sums
// (QK_NORM_PREFILL_THREADS_PER_THREADGROUP, gated_norm.metal:55); lanes 0, 1
// also produce the gates of v-heads 2hk, 2hk+1. Lane i holds dims i and
// i + 64.
constexpr int kPrepWaves = 4;  // (t, hk) pairs per 256-thread block
__global__ __launch_bounds__(kPrepWaves * kWave) void gdn_prefill_prepare_kernel(
    const uint16_t* __restrict__ conv_out, const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
    const float* __restrict__ A_log, const uint16_t* __restrict__ dt_bias, float* __restrict__ qn,
    float* __restrict__ kn, float* __restrict__ g, float* __restrict__ beta, float* __restrict__ kq, uint32_t T) {
  const uint32_t pair = blockIdx.x * kPrepWaves + (threadIdx.x / kWave);
  if (pair >= T * kGdnHk) return;  // a whole wave
  const uint32_t t = pair / kGdnHk, hk = pair % kGdnHk, d = threadIdx.x % kWave;
  const uint16_t* row = conv_out + static_cast<size_t>(t) * kGdnConvDim;
  const float q0 = bf2f(row[hk * kGdnDk + d]), q1 = bf2f(row[hk * kGdnDk + 64 + d]);
  const float k0 = bf2f(row[kGdnKeyDim + hk * kGdnDk + d]), k1 = bf2f(row[kGdnKeyDim + hk * kGdnDk + 64 + d]);
  const float qs = tree128_wave(__fmul_rn(q0, q0), __fmul_rn(q1, q1));
  const float ks = tree128_wave(__fmul_rn(k0, k0), __fmul_rn(k1, k1));
  const float q_inv = 1.0f / sqrtf(qs + 1.0e-6f), k_inv = 1.0f / sqrtf(ks + 1.0e-6f);
  const float q_scale = 1.0f / sqrtf(static_cast<float>(kGdnDk));
  const size_t o = (static_cast<size_t>(t) * kGdnHk + hk) * kGdnDk + d;
  const float qo0 = __fmul_rn(__fmul_rn(q0, q_inv), q_scale), qo1 = __fmul_rn(__fmul_rn(q1, q_inv), q_scale);
  const float ko0 = __fmul_rn(k0, k_inv), ko1 = __fmul_rn(k1, k_inv);
  qn[o] = qo0;
  qn[o + 64] = qo1;
  kn[o] = ko0;
  kn[o + 64] = ko1;
  // k.q of the normalised pair: shared by every state row of the two v-heads.
  const float kqs = tree128_wave(__fmul_rn(ko0, qo0), __fmul_rn(ko1, qo1));
  if (kq && d == 0) kq[static_cast<size_t>(t) * kGdnHk + hk] = kqs;
  if (d < kGdnHv / kGdnHk) {
    const uint32_t hv = hk * (kGdnHv / kGdnHk) + d;
    const size_t go = static_cast<size_t>(t) * kGdnHv + hv;
    const float x = __fadd_rn(bf2f(a[go]), bf2f(dt_bias[hv]));
    const float softplus = __fadd_rn(fmaxf(x, 0.0f), logf(1.0f + expf(-fabsf(x))));
    g[go] = expf(__fmul_rn(-expf(A_log[hv]), softplus));
    beta[go] = 1.0f / (1.0f + expf(-bf2f(b[go])));
  }
}

// Token-sequential delta rule. Block = 16 state rows of one v-head (4 wave64s,
// each 16-lane DPP row owns one state row; lane j holds dk = 8j..8j+7 in
// registers for the whole prompt). Per token:
//   kq = k.q; d = S*decay; kv = d.k; ob = d.q; delta = (v - kv)*beta;
//   S = d + k*delta; y = bf16(ob + delta*kq)
// The per-token inputs (q, k of the k-head, gates, v of the block's rows) are
// staged through LDS in chunks of kGdnChunk tokens, double-buffered: the
// next chunk's global loads are in flight while the current chunk runs, so the
// sequential loop only waits on LDS. Outputs collect in LDS and leave once per
// chunk. (One wave per SIMD: the loop is instruction-issue bound, so a layout
// with more lanes per row and more waves per SIMD only adds reduction work.)
constexpr int kGdnPRowsPerBlock = 16;
constexpr int kGdnChunk = 32;

template <bool PRE_KQ>
__global__ __launch_bounds__(256) void gdn_prefill_kernel(float* __restrict__ state, const float* __restrict__ qn,
                                                          const float* __restrict__ kn,
                                                          const uint16_t* __restrict__ conv_out,
                                                          const float* __restrict__ g,
                                                          const float* __restrict__ beta,
                                                          const float* __restrict__ kqv,
                                                          uint16_t* __restrict__ y, uint32_t T,
                                                          uint32_t has_state) {
  __shared__ float4 sq[2][kGdnChunk][kGdnDk / 4];
  __shared__ float4 sk[2][kGdnChunk][kGdnDk / 4];
  __shared__ float4 sgk[2][kGdnChunk];  // decay, beta, k.q of each token (one LDS read)
  __shared__ float sv[2][kGdnChunk][kGdnPRowsPerBlock];
  __shared__ uint16_t sy[2][kGdnChunk][kGdnPRowsPerBlock];
  constexpr uint32_t blocks_per_head = kGdnDv / kGdnPRowsPerBlock;
  const uint32_t tid = threadIdx.x;
  const uint32_t hv = blockIdx.x / blocks_per_head;
  const uint32_t row0 = (blockIdx.x % blocks_per_head) * kGdnPRowsPerBlock;
  const uint32_t rb = tid >> 4, j = tid & 15;  // row in block, lane in DPP row
  const uint32_t hk = hv / (kGdnHv / kGdnHk);
  float4* srow = reinterpret_cast<float4*>(state + (static_cast<size_t>(hv) * kGdnDv + row0 + rb) * kGdnDk + 8 * j);
  float S[8];
  {
    const float4 s0 = has_state ? srow[0] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 s1 = has_state ? srow[1] : make_float4(0.f, 0.f, 0.f, 0.f);
    S[0] = s0.x; S[1] = s0.y; S[2] = s0.z; S[3] = s0.w;
    S[4] = s1.x; S[5] = s1.y; S[6] = s1.z; S[7] = s1.w;
  }
  // Chunk loader: q/k 32 tokens x 32 float4 = 4 float4 per thread each;
  // v 32 tokens x 16 rows = 2 per thread; gates by threads 0..31.
  const float4* q4 = reinterpret_cast<const float4*>(qn) + hk * (kGdnDk / 4);
  const float4* k4 = reinterpret_cast<const float4*>(kn) + hk * (kGdnDk / 4);
  constexpr uint32_t qk_step = kGdnKeyDim / 4;  // float4 per token
  float4 rq[4], rk[4];
  float rv[2], rg = 0.f, rbt = 0.f, rkq = 0.f;
  auto load = [&](uint32_t c0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t idx = tid + 256 * i, t = c0 + idx / 32, f = idx % 32;
      rq[i] = t < T ? q4[static_cast<size_t>(t) * qk_step + f] : make_float4(0.f, 0.f, 0.f, 0.f);
      rk[i] = t < T ? k4[static_cast<size_t>(t) * qk_step + f] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t idx = tid + 256 * i, t = c0 + idx / 16, r = idx % 16;
      rv[i] = t < T ? bf2f(conv_out[static_cast<size_t>(t) * kGdnConvDim + 2 * kGdnKeyDim + hv * kGdnDv + row0 + r])
                    : 0.f;
    }
    if (tid < kGdnChunk && c0 + tid < T) {
      rg = g[static_cast<size_t>(c0 + tid) * kGdnHv + hv];
      rbt = beta[static_cast<size_t>(c0 + tid) * kGdnHv + hv];
      if constexpr (PRE_KQ) rkq = kqv[static_cast<size_t>(c0 + tid) * kGdnHk + hk];
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t idx = tid + 256 * i;
      sq[buf][idx / 32][idx % 32] = rq[i];
      sk[buf][idx / 32][idx % 32] = rk[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t idx = tid + 256 * i;
      sv[buf][idx / 16][idx % 16] = rv[i];
    }
    if (tid < kGdnChunk) sgk[buf][tid] = make_float4(rg, rbt, rkq, 0.f);
  };

  // Per-token operands, read from LDS one token ahead into alternating sets.
  struct Tok {
    float4 qa, qc, ka, kc;
    float decay, beta, kq, v;
  };
  auto fetch = [&](Tok& o, int b, uint32_t tt) {
    o.qa = sq[b][tt][2 * j];
    o.qc = sq[b][tt][2 * j + 1];
    o.ka = sk[b][tt][2 * j];
    o.kc = sk[b][tt][2 * j + 1];
    const float4 gk = sgk[b][tt];
    o.decay = gk.x;
    o.beta = gk.y;
    o.kq = gk.z;
    o.v = sv[b][tt][rb];
  };
  // Outputs of a chunk collect in LDS and leave in one coalesced pass after
  // the chunk's barrier.
  auto token = [&](const Tok& o, int b, uint32_t tt) {
    const float q[8] = {o.qa.x, o.qa.y, o.qa.z, o.qa.w, o.qc.x, o.qc.y, o.qc.z, o.qc.w};
    const float k[8] = {o.ka.x, o.ka.y, o.ka.z, o.ka.w, o.kc.x, o.kc.y, o.kc.z, o.kc.w};
    float d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = S[i] * o.decay;
    // two independent partial sums per dot product shorten the chain
    const float kv = row16_sum((d[0] * k[0] + d[1] * k[1] + d[2] * k[2] + d[3] * k[3]) +
                               (d[4] * k[4] + d[5] * k[5] + d[6] * k[6] + d[7] * k[7]));
    const float ob = row16_sum((d[0] * q[0] + d[1] * q[1] + d[2] * q[2] + d[3] * q[3]) +
                               (d[4] * q[4] + d[5] * q[5] + d[6] * q[6] + d[7] * q[7]));
    const float delta = (o.v - kv) * o.beta;
#pragma unroll
    for (int i = 0; i < 8; ++i) S[i] = d[i] + k[i] * delta;
    float kqd = o.kq;
    if constexpr (!PRE_KQ)
      kqd = row16_sum((k[0] * q[0] + k[1] * q[1] + k[2] * q[2] + k[3] * q[3]) +
                      (k[4] * q[4] + k[5] * q[5] + k[6] * q[6] + k[7] * q[7]));
    // every lane of the row holds the same y; all of them store it (same
    // address, same bits), which keeps the loop free of exec-mask branches
    sy[b][tt][rb] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(ob + delta * kqd));
  };

  load(0);
  store(0);
  __syncthreads();
  int buf = 0;
  for (uint32_t c0 = 0; c0 < T; c0 += kGdnChunk, buf ^= 1) {
    const bool more = c0 + kGdnChunk < T;
    if (more) load(c0 + kGdnChunk);
    const uint32_t n = min(static_cast<uint32_t>(kGdnChunk), T - c0);
    Tok ta, tb;
    fetch(ta, buf, 0);
    if (n == kGdnChunk) {
      // full chunk: unrolled, every LDS operand at a constant offset
#pragma unroll
      for (uint32_t tt = 0; tt < kGdnChunk; tt += 2) {
        // each fetch is issued before the other token's arithmetic
        fetch(tb, buf, tt + 1);
        __builtin_amdgcn_sched_barrier(0);
        token(ta, buf, tt);
        __builtin_amdgcn_sched_barrier(0);
        if (tt + 2 < kGdnChunk) fetch(ta, buf, tt + 2);
        __builtin_amdgcn_sched_barrier(0);
        token(tb, buf, tt + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      uint32_t tt = 0;
      for (; tt + 1 < n; tt += 2) {
        fetch(tb, buf, tt + 1);
        token(ta, buf, tt);
        fetch(ta, buf, tt + 2 < n ? tt + 2 : tt + 1);
        token(tb, buf, tt + 1);
      }
      if (tt < n) token(ta, buf, tt);
    }
    if (more) store(buf ^ 1);
    __syncthreads();
    // 16 rows x n tokens of this chunk: two rows per thread
    {
      const uint32_t t_out = tid >> 3, r2 = 2 * (tid & 7);
      if (t_out < n) {
        const uint32_t pair = static_cast<uint32_t>(sy[buf][t_out][r2]) | (static_cast<uint32_t>(sy[buf][t_out][r2 + 1]) << 16);
        *reinterpret_cast<uint32_t*>(y + static_cast<size_t>(c0 + t_out) * kGdnValDim + hv * kGdnDv + row0 + r2) = pair;
      }
    }
  }
  srow[0] = make_float4(S[0], S[1], S[2], S[3]);
  srow[1] = make_float4(S[4], S[5], S[6], S[7]);
}

// out[r] = a[r] ‖ b[r] for rows of `width` bf16 (concat_two_rows_bf16, the
// drafter's fc input, src/model/mtp.zig:262-270). One uint4 per thread.
__global__ void concat_rows_kernel(const uint4* __restrict__ a, const uint4* __restrict__ b, uint4* __restrict__ out,
                                   uint32_t rows, uint32_t w8) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<size_t>(rows) * 2 * w8) return;
  const size_t r = i / (2 * w8), c = i % (2 * w8);
  out[i] = c < w8 ? a[r * w8 + c] : b[r * w8 + c - w8];
}

}  // namespace

namespace prg {

int launch_concat_rows(hipStream_t s, const uint16_t* a, const uint16_t* b, uint16_t* out, uint32_t rows,
                       uint32_t width) {
  const uint32_t w8 = width / 8;
  const size_t n = static_cast<size_t>(rows) * 2 * w8;
  hipLaunchKernelGGL(concat_rows_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s,
                     reinterpret_cast<const uint4*>(a), reinterpret_cast<const uint4*>(b), reinterpret_cast<uint4*>(out),
                     rows, w8);
  PRG_CHECK_LAUNCH("concat_rows");
  return PRG_OK;
}

size_t attn_prefill_scores_elems(uint32_t T, uint32_t prefix) {
  const size_t L = static_cast<size_t>(prefix) + T, ld = (L + 63) / 64 * 64;
  return static_cast<size_t>(kAttnQHeads) * T * ld;
}

int launch_attn_prefill_prepare(hipStream_t s, const uint16_t* qp, const uint16_t* q_w, const uint16_t* k_in,
                                const uint16_t* k_w, const uint16_t* v_in, uint16_t* q_out, uint16_t* gate_out,
                                uint16_t* cache_k, uint16_t* cache_v, uint32_t T, uint32_t start_rope,
                                uint32_t start_cache, uint32_t stride) {
  hipLaunchKernelGGL(attn_prefill_prepare_kernel, dim3((T * (kAttnQHeads + kAttnKvHeads) + kPrepRows - 1) / kPrepRows),
                     dim3(kPrepThreads), 0, s,
                     qp, q_w, k_in, k_w, v_in, q_out, gate_out, cache_k, cache_v, T, start_rope, start_cache, stride);
  PRG_CHECK_LAUNCH("attn_prefill_prepare");
  return PRG_OK;
}

int launch_attn_prefill(hipStream_t s, const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                        const uint16_t* gate, uint16_t* out, uint16_t* scores, size_t scores_cap, uint32_t T,
                        uint32_t prefix, uint32_t stride, float scale) {
  // scores_cap: bf16 elements the score block holds
  if (attn_prefill_scores_elems(T, prefix) > scores_cap)
    return set_error(PRG_ERR_INVALID_ARG, "attention prefill: %u tokens after %u need %zu score elements, %zu held",
                     T, prefix, attn_prefill_scores_elems(T, prefix), scores_cap);
  const uint32_t L = prefix + T, ld = (L + 63) / 64 * 64;
  const uint32_t rows = kAttnGroup * T;  // per kv head: q head in group x token
  GemmArgs sc;
  sc.a = q;
  sc.lda = static_cast<uint64_t>(kAttnQHeads) * kAttnHeadDim;  // next token
  sc.lda_hi = kAttnHeadDim;                                    // next q head of the group
  sc.a_group = T;
  sc.a_z = static_cast<uint64_t>(kAttnGroup) * kAttnHeadDim;
  sc.b = cache_k;
  sc.ldb = kAttnHeadDim;
  sc.b_z = static_cast<uint64_t>(stride) * kAttnHeadDim;
  sc.c = scores;
  sc.ldc = ld;
  sc.c_z = static_cast<uint64_t>(rows) * ld;
  sc.M = rows;
  sc.N = L;
  sc.K = kAttnHeadDim;
  sc.causal_T = T;
  sc.causal_prefix = prefix;
  if (int rc = launch_gemm_bf16(s, sc, kGemmStore, kAttnKvHeads, "attn_prefill.scores")) return rc;
  hipLaunchKernelGGL(attn_prefill_softmax_kernel, dim3(kAttnKvHeads * rows), dim3(kSoftmaxThreads), 0, s, scores, ld,
                     L, T, prefix, scale);
  PRG_CHECK_LAUNCH("attn_prefill.softmax");
  GemmArgs pv;
  pv.a = scores;
  pv.lda = ld;
  pv.a_z = static_cast<uint64_t>(rows) * ld;
  pv.b = cache_v;
  pv.ldb = stride;
  pv.b_z = static_cast<uint64_t>(kAttnHeadDim) * stride;
  pv.c = out;
  pv.res = gate;
  pv.ldc = static_cast<uint64_t>(kAttnQHeads) * kAttnHeadDim;
  pv.ldc_hi = kAttnHeadDim;
  pv.c_group = T;
  pv.c_z = static_cast<uint64_t>(kAttnGroup) * kAttnHeadDim;
  pv.M = rows;
  pv.N = kAttnHeadDim;
  pv.K = L;
  pv.causal_T = T;
  pv.causal_prefix = prefix;
  return launch_gemm_bf16(s, pv, kGemmSigmoidGate, kAttnKvHeads, "attn_prefill.values");
}

int launch_conv1d_prefill(hipStream_t s, float* state, const uint16_t* qkv, const uint16_t* w, uint16_t* out,
                          uint32_t T, uint32_t has_state) {
  const size_t threads = static_cast<size_t>(kGdnConvDim / 2) * ((T + kConvChunk - 1) / kConvChunk);
  hipLaunchKernelGGL(conv1d_prefill_kernel, dim3(static_cast<uint32_t>((threads + 255) / 256)), dim3(256), 0, s, state,
                     qkv, w, out, T, has_state);
  PRG_CHECK_LAUNCH("conv1d_prefill");
  hipLaunchKernelGGL(conv1d_prefill_state_kernel, dim3(kGdnConvDim / 256), dim3(256), 0, s, state, qkv, T, has_state);
  PRG_CHECK_LAUNCH("conv1d_prefill_state");
  return PRG_OK;
}

int launch_gdn_prefill_prepare(hipStream_t s, const uint16_t* conv_out, const uint16_t* a, const uint16_t* b,
                               const float* A_log, const uint16_t* dt_bias, float* qn, float* kn, float* g,
                               float* beta, float* kq, uint32_t T) {
  hipLaunchKernelGGL(gdn_prefill_prepare_kernel, dim3((T * kGdnHk + kPrepWaves - 1) / kPrepWaves),
                     dim3(kPrepWaves * kWave), 0, s, conv_out, a, b, A_log, dt_bias, qn, kn, g, beta, kq, T);
  PRG_CHECK_LAUNCH("gdn_prefill_prepare");
  return PRG_OK;
}

int launch_gdn_prefill(hipStream_t s, float* state, const float* qn, const float* kn, const uint16_t* conv_out,
                       const float* g, const float* beta, const float* kq, uint16_t* y, uint32_t T,
                       uint32_t has_state) {
  // kq == nullptr: the recurrence forms k.q itself
  if (kq)
    hipLaunchKernelGGL(gdn_prefill_kernel<true>, dim3(kGdnHv * (kGdnDv / kGdnPRowsPerBlock)), dim3(256), 0, s, state,
                       qn, kn, conv_out, g, beta, kq, y, T, has_state);
  else
    hipLaunchKernelGGL(gdn_prefill_kernel<false>, dim3(kGdnHv * (kGdnDv / kGdnPRowsPerBlock)), dim3(256), 0, s, state,
                       qn, kn, conv_out, g, beta, kq, y, T, has_state);
  PRG_CHECK_LAUNCH("gdn_prefill");
  return PRG_OK;
}

}  // namespace prg

extern "C" {

size_t prg_attn_prefill_scores_bytes(uint32_t token_count, uint32_t prefix_len) {
  return sizeof(uint16_t) * prg::attn_prefill_scores_elems(token_count, prefix_len);
}

int prg_attn_prefill_prepare_bf16(void* stream, const uint16_t* packed_q, const uint16_t* q_weight,
                                  const uint16_t* k_input, const uint16_t* k_weight,
                                  const uint16_t* v_input, uint16_t* q_output, uint16_t* gate_output,
                                  uint16_t* key_cache, uint16_t* value_cache, uint32_t token_count,
                                  uint32_t start_rope_pos, uint32_t start_cache_pos,
                                  uint32_t cache_stride_tokens) {
  PRG_CHECK_ARG(packed_q && q_weight && k_input && k_weight && v_input && q_output && gate_output && key_cache &&
                    value_cache,
                "prg_attn_prefill_prepare_bf16: null pointer");
  PRG_CHECK_ARG(token_count > 0, "prg_attn_prefill_prepare_bf16: token_count == 0");
  PRG_CHECK_ARG(static_cast<uint64_t>(start_cache_pos) + token_count <= cache_stride_tokens,
                "prg_attn_prefill_prepare_bf16: cache slots [%u, %u) exceed the stride %u", start_cache_pos,
                start_cache_pos + token_count, cache_stride_tokens);
  PRG_CHECK_ARG(static_cast<uint64_t>(token_count) * (kAttnQHeads + kAttnKvHeads) < (1ull << 31),
                "prg_attn_prefill_prepare_bf16: token_count %u too large", token_count);
  return prg::launch_attn_prefill_prepare(as_stream(stream), packed_q, q_weight, k_input, k_weight, v_input, q_output,
                                          gate_output, key_cache, value_cache, token_count, start_rope_pos,
                                          start_cache_pos, cache_stride_tokens);
}

int prg_attn_prefill_bf16(void* stream, const uint16_t* q, const uint16_t* key_cache,
                          const uint16_t* value_cache, const uint16_t* gate, uint16_t* out,
                          uint16_t* scores, uint32_t token_count, uint32_t prefix_len,
                          uint32_t cache_stride_tokens, float scale) {
  PRG_CHECK_ARG(q && key_cache && value_cache && gate && out && scores, "prg_attn_prefill_bf16: null pointer");
  PRG_CHECK_ARG(token_count > 0, "prg_attn_prefill_bf16: token_count == 0");
  PRG_CHECK_ARG(cache_stride_tokens % 8 == 0, "prg_attn_prefill_bf16: stride %u must be a multiple of 8",
                cache_stride_tokens);
  PRG_CHECK_ARG(static_cast<uint64_t>(prefix_len) + token_count <= cache_stride_tokens,
                "prg_attn_prefill_bf16: %u + %u tokens exceed the stride %u", prefix_len, token_count,
                cache_stride_tokens);
  PRG_CHECK_ARG(static_cast<uint64_t>(kAttnQHeads) * token_count < (1ull << 31),
                "prg_attn_prefill_bf16: token_count %u too large", token_count);
  // the caller sized scores with prg_attn_prefill_scores_bytes (op contract)
  return prg::launch_attn_prefill(as_stream(stream), q, key_cache, value_cache, gate, out, scores,
                                  prg::attn_prefill_scores_elems(token_count, prefix_len), token_count, prefix_len,
                                  cache_stride_tokens, scale);
}

int prg_conv1d_silu_prefill_bf16(void* stream, float* state, const uint16_t* qkv, const uint16_t* weight,
                                 uint16_t* out, uint32_t token_count, uint32_t conv_dim,
                                 uint32_t kernel_size, uint32_t has_previous_state) {
  PRG_CHECK_ARG(state && qkv && weight && out, "prg_conv1d_silu_prefill_bf16: null pointer");
  PRG_CHECK_ARG(conv_dim == prg::kGdnConvDim && kernel_size == prg::kGdnConvK,
                "prg_conv1d_silu_prefill_bf16: only conv_dim 8192, kernel 4 is built");
  PRG_CHECK_ARG(token_count > 0, "prg_conv1d_silu_prefill_bf16: token_count == 0");
  return prg::launch_conv1d_prefill(as_stream(stream), state, qkv, weight, out, token_count, has_previous_state);
}

int prg_gated_delta_prefill_prepare_bf16(void* stream, const uint16_t* conv_out, const uint16_t* a,
                                         const uint16_t* b, const float* A_log, const uint16_t* dt_bias,
                                         float* q_out, float* k_out, float* g_out, float* beta_out,
                                         float* kq_out, uint32_t token_count) {
  PRG_CHECK_ARG(conv_out && a && b && A_log && dt_bias && q_out && k_out && g_out && beta_out,
                "prg_gated_delta_prefill_prepare_bf16: null pointer");
  PRG_CHECK_ARG(token_count > 0, "prg_gated_delta_prefill_prepare_bf16: token_count == 0");
  return prg::launch_gdn_prefill_prepare(as_stream(stream), conv_out, a, b, A_log, dt_bias, q_out, k_out, g_out,
                                         beta_out, kq_out, token_count);
}

int prg_gated_delta_prefill_bf16(void* stream, float* state, const float* q, const float* k,
                                 const uint16_t* conv_out, const float* g, const float* beta, uint16_t* y,
                                 uint32_t token_count, uint32_t has_previous_state) {
  PRG_CHECK_ARG(state && q && k && conv_out && g && beta && y, "prg_gated_delta_prefill_bf16: null pointer");
  PRG_CHECK_ARG(token_count > 0, "prg_gated_delta_prefill_bf16: token_count == 0");
  return prg::launch_gdn_prefill(as_stream(stream), state, q, k, conv_out, g, beta, nullptr, y, token_count,
                                 has_previous_state);
}

}  // extern "C"
