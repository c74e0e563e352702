// GQA decode attention: prepare (q/gate split, q/k RMSNorm + RoPE, KV append),
// split-context flash-decode partials, and the merge + sigmoid-gate reduce.
//
// Reference semantics:
//   prepare   qwen35_q_gate_prepare_kv_append_pair_head_major_value_dim_major_bf16
//             shaders/attention.metal:327-421 (params :50-60 = block_attn.zig:43-53)
//   partials  sdpa_decode_prefix_flash_partials_bf16 shaders/attention_decode.metal:24-210
//   reduce    sdpa_decode_prefix_flash_reduce_gated_bf16 shaders/attention_decode.metal:215-243
//   compose   FullAttentionBlock.decodeStepBf16 src/model/block_attn.zig:261-359
//
// Cache layout (the reference's, src/model/state.zig:41-48): K [kv, stride, 256]
// token-major, V [kv, 256, stride] value-dim-major.
//
// gfx950 partials design: the 4 q heads of a kv head share every K/V byte.
// Each block owns a contiguous token range of one kv head; the number of
// ranges is fixed per cache (graph-stable) and sized to put >= 256 blocks on
// the chip at long context.
//   phase 1  16 lanes per token (one DPP row), 16 dims per lane as two dwordx4
//            loads; q.k for 4 heads with v_dot2c_f32_bf16; row-local DPP sum.
//   phase 2  wave g takes head g: max, exp, sum over the range (scores in LDS).
//   phase 3  P.V: 8 lanes x 16 B cover 64 consecutive tokens of one V row
//            (128 B, coalesced); 8 rows per wave load; fp32 FMA with p from
//            LDS; 8-lane DPP sum at the end.
#include <stdlib.h>

#include <mutex>

#include "attention.hpp"

namespace {

using namespace prg;

constexpr int kAttnThreads = 256;
// Split ranges are multiples of 32 tokens and at least 64. A lane reads V in
// 8-token pieces, so every read stays inside the split's 32-token-aligned
// range (and the cache stride, a multiple of 64).
constexpr uint32_t kAttnChunkAlign = 32;
// Each split holds at least one full 64-token tile: on a short context the
// trailing splits stay empty (neutral partials, an early exit) instead of
// spreading a few tokens over every block. Measured at a ~2k-token context
// (64 splits per kv head): 32 tokens per split 654 tok/s, 64 per split 662.
constexpr uint32_t kAttnMinChunk = 64;

// Tokens per split for L cached tokens over nsplit splits.
__host__ __device__ inline uint32_t attn_chunk(uint32_t L, uint32_t nsplit) {
  const uint32_t c = ((L + nsplit - 1) / nsplit + kAttnChunkAlign - 1) & ~(kAttnChunkAlign - 1);
  return c > kAttnMinChunk ? c : kAttnMinChunk;
}

template <int CTRL>
__device__ inline float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over each aligned group of 16 lanes; all 16 lanes get the same bits.
__device__ inline float row16_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  return v;
}
template <int CTRL>
__device__ inline float dpp_max(float v) {
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                          false)));
}
// Max / sum over all 64 lanes (every lane gets the result): DPP within each
// 16-lane row, then the 4 row values by readlane.
__device__ inline float wave_max_dpp(float v) {
  v = dpp_max<0x141>(dpp_max<0x140>(dpp_max<0x4E>(dpp_max<0xB1>(v))));
  const int x = __builtin_bit_cast(int, v);
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 48))));
}
__device__ inline float wave_sum_dpp(float v) {
  const int x = __builtin_bit_cast(int, row16_sum(v));
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 48)));
}
// Sum over each aligned group of 8 lanes.
__device__ inline float row8_sum(float v) {
  v = dpp_add<0xB1>(v);
  v = dpp_add<0x4E>(v);
  v = dpp_add<0x141>(v);
  return v;
}

__device__ inline float dot2(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// ------------------------------------------------------------------ prepare --
__global__ __launch_bounds__(kAttnThreads) void attn_prepare_kernel(const AttnPrepareArgs a0) {
  __shared__ float red[kAttnThreads / kWave];
  AttnPrepareArgs a = a0;  // token blockIdx.y's slices
  if (const uint32_t r = blockIdx.y) {
    a.packed_q += r * (2 * kAttnQHeads * kAttnHeadDim);
    a.k_in += r * (kAttnKvHeads * kAttnHeadDim);
    a.v_in += r * (kAttnKvHeads * kAttnHeadDim);
    a.q_out += r * (kAttnQHeads * kAttnHeadDim);
    a.gate_out += r * (kAttnQHeads * kAttnHeadDim);
    a.step += r;
  }
  const uint32_t tg = blockIdx.x;
  const bool use_q = tg < kAttnQHeads;
  const uint32_t head = use_q ? tg : tg - kAttnQHeads;
  const uint32_t col = threadIdx.x;  // 256 threads == head_dim
  const size_t row_base = static_cast<size_t>(head) * kAttnHeadDim;
  const size_t packed_base = static_cast<size_t>(head) * 2 * kAttnHeadDim;
  const uint16_t* w = use_q ? a.q_norm : a.k_norm;
  constexpr uint32_t half = kAttnRotary / 2;
  // Every input is loaded before the step scalars are read, so the loads do
  // not wait for the step block's load.
  const float v = bf2f(use_q ? a.packed_q[packed_base + col] : a.k_in[row_base + col]);
  const uint16_t side = use_q ? a.packed_q[packed_base + kAttnHeadDim + col] : a.v_in[row_base + col];
  const float v2 = col < half ? bf2f(use_q ? a.packed_q[packed_base + col + half] : a.k_in[row_base + col + half])
                              : 0.0f;
  const uint32_t cache_pos = a.step ? a.step->cache_pos : a.cache_pos_host;
  const uint32_t rope_pos = a.step ? a.step->rope_pos : a.rope_pos_host;
  if (cache_pos >= a.stride) return;  // never write outside the cache (host checks first)

  if (use_q)
    a.gate_out[row_base + col] = side;
  else
    a.value_cache[(row_base + col) * a.stride + cache_pos] = side;
  const float ss = block_sum<kAttnThreads>(v * v, red);
  const float inv_rms = rsqrtf(ss / static_cast<float>(kAttnHeadDim) + kAttnEps);

  uint16_t* dst = use_q ? a.q_out + row_base
                        : a.key_cache + (static_cast<size_t>(head) * a.stride + cache_pos) * kAttnHeadDim;
  if (col < half) {
    // partial NeoX RoPE on dims [0, 64): pairs (i, i + 32); normed values are
    // rounded to bf16 before rotation (attention.metal:391-392).
    const float x1 = round_bf(v * inv_rms * bf2f(w[col]));
    const float x2 = round_bf(v2 * inv_rms * bf2f(w[col + half]));
    const float inv_freq = powf(kAttnTheta, -(2.0f * static_cast<float>(col)) / static_cast<float>(kAttnRotary));
    const float angle = static_cast<float>(rope_pos) * inv_freq;
    const float c = cosf(angle), s = sinf(angle);
    dst[col] = f2bf(x1 * c - x2 * s);
    dst[col + half] = f2bf(x2 * c + x1 * s);
  } else if (col >= kAttnRotary) {
    dst[col] = f2bf(v * inv_rms * bf2f(w[col]));
  }
}

// ----------------------------------------------------------------- partials --
// Query token r = blockIdx.z (or blockIdx.y for the merge) of a launch:
// its q / gate / output rows, its partials and its step scalars.
__device__ inline AttnDecodeArgs attn_row_args(const AttnDecodeArgs& a0, uint32_t r) {
  AttnDecodeArgs a = a0;
  if (r) {
    a.q += r * (kAttnQHeads * kAttnHeadDim);
    a.gate += r * (kAttnQHeads * kAttnHeadDim);
    a.out += r * (kAttnQHeads * kAttnHeadDim);
    a.partials += static_cast<size_t>(r) * kAttnQHeads * a.nsplit * kAttnPartialStride;
    a.step += r;
    if (a.packed_q) a.packed_q += r * (2 * kAttnQHeads * kAttnHeadDim);
  }
  return a;
}

// Tokens the partials cover: all seq_len cached tokens, or, in the
// decode-step form, those before the first new token.
__device__ inline uint32_t attn_cached_tokens(const AttnDecodeArgs& a0) {
  const uint32_t L = a0.step ? a0.step->seq_len : a0.seq_len_host;
  return min(a0.packed_q ? L - 1 : L, a0.stride);
}

// RMSNorm with weight wt and partial NeoX RoPE at pos (dims [0, 64), pairs
// i, i + 32; normed values rounded to bf16 before the rotation,
// attention.metal:391-392) of one 256-wide head held by one wave: lane l
// holds dims l + 64k (k = 0..3) and gets their bf16 results in o[k]. The sum
// of squares has a fixed order: per 64-dim group the row16 DPP sums of its
// four 16-lane rows as (r0 + r1) + (r2 + r3), then the groups as
// (g0 + g1) + (g2 + g3); every row of a two-token launch runs this same code,
// so the verify rows equal single-token steps. No barrier: the rotary partner
// of dim d < 64 is dim d ^ 32, i.e. lane l ^ 32.
__device__ inline void norm_rope_wave(const float (&x)[4], const float (&wt)[4], uint32_t pos, int lane,
                                      uint16_t (&o)[4]) {
  float S[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int v = __builtin_bit_cast(int, row16_sum(x[k] * x[k]));
    S[k] = (__builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, 48)));
  }
  const float ss = (S[0] + S[1]) + (S[2] + S[3]);
  constexpr uint32_t half = kAttnRotary / 2;
  const uint32_t i = static_cast<uint32_t>(lane) & (half - 1);
  const float inv_freq = powf(kAttnTheta, -(2.0f * static_cast<float>(i)) / static_cast<float>(kAttnRotary));
  const float angle = static_cast<float>(pos) * inv_freq;
  const float c = cosf(angle);
  const float sn = sinf(angle);
  const float inv_rms = rsqrtf(ss / static_cast<float>(kAttnHeadDim) + kAttnEps);
  float n[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) n[k] = x[k] * inv_rms * wt[k];
  n[0] = round_bf(n[0]);  // dims [0, 64) rotate
  const float other = __shfl_xor(n[0], static_cast<int>(half), kWave);
  float r;
  if (static_cast<uint32_t>(lane) < half)
    r = n[0] * c - other * sn;
  else
    r = n[0] * c + other * sn;
  o[0] = f2bf(r);
#pragma unroll
  for (int k = 1; k < 4; ++k) o[k] = f2bf(n[k]);
}

// FRESH: the decode-step form (packed_q set). Every load that does not depend
// on the step scalars (q, the norm weights, the new tokens' k / v) is issued
// first, then the K / V tile of the split, all on straight-line code: behind
// a branch the compiler's wait at the join would also cover the loads issued
// before it, so q would be prepared only once the K / V tile had arrived.
// ROWS2: a two-token launch (the verify), whose row 1 takes row 0's new token
// as its last cached token; one-row launches compile without that path.
template <bool FRESH, bool ROWS2>
__global__ __launch_bounds__(kAttnThreads) void attn_partials_kernel(const AttnDecodeArgs a0) {
  extern __shared__ float sc[];  // [4][split_tokens + 2] scores, then probabilities
  __shared__ float mh[kAttnGroup], lh[kAttnGroup];
  // decode-step form: prepared q of the group's 4 heads, new tokens' k and v
  __shared__ uint16_t qf[kAttnGroup * kAttnHeadDim];
  __shared__ uint16_t kf[2 * kAttnHeadDim], vf[2 * kAttnHeadDim];
  const uint32_t row = ROWS2 ? blockIdx.z : 0u;
  const AttnDecodeArgs a = attn_row_args(a0, row);

  const uint32_t kvh = blockIdx.y;
  const uint32_t split = blockIdx.x;
  const uint32_t col = threadIdx.x;
  // Wave w prepares q head w of the group and, in the split that takes the
  // new tokens, new token w's k (lane l: dims l + 64k, with their norm
  // weights); thread col keeps the new tokens' v at dim col. Row 1 repeats
  // row 0 when the launch has one row.
  const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
  float xq[4] = {}, wq[4] = {}, xk[4] = {}, wk[4] = {};
  uint16_t vb[2] = {0, 0};
  if constexpr (FRESH) {
    const uint16_t* qsrc = a.packed_q + (static_cast<size_t>(kvh) * kAttnGroup + wv) * 2 * kAttnHeadDim;
    const uint32_t kr = min(static_cast<uint32_t>(wv), a0.rows - 1);
    const uint16_t* ksrc = a0.k_in + (static_cast<size_t>(kr) * kAttnKvHeads + kvh) * kAttnHeadDim;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      xq[k] = bf2f(qsrc[ln + 64 * k]);
      wq[k] = bf2f(a.q_norm[ln + 64 * k]);
      xk[k] = bf2f(ksrc[ln + 64 * k]);
      wk[k] = bf2f(a0.k_norm[ln + 64 * k]);
    }
#pragma unroll
    for (uint32_t j = 0; j < 2; ++j) {
      const uint32_t jr = min(j, a0.rows - 1);
      vb[j] = a0.v_in[(static_cast<size_t>(jr) * kAttnKvHeads + kvh) * kAttnHeadDim + col];
    }
  }
  // Row r partitions its own cached range [0, L_r), L_r = step[r].seq_len - 1,
  // exactly as a one-token step at its position would, so both rows of a
  // two-token launch equal single-token steps bit for bit (same splits, same
  // per-lane summation order).
  const uint32_t L = attn_cached_tokens(a);
  const uint32_t chunk = attn_chunk(L, a.nsplit);
  const uint32_t t0 = min(split * chunk, L);
  const uint32_t t1 = min(t0 + chunk, L);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float* part = a.partials + (static_cast<size_t>(kvh) * kAttnGroup * a.nsplit + split) * kAttnPartialStride;
  const size_t head_stride = static_cast<size_t>(a.nsplit) * kAttnPartialStride;
  // In the decode-step form the row's own new token is an extra token of the
  // split that holds its last cached token (split 0 on an empty cache). For
  // row 1 of a two-token launch that last cached token is row 0's new token:
  // its cache slot is being written by row 0's block in this same launch, so
  // it is taken from the k / v this block prepares (kf / vf row 0) in place
  // of the cache, at the same score index and lane slot (`virt`).
  constexpr bool fresh = FRESH;
  const uint32_t last = L == 0 ? 0u : (L - 1) / chunk;
  const bool in_last = fresh && split == last;
  const uint32_t nx = in_last ? 1u : 0u;        // the row's own new token
  const uint32_t nk = in_last ? row + 1 : 0u;   // new tokens whose k / v this block prepares
  const uint32_t nvirt = (ROWS2 && in_last) ? row : 0u;  // of them, cached tokens of this row

  if (t0 >= t1 && nx == 0) {  // empty range: neutral partial
    for (uint32_t i = threadIdx.x; i < kAttnGroup * kAttnPartialStride; i += kAttnThreads) {
      const uint32_t g = i / kAttnPartialStride, k = i % kAttnPartialStride;
      part[g * head_stride + k] = (k == 0) ? -INFINITY : 0.0f;
    }
    return;
  }
  const uint32_t T = t1 - t0;  // cached tokens of this split
  const uint32_t TX = T + nx;  // plus the new token
  const uint32_t Tc = T - nvirt;  // of them, read from the cache
  // split-local index of the cached token taken from vf row 0 (none: ~0u)
  const uint32_t vslot = nvirt ? T - 1 : ~0u;
  const uint32_t ld = a.split_tokens + 2;
  // A range of <= 64 tokens (every split of a cache up to 4096 tokens) issues
  // all of its K and V loads before any arithmetic: one memory round trip.
  const bool one_tile = T <= 64;
  const int jd = lane & 15, r = lane >> 4;
  const int rr = lane >> 3, ts = lane & 7;
  const uint16_t* kbase = a.key_cache + static_cast<size_t>(kvh) * a.stride * kAttnHeadDim + 16 * jd;
  const uint16_t* vbase = a.value_cache + (static_cast<size_t>(kvh) * kAttnHeadDim + 64 * w + rr) * a.stride;
  // The first 64-token K / V tile of the range (the whole range when T <= 64)
  // is loaded unconditionally: rows and tokens past T read clamped in-bounds
  // cache slots (which may hold anything) and are never used. Longer ranges
  // take it as their first tile.
  uint4 kt[4][2], vt[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t tt = min(t0 + 4 * w + r + 16 * i, a.stride - 1);
    const uint4* kp = reinterpret_cast<const uint4*>(kbase + static_cast<size_t>(tt) * kAttnHeadDim);
    kt[i][0] = kp[0];
    kt[i][1] = kp[1];
  }
  {
    const uint32_t tv = min(t0 + 8 * ts, a.stride - 8);
#pragma unroll
    for (int p = 0; p < 8; ++p)
      vt[p] = *reinterpret_cast<const uint4*>(vbase + static_cast<size_t>(8 * p) * a.stride + tv);
  }

  // ---- decode-step form: q of the group's 4 heads (one dim per thread, as
  // the prepare kernel computes it) and, in the split that takes them, the
  // new tokens' k (normalised + rotated) and v, appended to the cache by the
  // block of their own row.
  uint32_t qd[kAttnGroup][8];
  if constexpr (FRESH) {
    // positions of the new tokens (row 1 repeats row 0 when there is one row)
    uint32_t npos[2], ncpos[2];
#pragma unroll
    for (uint32_t j = 0; j < 2; ++j) {
      const uint32_t jr = min(j, a0.rows - 1);
      npos[j] = a0.step ? a0.step[jr].rope_pos : a0.rope_pos_host + j;
      ncpos[j] = a0.step ? a0.step[jr].cache_pos : a0.cache_pos_host + j;
    }
    {
      uint16_t o[4];
      norm_rope_wave(xq, wq, a.step ? a.step->rope_pos : a.rope_pos_host, ln, o);
#pragma unroll
      for (int k = 0; k < 4; ++k) qf[wv * kAttnHeadDim + ln + 64 * k] = o[k];
    }
    // new token j = wv (wave-uniform guard; no loads behind it)
    const uint32_t j = static_cast<uint32_t>(wv);
    if (j < nk) {
      const uint32_t pj = j == 0 ? npos[0] : npos[1];
      const uint32_t cj = j == 0 ? ncpos[0] : ncpos[1];
      uint16_t o[4];
      norm_rope_wave(xk, wk, pj, ln, o);
#pragma unroll
      for (int k = 0; k < 4; ++k) kf[j * kAttnHeadDim + ln + 64 * k] = o[k];
      if (j == row && cj < a.stride) {
        uint16_t* kdst = a.key_cache_w + (static_cast<size_t>(kvh) * a.stride + cj) * kAttnHeadDim;
#pragma unroll
        for (int k = 0; k < 4; ++k) kdst[ln + 64 * k] = o[k];
      }
    }
#pragma unroll
    for (uint32_t jj = 0; jj < 2; ++jj) {
      if (jj < nk) {
        vf[jj * kAttnHeadDim + col] = vb[jj];
        if (jj == row && ncpos[jj] < a.stride)
          a.value_cache_w[(static_cast<size_t>(kvh) * kAttnHeadDim + col) * a.stride + ncpos[jj]] = vb[jj];
      }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < static_cast<int>(kAttnGroup); ++g) {
      const uint4* qp = reinterpret_cast<const uint4*>(qf + g * kAttnHeadDim + 16 * jd);
      const uint4 q0 = qp[0], q1 = qp[1];
      qd[g][0] = q0.x; qd[g][1] = q0.y; qd[g][2] = q0.z; qd[g][3] = q0.w;
      qd[g][4] = q1.x; qd[g][5] = q1.y; qd[g][6] = q1.z; qd[g][7] = q1.w;
    }
  } else {
#pragma unroll
    for (int g = 0; g < static_cast<int>(kAttnGroup); ++g) {
      const uint4* qp =
          reinterpret_cast<const uint4*>(a.q + (static_cast<size_t>(kvh) * kAttnGroup + g) * kAttnHeadDim + 16 * jd);
      const uint4 q0 = qp[0], q1 = qp[1];
      qd[g][0] = q0.x; qd[g][1] = q0.y; qd[g][2] = q0.z; qd[g][3] = q0.w;
      qd[g][4] = q1.x; qd[g][5] = q1.y; qd[g][6] = q1.z; qd[g][7] = q1.w;
    }
  }

  // ---- phase 1: scores. lane -> (token row r = lane/16, dims 16*jd .. +16)
  auto score = [&](uint32_t tt, uint4 k0, uint4 k1, bool valid) {
    const uint32_t kd[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    float s[kAttnGroup];
#pragma unroll
    for (int g = 0; g < static_cast<int>(kAttnGroup); ++g) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = dot2(qd[g][i], kd[i], acc);
      s[g] = row16_sum(acc);
    }
    if (valid && jd == 0) {
#pragma unroll
      for (int g = 0; g < static_cast<int>(kAttnGroup); ++g) sc[g * ld + tt] = s[g] * a.scale;
    }
  };
  if (one_tile) {
    // rows past T compute on zeros and store nothing (row16_sum stays row-local)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t tt = 4 * w + r + 16 * i;
      if (4 * w + 16 * i < T) score(tt, kt[i][0], kt[i][1], tt < Tc);
    }
  } else {
    // The first 64 tokens (all read from the cache: T > 64, so Tc >= 64)
    // from the preloaded tile.
#pragma unroll
    for (int i = 0; i < 4; ++i) score(4 * w + r + 16 * i, kt[i][0], kt[i][1], true);
    // Four tokens per lane per pass: all eight K loads are issued before the
    // first dot product, so a wave keeps 8 KiB of K in flight.
    uint32_t tt = 4 * w + r + 64;
    for (; tt + 48 < T; tt += 64) {
      uint4 k4[4][2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4* kp = reinterpret_cast<const uint4*>(kbase + static_cast<size_t>(t0 + tt + 16 * i) * kAttnHeadDim);
        k4[i][0] = kp[0];
        k4[i][1] = kp[1];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) score(tt + 16 * i, k4[i][0], k4[i][1], tt + 16 * i < Tc);
    }
    for (; tt < T; tt += 16) {
      const uint4* kp = reinterpret_cast<const uint4*>(kbase + static_cast<size_t>(t0 + tt) * kAttnHeadDim);
      score(tt, kp[0], kp[1], tt < Tc);
    }
  }
  // The tokens prepared here (the cached virtual one, then the row's own new
  // token): 16-lane row j of wave 0 scores kf row j at index Tc + j. The
  // cache pass above stored nothing at those indices.
  if (nk > 0 && w == 0 && static_cast<uint32_t>(r) < nk) {
    const uint4* kp = reinterpret_cast<const uint4*>(kf + r * kAttnHeadDim + 16 * jd);
    score(Tc + r, kp[0], kp[1], true);
  }
  // The first two 64-token V tiles do not depend on the softmax: their loads
  // are issued here, so they stream in while phase 2 runs.
  const bool vpre = !one_tile && Tc >= 128;
  uint4 v2[2][8];
  auto load_v2 = [&](uint32_t tb, bool first) {  // first: tile 0 is the preloaded one
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int p = 0; p < 8; ++p)
        v2[h][p] = (first && h == 0) ? vt[p]
                                     : *reinterpret_cast<const uint4*>(vbase + static_cast<size_t>(8 * p) * a.stride +
                                                                       t0 + tb + 64 * h + 8 * ts);
  };
  if (vpre) load_v2(0, true);
  // The virtual cached token's value bits (vf row 0) replace what lane ts
  // read from its cache slot, which row 0's block is writing in this launch:
  // same lane, same element, so the summation order is a one-token step's.
  // Branch-free bit merge on the packed words: the mask selects the 16-bit
  // half of word c that holds the virtual token (element e of the lane's 8
  // tokens; e >= 8 in the other lanes, whose words stay as loaded).
  auto patch_virt = [&](uint32_t (&vd)[4], uint32_t e, int p) {
    const uint32_t bits = vf[64 * w + 8 * p + rr];
    const uint32_t dup = bits | (bits << 16);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t m = (e == static_cast<uint32_t>(2 * c) ? 0x0000FFFFu : 0u) |
                         (e == static_cast<uint32_t>(2 * c + 1) ? 0xFFFF0000u : 0u);
      vd[c] = (vd[c] & ~m) | (dup & m);
    }
  };
  __syncthreads();

  // ---- phase 2: softmax statistics, wave g owns head g.
  {
    const int g = w;
    float m = -INFINITY;
    for (uint32_t t = lane; t < TX; t += 64) m = fmaxf(m, sc[g * ld + t]);
    m = wave_max_dpp(m);
    float l = 0.0f;
    for (uint32_t t = lane; t < TX; t += 64) {
      const float s = sc[g * ld + t];
      const float p = (s == -INFINITY) ? 0.0f : expf(s - m);
      sc[g * ld + t] = p;
      l += p;
    }
    l = wave_sum_dpp(l);
    if (lane == 0) {
      mh[g] = m;
      lh[g] = l;
    }
  }
  __syncthreads();

  // ---- phase 3: P.V. wave w owns dims [64w, 64w+64): 8 passes x 8 rows.
  float acc[8][kAttnGroup];
#pragma unroll
  for (int p = 0; p < 8; ++p)
#pragma unroll
    for (int g = 0; g < static_cast<int>(kAttnGroup); ++g) acc[p][g] = 0.0f;
  uint32_t tb0 = 0;
  if (!one_tile) {
    // Two full 64-token tiles per pass: all sixteen V loads are issued before
    // the first FMA, so a wave keeps 16 KiB of V in flight. The tiles before
    // the virtual token only: each acc[p][g] sums its tiles in the same order
    // here and in the one-tile loop below, so where a pass ends changes no bits.
    for (; tb0 + 128 <= Tc; tb0 += 128) {
      if (tb0 > 0) load_v2(tb0, false);  // the first pair was loaded before phase 2
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t tl = tb0 + 64 * h + 8 * ts;
        float pv[kAttnGroup][8];
#pragma unroll
        for (int g = 0; g < static_cast<int>(kAttnGroup); ++g)
#pragma unroll
          for (int i = 0; i < 8; ++i) pv[g][i] = sc[g * ld + tl + i];
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const uint32_t vd[4] = {v2[h][p].x, v2[h][p].y, v2[h][p].z, v2[h][p].w};
          float v8[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v8[2 * i] = bf_lo(vd[i]);
            v8[2 * i + 1] = bf_hi(vd[i]);
          }
#pragma unroll
          for (int g = 0; g < static_cast<int>(kAttnGroup); ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[p][g] += pv[g][i] * v8[i];
        }
      }
    }
  }
  for (uint32_t tb = tb0; tb < T; tb += 64) {
    const uint32_t tl = tb + 8 * ts;  // first of this lane's 8 tokens (block-local)
    if (tl >= T) continue;
    const uint32_t nvalid = min(8u, T - tl);
    const bool vtile = ROWS2 && (vslot - tb) < 64u;  // wave-uniform
    float pv[kAttnGroup][8];
#pragma unroll
    for (int g = 0; g < static_cast<int>(kAttnGroup); ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) pv[g][i] = (static_cast<uint32_t>(i) < nvalid) ? sc[g * ld + tl + i] : 0.0f;
    uint4 vv[8];
    if (tb == 0) {  // the preloaded first tile
#pragma unroll
      for (int p = 0; p < 8; ++p) vv[p] = vt[p];
    } else {
#pragma unroll
      for (int p = 0; p < 8; ++p)
        vv[p] = *reinterpret_cast<const uint4*>(vbase + static_cast<size_t>(8 * p) * a.stride + t0 + tl);
    }
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      uint32_t vd[4] = {vv[p].x, vv[p].y, vv[p].z, vv[p].w};
      if constexpr (ROWS2)
        if (vtile) patch_virt(vd, vslot - tl, p);
      float v8[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v8[2 * i] = bf_lo(vd[i]);
        v8[2 * i + 1] = bf_hi(vd[i]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (static_cast<uint32_t>(i) >= nvalid) v8[i] = 0.0f;  // slots past seq_len may hold anything
#pragma unroll
      for (int g = 0; g < static_cast<int>(kAttnGroup); ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[p][g] += pv[g][i] * v8[i];
    }
  }
  if (nx > 0 && ts == 0) {  // the row's own new token (vf row nk - 1, score index T), once per dim
    const uint16_t* vown = vf + (nk - 1) * kAttnHeadDim + 64 * w + rr;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const float vv = bf2f(vown[8 * p]);
#pragma unroll
      for (int g = 0; g < static_cast<int>(kAttnGroup); ++g) acc[p][g] += sc[g * ld + T] * vv;
    }
  }
#pragma unroll
  for (int p = 0; p < 8; ++p)
#pragma unroll
    for (int g = 0; g < static_cast<int>(kAttnGroup); ++g) acc[p][g] = row8_sum(acc[p][g]);
  if (ts == 0) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const uint32_t d = 64 * w + 8 * p + rr;
#pragma unroll
      for (int g = 0; g < static_cast<int>(kAttnGroup); ++g) part[g * head_stride + 2 + d] = acc[p][g];
    }
  }
  if (threadIdx.x < kAttnGroup) {
    part[threadIdx.x * head_stride + 0] = mh[threadIdx.x];
    part[threadIdx.x * head_stride + 1] = lh[threadIdx.x];
  }
}

// -------------------------------------------------------------------- merge --
// Block (head h, quarter qt, row r) of 64 threads; thread t owns output dim
// d = 64 qt + t. The split statistics (m, denom) are merged first (weights
// in LDS), then each thread sums its dim over the splits with independent
// loads, and applies the sigmoid gate (from packed q in the decode-step form).
constexpr uint32_t kMaxSplits = 1024;
constexpr int kMergeThreads = 64;


__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(const AttnDecodeArgs a0) {
  __shared__ float wsh[kMaxSplits];
  const uint32_t row = blockIdx.z;
  const AttnDecodeArgs a = attn_row_args(a0, row);
  const uint32_t h = blockIdx.x, qt = blockIdx.y, t = threadIdx.x;
  const uint32_t d = 64 * qt + t;
  const bool fresh = a0.packed_q != nullptr;
  const float* base = a.partials + static_cast<size_t>(h) * a.nsplit * kAttnPartialStride;
  const uint16_t* gsrc = fresh ? a.packed_q + static_cast<size_t>(h) * 2 * kAttnHeadDim + kAttnHeadDim
                               : a.gate + static_cast<size_t>(h) * kAttnHeadDim;
  const uint16_t gbits = gsrc[d];
  constexpr uint32_t kPre = 64;
  float acc = 0.0f, den;
  if (a.nsplit <= kPre) {
    // Every split, read up front: a split without tokens holds the neutral
    // partial (m = -inf, denominator and accumulators 0), which adds exact
    // zeros, so no sequence length (a dependent load) is needed first.
    float pre[kPre];
#pragma unroll
    for (uint32_t c = 0; c < kPre; ++c) pre[c] = c < a.nsplit ? base[c * kAttnPartialStride + 2 + d] : 0.0f;
    const float mc = t < a.nsplit ? base[t * kAttnPartialStride] : -INFINITY;
    const float lc = t < a.nsplit ? base[t * kAttnPartialStride + 1] : 0.0f;
    const float m_all = wave_max_dpp(mc);
    const float wgt = (mc == -INFINITY) ? 0.0f : expf(mc - m_all);
    wsh[t] = wgt;
    den = wave_sum_dpp(lc * wgt);
    __syncthreads();  // wsh
#pragma unroll
    for (uint32_t c = 0; c < kPre; ++c)
      if (c < a.nsplit) acc += pre[c] * wsh[c];
  } else {
    // splits holding tokens (on an empty cache, split 0 holds the new tokens)
    const uint32_t L = attn_cached_tokens(a);  // this row's partition
    uint32_t nact = fresh ? 1u : 0u;
    if (L > 0) {
      const uint32_t chunk = attn_chunk(L, a.nsplit);
      nact = min(a.nsplit, (L + chunk - 1) / chunk);
    }
    float pre[kPre];
#pragma unroll
    for (uint32_t c = 0; c < kPre; ++c) pre[c] = c < nact ? base[c * kAttnPartialStride + 2 + d] : 0.0f;
    float m_local = -INFINITY;
    for (uint32_t c = t; c < nact; c += kMergeThreads) m_local = fmaxf(m_local, base[c * kAttnPartialStride]);
    const float m_all = wave_max_dpp(m_local);
    float den_local = 0.0f;
    for (uint32_t c = t; c < nact; c += kMergeThreads) {
      const float mc = base[c * kAttnPartialStride];
      const float wgt = (mc == -INFINITY) ? 0.0f : expf(mc - m_all);
      wsh[c] = wgt;
      den_local += base[c * kAttnPartialStride + 1] * wgt;
    }
    den = wave_sum_dpp(den_local);
    __syncthreads();  // wsh
#pragma unroll
    for (uint32_t c = 0; c < kPre; ++c)
      if (c < nact) acc += pre[c] * wsh[c];
#pragma unroll 8
    for (uint32_t c = kPre; c < nact; ++c) acc += base[c * kAttnPartialStride + 2 + d] * wsh[c];
  }
  const size_t i = static_cast<size_t>(h) * kAttnHeadDim + d;
  const float sig = 1.0f / (1.0f + expf(-bf2f(gbits)));
  a.out[i] = f2bf((acc / den) * sig);
}

}  // namespace

namespace prg {

// Most tokens one split may hold; PEREGRINE_ATTN_SPLIT_TOKENS overrides it
// (a power of two from 64 to 4096) for tuning.
static uint32_t attn_max_split_tokens() {
  static const uint32_t v = [] {
    const char* e = getenv("PEREGRINE_ATTN_SPLIT_TOKENS");
    const long t = e ? atol(e) : 0;
    return (t >= 64 && t <= 4096 && (t & (t - 1)) == 0) ? static_cast<uint32_t>(t) : 1024u;
  }();
  return v;
}

// Fewest splits per kv head; PEREGRINE_ATTN_MIN_SPLITS (a power of two,
// 16..256) overrides it for tuning.
static uint32_t attn_min_splits() {
  static const uint32_t v = [] {
    const char* e = getenv("PEREGRINE_ATTN_MIN_SPLITS");
    const long t = e ? atol(e) : 0;
    return (t >= 16 && t <= 256 && (t & (t - 1)) == 0) ? static_cast<uint32_t>(t) : 64u;
  }();
  return v;
}

uint32_t attn_num_splits(uint32_t capacity) {
  // >= attn_min_splits() splits per kv head (256 blocks by default) and
  // <= attn_max_split_tokens() per split.
  const uint32_t cap = attn_max_split_tokens();
  uint32_t n = attn_min_splits();
  while ((capacity + n - 1) / n > cap && n < kMaxSplits) n *= 2;
  return n;
}

uint32_t attn_split_tokens(uint32_t capacity, uint32_t nsplit) { return attn_chunk(capacity, nsplit); }

int launch_attn_prepare(hipStream_t s, const AttnPrepareArgs& a) {
  if (a.rows < 1 || a.rows > 2 || (a.rows == 2 && a.step == nullptr))
    return set_error(PRG_ERR_INVALID_ARG, "attn_prepare: rows %u (two rows need device step scalars)", a.rows);
  hipLaunchKernelGGL(attn_prepare_kernel, dim3(kAttnQHeads + kAttnKvHeads, a.rows), dim3(kAttnThreads), 0, s, a);
  PRG_CHECK_LAUNCH("attn_prepare");
  return PRG_OK;
}

int launch_attn_decode(hipStream_t s, const AttnDecodeArgs& a) {
  if (a.rows < 1 || a.rows > 2 || (a.rows == 2 && a.step == nullptr))
    return set_error(PRG_ERR_INVALID_ARG, "attn_decode: rows %u (two rows need device step scalars)", a.rows);
  if (a.packed_q && !(a.q_norm && a.k_in && a.v_in && a.k_norm && a.key_cache_w && a.value_cache_w))
    return set_error(PRG_ERR_INVALID_ARG, "attn_decode: the decode-step form needs every input");
  const size_t lds = static_cast<size_t>(kAttnGroup) * (a.split_tokens + 2) * sizeof(float);
  void (*partials)(const AttnDecodeArgs) =
      a.packed_q ? (a.rows == 2 ? attn_partials_kernel<true, true> : attn_partials_kernel<true, false>)
                 : (a.rows == 2 ? attn_partials_kernel<false, true> : attn_partials_kernel<false, false>);
  hipLaunchKernelGGL(partials, dim3(a.nsplit, kAttnKvHeads, a.rows), dim3(kAttnThreads), lds, s, a);
  PRG_CHECK_LAUNCH("attn_partials");
  hipLaunchKernelGGL(attn_merge_kernel, dim3(kAttnQHeads, kAttnHeadDim / kMergeThreads, a.rows), dim3(kMergeThreads),
                     0, s, a);
  PRG_CHECK_LAUNCH("attn_merge");
  return PRG_OK;
}

// ------------------------------------------------------- allocation-free --
// Partials of prg_attn_decode_noalloc_bf16 live in this file-scope device
// array: each GPU holds its own copy (4,227,072 bytes: 16 q heads x 256
// splits x 258 floats, i.e. caches of up to 256 splits, 262144 tokens at the
// default 1024 tokens per split) until the process ends. Host code must not
// pass `scratch` itself to a kernel: its device address is looked up once
// per device (attn_noalloc_setup) and kept in g_scratch.
constexpr uint32_t kNoAllocMaxSplits = 256;
constexpr size_t kNoAllocFloats = static_cast<size_t>(kAttnQHeads) * kNoAllocMaxSplits * kAttnPartialStride;
static __device__ __align__(256) float scratch[kNoAllocFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device (set up on first use).
int noalloc_scratch(float** out) {
  int dev = 0;
  PRG_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(PRG_ERR_INVALID_ARG, "allocation-free attention: device %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(PRG_ERR_HIP, "allocation-free attention: hipGetSymbolAddress: %s", hipGetErrorString(e));
    g_scratch[dev] = static_cast<float*>(p);
  }
  *out = g_scratch[dev];
  return PRG_OK;
}
}  // namespace

int attn_noalloc_setup() {
  float* p = nullptr;
  return noalloc_scratch(&p);
}

// Shared by the decode-attention entry points: argument checks, then the
// partials + merge launches with `partials` as the workspace.
static int attn_decode_entry(const char* name, void* stream, const uint16_t* q, const uint16_t* key_cache,
                             const uint16_t* value_cache, const uint16_t* gate, uint16_t* out, float* partials,
                             uint32_t cache_stride_tokens, uint32_t seq_len, float scale) {
  PRG_CHECK_ARG(q && key_cache && value_cache && gate && out && partials, "%s: null pointer", name);
  PRG_CHECK_ARG(cache_stride_tokens % 64 == 0, "%s: stride %u must be a multiple of 64", name, cache_stride_tokens);
  if (seq_len == 0 || seq_len > cache_stride_tokens)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "%s: seq_len %u outside (0, %u]", name, seq_len,
                     cache_stride_tokens);
  AttnDecodeArgs a{};
  a.q = q;
  a.key_cache = key_cache;
  a.value_cache = value_cache;
  a.gate = gate;
  a.out = out;
  a.partials = partials;
  a.stride = cache_stride_tokens;
  a.nsplit = attn_num_splits(cache_stride_tokens);
  a.split_tokens = attn_split_tokens(cache_stride_tokens, a.nsplit);
  a.seq_len_host = seq_len;
  a.step = nullptr;
  a.scale = scale;
  return launch_attn_decode(as_stream(stream), a);
}

}  // namespace prg

extern "C" {

int prg_attn_decode_prepare_bf16(void* stream, const uint16_t* packed_q, const uint16_t* q_weight,
                                 uint16_t* q_output, uint16_t* gate, const uint16_t* k_input,
                                 const uint16_t* v_input, const uint16_t* k_weight,
                                 uint16_t* key_cache, uint16_t* value_cache,
                                 uint32_t cache_stride_tokens, uint32_t dst_token_index,
                                 uint32_t position_offset) {
  PRG_CHECK_ARG(packed_q && q_weight && q_output && gate && k_input && v_input && k_weight && key_cache && value_cache,
                "prg_attn_decode_prepare_bf16: null pointer");
  if (dst_token_index >= cache_stride_tokens)
    return prg::set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prg_attn_decode_prepare_bf16: dst %u >= stride %u",
                          dst_token_index, cache_stride_tokens);
  prg::AttnPrepareArgs a{packed_q, q_weight, k_input, v_input, k_weight, q_output, gate, key_cache, value_cache,
                         cache_stride_tokens, dst_token_index, position_offset, nullptr};
  return prg::launch_attn_prepare(prg::as_stream(stream), a);
}

int prg_attn_decode_bf16(void* stream, const uint16_t* q, const uint16_t* key_cache,
                         const uint16_t* value_cache, const uint16_t* gate, uint16_t* out,
                         float* partials, uint32_t cache_stride_tokens, uint32_t seq_len,
                         float scale) {
  return prg::attn_decode_entry("prg_attn_decode_bf16", stream, q, key_cache, value_cache, gate, out, partials,
                                cache_stride_tokens, seq_len, scale);
}

int prg_attn_decode_noalloc_bf16(void* stream, const uint16_t* q, const uint16_t* key_cache,
                                 const uint16_t* value_cache, const uint16_t* gate, uint16_t* out,
                                 uint32_t cache_stride_tokens, uint32_t seq_len, float scale) {
  const char* name = "prg_attn_decode_noalloc_bf16";
  PRG_CHECK_ARG(cache_stride_tokens > 0, "%s: stride 0", name);
  const uint32_t nsplit = prg::attn_num_splits(cache_stride_tokens);
  if (nsplit > prg::kNoAllocMaxSplits)
    return prg::set_error(PRG_ERR_INVALID_ARG,
                          "%s: a cache of %u tokens needs %u splits (%zu partial bytes); this entry holds %u splits "
                          "(%zu bytes)",
                          name, cache_stride_tokens, nsplit, prg_attn_decode_partials_bytes(cache_stride_tokens),
                          prg::kNoAllocMaxSplits, prg::kNoAllocFloats * sizeof(float));
  float* partials = nullptr;
  if (int rc = prg::noalloc_scratch(&partials)) return rc;
  return prg::attn_decode_entry(name, stream, q, key_cache, value_cache, gate, out, partials, cache_stride_tokens,
                                seq_len, scale);
}

size_t prg_attn_decode_partials_bytes(uint32_t cache_stride_tokens) {
  const uint32_t n = prg::attn_num_splits(cache_stride_tokens);
  return static_cast<size_t>(prg::kAttnQHeads) * n * prg::kAttnPartialStride * sizeof(float);
}

size_t prg_attn_decode_step_workspace_bytes(uint32_t cache_stride_tokens) {
  return prg_attn_decode_partials_bytes(cache_stride_tokens);
}

int prg_attn_decode_step_bf16(void* stream, const uint16_t* packed_q, const uint16_t* q_weight,
                              const uint16_t* k_input, const uint16_t* v_input, const uint16_t* k_weight,
                              uint16_t* key_cache, uint16_t* value_cache, uint16_t* out, void* workspace,
                              uint32_t cache_stride_tokens, uint32_t cache_pos, uint32_t rope_pos, float scale) {
  const char* name = "prg_attn_decode_step_bf16";
  PRG_CHECK_ARG(packed_q && q_weight && k_input && v_input && k_weight && key_cache && value_cache && out && workspace,
                "%s: null pointer", name);
  PRG_CHECK_ARG(cache_stride_tokens % 64 == 0, "%s: stride %u must be a multiple of 64", name, cache_stride_tokens);
  if (cache_pos >= cache_stride_tokens)
    return prg::set_error(PRG_ERR_SEQUENCE_TOO_LONG, "%s: cache_pos %u >= stride %u", name, cache_pos,
                          cache_stride_tokens);
  prg::AttnDecodeArgs a{};
  a.partials = static_cast<float*>(workspace);
  a.key_cache = a.key_cache_w = key_cache;
  a.value_cache = a.value_cache_w = value_cache;
  a.out = out;
  a.stride = cache_stride_tokens;
  a.nsplit = prg::attn_num_splits(cache_stride_tokens);
  a.split_tokens = prg::attn_split_tokens(cache_stride_tokens, a.nsplit);
  a.seq_len_host = cache_pos + 1;
  a.cache_pos_host = cache_pos;
  a.rope_pos_host = rope_pos;
  a.scale = scale;
  a.packed_q = packed_q;
  a.q_norm = q_weight;
  a.k_in = k_input;
  a.v_in = v_input;
  a.k_norm = k_weight;
  return prg::launch_attn_decode(prg::as_stream(stream), a);
}

}  // extern "C"
