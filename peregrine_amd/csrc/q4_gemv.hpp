// Q4 GEMV family for gfx950 — shared kernel template and launch parameters.
//
// Math (MLX affine 4-bit, group 64; reference shaders/linear.metal:12-19):
//   y[n] = sum_k x[k] * (s[n, k/64] * q[n, k] + b[n, k/64])
// factored per 32-value half-group as s * sum(q*x) + b * sum(x), as the
// reference does per 16-value lane chunk (shaders/linear_decode.metal:33-69).
//
// gfx950 design:
//   * 256-thread blocks = 4 wave64s; each wave owns ROWS consecutive output
//     rows of each weight matrix and sweeps the whole K range.
//   * Lane l reads 16 contiguous bytes (dwordx4 = 32 nibbles) per row per
//     2048-wide K step, so one wave load covers 1 KiB of a row, fully
//     coalesced. All ROWS x ITERS weight loads are issued up front.
//   * Dequant stays in registers: a nibble pair is OR-ed into the mantissa
//     of two bf16 lanes (0x4300 | q == 128 + q exactly) and multiplied with the
//     matching activation pair by v_dot2c_f32_bf16 with fp32 accumulation;
//     the 128*sum(x) offset is removed once per half-group.
//   * x is staged once per block in LDS, pre-permuted so that the pair
//     (x[8j+i], x[8j+i+4]) lines up with nibbles i and i+4 of word j.
//     An optional fused RMSNorm prologue normalises x while staging it.
//   * Partial sums are reduced across the wave with DPP row ops + readlane.
//   * Up to 4 independent weight matrices ("segments") that share x run in
//     one launch (e.g. in_proj qkv | z | a | b), cutting launches per layer.
#pragma once

#include "common.hpp"
#include "norm.hpp"
#include "gdn.hpp"

namespace prg {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kGemvKStep = 2048;  // K values one wave consumes per step
constexpr int kGemvMaxIters = 8;  // in_dim <= 16384
constexpr int kGemvMaxSegs = 4;

enum GemvEpi : int {
  kEpiPlain = 0,     // out = bf16(dot)
  kEpiResidual = 1,  // out = bf16(float(bf16(dot)) + float(res))
  kEpiSiluGate = 2,  // out = bf16(silu(bf16(gate)) * bf16(up))   (two matrices)
  kEpiArgmax = 3,    // per 8 rows: first strict max of bf16(dot) -> partial
};

struct GemvSeg {
  const uint32_t* w[2];  // matrix 0 (and 1 = up for silu-gate)
  const uint16_t* s[2];
  const uint16_t* b[2];
  uint16_t* out[2];           // per activation row m
  const uint16_t* res[2];     // per activation row m (residual epilogue)
  float* pval[2];             // per activation row m (argmax epilogue)
  uint32_t* pidx[2];
  // Optional conv1d+SiLU epilogue (plain epilogue, M == 1): the bf16 GEMV
  // output x of row c feeds the depthwise causal conv of channel c, whose f32
  // state [3, conv_dim] is rolled in place; out receives the conv output.
  // This fuses in_proj_qkv with conv1d_silu_decode_bf16 (block_linear.zig:230-240).
  float* conv_state;
  const uint16_t* conv_w;     // bf16 [conv_dim, 4]
  uint32_t conv_dim;
  uint32_t rows;              // output rows of this segment
  uint32_t block_begin;       // first block index of this segment
};

struct GemvParams {
  GemvSeg seg[kGemvMaxSegs];
  const uint16_t* x[2];       // activation rows (M of them)
  const uint16_t* norm_w;     // fused RMSNorm weight (NORM variants)
  float eps;
  uint32_t K;
  uint32_t nseg;
  uint32_t tail_lanes;        // active lanes in the last K step (64 if full)
};

// ------------------------------------------------------------ device ---------
__device__ inline float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Sum of a float over all 64 lanes; the result is wave-uniform. Lanes of a
// 16-lane row are combined with DPP (quad_perm, half-mirror, mirror), after
// which all 16 hold the same bits; the 4 row sums are read with readlane.
__device__ inline float wave_sum_uniform(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  const int iv = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
  return (r0 + r1) + (r2 + r3);
}

// 8 bf16 (as a uint4 of pairs (x0,x1),(x2,x3),(x4,x5),(x6,x7)) ->
// dot2 order (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ inline uint4 permute_pairs(uint4 v) {
  uint4 o;
  o.x = (v.x & 0xffffu) | (v.z << 16);
  o.y = (v.x >> 16) | (v.z & 0xffff0000u);
  o.z = (v.y & 0xffffu) | (v.w << 16);
  o.w = (v.y >> 16) | (v.w & 0xffff0000u);
  return o;
}

// Stage the M activation rows into LDS (permuted pairs). With NORM, each row
// is RMS-normalised first: out = bf16(x * rsqrt(mean(x^2) + eps) * w), the
// rmsnorm_bf16 formula (reference shaders/rmsnorm.metal:80-116).
template <int M, bool NORM>
__device__ inline void gemv_stage_x(const GemvParams& p, uint32_t* xs, float* red) {
  const uint32_t n8 = p.K / 8;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint4* src = reinterpret_cast<const uint4*>(p.x[m]);
    uint4* dst = reinterpret_cast<uint4*>(xs + m * (p.K / 2));
    if constexpr (NORM) {
      static_assert(kGemvThreads == kNormThreads, "fused norm shares the standalone reduction");
      const float scale = rms_scale(src, n8, p.K, p.eps, red);
      const uint4* wsrc = reinterpret_cast<const uint4*>(p.norm_w);
      for (uint32_t g = threadIdx.x; g < n8; g += kGemvThreads)
        dst[g] = permute_pairs(rms_apply(src[g], wsrc[g], scale));
    } else {
      for (uint32_t g = threadIdx.x; g < n8; g += kGemvThreads) dst[g] = permute_pairs(src[g]);
    }
  }
}

template <int M, int ROWS, int ITERS, int EPI, bool NORM>
__global__ __launch_bounds__(kGemvThreads) void q4_gemv_kernel(const GemvParams p) {
  constexpr int NMAT = (EPI == kEpiSiluGate) ? 2 : 1;
  extern __shared__ uint32_t xs[];  // [M][K/2] permuted bf16 pairs
  __shared__ float red[kGemvWaves];

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;

  // Segment lookup (uniform).
  const uint32_t bid = blockIdx.x;
  uint32_t si = 0;
  for (uint32_t i = 1; i < p.nseg; ++i)
    if (bid >= p.seg[i].block_begin) si = i;
  const GemvSeg& sg = p.seg[si];
  const uint32_t row0 = (bid - sg.block_begin) * (kGemvWaves * ROWS) + wid * ROWS;
  const uint32_t nrows = sg.rows;
  const uint32_t K = p.K;
  const uint32_t words_per_row = K / 8;
  const uint32_t groups = K / 64;
  const bool tail_active = lane < static_cast<int>(p.tail_lanes);

  // 1) issue every weight load for this wave's rows.
  u32x4 wv[NMAT][ROWS][ITERS];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const uint32_t row = min(row0 + r, nrows - 1);
      const u32x4* wp = reinterpret_cast<const u32x4*>(sg.w[mat] + static_cast<size_t>(row) * words_per_row) + lane;
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        if (it < ITERS - 1 || tail_active)
          wv[mat][r][it] = __builtin_nontemporal_load(wp + it * (kGemvKStep / 32));
        else
          wv[mat][r][it] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  // 2) stage activations (and the fused norm) while the loads are in flight.
  gemv_stage_x<M, NORM>(p, xs, red);
  __syncthreads();

  // 3) dequant + dot.
  float acc[NMAT][ROWS][M];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[mat][r][m] = 0.0f;

  constexpr uint32_t kMask = 0x000F000Fu;
  constexpr uint32_t kMagic = 0x43004300u;  // bf16 pair (128, 128)
  constexpr uint32_t kOnes = 0x3F803F80u;   // bf16 pair (1, 1)

#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    if (it == ITERS - 1 && !tail_active) break;
    uint32_t xp[M][16];
    float xsum[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4* xl = reinterpret_cast<const uint4*>(xs + m * (K / 2) + it * (kGemvKStep / 2) + lane * 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = xl[q];
        xp[m][4 * q + 0] = v.x;
        xp[m][4 * q + 1] = v.y;
        xp[m][4 * q + 2] = v.z;
        xp[m][4 * q + 3] = v.w;
      }
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) s = dot2_bf16(xp[m][j], kOnes, s);
      xsum[m] = s;
    }
    const uint32_t group = it * (kGemvKStep / 64) + (lane >> 1);
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        const uint32_t row = min(row0 + r, nrows - 1);
        const size_t meta = static_cast<size_t>(row) * groups + group;
        const float sc = bf2f(sg.s[mat][meta]);
        const float bi = bf2f(sg.b[mat][meta]);
        const u32x4 w4 = wv[mat][r][it];
        const uint32_t wd[4] = {w4[0], w4[1], w4[2], w4[3]};
        float aq[M];
#pragma unroll
        for (int m = 0; m < M; ++m) aq[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t word = wd[j];
          const uint32_t t0 = (word & kMask) | kMagic;
          const uint32_t t1 = ((word >> 4) & kMask) | kMagic;
          const uint32_t t2 = ((word >> 8) & kMask) | kMagic;
          const uint32_t t3 = ((word >> 12) & kMask) | kMagic;
#pragma unroll
          for (int m = 0; m < M; ++m) {
            aq[m] = dot2_bf16(t0, xp[m][4 * j + 0], aq[m]);
            aq[m] = dot2_bf16(t1, xp[m][4 * j + 1], aq[m]);
            aq[m] = dot2_bf16(t2, xp[m][4 * j + 2], aq[m]);
            aq[m] = dot2_bf16(t3, xp[m][4 * j + 3], aq[m]);
          }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float qx = aq[m] - 128.0f * xsum[m];  // sum(q * x)
          acc[mat][r][m] += sc * qx + bi * xsum[m];
        }
      }
    }
  }

  // 4) reduce across the wave and write.
  float tot[NMAT][ROWS][M];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) tot[mat][r][m] = wave_sum_uniform(acc[mat][r][m]);

  if (lane != 0) return;
  if constexpr (EPI == kEpiArgmax) {
    static_assert(ROWS == 8, "argmax partials cover 8 rows");
    if (row0 >= nrows) return;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float best = round_bf(tot[0][0][m]);
      uint32_t best_i = row0;
#pragma unroll
      for (int r = 1; r < ROWS; ++r) {
        const float v = round_bf(tot[0][r][m]);
        if (v > best) {
          best = v;
          best_i = row0 + r;
        }
      }
      sg.pval[m][row0 / 8] = best;
      sg.pidx[m][row0 / 8] = best_i;
    }
  } else {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const uint32_t row = row0 + r;
      if (row >= nrows) break;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        uint16_t o;
        if constexpr (EPI == kEpiPlain) {
          if (M == 1 && sg.conv_state != nullptr)
            o = conv1d_silu_step(sg.conv_state, sg.conv_w, sg.conv_dim, row, round_bf(tot[0][r][m]));
          else
            o = f2bf(tot[0][r][m]);
        } else if constexpr (EPI == kEpiResidual) {
          o = f2bf(round_bf(tot[0][r][m]) + bf2f(sg.res[m][row]));
        } else {
          const float g = round_bf(tot[0][r][m]);
          const float u = round_bf(tot[1][r][m]);
          o = f2bf(silu(g) * u);
        }
        sg.out[m][row] = o;
      }
    }
  }
}

// ------------------------------------------------------------- host ----------
// Launch one GEMV-family kernel. Segment block ranges are filled in here.
// Returns a PRG_ERR_* code.
int launch_q4_gemv(hipStream_t stream, GemvParams& p, int M, int rows_per_wave, int epi,
                   bool norm, const char* name);

// Rows per wave picked for a launch of `total_rows` rows at in_dim K.
int gemv_rows_per_wave(uint32_t total_rows, uint32_t K, int epi, int M);

// Final argmax over partials + advance of the device token loop.
int launch_argmax_advance(hipStream_t s, const float* values, const uint32_t* indices, uint32_t n,
                          DecodeCtl* ctl, const uint32_t* prompt, uint32_t* predictions);
// Advance with the next token forced from prompt (no lm_head this step).
int launch_advance_forced(hipStream_t s, DecodeCtl* ctl, const uint32_t* prompt);

}  // namespace prg
