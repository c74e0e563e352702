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
//   * Dequant stays in registers: v_perm_b32 places each nibble under the
//     byte 0x43 (bf16 0x43qq == 128 + q exactly), two per dword, and
//     v_dot2c_f32_bf16 multiplies them with the matching activation pair in
//     fp32; one of the two dot2 chains of a half-group starts at -128*sum(x),
//     which removes the offset.
//   * x is staged once per block in LDS, pre-permuted so each activation pair
//     lines up with the nibble pair the unpack produces.
//     An optional fused RMSNorm prologue normalises x while staging it.
//   * One-row-per-wave launches work in rounds of four groups: the four rows'
//     lane partials are reduced together (v_permlane32/16_swap halve the
//     lanes while trading rows, then a DPP row sum), and one lane per row runs
//     the epilogue. Multi-row launches reduce per row with DPP + readlane.
//   * Up to 4 independent weight matrices ("segments") that share x run in
//     one launch (e.g. in_proj qkv | z | a | b), cutting launches per layer.
#pragma once

#include <type_traits>

#include "common.hpp"
#include "norm.hpp"
#include "gdn.hpp"

namespace prg {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kGemvKStep = 2048;  // K values one wave consumes per step
constexpr int kGemvMaxIters = 8;  // in_dim <= 16384
constexpr int kGemvMaxSegs = 4;

// Prologue applied to x while it is staged.
enum GemvNorm : int {
  kNormNone = 0,
  kNormRms = 1,    // RMSNorm over the whole row with norm_w [K] (rmsnorm.metal:80-116)
  kNormGated = 2,  // per 128-wide head: RMSNorm with norm_w [128], times gz = silu(z) (gated_norm.metal:163-189)
};

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
  // Optional conv1d+SiLU epilogue (plain epilogue): the bf16 GEMV output x
  // of row c feeds the depthwise causal conv of channel c, whose f32 state
  // [3, conv_dim] is rolled; out receives the conv output. This fuses
  // in_proj_qkv with conv1d_silu_decode_bf16 (block_linear.zig:230-240).
  // M == 1: the rolled state goes to conv_state_out (nullptr: in place).
  // M == 2 (two consecutive tokens): the state after row 0 goes to
  // conv_state_out and the state after row 1 back to conv_state.
  float* conv_state;
  float* conv_state_out;
  const uint16_t* conv_w;     // bf16 [conv_dim, 4]
  uint32_t conv_dim;
  // Optional SiLU epilogue (plain epilogue): row c of activation row m
  // writes silu(bf16(dot)) in f32 to silu_out[m] instead of bf16 to out (the
  // GDN z gate).
  float* silu_out[2];
  // Decode-layout copies of w / s / b (q4_gemv_t16.hpp); null when absent.
  const uint32_t* tw[2];
  const uint16_t* ts[2];
  const uint16_t* tb[2];
  uint32_t rows;              // output rows of this segment
  uint32_t block_begin;       // first group index of this segment (set by the launcher)
};

struct GemvParams {
  GemvSeg seg[kGemvMaxSegs];
  const uint16_t* x[2];       // activation rows (M of them)
  const uint16_t* norm_w;     // fused RMSNorm weight (NORM variants)
  const float* gz[2];         // per activation row: silu(z) in f32 for kNormGated
  float eps;
  uint32_t K;
  uint32_t nseg;
  uint32_t tail_lanes;        // active lanes in the last K step (64 if full)
  uint32_t total_groups;      // groups of ROWS rows over all segments (set by the launcher)
  // kEpiArgmax: if set, each wave writes one entry (its best partial under the
  // final argmax's order) to pval / pidx[wave] instead of one per 8 rows, and
  // the launch's wave count goes here (the grid is capped at kArgmaxMaxWaves).
  uint32_t* argmax_waves;
  // If set, block 0 also writes activation row m as staged (normalised with
  // NORM, bf16 pairs in the dot order of unpack_q4_word: K / 2 dwords) to
  // x_image[m], for a consumer that needs the same normalised row.
  uint32_t* x_image[2];
};

constexpr uint32_t kArgmaxMaxWaves = 4096;

// The final argmax's order on partials (value, partial position p): among
// equal maxima the winner minimises (bitreverse8(p mod 256), p div 256), the
// effective order of the reference's 256-thread scan and halving tree
// (shaders/argmax.metal:6-43); NaN and -inf never win. A strict total order,
// so any reduction tree picks the same winner.
__device__ inline uint32_t argmax_tie_key(uint32_t p) {
  return ((__builtin_bitreverse32(p & 255u) >> 24) << 24) | (p >> 8);
}
__device__ inline bool argmax_better(float v, uint32_t p, float bv, uint32_t bp) {
  // true when (v, p) beats (bv, bp)
  if (!(v > -INFINITY)) return false;
  if (!(bv > -INFINITY)) return true;
  if (v > bv) return true;
  if (v < bv) return false;
  return argmax_tie_key(p) < argmax_tie_key(bp);
}

// ------------------------------------------------------------ device ---------
__device__ inline float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// 8 bf16 (as a uint4 of pairs (x0,x1),(x2,x3),(x4,x5),(x6,x7)) -> the dot2
// order of the nibble unpack below: (x0,x2),(x4,x6),(x1,x3),(x5,x7).
__device__ inline uint4 permute_pairs(uint4 v) {
  uint4 o;
  o.x = (v.x & 0xffffu) | (v.y << 16);
  o.y = (v.z & 0xffffu) | (v.w << 16);
  o.z = (v.x >> 16) | (v.y & 0xffff0000u);
  o.w = (v.z >> 16) | (v.w & 0xffff0000u);
  return o;
}

// Unpack one packed word (nibbles n0..n7, n0 lowest) into four bf16 pairs of
// the exact values 128 + q: (n0,n2), (n4,n6), (n1,n3), (n5,n7). The low and
// high nibbles are isolated as bytes, then v_perm_b32 interleaves each nibble
// byte with the byte 0x43 (bf16 0x43qq == 128 + q, q <= 15).
__device__ inline void unpack_q4_word(uint32_t word, uint32_t (&t)[4]) {
  constexpr uint32_t kHigh = 0x43434343u;
  const uint32_t lo = word & 0x0F0F0F0Fu;         // bytes n0 n2 n4 n6
  const uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;  // bytes n1 n3 n5 n7
  // selector byte k: 0..3 = byte of the 2nd operand, 4..7 = byte of kHigh
  t[0] = __builtin_amdgcn_perm(kHigh, lo, 0x04010400u);
  t[1] = __builtin_amdgcn_perm(kHigh, lo, 0x04030402u);
  t[2] = __builtin_amdgcn_perm(kHigh, hi, 0x04010400u);
  t[3] = __builtin_amdgcn_perm(kHigh, hi, 0x04030402u);
}

// Register buffer holding one group's weights for one wave: ROWS rows of each
// of NMAT matrices, ITERS K-steps, plus the matching scale and bias bits.
// Scale and bias stay in separate registers as loaded: combining them when
// the loads are issued would make the wave wait for the prefetched group's
// loads right away, i.e. one full memory latency per group.
template <int NMAT, int ROWS, int ITERS>
struct GemvBuf {
  u32x4 w[NMAT][ROWS][ITERS];
  uint16_t sc[NMAT][ROWS][ITERS];  // bf16 scale bits, widened where they are used
  uint16_t bi[NMAT][ROWS][ITERS];  // bf16 bias bits
};

// Where group g of the launch lives: segment index and first row.
struct GemvLoc {
  uint32_t seg;
  uint32_t row0;
};

template <int ROWS>
__device__ inline GemvLoc gemv_locate(const GemvParams& p, uint32_t g) {
  uint32_t si = 0;
  for (uint32_t i = 1; i < p.nseg; ++i)
    if (g >= p.seg[i].block_begin) si = i;
  return GemvLoc{si, (g - p.seg[si].block_begin) * ROWS};
}

template <int NMAT, int ROWS, int ITERS, bool TAIL>
__device__ inline void gemv_load(const GemvParams& p, uint32_t g, int lane, bool tail_active,
                                 GemvBuf<NMAT, ROWS, ITERS>& b) {
  const GemvLoc loc = gemv_locate<ROWS>(p, g);
  const GemvSeg& sg = p.seg[loc.seg];
  const uint32_t words_per_row = p.K / 8, groups = p.K / 64;
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const uint32_t row = min(loc.row0 + r, sg.rows - 1);
      const u32x4* wp = reinterpret_cast<const u32x4*>(sg.w[mat] + static_cast<size_t>(row) * words_per_row) + lane;
      const size_t meta = static_cast<size_t>(row) * groups + (lane >> 1);
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        if (!TAIL || it < ITERS - 1 || tail_active) {
          b.w[mat][r][it] = __builtin_nontemporal_load(wp + it * (kGemvKStep / 32));
          b.sc[mat][r][it] = sg.s[mat][meta + it * (kGemvKStep / 64)];
          b.bi[mat][r][it] = sg.b[mat][meta + it * (kGemvKStep / 64)];
        } else {
          b.w[mat][r][it] = u32x4{0u, 0u, 0u, 0u};
          b.sc[mat][r][it] = 0;
          b.bi[mat][r][it] = 0;
        }
      }
    }
  }
}

// Activation pairs of one lane for one K-step (16 dwords) + their sum.
template <int M>
struct XStep {
  uint32_t xp[M][16];
  float xsum[M];
  float xoff[M];  // -128 * xsum, exact: the 128 + q offset of the unpacked nibbles
};

template <int M>
__device__ inline void gemv_read_x(const uint32_t* xs, uint32_t K, int it, int lane, XStep<M>& x) {
  constexpr uint32_t kOnes = 0x3F803F80u;  // bf16 pair (1, 1)
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint4* xl = reinterpret_cast<const uint4*>(xs + m * (K / 2) + it * (kGemvKStep / 2) + lane * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 v = xl[q];
      x.xp[m][4 * q + 0] = v.x;
      x.xp[m][4 * q + 1] = v.y;
      x.xp[m][4 * q + 2] = v.z;
      x.xp[m][4 * q + 3] = v.w;
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s = dot2_bf16(x.xp[m][j], kOnes, s);
    x.xsum[m] = s;
    x.xoff[m] = -128.0f * s;
  }
}

// acc[mat][r][m] += s*sum(q*x) + b*sum(x) over this lane's 32 values of step it.
template <int M, int NMAT, int ROWS, int ITERS>
__device__ inline void gemv_dot_step(const GemvBuf<NMAT, ROWS, ITERS>& b, int it, const XStep<M>& x,
                                     float (&acc)[NMAT][ROWS][M]) {
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const u32x4 w4 = b.w[mat][r][it];
      const uint32_t wd[4] = {w4[0], w4[1], w4[2], w4[3]};
      // Two dot2 chains per activation row (the other matrices, rows and
      // K-steps give the scheduler more independent chains); the first starts
      // at -128 * sum(x), so the chains add up to sum(q * x) directly.
      float aq[M][2];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        aq[m][0] = x.xoff[m];
        aq[m][1] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t t[4];
        unpack_q4_word(wd[j], t);
#pragma unroll
        for (int m = 0; m < M; ++m) {
#pragma unroll
          for (int c = 0; c < 4; ++c) aq[m][c & 1] = dot2_bf16(t[c], x.xp[m][4 * j + c], aq[m][c & 1]);
        }
      }
      const float sc = bf_lo(static_cast<uint32_t>(b.sc[mat][r][it]));
      const float bi = bf_lo(static_cast<uint32_t>(b.bi[mat][r][it]));
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float qx = aq[m][0] + aq[m][1];  // sum(q * x)
        // explicit fma order: every instantiation (M = 1 or 2, any rows per
        // wave) rounds the same way, which the two-token verify relies on
        acc[mat][r][m] = __fmaf_rn(bi, x.xsum[m], __fmaf_rn(sc, qx, acc[mat][r][m]));
      }
    }
  }
}

// Where one finished row goes (all epilogues but argmax), selected per lane.
struct GemvRowDst {
  uint16_t* out[2];
  float* silu_out[2];
  const uint16_t* res[2];
  float* conv_state;
  float* conv_state_out;
  const uint16_t* conv_w;
  uint32_t conv_dim;
  uint32_t row;
};

__device__ inline GemvRowDst gemv_row_dst(const GemvSeg& sg, uint32_t row) {
  GemvRowDst d;
  d.out[0] = sg.out[0];
  d.out[1] = sg.out[1];
  d.silu_out[0] = sg.silu_out[0];
  d.silu_out[1] = sg.silu_out[1];
  d.res[0] = sg.res[0];
  d.res[1] = sg.res[1];
  d.conv_state = sg.conv_state;
  d.conv_state_out = sg.conv_state_out ? sg.conv_state_out : sg.conv_state;
  d.conv_w = sg.conv_w;
  d.conv_dim = sg.conv_dim;
  d.row = row;
  return d;
}

// Epilogue of one row: tot[mat][m] are its finished dot products.
template <int M, int NMAT, int EPI>
__device__ inline void gemv_store_row(const GemvRowDst& d, const float (&tot)[NMAT][M]) {
  if constexpr (EPI == kEpiPlain) {
    if (d.silu_out[0] != nullptr) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float zb = round_bf(tot[0][m]);
        d.silu_out[m][d.row] = zb / (1.0f + expf(-zb));
      }
      return;
    }
    if constexpr (M == 2) {
      if (d.conv_state != nullptr) {
        uint16_t o0, o1;
        conv1d_silu_step2(d.conv_state, d.conv_state_out, d.conv_state, d.conv_w, d.conv_dim, d.row,
                          round_bf(tot[0][0]), round_bf(tot[0][1]), o0, o1);
        d.out[0][d.row] = o0;
        d.out[1][d.row] = o1;
        return;
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    uint16_t o;
    if constexpr (EPI == kEpiPlain) {
      if (M == 1 && d.conv_state != nullptr)
        o = conv1d_silu_step(d.conv_state, d.conv_state_out, d.conv_w, d.conv_dim, d.row, round_bf(tot[0][m]));
      else
        o = f2bf(tot[0][m]);
    } else if constexpr (EPI == kEpiResidual) {
      o = f2bf(round_bf(tot[0][m]) + bf2f(d.res[m][d.row]));
    } else {
      o = f2bf(silu(round_bf(tot[0][m])) * round_bf(tot[NMAT - 1][m]));
    }
    d.out[m][d.row] = o;
  }
}

// Transposed reduction of four groups' accumulators (one row each) across
// the wave: v[q][e] is lane-partial e of group q. Lanes l and l^32 are merged
// with v_permlane32_swap (groups q and q+2 trade halves), then l and l^16 with
// v_permlane16_swap (q and q+1), so 16-lane row r ends up holding group r,
// which a DPP row sum finishes. 10 ops per value instead of a full 64-lane
// reduction per group; the combination order of every value is the same for
// any E, so M = 1 and M = 2 launches give identical bits per row.
template <int E>
__device__ inline void reduce4_rows(float (&v)[4][E]) {
#pragma unroll
  for (int e = 0; e < E; ++e) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      float a = v[q][e], b = v[q + 2][e];
      swap32(a, b);
      v[q][e] = a + b;
    }
    float a = v[0][e], b = v[1][e];
    swap16(a, b);
    v[0][e] = row16_sum(a + b);
  }
}

// Reduce one group's accumulators across the wave and write its outputs.
// (wbv, wbi): the wave's running best partial and its row when the argmax
// epilogue writes per wave (p.argmax_waves).
template <int M, int NMAT, int ROWS, int EPI>
__device__ inline void gemv_epilogue(const GemvParams& p, const GemvLoc& loc, int lane,
                                     float (&acc)[NMAT][ROWS][M], float (&wbv)[M], uint32_t (&wbi)[M]) {
  float tot[NMAT][ROWS][M];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) tot[mat][r][m] = wave_sum_uniform(acc[mat][r][m]);
  if (lane != 0) return;
  const GemvSeg& sg = p.seg[loc.seg];
  const uint32_t row0 = loc.row0;
  if constexpr (EPI == kEpiArgmax) {
    static_assert(ROWS == 8, "argmax partials cover 8 rows");
    if (row0 >= sg.rows) return;
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
      if (p.argmax_waves != nullptr) {
        // the group's partial position is best_i / 8 (= row0 / 8)
        if (argmax_better(best, best_i >> 3, wbv[m], wbi[m] >> 3)) {
          wbv[m] = best;
          wbi[m] = best_i;
        }
      } else {
        sg.pval[m][row0 / 8] = best;
        sg.pidx[m][row0 / 8] = best_i;
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const uint32_t row = row0 + r;
      if (row >= sg.rows) break;
      if constexpr (EPI == kEpiPlain && M == 2) {
        if (sg.silu_out[0] == nullptr && sg.conv_state != nullptr) {
          uint16_t o0, o1;
          conv1d_silu_step2(sg.conv_state, sg.conv_state_out, sg.conv_state, sg.conv_w, sg.conv_dim, row,
                            round_bf(tot[0][r][0]), round_bf(tot[0][r][1]), o0, o1);
          sg.out[0][row] = o0;
          sg.out[1][row] = o1;
          continue;
        }
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        uint16_t o;
        if constexpr (EPI == kEpiPlain) {
          if (sg.silu_out[0] != nullptr) {
            const float zb = round_bf(tot[0][r][m]);
            sg.silu_out[m][row] = zb / (1.0f + expf(-zb));
            continue;
          }
          if (M == 1 && sg.conv_state != nullptr)
            o = conv1d_silu_step(sg.conv_state, sg.conv_state_out ? sg.conv_state_out : sg.conv_state, sg.conv_w,
                                 sg.conv_dim, row, round_bf(tot[0][r][m]));
          else
            o = f2bf(tot[0][r][m]);
        } else if constexpr (EPI == kEpiResidual) {
          o = f2bf(round_bf(tot[0][r][m]) + bf2f(sg.res[m][row]));
        } else {
          const float gt = round_bf(tot[0][r][m]);
          const float up = round_bf(tot[1][r][m]);
          o = f2bf(silu(gt) * up);
        }
        sg.out[m][row] = o;
      }
    }
  }
}

// Persistent, software-pipelined GEMV. Work is split into "groups" of ROWS
// consecutive rows of one segment; wave w of the grid handles groups
// w, w + W, w + 2W, ... (W = waves in the grid). Each wave keeps two register
// buffers: while it dequantises and reduces group g the loads of group g + W
// are in flight, so HBM streaming overlaps the VALU work. The activation rows
// (and fused-norm weights) are loaded before any weight so they return first;
// the norm and LDS staging then run while the first group streams in. With XREG the lane's activation pairs for every
// K-step stay in registers for the whole kernel.
template <int M, int ROWS, int ITERS, int EPI, int NORM, bool TAIL>
__global__ __launch_bounds__(kGemvThreads) void q4_gemv_kernel(const GemvParams p) {
  constexpr int NMAT = (EPI == kEpiSiluGate) ? 2 : 1;
  constexpr bool XREG = ITERS * M <= 4;  // <= 64 VGPRs of activation pairs
  extern __shared__ uint32_t xs[];  // [M][K/2] permuted bf16 pairs
  __shared__ float red[M * kGemvWaves];  // per activation row: the waves' sums of squares

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const uint32_t W = gridDim.x * kGemvWaves;
  const uint32_t G = p.total_groups;
  const bool tail_active = !TAIL || lane < static_cast<int>(p.tail_lanes);
  const uint32_t n8 = p.K / 8;

  // 1) activations (+ norm weights, + gates): one uint4 (8 values) per thread
  // per K-step. Without a K tail (K == ITERS * 2048) every thread's units
  // exist, and these loads and the first group's (below) are issued on
  // straight-line code: behind a branch the compiler's wait before the
  // staging would also cover the first group's weights, so the staging (and
  // the norm's reductions) would start only when those arrive.
  constexpr int XU = (ITERS * (kGemvKStep / 8) + kGemvThreads - 1) / kGemvThreads;  // uint4 units per thread
  uint4 xv[M][XU];
  uint4 nw[NORM != kNormNone ? XU : 1];
  float4 zv[NORM == kNormGated ? M : 1][NORM == kNormGated ? XU : 1][2];
#pragma unroll
  for (int it = 0; it < XU; ++it) {
    const uint32_t gi = it * kGemvThreads + threadIdx.x;
    const bool in_k = !TAIL || gi < n8;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if constexpr (TAIL)
        xv[m][it] = in_k ? reinterpret_cast<const uint4*>(p.x[m])[gi] : make_uint4(0, 0, 0, 0);
      else
        xv[m][it] = reinterpret_cast<const uint4*>(p.x[m])[gi];
    }
    if constexpr (NORM == kNormRms) {
      if constexpr (TAIL)
        nw[it] = in_k ? reinterpret_cast<const uint4*>(p.norm_w)[gi] : make_uint4(0, 0, 0, 0);
      else
        nw[it] = reinterpret_cast<const uint4*>(p.norm_w)[gi];
    }
    if constexpr (NORM == kNormGated) {
      // 8 values of head gi / 16: weight entries 8 (gi % 16) .. +8 of the [128] vector.
      nw[it] = reinterpret_cast<const uint4*>(p.norm_w)[gi % (kGdnDv / 8)];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float4* zp = reinterpret_cast<const float4*>(p.gz[m]) + 2 * gi;
        if constexpr (TAIL) {
          zv[m][it][0] = zv[m][it][1] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (in_k) {
            zv[m][it][0] = zp[0];
            zv[m][it][1] = zp[1];
          }
        } else {
          zv[m][it][0] = zp[0];
          zv[m][it][1] = zp[1];
        }
      }
    }
  }

  // 2) the first group's weights. The wave handles n groups (wave-uniform);
  // a wave with none (the grid's last block only) loads the last group and
  // leaves it unused, so the load needs no branch.
  constexpr bool kRounds = (ROWS == 1 && EPI != kEpiArgmax);
  GemvBuf<NMAT, ROWS, ITERS> b0, b1;
  uint32_t g = blockIdx.x * kGemvWaves + wid;
  uint32_t n = g < G ? (G - 1 - g) / W + 1 : 0;
  gemv_load<NMAT, ROWS, ITERS, TAIL>(p, g < G ? g : G - 1, lane, tail_active, b0);

  // 3) stage x into LDS (normalised with NORM), then into registers.
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float scale = 1.0f;
    if constexpr (NORM == kNormRms) {
      float ss = 0.0f;
#pragma unroll
      for (int it = 0; it < XU; ++it) {
        const uint32_t d[4] = {xv[m][it].x, xv[m][it].y, xv[m][it].z, xv[m][it].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = bf_lo(d[i]), b = bf_hi(d[i]);
          ss = __fmaf_rn(a, a, ss);
          ss = __fmaf_rn(b, b, ss);
        }
      }
      // one barrier per activation row (each has its own slots); the same
      // reduction as the standalone RMSNorm, so both give identical bits
      const float total = block_sum256_dpp(ss, red + m * kGemvWaves);
      scale = 1.0f / sqrtf(__fadd_rn(total / static_cast<float>(p.K), p.eps));
    }
    uint4* dst = reinterpret_cast<uint4*>(xs + m * (p.K / 2));
#pragma unroll
    for (int it = 0; it < XU; ++it) {
      const uint32_t gi = it * kGemvThreads + threadIdx.x;
      if constexpr (NORM == kNormGated) {
        // The 16 lanes of a DPP row hold the 128 values of one head.
        float ss = 0.0f;
        const uint32_t d[4] = {xv[m][it].x, xv[m][it].y, xv[m][it].z, xv[m][it].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = bf_lo(d[i]), b = bf_hi(d[i]);
          ss = __fmaf_rn(a, a, ss);
          ss = __fmaf_rn(b, b, ss);
        }
        const float hscale = rsqrtf(__fadd_rn(__fmul_rn(row16_sum(ss), 1.0f / kGdnDv), p.eps));
        if (!TAIL || gi < n8)
          dst[gi] = permute_pairs(gated_rms_apply(xv[m][it], nw[it], zv[m][it][0], zv[m][it][1], hscale));
      } else if (!TAIL || gi < n8) {
        uint4 v;
        if constexpr (NORM == kNormRms)
          v = permute_pairs(rms_apply(xv[m][it], nw[it], scale));
        else
          v = permute_pairs(xv[m][it]);
        dst[gi] = v;
        // block 0 only (its waves may wait for this store together with the
        // first group's weights; the other blocks take no store)
        if (p.x_image[m] != nullptr && blockIdx.x == 0) reinterpret_cast<uint4*>(p.x_image[m])[gi] = v;
      }
    }
  }
  // Keep the first group's scale / bias register copies below the barrier:
  // moved above it they would make every wave wait for that group's loads.
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);

  XStep<M> xr[XREG ? ITERS : 1];
  if constexpr (XREG) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) gemv_read_x<M>(xs, p.K, it, lane, xr[it]);
  }

  auto accumulate = [&](const GemvBuf<NMAT, ROWS, ITERS>& b, float (&acc)[NMAT][ROWS][M]) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[mat][r][m] = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      if (TAIL && it == ITERS - 1 && !tail_active) break;
      if constexpr (XREG) {
        gemv_dot_step<M>(b, it, xr[it], acc);
      } else {
        XStep<M> x;
        gemv_read_x<M>(xs, p.K, it, lane, x);
        gemv_dot_step<M>(b, it, x, acc);
      }
    }
  };

  // 4) The pipeline: group i + 1 streams into the other register buffer
  // while group i is dequantised. Every prefetch load is issued on
  // straight-line code whose continuation always uses it: a prefetch under a
  // branch joins a path without it, and the compiler's wait counts at the
  // join then cover the prefetched loads as well, i.e. the wave waits for the
  // next group's loads before it dequantises the current one.
  if constexpr (kRounds) {
    // Rounds of up to four groups g + jW (j < NV); MORE says that another
    // round follows, so the round's last group prefetches the next round's
    // first. One transposed reduction per round, then a one-lane-per-group
    // epilogue.
    constexpr int E = NMAT * M;
    auto step = [&](const GemvBuf<NMAT, 1, ITERS>& cur, float (&vq)[E]) {
      float acc[NMAT][1][M];
      accumulate(cur, acc);
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int m = 0; m < M; ++m) vq[mat * M + m] = acc[mat][0][m];
    };
    auto round = [&](auto nv_c, auto more_c) {
      constexpr int NV = decltype(nv_c)::value;
      constexpr bool MORE = decltype(more_c)::value;
      float v[4][E];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < E; ++e) v[q][e] = 0.0f;
      if constexpr (NV > 1 || MORE) gemv_load<NMAT, 1, ITERS, TAIL>(p, g + W, lane, tail_active, b1);
      step(b0, v[0]);
      if constexpr (NV > 1) {
        if constexpr (NV > 2 || MORE) gemv_load<NMAT, 1, ITERS, TAIL>(p, g + 2 * W, lane, tail_active, b0);
        step(b1, v[1]);
      }
      if constexpr (NV > 2) {
        if constexpr (NV > 3 || MORE) gemv_load<NMAT, 1, ITERS, TAIL>(p, g + 3 * W, lane, tail_active, b1);
        step(b0, v[2]);
      }
      if constexpr (NV > 3) {
        if constexpr (MORE) gemv_load<NMAT, 1, ITERS, TAIL>(p, g + 4 * W, lane, tail_active, b0);
        step(b1, v[3]);
      }
      reduce4_rows<E>(v);
      // 16-lane row q now holds group g + qW; its first lane writes the row.
      GemvRowDst dst{};
      bool valid = false;
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const GemvLoc loc = gemv_locate<1>(p, g + q * W);
        const GemvRowDst dq = gemv_row_dst(p.seg[loc.seg], loc.row0);
        if ((lane >> 4) == q) {
          dst = dq;
          valid = true;
        }
      }
      if (valid && (lane & 15) == 0) {
        float tot[NMAT][M];
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int m = 0; m < M; ++m) tot[mat][m] = v[0][mat * M + m];
        gemv_store_row<M, NMAT, EPI>(dst, tot);
      }
    };
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    using C3 = std::integral_constant<int, 3>;
    using C4 = std::integral_constant<int, 4>;
    while (n > 4) {
      round(C4{}, std::true_type{});
      g += 4 * W;
      n -= 4;
    }
    switch (n) {
      case 4: round(C4{}, std::false_type{}); break;
      case 3: round(C3{}, std::false_type{}); break;
      case 2: round(C2{}, std::false_type{}); break;
      case 1: round(C1{}, std::false_type{}); break;
      default: break;
    }
  } else {
    float wbv[M];
    uint32_t wbi[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      wbv[m] = -INFINITY;
      wbi[m] = 0xffffffffu;  // no partial yet (never compared: -inf never wins)
    }
    auto process = [&](const GemvBuf<NMAT, ROWS, ITERS>& b, uint32_t grp) {
      float acc[NMAT][ROWS][M];
      accumulate(b, acc);
      gemv_epilogue<M, NMAT, ROWS, EPI>(p, gemv_locate<ROWS>(p, grp), lane, acc, wbv, wbi);
    };
    while (n > 2) {
      gemv_load<NMAT, ROWS, ITERS, TAIL>(p, g + W, lane, tail_active, b1);
      process(b0, g);
      gemv_load<NMAT, ROWS, ITERS, TAIL>(p, g + 2 * W, lane, tail_active, b0);
      process(b1, g + W);
      g += 2 * W;
      n -= 2;
    }
    if (n == 2) {
      gemv_load<NMAT, ROWS, ITERS, TAIL>(p, g + W, lane, tail_active, b1);
      process(b0, g);
      process(b1, g + W);
    } else if (n == 1) {
      process(b0, g);
    }
    if constexpr (EPI == kEpiArgmax) {
      if (p.argmax_waves != nullptr && lane == 0) {
        const uint32_t wave = blockIdx.x * kGemvWaves + wid;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          p.seg[0].pval[m][wave] = wbv[m];
          p.seg[0].pidx[m][wave] = wbi[m];
        }
        if (wave == 0) *p.argmax_waves = gridDim.x * kGemvWaves;
      }
    }
  }
}

// ------------------------------------------------------------- host ----------
// Instantiated per epilogue in q4_gemv_inst_*.hip. Returns 0, or -1 when no
// kernel variant exists for (M, rows, iters).
template <int EPI, int NORM>
int launch_m(hipStream_t s, const GemvParams& p, int M, int rows, int iters, size_t lds);

// Launch one GEMV-family kernel. Segment block ranges are filled in here.
// Returns a PRG_ERR_* code.
int launch_q4_gemv(hipStream_t stream, GemvParams& p, int M, int rows_per_wave, int epi,
                   int norm, const char* name);

// Rows per wave picked for a launch of `total_rows` rows at in_dim K.
int gemv_rows_per_wave(uint32_t total_rows, uint32_t K, int epi, int M);

// Final argmax over the per-wave entries of an argmax GEMV launched with
// GemvParams::argmax_waves = count (values / rows hold kArgmaxMaxWaves
// entries), with and without the control-block update.
int launch_argmax_waves_advance(hipStream_t s, const float* values, const uint32_t* rows, const uint32_t* count,
                                DecodeCtl* ctl, const uint32_t* prompt, uint32_t* predictions);
// M (1 or 2) activation rows in one launch: row m's entries -> out[m][0].
int launch_argmax_waves(hipStream_t s, int M, const float* const* values, const uint32_t* const* rows,
                        const uint32_t* count, uint32_t* const* out);
// Advance with the next token forced from prompt (no lm_head this step).
int launch_advance_forced(hipStream_t s, DecodeCtl* ctl, const uint32_t* prompt);

}  // namespace prg
