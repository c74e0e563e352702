// Q4 GEMV on the matrix cores over the decode layout (see q4_gemv_t16.hpp):
// the repack kernel, the GEMV kernel template and its launcher.
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "q4_gemv_t16.hpp"

namespace prg {

constexpr uint32_t kT16Steps = 2;  // 1 KiB wave loads per window

typedef __bf16 t16_bf16x8 __attribute__((ext_vector_type(8)));
typedef float t16_f32x4 __attribute__((ext_vector_type(4)));

// MLX layout -> decode layout. Unit o (16 bytes) = (tile, window, step, lane).
__global__ __launch_bounds__(256) void t16_repack_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                                         const uint16_t* __restrict__ b, uint32_t* __restrict__ tw,
                                                         uint16_t* __restrict__ ts, uint16_t* __restrict__ tb,
                                                         uint32_t N, uint32_t K) {
  const uint32_t wins = K / kT16WinK;
  const size_t units = static_cast<size_t>(N / kT16Rows) * wins * kT16Steps * kWave;
  for (size_t o = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; o < units;
       o += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const uint32_t lane = static_cast<uint32_t>(o & 63), st = static_cast<uint32_t>((o >> 6) & 1);
    const size_t tile_win = o >> 7;
    const uint32_t win = static_cast<uint32_t>(tile_win % wins);
    const uint32_t tile = static_cast<uint32_t>(tile_win / wins);
    const uint32_t row = tile * kT16Rows + (lane & 15);
    const uint32_t word = win * 32 + st * 16 + 4 * (lane >> 4);
    reinterpret_cast<uint4*>(tw)[o] = *reinterpret_cast<const uint4*>(w + static_cast<size_t>(row) * (K / 8) + word);
    if (st == 0) {
      const size_t mo = tile_win * kWave + lane;
      const size_t mi = static_cast<size_t>(row) * (K / 64) + win * 4 + (lane >> 4);
      ts[mo] = s[mi];
      tb[mo] = b[mi];
    }
  }
}

namespace {

// Segment and tile-within-segment of launch tile t (segment tile ranges in
// GemvSeg::block_begin).
struct T16Loc {
  uint32_t seg;
  uint32_t tile;
};
__device__ inline T16Loc t16_locate(const GemvParams& p, uint32_t t) {
  uint32_t si = 0;
  for (uint32_t i = 1; i < p.nseg; ++i)
    if (t >= p.seg[i].block_begin) si = i;
  return T16Loc{si, t - p.seg[si].block_begin};
}

// One window of one wave: two 1 KiB steps per matrix plus the lane's scale
// and bias bits (kept as loaded until the window is used).
template <int NMAT>
struct T16Win {
  u32x4 w[NMAT][kT16Steps];
  uint16_t sc[NMAT];
  uint16_t bi[NMAT];
};

// Window u (0..NW-1) of wave w's K range of launch tile t.
template <int NMAT, int S, int NW>
__device__ inline void t16_load(const GemvParams& p, uint32_t t, int w, int u, int lane, T16Win<NMAT>& b) {
  constexpr uint32_t kWins = NW * S;  // windows per row
  const T16Loc loc = t16_locate(p, t);
  const GemvSeg& sg = p.seg[loc.seg];
  const size_t win = static_cast<size_t>(loc.tile) * kWins + NW * w + u;
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const u32x4* wp = reinterpret_cast<const u32x4*>(sg.tw[mat]) + win * (kT16Steps * kWave) + lane;
#pragma unroll
    for (int st = 0; st < static_cast<int>(kT16Steps); ++st) b.w[mat][st] = __builtin_nontemporal_load(wp + st * kWave);
    b.sc[mat] = sg.ts[mat][win * kWave + lane];
    b.bi[mat] = sg.tb[mat][win * kWave + lane];
  }
}

// Sum of lanes j, j + 16, j + 32, j + 48 as (v[j] + v[j+32]) + (v[j+16] + v[j+48]);
// all four lanes receive the same bits.
__device__ inline float sum_c4(float v) {
  float a = v, b = v;
  swap32(a, b);
  v = a + b;
  a = v;
  b = v;
  swap16(a, b);
  return a + b;
}

// NW windows (1 to 4) per wave: K = 256 NW S.
template <int M, int NMAT, int S, int NW, int EPI, int NORM>
__global__ __launch_bounds__(S * kWave) void q4_gemv_t16_kernel(const GemvParams p) {
  static_assert(NW >= 1 && NW <= 4, "one to four windows per wave");
  constexpr uint32_t K = kT16WinK * NW * S;
  constexpr uint32_t kThreads = S * kWave;
  constexpr uint32_t kUnits = K / 8;  // uint4 units of one activation row
  // units per thread: when the row does not fill the last pass, the threads
  // past it skip that pass (a wave-uniform test: kUnits % 64 == 0)
  constexpr int XU = static_cast<int>((kUnits + kThreads - 1) / kThreads);
  static_assert(kUnits % kWave == 0, "whole waves per pass");
  auto staged_unit = [&](int it) { return kUnits % kThreads == 0 || it * kThreads + threadIdx.x < kUnits; };
  constexpr uint32_t kGroups = K / 64;
  constexpr uint32_t kZero = M * K / 2;  // dword offset of the 64-byte zero block
  // x as permuted bf16 pairs (M rows), then 16 zero dwords
  __shared__ __align__(16) uint32_t xs[M * K / 2 + 16];
  __shared__ float xg[M * kGroups];           // per-group sums of the staged x
  __shared__ float red[2][S][NMAT][M][16];    // per-wave row sums, double-buffered over tiles
  __shared__ float nred[M][S];                // RMSNorm partial sums of squares

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int c = lane >> 4;
  const uint32_t tiles = p.total_groups;
  uint32_t tile = blockIdx.x;

  // 1) activations (and norm weights) first so they return first, then this
  // wave's first window of its first tile; the second is issued once x is
  // staged. Every wave's x loads queue behind the weight loads its CU has
  // already issued, and the staging gates the first matrix instructions, so
  // fewer bytes ahead of them (one window per wave instead of two) bring x in
  // sooner.
  uint4 xv[M][XU];
  uint4 nw[NORM != kNormNone ? XU : 1];
  float4 zv[NORM == kNormGated ? M : 1][NORM == kNormGated ? XU : 1][2];
#pragma unroll
  for (int it = 0; it < XU; ++it) {
    // threads past the row load unit 0 and never use it
    const uint32_t gi = staged_unit(it) ? it * kThreads + tid : 0u;
#pragma unroll
    for (int m = 0; m < M; ++m) xv[m][it] = reinterpret_cast<const uint4*>(p.x[m])[gi];
    if constexpr (NORM == kNormRms) nw[it] = reinterpret_cast<const uint4*>(p.norm_w)[gi];
    if constexpr (NORM == kNormGated) {
      // 8 values of head gi / 16: entries 8 (gi % 16) .. +8 of the [128] weight
      nw[it] = reinterpret_cast<const uint4*>(p.norm_w)[gi % (kGdnDv / 8)];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float4* zp = reinterpret_cast<const float4*>(p.gz[m]) + 2 * gi;
        zv[m][it][0] = zp[0];
        zv[m][it][1] = zp[1];
      }
    }
  }
  T16Win<NMAT> b0, b1;
  t16_load<NMAT, S, NW>(p, tile, w, 0, lane, b0);

  // 2) normalise, stage x as the permuted pairs of the nibble unpack, and the
  // per-group sums of the staged values.
  float scale[M];
#pragma unroll
  for (int m = 0; m < M; ++m) scale[m] = 1.0f;
  if constexpr (NORM == kNormRms) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float ss = 0.0f;
#pragma unroll
      for (int it = 0; it < XU; ++it) {
        const uint32_t d[4] = {xv[m][it].x, xv[m][it].y, xv[m][it].z, xv[m][it].w};
        if (!staged_unit(it)) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = bf_lo(d[i]), b = bf_hi(d[i]);
          ss = __fmaf_rn(a, a, ss);
          ss = __fmaf_rn(b, b, ss);
        }
      }
      ss = wave_sum_uniform(ss);
      if (lane == 0) nred[m][w] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float total;
      if constexpr (S == 4) {
        // the order of block_sum256_dpp: a 256-thread launch normalises to the same bits
        total = (nred[m][0] + nred[m][1]) + (nred[m][2] + nred[m][3]);
      } else {
        total = nred[m][0];
#pragma unroll
        for (int ww = 1; ww < S; ++ww) total += nred[m][ww];
      }
      scale[m] = 1.0f / sqrtf(__fadd_rn(total / static_cast<float>(K), p.eps));
    }
  }
  constexpr uint32_t kOnes = 0x3F803F80u;  // bf16 pair (1, 1)
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int it = 0; it < XU; ++it) {
      if (!staged_unit(it)) continue;
      const uint32_t gi = it * kThreads + tid;
      uint4 v;
      if constexpr (NORM == kNormRms) {
        v = permute_pairs(rms_apply(xv[m][it], nw[it], scale[m]));
      } else if constexpr (NORM == kNormGated) {
        // The 16 lanes of a DPP row hold the 128 values of one head: the
        // per-head RMSNorm of q4_gemv_kernel's gated prologue, same order.
        float ss = 0.0f;
        const uint32_t d[4] = {xv[m][it].x, xv[m][it].y, xv[m][it].z, xv[m][it].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = bf_lo(d[i]), b = bf_hi(d[i]);
          ss = __fmaf_rn(a, a, ss);
          ss = __fmaf_rn(b, b, ss);
        }
        const float hscale = rsqrtf(__fadd_rn(__fmul_rn(row16_sum(ss), 1.0f / kGdnDv), p.eps));
        v = permute_pairs(gated_rms_apply(xv[m][it], nw[it], zv[m][it][0], zv[m][it][1], hscale));
      } else {
        v = permute_pairs(xv[m][it]);
      }
      reinterpret_cast<uint4*>(xs + m * (K / 2))[gi] = v;
      if (p.x_image[m] != nullptr && blockIdx.x == 0) reinterpret_cast<uint4*>(p.x_image[m])[gi] = v;
      float sm = dot2_bf16(v.x, kOnes, 0.0f);
      sm = dot2_bf16(v.y, kOnes, sm);
      sm = dot2_bf16(v.z, kOnes, sm);
      sm = dot2_bf16(v.w, kOnes, sm);
      // the 8 units of a group sit in 8 consecutive lanes: DPP butterfly
      // (quad_perm 1032, quad_perm 2301, half-row mirror); every lane of the
      // 8 gets the same bits
      sm += dpp_f<0xB1>(sm);
      sm += dpp_f<0x4E>(sm);
      sm += dpp_f<0x141>(sm);
      if ((gi & 7) == 0) xg[m * kGroups + gi / 8] = sm;
    }
  }
  if (tid < 16) xs[kZero + tid] = 0u;
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NW >= 2) t16_load<NMAT, S, NW>(p, tile, w, 1, lane, b1);

  // 3) A operand: lane (i = lane & 15, c) holds row i = 4 h + m, k-chunk c.
  // It carries x_m only when chunk c of step st lies in group slot h of the
  // window (h == 2 st + c / 2); otherwise it reads the zero block.
  const int ia = lane & 15;
  const int ha = ia >> 2, ma = ia & 3;
  uint32_t aoff[2], ainc[2];  // dwords
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const bool data = ma < M && ha == 2 * st + (c >> 1);
    aoff[st] = data ? static_cast<uint32_t>(ma) * (K / 2) + 128u * NW * w + 64u * st + 16u * c : kZero;
    ainc[st] = data ? 128u : 0u;
  }
  // Group sums of the lane's group slot c in each of the wave's windows.
  float xsum[NW][M];
#pragma unroll
  for (int u = 0; u < NW; ++u)
#pragma unroll
    for (int m = 0; m < M; ++m) xsum[u][m] = xg[m * kGroups + 4 * NW * w + 4 * u + c];

  auto window = [&](const T16Win<NMAT>& b, int u, float (&acc)[NMAT][M]) {
    t16_f32x4 C[NMAT];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) C[mat] = t16_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      t16_bf16x8 A[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) A[t] = *reinterpret_cast<const t16_bf16x8*>(xs + aoff[st] + u * ainc[st] + 4 * t);
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          uint32_t q[4];
          unpack_q4_word(b.w[mat][st][t], q);
          const uint4 bv = make_uint4(q[0], q[1], q[2], q[3]);
          C[mat] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t], __builtin_bit_cast(t16_bf16x8, bv), C[mat], 0, 0, 0);
        }
      }
    }
    // lane (j, c): C[mat][m] = sum (128 + q) x_m over group 4u + c of row j
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      const float sc = bf_lo(static_cast<uint32_t>(b.sc[mat]));
      const float bi = bf_lo(static_cast<uint32_t>(b.bi[mat]));
      const float bq = __fmaf_rn(-128.0f, sc, bi);
#pragma unroll
      for (int m = 0; m < M; ++m) acc[mat][m] = __fmaf_rn(bq, xsum[u][m], __fmaf_rn(sc, C[mat][m], acc[mat][m]));
    }
  };

  float wbv[M];
  uint32_t wbi[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    wbv[m] = -INFINITY;
    wbi[m] = 0xffffffffu;  // no partial yet (never compared: -inf never wins)
  }
  int buf = 0;

  // One tile: NW windows, the next tile's first two windows prefetched (PF)
  // while the last two are computed, then the row sums and epilogue.
  auto tile_body = [&](uint32_t t, uint32_t nt, auto pf) {
    constexpr bool PF = decltype(pf)::value;
    float acc[NMAT][M];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[mat][m] = 0.0f;
    if constexpr (NW == 4) {
      window(b0, 0, acc);
      t16_load<NMAT, S, NW>(p, t, w, 2, lane, b0);
      window(b1, 1, acc);
      t16_load<NMAT, S, NW>(p, t, w, 3, lane, b1);
      window(b0, 2, acc);
      if constexpr (PF) t16_load<NMAT, S, NW>(p, nt, w, 0, lane, b0);
      window(b1, 3, acc);
      if constexpr (PF) t16_load<NMAT, S, NW>(p, nt, w, 1, lane, b1);
    } else if constexpr (NW == 3) {
      window(b0, 0, acc);
      t16_load<NMAT, S, NW>(p, t, w, 2, lane, b0);
      window(b1, 1, acc);
      if constexpr (PF) t16_load<NMAT, S, NW>(p, nt, w, 1, lane, b1);
      window(b0, 2, acc);
      if constexpr (PF) t16_load<NMAT, S, NW>(p, nt, w, 0, lane, b0);
    } else if constexpr (NW == 2) {
      window(b0, 0, acc);
      if constexpr (PF) t16_load<NMAT, S, NW>(p, nt, w, 0, lane, b0);
      window(b1, 1, acc);
      if constexpr (PF) t16_load<NMAT, S, NW>(p, nt, w, 1, lane, b1);
    } else {
      window(b0, 0, acc);
      if constexpr (PF) t16_load<NMAT, S, NW>(p, nt, w, 0, lane, b0);
    }
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float v = sum_c4(acc[mat][m]);
        if (lane < 16) red[buf][w][mat][m][lane] = v;
      }
    __syncthreads();
    if (w == 0) {
      const T16Loc loc = t16_locate(p, t);
      const GemvSeg& sg = p.seg[loc.seg];
      const uint32_t row0 = loc.tile * kT16Rows;
      float tot[NMAT][M];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int m = 0; m < M; ++m) {
          float sum = 0.0f;
          if (lane < 16) {
            sum = red[buf][0][mat][m][lane];
#pragma unroll
            for (int ww = 1; ww < S; ++ww) sum += red[buf][ww][mat][m][lane];
          }
          tot[mat][m] = sum;
        }
      if constexpr (EPI == kEpiArgmax) {
        // Per 8-row partial: the first strict maximum of bf16(dot); a partial
        // whose first row is NaN stays NaN and never wins (argmax_better).
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const int vb = __builtin_bit_cast(int, round_bf(tot[0][m]));
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float best = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vb, 8 * h));
            uint32_t bi = 0;
#pragma unroll
            for (int r = 1; r < 8; ++r) {
              const float v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vb, 8 * h + r));
              if (v > best) {
                best = v;
                bi = r;
              }
            }
            const uint32_t row = row0 + 8 * h + bi;
            if (argmax_better(best, row >> 3, wbv[m], wbi[m] >> 3)) {
              wbv[m] = best;
              wbi[m] = row;
            }
          }
        }
      } else {
        if (lane < 16) gemv_store_row<M, NMAT, EPI>(gemv_row_dst(sg, row0 + lane), tot);
      }
    }
    buf ^= 1;
  };

  for (;;) {
    const uint32_t nt = tile + gridDim.x;
    if (nt < tiles) {
      tile_body(tile, nt, std::true_type{});
      tile = nt;
    } else {
      tile_body(tile, tile, std::false_type{});
      break;
    }
  }

  if constexpr (EPI == kEpiArgmax) {
    if (tid == 0) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        p.seg[0].pval[m][blockIdx.x] = wbv[m];
        p.seg[0].pidx[m][blockIdx.x] = wbi[m];
      }
      if (blockIdx.x == 0) *p.argmax_waves = gridDim.x;
    }
  }
}

// Kernel variants: (NMAT, S, NW, EPI, NORM) x M in {1, 2}; K = 256 NW S.
#define PRG_T16_VARIANTS(X)                    \
  X(2, 4, 4, kEpiSiluGate, kNormRms)           \
  X(1, 16, 1, kEpiResidual, kNormGated)        \
  X(1, 16, 1, kEpiResidual, kNormNone)         \
  X(1, 8, 2, kEpiResidual, kNormGated)         \
  X(1, 8, 2, kEpiResidual, kNormNone)          \
  X(1, 4, 4, kEpiResidual, kNormGated)         \
  X(1, 4, 4, kEpiResidual, kNormNone)          \
  X(1, 4, 4, kEpiPlain, kNormRms)              \
  X(1, 4, 4, kEpiPlain, kNormNone)             \
  X(1, 8, 4, kEpiPlain, kNormNone)             \
  X(1, 12, 4, kEpiPlain, kNormNone)            \
  X(1, 16, 3, kEpiResidual, kNormNone)         \
  X(1, 12, 4, kEpiResidual, kNormNone)         \
  X(1, 4, 4, kEpiArgmax, kNormRms)             \
  X(1, 4, 4, kEpiArgmax, kNormNone)

// Launches (or, with grid == 0, only looks up) the variant with NW windows
// per wave for the launch's K (S = K / (256 NW)); -1 if none.
int t16_dispatch(hipStream_t s, const GemvParams& p, int M, int nmat, int epi, int norm, uint32_t grid, int nw) {
  const uint32_t K = p.K;
#define PRG_T16_CASE(NM, SS, NWW, EP, NO)                                                                          \
  if (nmat == NM && K == kT16WinK * NWW * SS && epi == EP && norm == NO && NWW == nw) {                        \
    if (grid == 0) return 0;                                                                                     \
    if (M == 1)                                                                                                  \
      hipLaunchKernelGGL((q4_gemv_t16_kernel<1, NM, SS, NWW, EP, NO>), dim3(grid), dim3(SS * kWave), 0, s, p);   \
    else                                                                                                         \
      hipLaunchKernelGGL((q4_gemv_t16_kernel<2, NM, SS, NWW, EP, NO>), dim3(grid), dim3(SS * kWave), 0, s, p);   \
    return 0;                                                                                                    \
  }
  PRG_T16_VARIANTS(PRG_T16_CASE)
#undef PRG_T16_CASE
  return -1;
}

}  // namespace

bool t16_shape_ok(uint32_t N, uint32_t K) {
  return N > 0 && N % kT16Rows == 0 && K >= kT16WaveK && K % kT16WaveK == 0 && K <= 16384;
}

int launch_t16_repack(hipStream_t s, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      uint32_t* tw, uint16_t* ts, uint16_t* tb, uint32_t N, uint32_t K) {
  PRG_CHECK_ARG(w && scales && biases && tw && ts && tb, "t16 repack: null pointer");
  PRG_CHECK_ARG(t16_shape_ok(N, K), "t16 repack: shape %u x %u (rows %% 16, K %% 1024)", N, K);
  const size_t units = static_cast<size_t>(N / kT16Rows) * (K / kT16WinK) * kT16Steps * kWave;
  const uint32_t blocks = static_cast<uint32_t>(std::min<size_t>((units + 255) / 256, 8192));
  hipLaunchKernelGGL(t16_repack_kernel, dim3(blocks), dim3(256), 0, s, w, scales, biases, tw, ts, tb, N, K);
  PRG_CHECK_LAUNCH("t16 repack");
  return PRG_OK;
}

// Launches of at most this many tiles (a 4096-row matrix has 256) take the
// fewest windows per wave that have a kernel, i.e. the most waves per tile;
// larger launches take four. PEREGRINE_T16_FEW overrides the threshold and
// PEREGRINE_T16_NWSKIP (bit 1 << nw) excludes window counts (tuning).
static uint32_t t16_env(const char* name, uint32_t dflt) {
  const char* e = getenv(name);
  return e ? static_cast<uint32_t>(atoi(e)) : dflt;
}
static uint32_t t16_few_tiles() {
  static const uint32_t v = t16_env("PEREGRINE_T16_FEW", 384u);
  return v;
}
static uint32_t t16_nw_skip() {
  static const uint32_t v = t16_env("PEREGRINE_T16_NWSKIP", 0u);
  return v;
}

static uint32_t t16_tiles(const GemvParams& p) {
  uint32_t tiles = 0;
  for (uint32_t i = 0; i < p.nseg; ++i) tiles += p.seg[i].rows / kT16Rows;
  return tiles;
}

// The variant a launch takes (*nw windows per wave); -1 when there is none.
// Argmax launches loop over tiles and take four windows.
static int t16_pick(const GemvParams& p, int M, int nmat, int epi, int norm, int* nw) {
  const bool few = epi != kEpiArgmax && t16_tiles(p) <= t16_few_tiles();
  static const int kFew[4] = {1, 2, 3, 4}, kMany[4] = {4, 3, 2, 1};
  for (int c : few ? kFew : kMany) {
    if (c != 4 && (t16_nw_skip() >> c & 1u)) continue;
    if (t16_dispatch(nullptr, p, M, nmat, epi, norm, 0, c) == 0) {
      *nw = c;
      return 0;
    }
  }
  return -1;
}

bool t16_usable(const GemvParams& p, int M, int epi, int norm) {
  if (M < 1 || M > 2 || p.nseg < 1 || p.nseg > kGemvMaxSegs) return false;
  if (p.K % kT16WaveK != 0 && p.K % (2 * kT16WinK) != 0) return false;
  if (epi == kEpiArgmax && (p.nseg != 1 || p.argmax_waves == nullptr)) return false;
  const int nmat = epi == kEpiSiluGate ? 2 : 1;
  for (uint32_t i = 0; i < p.nseg; ++i) {
    const GemvSeg& sg = p.seg[i];
    if (sg.rows == 0 || sg.rows % kT16Rows != 0) return false;
    for (int mat = 0; mat < nmat; ++mat)
      if (!sg.tw[mat] || !sg.ts[mat] || !sg.tb[mat]) return false;
  }
  int nw = 0;
  return t16_pick(p, M, nmat, epi, norm, &nw) == 0;
}

int launch_q4_gemv_t16(hipStream_t s, GemvParams& p, int M, int epi, int norm, const char* name) {
  if (!t16_usable(p, M, epi, norm))
    return set_error(PRG_ERR_INVALID_ARG, "%s: no T16 GEMV for M=%d epilogue %d norm %d K=%u (%u segments)", name, M,
                     epi, norm, p.K, p.nseg);
  if (norm == kNormRms && p.norm_w == nullptr) return set_error(PRG_ERR_INVALID_ARG, "%s: RMSNorm weight", name);
  if (norm == kNormGated && (p.norm_w == nullptr || p.gz[0] == nullptr || (M == 2 && p.gz[1] == nullptr)))
    return set_error(PRG_ERR_INVALID_ARG, "%s: gated norm needs norm_w and gz", name);
  uint32_t tiles = 0;
  for (uint32_t i = 0; i < p.nseg; ++i) {
    p.seg[i].block_begin = tiles;
    tiles += p.seg[i].rows / kT16Rows;
  }
  p.total_groups = tiles;
  p.tail_lanes = 64;
  const uint32_t grid = epi == kEpiArgmax ? std::min<uint32_t>(tiles, kArgmaxMaxWaves) : tiles;
  const int nmat = epi == kEpiSiluGate ? 2 : 1;
  int nw = 0;
  if (t16_pick(p, M, nmat, epi, norm, &nw) != 0 || t16_dispatch(s, p, M, nmat, epi, norm, grid, nw) != 0)
    return set_error(PRG_ERR_INVALID_ARG, "%s: no T16 kernel", name);
  PRG_CHECK_LAUNCH(name);
  return PRG_OK;
}

}  // namespace prg

// ------------------------------------------------------------- C ABI -------
namespace {

prg::GemvParams t16_one_seg(const uint32_t* tw, const uint16_t* ts, const uint16_t* tb, uint32_t rows, uint32_t K) {
  prg::GemvParams p{};
  p.nseg = 1;
  p.K = K;
  p.seg[0].tw[0] = tw;
  p.seg[0].ts[0] = ts;
  p.seg[0].tb[0] = tb;
  p.seg[0].rows = rows;
  return p;
}

int t16_check(const char* name, const void* x, const void* tw, const void* ts, const void* tb, uint32_t out_dim,
              uint32_t in_dim) {
  PRG_CHECK_ARG(x && tw && ts && tb, "%s: null pointer", name);
  PRG_CHECK_ARG(prg::t16_shape_ok(out_dim, in_dim), "%s: shape %u x %u (out_dim %% 16, in_dim %% 1024)", name, out_dim,
                in_dim);
  // the kernels read x and the packed words 16 bytes at a time
  PRG_CHECK_ARG(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(tw) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(ts) % 2 == 0 && reinterpret_cast<uintptr_t>(tb) % 2 == 0,
                "%s: x and the packed words must be 16-byte aligned", name);
  return PRG_OK;
}

constexpr size_t kT16ArgmaxWs = 2 * prg::kArgmaxMaxWaves * (sizeof(float) + sizeof(uint32_t)) + 256;

}  // namespace

extern "C" {

int prg_q4_repack_t16(void* stream, const uint32_t* w, const uint16_t* scales, const uint16_t* biases, uint32_t* tw,
                      uint16_t* ts, uint16_t* tb, uint32_t out_dim, uint32_t in_dim) {
  return prg::launch_t16_repack(prg::as_stream(stream), w, scales, biases, tw, ts, tb, out_dim, in_dim);
}

int prg_q4_gemv_t16_bf16(void* stream, const uint16_t* x, const uint32_t* tw, const uint16_t* ts, const uint16_t* tb,
                         uint16_t* y, uint32_t token_count, uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv_t16_bf16";
  if (int rc = t16_check(name, x, tw, ts, tb, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(y != nullptr, "%s: null output", name);
  if (token_count == 0) return prg::set_error(PRG_ERR_EMPTY_INPUT, "%s: token_count == 0", name);
  hipStream_t s = prg::as_stream(stream);
  for (uint32_t t = 0; t < token_count; t += 2) {
    const int M = (token_count - t >= 2) ? 2 : 1;
    prg::GemvParams p = t16_one_seg(tw, ts, tb, out_dim, in_dim);
    for (int m = 0; m < M; ++m) {
      p.x[m] = x + static_cast<size_t>(t + m) * in_dim;
      p.seg[0].out[m] = y + static_cast<size_t>(t + m) * out_dim;
    }
    if (!prg::t16_usable(p, M, prg::kEpiPlain, prg::kNormNone))
      return prg::set_error(PRG_ERR_INVALID_ARG, "%s: in_dim %u (4096, 8192 or 12288)", name, in_dim);
    if (int rc = prg::launch_q4_gemv_t16(s, p, M, prg::kEpiPlain, prg::kNormNone, name)) return rc;
  }
  return PRG_OK;
}

int prg_q4_gemv_t16_silu_gate_norm_bf16(void* stream, const uint16_t* x, const uint16_t* norm_weight, float eps,
                                        const uint32_t* gate_tw, const uint16_t* gate_ts, const uint16_t* gate_tb,
                                        const uint32_t* up_tw, const uint16_t* up_ts, const uint16_t* up_tb,
                                        uint16_t* out, uint32_t out_dim, uint32_t in_dim) {
  const char* name = "prg_q4_gemv_t16_silu_gate_norm_bf16";
  if (int rc = t16_check(name, x, gate_tw, gate_ts, gate_tb, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(norm_weight && up_tw && up_ts && up_tb && out, "%s: null pointer", name);
  prg::GemvParams p = t16_one_seg(gate_tw, gate_ts, gate_tb, out_dim, in_dim);
  p.seg[0].tw[1] = up_tw;
  p.seg[0].ts[1] = up_ts;
  p.seg[0].tb[1] = up_tb;
  p.seg[0].out[0] = out;
  p.x[0] = x;
  p.norm_w = norm_weight;
  p.eps = eps;
  if (!prg::t16_usable(p, 1, prg::kEpiSiluGate, prg::kNormRms))
    return prg::set_error(PRG_ERR_INVALID_ARG, "%s: in_dim %u (4096)", name, in_dim);
  return prg::launch_q4_gemv_t16(prg::as_stream(stream), p, 1, prg::kEpiSiluGate, prg::kNormRms, name);
}

size_t prg_q4_gemv_t16_argmax_workspace_bytes(void) { return kT16ArgmaxWs; }

int prg_q4_gemv_t16_argmax_bf16(void* stream, const uint16_t* x, const uint32_t* tw, const uint16_t* ts,
                                const uint16_t* tb, uint32_t* out_index, uint32_t token_count, uint32_t out_dim,
                                uint32_t in_dim, void* workspace) {
  const char* name = "prg_q4_gemv_t16_argmax_bf16";
  if (int rc = t16_check(name, x, tw, ts, tb, out_dim, in_dim)) return rc;
  PRG_CHECK_ARG(out_index && workspace, "%s: null output or workspace", name);
  PRG_CHECK_ARG(token_count == 1 || token_count == 2, "%s: token_count %u (1 or 2)", name, token_count);
  const int M = static_cast<int>(token_count);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* vals[2] = {reinterpret_cast<float*>(ws), reinterpret_cast<float*>(ws) + prg::kArgmaxMaxWaves};
  uint32_t* rows[2] = {reinterpret_cast<uint32_t*>(ws + 2 * prg::kArgmaxMaxWaves * sizeof(float)),
                       reinterpret_cast<uint32_t*>(ws + 2 * prg::kArgmaxMaxWaves * sizeof(float)) +
                           prg::kArgmaxMaxWaves};
  uint32_t* count = reinterpret_cast<uint32_t*>(ws + 2 * prg::kArgmaxMaxWaves * (sizeof(float) + sizeof(uint32_t)));
  prg::GemvParams p = t16_one_seg(tw, ts, tb, out_dim, in_dim);
  for (int m = 0; m < M; ++m) {
    p.x[m] = x + static_cast<size_t>(m) * in_dim;
    p.seg[0].pval[m] = vals[m];
    p.seg[0].pidx[m] = rows[m];
  }
  p.argmax_waves = count;
  if (!prg::t16_usable(p, M, prg::kEpiArgmax, prg::kNormNone))
    return prg::set_error(PRG_ERR_INVALID_ARG, "%s: in_dim %u (4096)", name, in_dim);
  hipStream_t s = prg::as_stream(stream);
  if (int rc = prg::launch_q4_gemv_t16(s, p, M, prg::kEpiArgmax, prg::kNormNone, name)) return rc;
  const float* cv[2] = {vals[0], vals[1]};
  const uint32_t* cr[2] = {rows[0], rows[1]};
  uint32_t* outs[2] = {out_index, out_index + 1};
  return prg::launch_argmax_waves(s, M, cv, cr, count, outs);
}

}  // extern "C"
