// MFMA GEMM for the prompt path (declarations and tiling notes in gemm.hpp).
//
// Reference kernels this replaces:
//   linear_q4_affine_group64_prefill_qmm_m32n64_nt_bf16_tiles_{,residual_add_}bf16
//       shaders/linear.metal:780-988 (host Q4Linear.encodePrefillQmm*, linear_q4.zig:197-233)
//   the prepared-dense route (q4_dequantize_bf16 + MLX bf16 NT GEMM), same numbers
//       src/model/mlx_nt.zig:139-162
//   attention score / value GEMMs of the materialised prefill
//       src/model/block_attn.zig:75-109, 500-631
//   silu_mul_pair_inplace_bf16 / sigmoid_mul_pair_inplace_bf16 as epilogues
//       shaders/elementwise.metal:64-99
#include <stdlib.h>

#include <algorithm>

#include "gemm.hpp"

namespace {

using namespace prg;

constexpr int kBM = 128, kBN = 128, kBK = 64, kGemmThreads = 256;
static_assert(kBM == kGemmBf16RowTile && kBK == kGemmBf16KStep, "causal_pv_columns follows this tiling");
constexpr int kLdsRow = kBK + 8;  // bf16 per LDS row (144 bytes)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ inline const uint16_t* row_ptr(const uint16_t* base, uint64_t ld, uint64_t ld_hi, uint32_t group,
                                          uint32_t m) {
  if (group) return base + static_cast<uint64_t>(m / group) * ld_hi + static_cast<uint64_t>(m % group) * ld;
  return base + static_cast<uint64_t>(m) * ld;
}

// Two f32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ inline uint32_t pack_bf16(float lo, float hi) {
  const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// One Q4 word (8 nibbles, nibble j = column j) -> 8 bf16(s*q + b) in column
// order. s*q is exact in f32 (8-bit by 4-bit significands), so the fma rounds
// once, exactly like the reference's separate multiply and add.
__device__ inline uint4 dequant_word(uint32_t w, float s, float b) {
  uint32_t lo = w & 0x0F0F0F0Fu;         // columns 0, 2, 4, 6 in bytes 0..3
  uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // columns 1, 3, 5, 7
  // Hide the masks from the optimiser so each byte converts with one
  // v_cvt_f32_ubyteN instead of a bit-field extract plus a convert.
  asm("" : "+v"(lo), "+v"(hi));
  uint4 r;
  r.x = pack_bf16(fmaf(s, static_cast<float>(lo & 0xffu), b), fmaf(s, static_cast<float>(hi & 0xffu), b));
  r.y = pack_bf16(fmaf(s, static_cast<float>((lo >> 8) & 0xffu), b), fmaf(s, static_cast<float>((hi >> 8) & 0xffu), b));
  r.z = pack_bf16(fmaf(s, static_cast<float>((lo >> 16) & 0xffu), b), fmaf(s, static_cast<float>((hi >> 16) & 0xffu), b));
  r.w = pack_bf16(fmaf(s, static_cast<float>(lo >> 24), b), fmaf(s, static_cast<float>(hi >> 24), b));
  return r;
}

// 8 bf16 at columns [k, k+8) of a row; columns >= K read as zero.
__device__ inline uint4 load8(const uint16_t* row, uint32_t k, uint32_t K) {
  if (!row) return make_uint4(0, 0, 0, 0);
  if (k + 8 <= K) return *reinterpret_cast<const uint4*>(row + k);
  uint32_t v[4] = {0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (k + e < K) v[e >> 1] |= static_cast<uint32_t>(row[k + e]) << (16 * (e & 1));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

template <bool Q4, int EPI>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(const GemmArgs g) {
  // two LDS stages: step k's tiles are read by the matrix cores while step
  // k+1's are written
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][kBM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][kBN * kLdsRow];
  constexpr bool kPair = (EPI == kGemmSiluPair);
  constexpr uint32_t kTileN = kPair ? kBN / 2 : kBN;  // output columns per block

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t tiles_m = (g.M + kBM - 1) / kBM;
  const uint32_t tn = blockIdx.x / tiles_m;
  uint32_t seg = 0;  // Q4 weight segment of this output tile
  if constexpr (Q4 && !kPair) {
#pragma unroll
    for (int i = 1; i < kGemmMaxSegs; ++i)
      if (i < static_cast<int>(g.nq) && tn >= g.q[i].tile0) seg = i;
  }
  const uint32_t m0 = (blockIdx.x % tiles_m) * kBM;
  const uint32_t n0 = (tn - (Q4 ? g.q[seg].tile0 : 0)) * kTileN;
  const uint32_t N = Q4 ? g.q[seg].n : g.N;
  const uint64_t z = blockIdx.z;
  const uint32_t K = g.K;
  // Causal attention: the last column any row of this tile sees (rows of one
  // tile may span two q heads; then the tile holds token T - 1).
  uint32_t k_end = K;
  if (!Q4 && g.causal_T != 0) {
    const uint32_t last = g.causal_prefix + min(g.causal_T - 1, m0 % g.causal_T + (kBM - 1));
    if (EPI == kGemmStore && n0 > last) return;  // scores: every column masked
    if (EPI == kGemmSigmoidGate) k_end = causal_pv_columns(m0, g.causal_T, g.causal_prefix, K);  // P.V: zeros past it
  }

  // Global -> register staging. A (and bf16 B): 16-byte chunk i of this
  // thread is row (tid/8 + 32 i), columns k0 + 8*(tid%8) .. +8.
  const int ld_row = tid >> 3, ld_c8 = (tid & 7) * 8;
  const uint16_t* a_row[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t m = m0 + ld_row + 32 * i;
    a_row[i] = m < g.M ? row_ptr(g.a + z * g.a_z, g.lda, g.lda_hi, g.a_group, m) : nullptr;
  }
  uint4 ra[4];
  // Q4 B: thread owns tile row tid/2 and half tid%2 of each 64-column group.
  const int q_row = tid >> 1, q_half = tid & 1;
  const uint32_t* q_w = nullptr;
  const uint16_t *q_s = nullptr, *q_b = nullptr;
  const uint16_t* b_row[4];
  uint4 rb[4];
  uint4 rw = make_uint4(0, 0, 0, 0);
  uint16_t rs = 0, rbias = 0;
  if constexpr (Q4) {
    const GemmQ4& Q = g.q[kPair ? (q_row >> 6) : seg];
    const uint32_t n = n0 + (kPair ? (q_row & 63) : q_row);
    if (n < N) {
      q_w = Q.w + static_cast<uint64_t>(n) * (K / 8) + q_half * 4;
      q_s = Q.s + static_cast<uint64_t>(n) * (K / 64);
      q_b = Q.b + static_cast<uint64_t>(n) * (K / 64);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t n = n0 + ld_row + 32 * i;
      b_row[i] = n < N ? g.b + z * g.b_z + static_cast<uint64_t>(n) * g.ldb : nullptr;
    }
  }

  auto load = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ra[i] = load8(a_row[i], k0 + ld_c8, K);
    if constexpr (Q4) {
      if (q_w) {
        rw = *reinterpret_cast<const uint4*>(q_w + k0 / 8);
        rs = q_s[k0 / 64];
        rbias = q_b[k0 / 64];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) rb[i] = load8(b_row[i], k0 + ld_c8, K);
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Fragment rows: 16x32 A block i of this wave, 16x32 B block j.
  const int frow = lane & 15, fk = (lane >> 4) * 8;
  int brow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) brow[j] = kPair ? ((j < 2) ? wn * 32 + 16 * j : 64 + wn * 32 + 16 * (j - 2)) : wn * 64 + 16 * j;

  // Registers -> LDS stage st (A as loaded, Q4 B dequantised once here).
  auto store_stage = [&](int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&sA[st][(ld_row + 32 * i) * kLdsRow + ld_c8]) = ra[i];
    if constexpr (Q4) {
      const float s = bf2f(rs), b = bf2f(rbias);
      uint4* dst = reinterpret_cast<uint4*>(&sB[st][q_row * kLdsRow + q_half * 32]);
      dst[0] = dequant_word(rw.x, s, b);
      dst[1] = dequant_word(rw.y, s, b);
      dst[2] = dequant_word(rw.z, s, b);
      dst[3] = dequant_word(rw.w, s, b);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&sB[st][(ld_row + 32 * i) * kLdsRow + ld_c8]) = rb[i];
    }
  };

  // One barrier per K step: step k+1 is stored into the other stage and step
  // k+2's global loads are issued before the matrix cores run on stage k; the
  // barrier then both publishes stage k+1 and retires the reads of stage k.
  load(0);
  store_stage(0);
  if (kBK < k_end) load(kBK);
  __syncthreads();
  int st = 0;
  for (uint32_t k0 = 0; k0 < k_end; k0 += kBK, st ^= 1) {
    if (k0 + kBK < k_end) {
      store_stage(st ^ 1);
      if (k0 + 2 * kBK < k_end) load(k0 + 2 * kBK);
    }
    const uint16_t* A = sA[st];
    const uint16_t* B = sB[st];
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      bf16x8 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&A[(wm * 64 + 16 * i + frow) * kLdsRow + kk + fk]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = *reinterpret_cast<const bf16x8*>(&B[(brow[j] + frow) * kLdsRow + kk + fk]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // Epilogue: lane holds rows 4*(lane/16) + r, column lane%16 of each block.
  const int crow = 4 * (lane >> 4), ccol = lane & 15;
  // Q4: segment output [M, n] row-major; bf16: two-level rows, z offset.
  uint16_t* C = Q4 ? g.q[seg].c : g.c + z * g.c_z;
  const uint16_t* R = g.res ? (Q4 ? g.res : g.res + z * g.c_z) : nullptr;
  const uint64_t ldc = Q4 ? N : g.ldc, ldc_hi = Q4 ? 0 : g.ldc_hi;
  const uint32_t c_group = Q4 ? 0 : g.c_group;
  if constexpr (kPair) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t m = m0 + wm * 64 + 16 * i + crow + r;
        if (m >= g.M) continue;
        uint16_t* out = const_cast<uint16_t*>(row_ptr(C, ldc, ldc_hi, c_group, m));
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t n = n0 + wn * 32 + 16 * j + ccol;
          if (n >= N) continue;
          const float gate = round_bf(acc[i][j][r]), up = round_bf(acc[i][j + 2][r]);
          out[n] = f2bf(silu(gate) * up);
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t m = m0 + wm * 64 + 16 * i + crow + r;
        if (m >= g.M) continue;
        uint16_t* out = const_cast<uint16_t*>(row_ptr(C, ldc, ldc_hi, c_group, m));
        const uint16_t* rin = R ? row_ptr(R, ldc, ldc_hi, c_group, m) : nullptr;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t n = n0 + wn * 64 + 16 * j + ccol;
          if (n >= N) continue;
          const float v = acc[i][j][r];
          if constexpr (EPI == kGemmStore) {
            out[n] = f2bf(v);
          } else if constexpr (EPI == kGemmResidual) {
            out[n] = f2bf(round_bf(v) + bf2f(rin[n]));
          } else {
            out[n] = f2bf(round_bf(v) * sigmoid(bf2f(rin[n])));
          }
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Q4 weights: BM-row x 128-weight-row tiles (BM = 256 or 192), 8 waves (4 along
// M x 2 along N, (BM/4) x 64 each). Every weight element is dequantised once
// per BM activation rows.
//
// Pipeline per 64-k step s (one barrier per step), three LDS stages in a ring:
//   - stage s is consumed: fragments of its second 32-k half are read while the
//     matrix cores run the first half, then the first half of stage s+1 (written
//     during step s-1 and published by the previous barrier) while they run the
//     second;
//   - stage s+2 is written from registers holding the global data of step s+2
//     (issued two steps earlier), and the global loads of step s+4 are issued.
// LDS rows are 128 B with 16-byte chunk c of row r stored at chunk c ^ (r & 7):
// the coalesced staging writes (8 lanes = one row) and the MFMA fragment reads
// (lanes = 16 rows x 4 chunks) both run at the full LDS rate on gfx950.
constexpr int kQ4Threads = 512, kQ4Stages = 3;
constexpr uint32_t kQ4BBytes = 128 * 128;
constexpr uint32_t kBufferWord3 = 0x00020000;  // raw buffer descriptor, 32-bit data format

__device__ inline __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferWord3);
}

// DENSE: every segment has its prepared bf16 copy (GemmQ4::dense, the values
// dequant_word produces), staged as is: the same LDS tile, hence the same
// results bit for bit, without the per-tile dequantisation.
template <int EPI, int BM, bool DENSE>
__global__ __launch_bounds__(kQ4Threads) void gemm_q4_kernel(const GemmArgs g) {
  static_assert(BM == 256 || BM == 192, "row tile");
  constexpr int WTM = BM / 4, IM = WTM / 16;  // wave tile rows, 16-row MFMA blocks per wave
  constexpr uint32_t kQ4ABytes = BM * 128, kQ4Stage = kQ4ABytes + kQ4BBytes;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kQ4Stages * kQ4Stage];
  constexpr bool kPair = (EPI == kGemmSiluPair);
  constexpr uint32_t kTileN = kPair ? 64 : 128;  // output columns per block

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // Block -> tile: block b runs on XCD b % 8; each XCD walks a contiguous range
  // of tiles, ordered tm-fastest within groups of 4 tile rows, so the blocks
  // resident on one XCD share A rows and weight columns in its L2.
  const uint32_t tiles_m = (g.M + BM - 1) / BM;
  uint32_t tm, tn;
  {
    const uint32_t T = gridDim.x, b = blockIdx.x, x = b % 8, q = T / 8, r = T % 8;
    const uint32_t L = x * q + (x < r ? x : r) + b / 8;
    const uint32_t tiles_n = T / tiles_m;
    const uint32_t width = 4 * tiles_n, first = (L / width) * 4;
    const uint32_t gs = tiles_m - first < 4u ? tiles_m - first : 4u;
    tm = first + (L % width) % gs;
    tn = (L % width) / gs;
  }
  uint32_t seg = 0;
  if constexpr (!kPair) {
#pragma unroll
    for (int i = 1; i < kGemmMaxSegs; ++i)
      if (i < static_cast<int>(g.nq) && tn >= g.q[i].tile0) seg = i;
  }
  const uint32_t m0 = tm * BM;
  const uint32_t n0 = (tn - g.q[seg].tile0) * kTileN;
  const uint32_t N = g.q[seg].n;
  const uint32_t K = g.K, steps = K / kBK;

  // A: thread t stages rows (t >> 3) + 64 i (i < BM / 64), chunk t & 7; rows >= M
  // read as zero. Each row's offset is in the per-lane (VGPR) offset, which
  // the buffer range check covers; only the step's k offset, always inside a
  // row, goes in the scalar offset.
  const __amdgpu_buffer_rsrc_t a_rsrc = buffer_rsrc(g.a, static_cast<uint32_t>(static_cast<uint64_t>(g.M) * g.lda * 2));
  const uint32_t ar = tid >> 3, ac = tid & 7;
  uint32_t a_voff[BM / 64];
#pragma unroll
  for (int i = 0; i < BM / 64; ++i) a_voff[i] = static_cast<uint32_t>(((m0 + ar + 64 * i) * g.lda + ac * 8) * 2);
  const uint32_t a_lds = ar * 128 + ((ac ^ (ar & 7)) << 4);
  // B: thread t dequantises word t & 7 (columns 8 (t&7) .. +8 of the step) of
  // tile rows (t >> 3) + 64 j. Pair: j = 0 gate, j = 1 up (same output columns).
  const uint32_t br = tid >> 3, bw = tid & 7;
  __amdgpu_buffer_rsrc_t w_rsrc[2];
  uint32_t w_off[2];
  const uint16_t *ps[2], *pb[2];
  uint32_t b_lds[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const GemmQ4& Q = g.q[kPair ? j : seg];
    const uint32_t row = kPair ? n0 + br : n0 + br + 64 * j;
    const uint32_t nn = row < N ? row : N - 1;  // rows past N are computed, never stored
    if constexpr (DENSE) {
      // 16 bytes = the 8 prepared values of word bw of the step
      w_rsrc[j] = buffer_rsrc(Q.dense, static_cast<uint32_t>(static_cast<uint64_t>(N) * K * 2));
      w_off[j] = nn * (K * 2) + bw * 16;
    } else {
      w_rsrc[j] = buffer_rsrc(Q.w, static_cast<uint32_t>(static_cast<uint64_t>(N) * K / 2));
      w_off[j] = nn * (K / 2) + bw * 4;
    }
    ps[j] = Q.s + static_cast<uint64_t>(nn) * (K / 64);
    pb[j] = Q.b + static_cast<uint64_t>(nn) * (K / 64);
    const uint32_t lrow = br + 64 * j;
    b_lds[j] = kQ4ABytes + lrow * 128 + ((bw ^ (lrow & 7)) << 4);
  }

  u32x4 ra[2][BM / 64];
  uint32_t rw[2][2];
  uint16_t rs[2][2], rb[2][2];
  u32x4 rd[DENSE ? 2 : 1][2];
  auto gload = [&](int set, uint32_t ks) {
#pragma unroll
    for (int i = 0; i < BM / 64; ++i) ra[set][i] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_voff[i], ks * 128, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (DENSE) {
        rd[set][j] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc[j], w_off[j], ks * 128, 0);
      } else {
        rw[set][j] = __builtin_amdgcn_raw_buffer_load_b32(w_rsrc[j], w_off[j], ks * 32, 0);
        rs[set][j] = ps[j][ks];
        rb[set][j] = pb[j][ks];
      }
    }
  };
  auto store_a = [&](int set, uint32_t stage) {
    uint8_t* base = lds + stage * kQ4Stage + a_lds;
#pragma unroll
    for (int i = 0; i < BM / 64; ++i) *reinterpret_cast<u32x4*>(base + i * 8192) = ra[set][i];
  };
  auto store_b = [&](int set, uint32_t stage) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (DENSE) {
        *reinterpret_cast<u32x4*>(lds + stage * kQ4Stage + b_lds[j]) = rd[set][j];
      } else {
        const uint4 d = dequant_word(rw[set][j], bf2f(rs[set][j]), bf2f(rb[set][j]));
        *reinterpret_cast<uint4*>(lds + stage * kQ4Stage + b_lds[j]) = d;
      }
    }
  };

  // MFMA fragments: lane holds row (lane & 15) of a 16-row block, chunk
  // (lane >> 4) + 4 kk of the 64-k step.
  const uint32_t fsw = (lane >> 4) ^ (lane & 7);
  const uint32_t fa0 = (wm * WTM + (lane & 15)) * 128 + (fsw << 4);
  const uint32_t fa1 = (wm * WTM + (lane & 15)) * 128 + ((fsw ^ 4) << 4);
  uint32_t fb0[4], fb1[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t brow = kPair ? ((j < 2) ? wn * 32 + 16 * j : 64 + wn * 32 + 16 * (j - 2)) : wn * 64 + 16 * j;
    fb0[j] = kQ4ABytes + (brow + (lane & 15)) * 128 + (fsw << 4);
    fb1[j] = kQ4ABytes + (brow + (lane & 15)) * 128 + ((fsw ^ 4) << 4);
  }
  bf16x8 fa[2][IM], fb[2][4];
  auto fread = [&](int f, uint32_t stage, int kk) {
    const uint8_t* base = lds + stage * kQ4Stage;
#pragma unroll
    for (int i = 0; i < IM; ++i) fa[f][i] = *reinterpret_cast<const bf16x8*>(base + (kk ? fa1 : fa0) + i * 2048);
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[f][j] = *reinterpret_cast<const bf16x8*>(base + (kk ? fb1[j] : fb0[j]));
  };
  f32x4 acc[IM][4];
#pragma unroll
  for (int i = 0; i < IM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mfma = [&](int f) {
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[f][i], fb[f][j], acc[i][j], 0, 0, 0);
  };
  // Steps past the end reload the last one (kept in bounds, never consumed).
  auto clampk = [&](uint32_t k) { return k < steps ? k : steps - 1; };

  gload(0, 0);
  gload(1, clampk(1));
  store_a(0, 0);
  store_b(0, 0);
  gload(0, clampk(2));
  store_a(1, 1);
  store_b(1, 1);
  gload(1, clampk(3));
  __syncthreads();
  fread(0, 0, 0);

  uint32_t st0 = 0;  // stage of step s
  auto step = [&](int set, uint32_t s) {
    const uint32_t st1 = st0 == kQ4Stages - 1 ? 0 : st0 + 1;
    const uint32_t st2 = st1 == kQ4Stages - 1 ? 0 : st1 + 1;
    store_a(set, st2);
    fread(1, st0, 1);
    mfma(0);
    store_b(set, st2);
    gload(set, clampk(s + 4));
    fread(0, st1, 0);
    mfma(1);
    // Spread the LDS traffic, the global loads and the dequantisation between
    // the matrix instructions of the step.
#pragma unroll
    for (int i = 0; i < IM * 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
    }
#pragma unroll
    for (int i = 0; i < IM * 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
    }
    __syncthreads();
    st0 = st1;
  };
  uint32_t s = 0;
  for (; s + 1 < steps; s += 2) {
    step(0, s);
    step(1, s + 1);
  }
  if (s < steps) step(0, s);

  // Epilogue: lane holds rows 4 (lane / 16) + r, column lane % 16 of each block.
  const int crow = 4 * (lane >> 4), ccol = lane & 15;
  uint16_t* C = g.q[seg].c;
  if constexpr (kPair) {
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t m = m0 + wm * WTM + 16 * i + crow + r;
        if (m >= g.M) continue;
        uint16_t* out = C + static_cast<uint64_t>(m) * N;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t n = n0 + wn * 32 + 16 * j + ccol;
          if (n >= N) continue;
          const float gate = round_bf(acc[i][j][r]), up = round_bf(acc[i][j + 2][r]);
          out[n] = f2bf(silu(gate) * up);
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t m = m0 + wm * WTM + 16 * i + crow + r;
        if (m >= g.M) continue;
        uint16_t* out = C + static_cast<uint64_t>(m) * N;
        const uint16_t* rin = (EPI == kGemmResidual) ? g.res + static_cast<uint64_t>(m) * N : nullptr;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t n = n0 + wn * 64 + 16 * j + ccol;
          if (n >= N) continue;
          const float v = acc[i][j][r];
          if constexpr (EPI == kGemmStore) {
            out[n] = f2bf(v);
          } else {
            out[n] = f2bf(round_bf(v) + bf2f(rin[n]));
          }
        }
      }
  }
}

// MFMA GEMM over the prepared dense copies with 256 weight rows per block and
// BM prompt rows (256 or 320), epilogues SiLU pair (the 128 gate and 128 up
// rows of 128 output columns) or store (256 output columns of one weight
// segment; segments start at multiples of 256 tiles' columns, tile0 counted in
// 256-column tiles). 8 waves as 2 along M x 4 along N; wave (wm, wn) owns rows
// BM/2 wm .. +BM/2 and four 16-column fragment blocks: for the pair, blocks
// 0, 1 of gate and 2, 3 of up for the same output columns 32 wn .. +32, so the
// epilogue pairs acc[i][j] with acc[i][j + 2] in registers; for the store,
// output columns 64 wn .. +64. Per output element the matrix instructions
// are those of gemm_q4_kernel in the same k order (16x16x32 blocks of k 32 s
// .. 32 s + 31 with the same lane -> k map), so every row tile and both
// kernels give the same bits.
//
// Pipeline per 32-k step s (one barrier per step), LDS stages of
// (BM + 256) x 64 bytes, as many as fit in 160 KB (5 at BM = 256, 4 at 320):
// the step s + NS - 1 loads go straight into LDS (buffer_load_dwordx4 ...
// lds: 64 lanes x 16 B = 1 KB of 64-byte rows per instruction; 4 per wave
// per step, 5 for the waves that also take the rows past 256), the step's
// fragments are read and its matrix instructions run, then each wave waits
// until its step s + 1 loads have landed (the newer ones may still be in
// flight) before the barrier. Rows of A past M and weight rows past N fall
// outside the buffer range and read as zero (their row offset is in the
// range-checked per-lane offset).
constexpr int kDmaThreads = 512, kDmaBK = 32;
constexpr uint32_t kLdsBytes = 160 * 1024;

// One direct-to-LDS load: 16 bytes per lane at LDS address m0 + 16 * lane.
// m0 is written only here; nothing else in the kernel reads it (no indirect
// register indexing or GWS / ordered-count operations).
__device__ inline void lds_load16(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}
// s_waitcnt with vmcnt <= n and the other counters left alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
#define PRG_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14))

template <int EPI, int BM>
__global__ __launch_bounds__(kDmaThreads) void gemm_dma_kernel(const GemmArgs g) {
  static_assert(BM == 256 || BM == 320, "row tile");
  static_assert(EPI == kGemmSiluPair || EPI == kGemmStore, "epilogue");
  constexpr bool kPair = EPI == kGemmSiluPair;
  constexpr uint32_t kStage = (BM + 256) * kDmaBK * 2;
  constexpr int NS = static_cast<int>(kLdsBytes / kStage);  // 5 or 4
  constexpr int IM = BM / 32;                               // 16-row blocks per wave
  constexpr int kExtra = BM / 16 - 16;                      // waves that load a third A group
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const bool extra = wave < kExtra;
  const uint32_t K = g.K, steps = K / kDmaBK;
  // Block -> tile as in gemm_q4_kernel: each XCD walks a contiguous range,
  // tm-fastest within groups of 4 tile rows.
  const uint32_t tiles_m = (g.M + BM - 1) / BM;
  uint32_t tm, tn;
  {
    const uint32_t T = gridDim.x, b = blockIdx.x, x = b % 8, q = T / 8, r = T % 8;
    const uint32_t L = x * q + (x < r ? x : r) + b / 8;
    const uint32_t tiles_n = T / tiles_m;
    const uint32_t width = 4 * tiles_n, first = (L / width) * 4;
    const uint32_t gs = tiles_m - first < 4u ? tiles_m - first : 4u;
    tm = first + (L % width) % gs;
    tn = (L % width) / gs;
  }
  uint32_t seg = 0;
  if constexpr (!kPair) {
#pragma unroll
    for (int i = 1; i < kGemmMaxSegs; ++i)
      if (i < static_cast<int>(g.nq) && tn >= g.q[i].tile0) seg = i;
  }
  const GemmQ4& q0 = g.q[seg];
  const uint32_t N = q0.n;
  const uint32_t m0 = tm * BM, n0 = kPair ? tn * 128 : (tn - q0.tile0) * 256;
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(g.a, static_cast<uint32_t>(static_cast<uint64_t>(g.M) * g.lda * 2));
  const __amdgpu_buffer_rsrc_t rw0 = buffer_rsrc(q0.dense, static_cast<uint32_t>(static_cast<uint64_t>(N) * K * 2));
  const __amdgpu_buffer_rsrc_t rw1 =
      kPair ? buffer_rsrc(g.q[1].dense, static_cast<uint32_t>(static_cast<uint64_t>(N) * K * 2)) : rw0;
  // Wave w loads A rows 16 (w + 8 h) .. +15 for h = 0, 1 (and 256 + 16 w when
  // it is one of the kExtra), and 16 weight rows into LDS rows BM + 16 w and
  // BM + 128 + 16 w: gate and up row n0 + 16 w (pair), or rows n0 + 16 w and
  // n0 + 128 + 16 w of the segment (store); lane l: row + l / 4, chunk l % 4.
  const uint32_t lrow = 16 * wave + (lane >> 2), lch = 8 * (lane & 3);
  uint32_t va[3];
#pragma unroll
  for (int h = 0; h < 3; ++h) va[h] = static_cast<uint32_t>(((m0 + lrow + 128 * h) * g.lda + lch) * 2);
  const uint32_t vw0 = ((n0 + lrow) * K + lch) * 2;
  const uint32_t vw1 = kPair ? vw0 : ((n0 + 128 + lrow) * K + lch) * 2;
  // LDS byte address of the ring (the address-space cast is a C-style cast)
  const uint32_t lbase = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)lds));
  auto issue = [&](uint32_t ks, uint32_t stage) {
    const uint32_t sb = lbase + stage * kStage + 1024 * wave;
    lds_load16(ra, sb, va[0], ks * 64);
    lds_load16(ra, sb + 128 * 64, va[1], ks * 64);
    if (kExtra > 0 && extra) lds_load16(ra, sb + 256 * 64, va[2], ks * 64);
    lds_load16(rw0, sb + BM * 64, vw0, ks * 64);
    lds_load16(rw1, sb + (BM + 128) * 64, vw1, ks * 64);
  };
  // this wave's loads newer than the ones of the step it needs next
  auto wait_next = [&]() {
    if (kExtra > 0 && extra)
      PRG_WAIT_VMCNT(5 * (NS - 2));
    else
      PRG_WAIT_VMCNT(4 * (NS - 2));
  };
  // fragments: lane -> row (lane & 15) of a 16-row block, 16-byte chunk lane >> 4
  const uint32_t fa = (wm * (BM / 2) + (lane & 15)) * 64 + (lane >> 4) * 16;
  uint32_t fb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t brow = kPair ? (j < 2 ? 0 : 128) + wn * 32 + 16 * (j & 1) : wn * 64 + 16 * j;
    fb[j] = (BM + brow + (lane & 15)) * 64 + (lane >> 4) * 16;
  }
  f32x4 acc[IM][4];
#pragma unroll
  for (int i = 0; i < IM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Steps past the end reload the last one (in bounds, never consumed).
  auto clampk = [&](uint32_t k) { return k < steps ? k : steps - 1; };

#pragma unroll
  for (int i = 0; i < NS - 1; ++i) issue(clampk(i), i);
  wait_next();
  __syncthreads();
  uint32_t st = 0;
  for (uint32_t s = 0; s < steps; ++s) {
    // stage of step s + NS - 1: the one step s - 1 read, released by the last barrier
    issue(clampk(s + NS - 1), st == 0 ? NS - 1 : st - 1);
    const uint8_t* base = lds + st * kStage;
    bf16x8 fav[IM], fbv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fbv[j] = *reinterpret_cast<const bf16x8*>(base + fb[j]);
#pragma unroll
    for (int i = 0; i < IM; ++i) fav[i] = *reinterpret_cast<const bf16x8*>(base + fa + i * 1024);
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fav[i], fbv[j], acc[i][j], 0, 0, 0);
    // the first matrix instructions start as soon as their fragments arrive
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    }
    if constexpr (IM > 8) __builtin_amdgcn_sched_group_barrier(0x100, IM - 8, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 4 * IM - 4, 0);
    wait_next();  // this wave's step s + 1 loads have landed
    __syncthreads();
    st = st + 1 == NS ? 0 : st + 1;
  }
  PRG_WAIT_VMCNT(0);

  // Epilogue: lane holds rows 4 (lane / 16) + r, column lane % 16 of each block.
  const int crow = 4 * (lane >> 4), ccol = lane & 15;
  uint16_t* C = q0.c;
#pragma unroll
  for (int i = 0; i < IM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t m = m0 + wm * (BM / 2) + 16 * i + crow + r;
      if (m >= g.M) continue;
      uint16_t* out = C + static_cast<uint64_t>(m) * N;
      if constexpr (kPair) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t n = n0 + wn * 32 + 16 * j + ccol;
          if (n >= N) continue;
          const float gate = round_bf(acc[i][j][r]), up = round_bf(acc[i][j + 2][r]);
          out[n] = f2bf(silu(gate) * up);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t n = n0 + wn * 64 + 16 * j + ccol;
          if (n >= N) continue;
          out[n] = f2bf(acc[i][j][r]);
        }
      }
    }
}

// Row tile per launch: one block per CU (the LDS ring holds one), so a launch
// takes about (rounds of 256 blocks) x BM. 192-row tiles win where they save a
// mostly empty last tile or round (a 1600-row prompt: 7 x 256 rows -> 9 x 192);
// 2048-row chunks and the N = 4096 projections keep 256.
inline uint32_t gemm_device_cus() {
  static const uint32_t cus = []() -> uint32_t {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 256u;
    return static_cast<uint32_t>(prop.multiProcessorCount);
  }();
  return cus;
}

template <int EPI, int BM>
int launch_q4_bm(hipStream_t s, const GemmArgs& g, uint32_t tiles_n, const char* name) {
  const uint32_t tiles = ((g.M + BM - 1) / BM) * tiles_n;
  bool dense = true;
  for (uint32_t i = 0; i < g.nq; ++i) dense = dense && g.q[i].dense != nullptr;
  if (dense)
    hipLaunchKernelGGL((gemm_q4_kernel<EPI, BM, true>), dim3(tiles), dim3(kQ4Threads), 0, s, g);
  else
    hipLaunchKernelGGL((gemm_q4_kernel<EPI, BM, false>), dim3(tiles), dim3(kQ4Threads), 0, s, g);
  PRG_CHECK_LAUNCH(name);
  return PRG_OK;
}

// Rounds of gemm_dma_kernel blocks in units of gemm_q4_kernel rows (its cost
// model: a round of BM-row tiles costs BM; one unit ~ 0.255 us at K = 4096),
// from 1600-token ingest traces: 256-row direct-to-LDS rounds 113 us (445); a
// 320-row round takes 123 / 131 / 139 / 147 us with 80 / 200 / 250 / 240 x 2
// blocks, i.e. mostly the per-block time, so 530 stands for it (q / k / v and
// in_proj take it; the 80-block N = 4096 launches stay on gemm_q4_kernel).
// PEREGRINE_GEMM_DMA = 0 / 256 / 320 forces the 192 / 256-row kernel or that
// row tile of this one, whatever the estimate (all give the same bits).
constexpr uint64_t kDmaRoundCost256 = 445, kDmaRoundCost320 = 530;

inline int dma_override() {
  const char* e = getenv("PEREGRINE_GEMM_DMA");
  if (e == nullptr || e[0] == '\0') return -1;
  return atoi(e);
}

// g: as launch_gemm_q4 leaves it (segments' tile0 in 128-column tiles).
template <int EPI, int BM>
int launch_dma(hipStream_t s, GemmArgs g, uint32_t tiles_n, const char* name) {
  uint64_t rows = 0;
  for (uint32_t i = 0; i < g.nq; ++i) rows = std::max<uint64_t>(rows, g.q[i].n);
  PRG_CHECK_ARG((rows + 256) * g.K * 2 < (1ull << 32) && static_cast<uint64_t>(g.M + BM) * g.lda * 2 < (1ull << 32),
                "%s: operands too large for 32-bit offsets", name);
  if constexpr (EPI == kGemmStore) {
    uint32_t tile = 0;
    for (uint32_t i = 0; i < g.nq; ++i) {
      g.q[i].tile0 = tile;
      tile += (g.q[i].n + 255) / 256;
    }
  }
  const uint32_t tiles = ((g.M + BM - 1) / BM) * tiles_n;
  hipLaunchKernelGGL((gemm_dma_kernel<EPI, BM>), dim3(tiles), dim3(kDmaThreads), 0, s, g);
  PRG_CHECK_LAUNCH(name);
  return PRG_OK;
}

template <int EPI>
int launch_q4_t(hipStream_t s, const GemmArgs& g, const char* name) {
  const uint32_t tiles_n = (EPI == kGemmSiluPair) ? (g.q[0].n + 63) / 64
                                                  : g.q[g.nq - 1].tile0 + (g.q[g.nq - 1].n + 127) / 128;
  const uint32_t cus = gemm_device_cus();
  auto cost = [&](uint32_t bm) -> uint64_t {
    const uint32_t blocks = ((g.M + bm - 1) / bm) * tiles_n;
    return static_cast<uint64_t>((blocks + cus - 1) / cus) * bm;
  };
  if constexpr (EPI == kGemmSiluPair || EPI == kGemmStore) {
    bool dense = true;
    for (uint32_t i = 0; i < g.nq; ++i) dense = dense && g.q[i].dense != nullptr;
    if (dense) {
      // columns per block: 128 outputs of the pair, 256 of a store segment
      uint32_t tiles_nd = 0;
      if constexpr (EPI == kGemmSiluPair) {
        tiles_nd = (g.q[0].n + 127) / 128;
      } else {
        for (uint32_t i = 0; i < g.nq; ++i) tiles_nd += (g.q[i].n + 255) / 256;
      }
      auto cost_dma = [&](uint32_t bm, uint64_t round) -> uint64_t {
        const uint32_t blocks = ((g.M + bm - 1) / bm) * tiles_nd;
        return static_cast<uint64_t>((blocks + cus - 1) / cus) * round;
      };
      const uint64_t c256 = cost_dma(256, kDmaRoundCost256), c320 = cost_dma(320, kDmaRoundCost320);
      const uint64_t cold = std::min(cost(192), cost(256));
      int pick = dma_override();
      if (pick < 0) pick = std::min(c256, c320) < cold ? (c320 < c256 ? 320 : 256) : 0;
      if (pick == 320) return launch_dma<EPI, 320>(s, g, tiles_nd, name);
      if (pick == 256) return launch_dma<EPI, 256>(s, g, tiles_nd, name);
    }
  }
  if (cost(192) < cost(256)) return launch_q4_bm<EPI, 192>(s, g, tiles_n, name);
  return launch_q4_bm<EPI, 256>(s, g, tiles_n, name);
}

template <bool Q4, int EPI>
int launch_t(hipStream_t s, const GemmArgs& g, uint32_t batch, const char* name) {
  constexpr uint32_t kTileN = (EPI == kGemmSiluPair) ? kBN / 2 : kBN;
  uint32_t tiles_n = (g.N + kTileN - 1) / kTileN;
  if (Q4) tiles_n = (EPI == kGemmSiluPair) ? (g.q[0].n + kTileN - 1) / kTileN : g.q[g.nq - 1].tile0 +
                    (g.q[g.nq - 1].n + kTileN - 1) / kTileN;
  const uint32_t tiles = ((g.M + kBM - 1) / kBM) * tiles_n;
  hipLaunchKernelGGL((gemm_kernel<Q4, EPI>), dim3(tiles, 1, batch), dim3(kGemmThreads), 0, s, g);
  PRG_CHECK_LAUNCH(name);
  return PRG_OK;
}

int check_common(const GemmArgs& g, int epi, const char* name) {
  PRG_CHECK_ARG(g.a, "%s: null A", name);
  PRG_CHECK_ARG(g.M > 0 && g.N > 0 && g.K > 0, "%s: empty problem M=%u N=%u K=%u", name, g.M, g.N, g.K);
  PRG_CHECK_ARG(g.lda % 8 == 0 && g.lda_hi % 8 == 0 && g.a_z % 8 == 0,
                "%s: A row strides must be multiples of 8 elements", name);
  PRG_CHECK_ARG(reinterpret_cast<uintptr_t>(g.a) % 16 == 0, "%s: A must be 16-byte aligned", name);
  PRG_CHECK_ARG(epi >= kGemmStore && epi <= kGemmSigmoidGate, "%s: bad epilogue %d", name, epi);
  PRG_CHECK_ARG((epi != kGemmResidual && epi != kGemmSigmoidGate) || g.res, "%s: epilogue needs res", name);
  PRG_CHECK_ARG(static_cast<uint64_t>((g.M + kBM - 1) / kBM) * ((g.N + kBN - 1) / kBN) * 2 < (1ull << 31),
                "%s: grid too large", name);
  return PRG_OK;
}

}  // namespace

namespace {

// Prepared bf16 copy of a Q4 matrix: dense[n][k] = bf16(s*q + b), the values
// the Q4 GEMM stages (dequant_word). One thread per 8-value word.
__global__ __launch_bounds__(256) void dequant_dense_kernel(const uint32_t* __restrict__ w,
                                                            const uint16_t* __restrict__ sc,
                                                            const uint16_t* __restrict__ bi, uint4* __restrict__ out,
                                                            uint64_t words, uint32_t K) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= words) return;
  const uint64_t grp = i / 8;  // 8 words of a row per 64-value group; K % 64 == 0
  (void)K;
  out[i] = dequant_word(__builtin_nontemporal_load(w + i), bf2f(sc[grp]), bf2f(bi[grp]));
}

}  // namespace

namespace prg {

int launch_dequant_dense(hipStream_t s, const uint32_t* w, const uint16_t* sc, const uint16_t* bi, uint16_t* out,
                         uint32_t n, uint32_t K, const char* name) {
  PRG_CHECK_ARG(w && sc && bi && out, "%s: null pointer", name);
  PRG_CHECK_ARG(n > 0 && K > 0 && K % 64 == 0, "%s: shape %u x %u (K must be a multiple of 64)", name, n, K);
  PRG_CHECK_ARG(reinterpret_cast<uintptr_t>(out) % 16 == 0, "%s: output must be 16-byte aligned", name);
  const uint64_t words = static_cast<uint64_t>(n) * K / 8;
  const uint64_t blocks = (words + 255) / 256;
  PRG_CHECK_ARG(blocks < (1ull << 31), "%s: matrix too large", name);
  hipLaunchKernelGGL(dequant_dense_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, w, sc, bi,
                     reinterpret_cast<uint4*>(out), words, K);
  PRG_CHECK_LAUNCH(name);
  return PRG_OK;
}

int launch_gemm_q4(hipStream_t s, GemmArgs g, int epi, const char* name) {
  PRG_CHECK_ARG(g.nq >= 1 && g.nq <= kGemmMaxSegs, "%s: %u weight segments", name, g.nq);
  PRG_CHECK_ARG(epi != kGemmSiluPair || g.nq == 2, "%s: the SiLU pair takes exactly two weights", name);
  PRG_CHECK_ARG(epi != kGemmResidual || g.nq == 1, "%s: the residual epilogue takes one weight", name);
  PRG_CHECK_ARG(epi != kGemmSigmoidGate, "%s: the sigmoid gate epilogue takes bf16 B", name);
  uint32_t tile = 0;
  g.N = 0;
  for (uint32_t i = 0; i < g.nq; ++i) {
    GemmQ4& q = g.q[i];
    PRG_CHECK_ARG(q.w && q.s && q.b && q.n > 0, "%s: Q4 segment %u incomplete", name, i);
    PRG_CHECK_ARG(reinterpret_cast<uintptr_t>(q.w) % 16 == 0, "%s: Q4 weight must be 16-byte aligned", name);
    PRG_CHECK_ARG(epi == kGemmSiluPair ? (i == 1 || q.c) : q.c != nullptr, "%s: null output", name);
    PRG_CHECK_ARG(epi != kGemmSiluPair || q.n == g.q[0].n, "%s: gate and up differ in size", name);
    q.tile0 = tile;
    tile += (q.n + kBN - 1) / kBN;
    g.N += q.n;
  }
  if (int rc = check_common(g, epi, name)) return rc;
  PRG_CHECK_ARG(g.K % 64 == 0, "%s: in_dim %u must be a multiple of 64", name, g.K);
  // 32-bit buffer offsets: the A rows of the last tile and every weight matrix
  // must lie within 4 GiB of their base.
  PRG_CHECK_ARG(static_cast<uint64_t>(g.M + 256) * g.lda * 2 < (1ull << 32), "%s: A too large (M=%u lda=%llu)", name,
                g.M, static_cast<unsigned long long>(g.lda));
  for (uint32_t i = 0; i < g.nq; ++i) {
    PRG_CHECK_ARG(static_cast<uint64_t>(g.q[i].n) * g.K / 2 < (1ull << 32), "%s: Q4 segment %u too large", name, i);
    PRG_CHECK_ARG(!g.q[i].dense || (static_cast<uint64_t>(g.q[i].n) * g.K * 2 < (1ull << 32) &&
                                    reinterpret_cast<uintptr_t>(g.q[i].dense) % 16 == 0),
                  "%s: prepared bf16 copy of segment %u too large or misaligned", name, i);
  }
  PRG_CHECK_ARG(g.a_group == 0 && g.a_z == 0, "%s: Q4 GEMM takes plain [M, K] activations", name);
  switch (epi) {
    case kGemmStore: return launch_q4_t<kGemmStore>(s, g, name);
    case kGemmResidual: return launch_q4_t<kGemmResidual>(s, g, name);
    default: return launch_q4_t<kGemmSiluPair>(s, g, name);
  }
}

int launch_gemm_bf16(hipStream_t s, const GemmArgs& g, int epi, uint32_t batch, const char* name) {
  if (int rc = check_common(g, epi, name)) return rc;
  PRG_CHECK_ARG(g.c, "%s: null C", name);
  PRG_CHECK_ARG(g.b, "%s: null B", name);
  PRG_CHECK_ARG(epi != kGemmSiluPair, "%s: the SiLU pair epilogue takes Q4 weights", name);
  PRG_CHECK_ARG(g.ldb % 8 == 0 && g.b_z % 8 == 0 && reinterpret_cast<uintptr_t>(g.b) % 16 == 0,
                "%s: B rows must be 16-byte aligned", name);
  PRG_CHECK_ARG(batch >= 1 && batch <= 65535, "%s: batch %u", name, batch);
  switch (epi) {
    case kGemmStore: return launch_t<false, kGemmStore>(s, g, batch, name);
    case kGemmResidual: return launch_t<false, kGemmResidual>(s, g, batch, name);
    default: return launch_t<false, kGemmSigmoidGate>(s, g, batch, name);
  }
}

}  // namespace prg

extern "C" {

int prg_q4_qmm_bf16(void* stream, const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                    const uint16_t* biases, uint16_t* out, uint32_t token_count, uint32_t out_dim,
                    uint32_t in_dim) {
  PRG_CHECK_ARG(x && w && scales && biases && out, "prg_q4_qmm_bf16: null pointer");
  GemmArgs g;
  g.a = x;
  g.lda = in_dim;
  g.q[0] = GemmQ4{w, scales, biases, out, out_dim, 0};
  g.nq = 1;
  g.M = token_count;
  g.K = in_dim;
  return launch_gemm_q4(as_stream(stream), g, kGemmStore, "prg_q4_qmm_bf16");
}

int prg_q4_qmm_residual_add_bf16(void* stream, const uint16_t* x, const uint32_t* w,
                                 const uint16_t* scales, const uint16_t* biases,
                                 const uint16_t* residual, uint16_t* out, uint32_t token_count,
                                 uint32_t out_dim, uint32_t in_dim) {
  PRG_CHECK_ARG(x && w && scales && biases && residual && out, "prg_q4_qmm_residual_add_bf16: null pointer");
  GemmArgs g;
  g.a = x;
  g.lda = in_dim;
  g.q[0] = GemmQ4{w, scales, biases, out, out_dim, 0};
  g.nq = 1;
  g.res = residual;
  g.M = token_count;
  g.K = in_dim;
  return launch_gemm_q4(as_stream(stream), g, kGemmResidual, "prg_q4_qmm_residual_add_bf16");
}

int prg_q4_qmm_silu_gate_bf16(void* stream, const uint16_t* x, const uint32_t* gate_w,
                              const uint16_t* gate_scales, const uint16_t* gate_biases,
                              const uint32_t* up_w, const uint16_t* up_scales,
                              const uint16_t* up_biases, uint16_t* out, uint32_t token_count,
                              uint32_t out_dim, uint32_t in_dim) {
  PRG_CHECK_ARG(x && gate_w && gate_scales && gate_biases && up_w && up_scales && up_biases && out,
                "prg_q4_qmm_silu_gate_bf16: null pointer");
  GemmArgs g;
  g.a = x;
  g.lda = in_dim;
  g.q[0] = GemmQ4{gate_w, gate_scales, gate_biases, out, out_dim, 0};
  g.q[1] = GemmQ4{up_w, up_scales, up_biases, nullptr, out_dim, 0};
  g.nq = 2;
  g.M = token_count;
  g.K = in_dim;
  return launch_gemm_q4(as_stream(stream), g, kGemmSiluPair, "prg_q4_qmm_silu_gate_bf16");
}

}  // extern "C"
