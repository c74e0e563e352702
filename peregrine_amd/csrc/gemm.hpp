// MFMA GEMM for the prompt (prefill) path: C = A * B^T with bf16 operands and
// fp32 accumulation on the gfx950 matrix cores.
//
//   A  bf16 [M, K] (activations, attention probabilities, queries)
//   B  either Q4 weights in the MLX affine group-64 format, dequantised in the
//      kernel to bf16(s*q + b) exactly as the reference's prefill QMM rounds
//      them (shaders/linear.metal:862-873), or a bf16 matrix [N, K] (the K
//      cache for scores, the value-dim-major V cache for P*V)
//   C  bf16 [M, N]
//
// Rows of A and C may be addressed in two levels, row m at
//   base + (m / group) * ld_hi + (m % group) * ld
// which lets the attention GEMMs read queries and write contexts in the
// [token, head, dim] layout directly (rows = head-in-group x token).
//
// Tiling: 256 threads (4 wave64s as 2x2) own a 128x128 output tile; each wave a
// 64x64 sub-tile of 4x4 v_mfma_f32_16x16x32_bf16 blocks. K advances 64 at a
// time (one Q4 scale group) through LDS with a register prefetch of the next
// step's global data. LDS rows are padded to 72 bf16 so the 16-byte fragment
// reads of 16 consecutive rows hit distinct banks.
#pragma once

#include "common.hpp"

namespace prg {

enum GemmEpi : int {
  kGemmStore = 0,     // C = bf16(acc)
  kGemmResidual = 1,  // C = bf16(float(bf16(acc)) + res)          (linear.metal:932-937)
  kGemmSiluPair = 2,  // C = bf16(silu(bf16(acc_gate)) * bf16(acc_up)), two Q4 matrices
                      //     (qmm + silu_mul_pair_inplace_bf16, elementwise.metal:64-73)
  kGemmSigmoidGate = 3,  // C = bf16(float(bf16(acc)) * sigmoid(gate))  (attention context,
                         //     elementwise.metal:88-99); `res` points at the gate
};

constexpr int kGemmMaxSegs = 4;
// Row tile and K step of the bf16 GEMM (attention scores and P.V). The P.V
// GEMM of a causal prefill reads a tile's probabilities up to its last visible
// column rounded up to the K step; the softmax writes its zeros that far.
constexpr uint32_t kGemmBf16RowTile = 128, kGemmBf16KStep = 64;
// Columns [0, result) of the probability rows that the P.V tile holding row
// `row` (of rows = 4 x T per kv head) reads.
__host__ __device__ inline uint32_t causal_pv_columns(uint32_t row, uint32_t T, uint32_t prefix, uint32_t L) {
  const uint32_t m0 = row / kGemmBf16RowTile * kGemmBf16RowTile;
  const uint32_t t_last = m0 % T + (kGemmBf16RowTile - 1) < T ? m0 % T + (kGemmBf16RowTile - 1) : T - 1;
  const uint32_t end = (prefix + t_last + kGemmBf16KStep) / kGemmBf16KStep * kGemmBf16KStep;
  return end < L ? end : L;
}

struct GemmQ4 {
  const uint32_t* w = nullptr;  // u32 [n, K/8]
  const uint16_t* s = nullptr;  // bf16 [n, K/64]
  const uint16_t* b = nullptr;
  uint16_t* c = nullptr;        // bf16 [M, n]
  uint32_t n = 0;
  uint32_t tile0 = 0;           // first output tile of the segment (set by the launcher)
  // Optional prepared copy bf16 [n, K] = dequantised w (launch_dequant_dense).
  // When every segment has one, the kernel stages it instead of
  // dequantising per tile; the results are the same bit for bit.
  const uint16_t* dense = nullptr;
};

struct GemmArgs {
  // A: bf16
  const uint16_t* a = nullptr;
  uint64_t lda = 0, lda_hi = 0, a_z = 0;
  uint32_t a_group = 0;  // 0 = no second level
  // B, bf16 mode: row n at b + n * ldb; columns k >= K read as zero
  const uint16_t* b = nullptr;
  uint64_t ldb = 0, b_z = 0;
  // B, Q4 mode: up to 4 weight segments sharing A, each with its own output
  // [M, n] (one launch for projections that read the same activations). The
  // SiLU pair epilogue takes gate in q[0] and up in q[1] (same n, output
  // q[0].c).
  GemmQ4 q[kGemmMaxSegs];
  uint32_t nq = 0;
  // C (bf16 mode; and the residual / gate input, same addressing)
  uint16_t* c = nullptr;
  const uint16_t* res = nullptr;
  uint64_t ldc = 0, ldc_hi = 0, c_z = 0;
  uint32_t c_group = 0;
  uint32_t M = 0, N = 0, K = 0;
  // Causal attention (bf16 mode; 0 = off): row m is token m % causal_T of the
  // chunk and sees columns [0, causal_prefix + token]. The scores GEMM skips
  // tiles past every row's last visible column (the softmax masks them); the
  // P.V GEMM stops K there (the probabilities past it are exact zeros).
  uint32_t causal_T = 0, causal_prefix = 0;
};

// Q4 weights in g.q[0..nq). K % 64 == 0; A rows 16-byte aligned (lda % 8 == 0).
// The residual epilogue reads g.res [M, q[0].n].
int launch_gemm_q4(hipStream_t s, GemmArgs g, int epi, const char* name);
// Prepared bf16 copy out [n, K] of Q4 weights (w, sc, bi): the values the Q4
// GEMM dequantises per tile.
int launch_dequant_dense(hipStream_t s, const uint32_t* w, const uint16_t* sc, const uint16_t* bi, uint16_t* out,
                         uint32_t n, uint32_t K, const char* name);
// bf16 B, `batch` independent problems along grid.z (offsets a_z, b_z, c_z).
int launch_gemm_bf16(hipStream_t s, const GemmArgs& g, int epi, uint32_t batch, const char* name);

}  // namespace prg
