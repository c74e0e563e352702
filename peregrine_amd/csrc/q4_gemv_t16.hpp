// Q4 GEMV on the matrix cores over the decode layout of the weights.
//
// Math: the MLX affine Q4 group-64 GEMV of q4_gemv.hpp (reference
// shaders/linear.metal:12-19, shaders/linear_decode.metal:13-74),
//   y[n] = sum_g s[n,g] * sum_{k in g} q[n,k] x[k] + b[n,g] * sum_{k in g} x[k].
//
// Decode layout (a copy of an MLX-layout matrix, written once by
// launch_t16_repack): rows in tiles of 16, K in windows of 256. The 2 KiB of
// one (tile, window) are two 1 KiB steps; in step st, lane l = j + 16 c
// (j = l & 15, c = l >> 4) holds the 16 bytes of row 16 tile + j at words
// 32 win + 16 st + 4 c .. +3 of the row, so one dwordx4 wave load reads 1 KiB
// of contiguous memory. Scales and biases follow the same order: entry
// 64 (tile * windows + win) + l is group 4 win + c of row 16 tile + j.
//
// Kernel: a tile's K range is split over the S waves of a block, four
// windows per wave (S = K / 1024), or two (S = K / 512) when the launch has
// few tiles, so a 4096-row matrix still runs 8 waves per tile. Each unpacked word (v_perm_b32 under the byte 0x43:
// bf16 128 + q) is the B operand of a v_mfma_f32_16x16x32_bf16 whose 16
// columns are the tile's rows; the A operand is x from LDS with row i = 4 h + m
// holding activation row m only for the k of group slot h of the window
// (zero elsewhere), so after a window the accumulator lane (j, h) holds
// sum (128 + q) x over group h of row j for each m. The scale and bias are
// applied per window and lane: acc += s * C + (b - 128 s) * sum(x). The four
// lanes of a row and the S waves are summed in a fixed order at the end of
// the tile, so each row's bits do not depend on M: the two-token verify
// (M = 2) reproduces the single-token step (M = 1) row by row.
#pragma once

#include "q4_gemv.hpp"

namespace prg {

constexpr uint32_t kT16Rows = 16;    // rows per tile
constexpr uint32_t kT16WinK = 256;   // K values per window
constexpr uint32_t kT16WaveK = 1024; // K values per wave (four windows)

// The decode layout stores exactly the MLX bytes (N K / 2 of weights, N K / 64
// scales and biases), permuted; shapes it supports: N % 16 == 0, K a multiple
// of 1024 up to 16384.
bool t16_shape_ok(uint32_t N, uint32_t K);

// MLX layout -> decode layout (all three arrays). Returns a PRG_ERR_* code.
int launch_t16_repack(hipStream_t s, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      uint32_t* tw, uint16_t* ts, uint16_t* tb, uint32_t N, uint32_t K);

// True when every segment of p carries decode-layout copies (GemvSeg::tw..)
// and a T16 kernel exists for (M, epilogue, norm, K).
bool t16_usable(const GemvParams& p, int M, int epi, int norm);

// Launch the T16 GEMV (segment tile ranges are filled in here). Argmax
// launches write one entry per block (grid <= kArgmaxMaxWaves) to
// pval / pidx and the block count to p.argmax_waves, like q4_gemv_kernel's
// per-wave entries. Returns a PRG_ERR_* code.
int launch_q4_gemv_t16(hipStream_t s, GemvParams& p, int M, int epi, int norm, const char* name);

}  // namespace prg
