// Shared device/host helpers for the gfx950 decode-path kernels.
//
// Numeric conventions (every kernel follows them):
//   * activations, norm weights, Q4 scales/biases are bf16 stored as uint16_t;
//   * accumulation is fp32;
//   * f32 -> bf16 is round-to-nearest-even (NaN stays NaN, quieted).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "peregrine_hip.h"

namespace prg {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Per-decode-step scalars. The decode graph keeps them in device memory so one
// captured graph serves every position; kernels read them at run time.
// (Names follow DeviceModel.forwardNextToken's arguments, model.zig:1564-1575.)
struct StepScalars {
  uint32_t token;      // input token id
  uint32_t cache_pos;  // KV slot written this step
  uint32_t rope_pos;   // RoPE position; GDN state is used iff rope_pos != 0
  uint32_t seq_len;    // tokens attended (cache_pos + 1 without a prefix)
};

// Device-resident control block of the token loop (decode_loop.zig:96-160
// without a prefix): step n consumes tokens[n] at position n and records the
// greedy prediction for position n+1 in predictions[n]. While n+1 < prompt_len
// the next input is forced to prompt[n+1] (prompt ingestion / teacher forcing),
// afterwards it is the prediction itself.
struct DecodeCtl {
  StepScalars s;
  uint32_t n;
  uint32_t prompt_len;
  uint32_t capacity;  // KV cache slots; positions never advance past it
  uint32_t overflow;  // set when a step would have exceeded capacity
  // rope_pos - cache_pos (mod 2^32) of the step the loop was entered with,
  // kept for every later step: rope_pos = cache_pos + rope_off.
  uint32_t rope_off;
};

// ---------------------------------------------------------------- bf16 -------
__host__ __device__ inline float bf2f(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// f32 -> bf16 bits: round to nearest even, NaN -> the quiet NaN
// (u >> 16) | 0x40 (the conversion the reference's shaders apply with
// bfloat(f)). One v_cvt_pk_bf16_f32: gfx950's conversion gives exactly these
// bits for every one of the 2^32 inputs (checked exhaustively on the MI355X
// against the bit expression (u + 0x7fff + ((u >> 16) & 1)) >> 16 with the
// NaN case; prg_f32_to_bf16's GPU test pins it against the oracle).
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));
typedef float f32x2_cvt __attribute__((ext_vector_type(2)));
__device__ inline uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }
// Two values in one conversion: lo in bits 0..15, hi in bits 16..31.
__device__ inline uint32_t f2bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_cvt{lo, hi}, bf16x2_cvt));
}

// Round an f32 to the nearest bf16 value and return it as f32.
__device__ inline float round_bf(float f) { return bf2f(f2bf(f)); }

// Low / high bf16 of a packed pair, widened to f32.
__device__ inline float bf_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ inline float bf_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// ------------------------------------------------------------ wave ops -------
constexpr int kWave = 64;

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Sum over aligned groups of `W` lanes (W a power of two <= 64).
template <int W>
__device__ inline float group_sum(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

template <int W>
__device__ inline float group_max(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Block-wide sum for a block of NT threads (NT multiple of 64). `red` must hold
// NT/64 floats of shared memory. Every thread gets the total. The combination
// order is fixed (wave sums, then wave 0..n-1 in order), so every block that
// runs this on the same data produces the same bits.
template <int NT>
__device__ inline float block_sum(float v, float* red) {
  constexpr int NW = NT / kWave;
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  return t;
}

// v_mov_dpp of an f32 (CTRL a DPP control: 0xB1 / 0x4E quad xor 1 / 2,
// 0x141 row_half_mirror, 0x140 row_mirror).
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each 16-lane DPP row. Every lane of the row receives the same bits:
// each step adds a lane's value to its partner's in an order both partners
// share (a + b == b + a), so the rows stay uniform.
__device__ inline float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
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

// Sum over a 256-thread block in a fixed order: wave_sum_uniform per wave,
// then (w0 + w1) + (w2 + w3) from LDS. One barrier; red (4 floats) may be
// written again only after another barrier. Every thread gets the total.
__device__ inline float block_sum256_dpp(float v, float* red) {
  v = wave_sum_uniform(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// v_permlane32_swap / v_permlane16_swap of two floats: returns {new a, new b}.
// Both results are copied out of the builtin's pair into scalars before use.
__device__ inline void swap32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                  false, false);
  const uint32_t x = r[0], y = r[1];
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
__device__ inline void swap16(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                  false, false);
  const uint32_t x = r[0], y = r[1];
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}

// Sum over each 32-lane half of the wave with DPP and one v_permlane16_swap
// (no LDS round trips); every lane of a half receives the same bits:
// (even row total) + (odd row total).
__device__ inline float half_sum32(float v) {
  v = row16_sum(v);
  float a = v, b = v;
  swap16(a, b);  // each lane now holds its own row's total and its partner row's
  return a + b;
}

__device__ inline float silu(float g) { return g / (1.0f + expf(-g)); }
__device__ inline float sigmoid(float g) { return 1.0f / (1.0f + expf(-g)); }

}  // namespace prg

// ------------------------------------------------------------- host side -----
namespace prg {

// Records a message for prg_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace prg

#define PRG_CHECK_ARG(cond, ...)                                      \
  do {                                                                \
    if (!(cond)) return ::prg::set_error(PRG_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)

#define PRG_CHECK_LAUNCH(name)                                                    \
  do {                                                                            \
    hipError_t e__ = hipGetLastError();                                           \
    if (e__ != hipSuccess)                                                        \
      return ::prg::set_error(PRG_ERR_HIP, "%s: launch failed: %s", name,         \
                              hipGetErrorString(e__));                            \
  } while (0)

#define PRG_HIP(call)                                                             \
  do {                                                                            \
    hipError_t e__ = (call);                                                      \
    if (e__ != hipSuccess)                                                        \
      return ::prg::set_error(PRG_ERR_HIP, "%s: %s", #call, hipGetErrorString(e__)); \
  } while (0)
