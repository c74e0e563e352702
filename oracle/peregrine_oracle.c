/*
 * peregrine_oracle.c — TEST INFRASTRUCTURE (parity checker + CPU baseline).
 * Scalar restatement of the reference shader semantics; see the header.
 * Built with -ffp-contract=off so every multiply and add rounds separately,
 * as the reference source is written (build.zig:133-134: no fast-math).
 */
#include "peregrine_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ threads ---- */
static int g_threads = 1;

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 256 ? 256 : n); }
int orc_get_threads(void) { return g_threads; }

typedef void (*range_fn)(void *ctx, size_t begin, size_t end);
typedef struct {
  range_fn fn;
  void *ctx;
  size_t begin, end;
} range_job;

static void *range_thread(void *arg) {
  range_job *j = (range_job *)arg;
  j->fn(j->ctx, j->begin, j->end);
  return NULL;
}

/* Split [0, n) into contiguous chunks; each output row is computed by exactly
 * one thread with the same arithmetic, so results are thread-count invariant. */
static void parallel_for(size_t n, range_fn fn, void *ctx) {
  int t = g_threads;
  if (t <= 1 || n < 2) {
    fn(ctx, 0, n);
    return;
  }
  if ((size_t)t > n) t = (int)n;
  pthread_t th[256];
  range_job jobs[256];
  size_t chunk = (n + t - 1) / t;
  int launched = 0;
  for (int i = 0; i < t; ++i) {
    size_t b = (size_t)i * chunk, e = b + chunk;
    if (b >= n) break;
    if (e > n) e = n;
    jobs[i].fn = fn;
    jobs[i].ctx = ctx;
    jobs[i].begin = b;
    jobs[i].end = e;
    if (pthread_create(&th[i], NULL, range_thread, &jobs[i]) != 0) {
      fn(ctx, b, e);
      jobs[i].fn = NULL;
    }
    launched = i + 1;
  }
  for (int i = 0; i < launched; ++i)
    if (jobs[i].fn) pthread_join(th[i], NULL);
}

/* -------------------------------------------------------------- bf16 ----- */
float orc_bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float rbf(float f) { return orc_bf2f(orc_f2bf(f)); }

/* Metal simd_sum over a 32-lane simdgroup, restated as an xor butterfly
 * (offsets 16, 8, 4, 2, 1); lane 0's value is returned. */
static float simd_sum32(float *v) {
  float t[32];
  for (int off = 16; off > 0; off >>= 1) {
    for (int l = 0; l < 32; ++l) t[l] = v[l] + v[l ^ off];
    memcpy(v, t, sizeof(t));
  }
  return v[0];
}

/* ------------------------------------------------------- A1 dequant ------ */
/* shaders/linear.metal:422-444: q = (packed >> 4*(k&7)) & 0xF,
 * out = bfloat(scale * float(q) + bias). */
void orc_q4_dequantize_bf16(const uint32_t *w, const uint16_t *s, const uint16_t *b,
                            uint16_t *out, uint32_t N, uint32_t K) {
  const uint32_t words = K / 8, groups = K / 64;
  for (uint32_t n = 0; n < N; ++n)
    for (uint32_t k = 0; k < K; ++k) {
      const uint32_t packed = w[(size_t)n * words + k / 8];
      const uint32_t q = (packed >> ((k & 7u) * 4u)) & 0x0fu;
      const size_t meta = (size_t)n * groups + k / 64;
      const float scale = orc_bf2f(s[meta]);
      const float bias = orc_bf2f(b[meta]);
      out[(size_t)n * K + k] = orc_f2bf(scale * (float)q + bias);
    }
}

/* ----------------------------------------------------------- A2 dots ----- */
typedef struct {
  const uint16_t *x;
  uint32_t M;
  const uint32_t *w;
  const uint16_t *s, *b;
  float *dots;
  uint32_t N, K;
} dots_ctx;

/* One output row n for M activation rows, following
 * q4_decode_group64_compute4_bf16 (shaders/linear_decode.metal:13-74) and its
 * x2 sibling (:76-159): lane L handles values [k + 16L, k + 16L + 16) of each
 * 512-wide step; x values 1..3 of each 4 are pre-divided by 16/256/4096 and
 * multiplied by the unshifted masked nibble; result[L] += scale*quant_acc +
 * bias*input_sum; finally simd_sum. */
static void dots_row(const dots_ctx *c, uint32_t n) {
  const uint32_t K = c->K;
  const uint32_t bytes_per_row = K / 2, group_count = K / 64;
  const uint8_t *wb = (const uint8_t *)c->w + (size_t)n * bytes_per_row;
  for (uint32_t m = 0; m < c->M; ++m) {
    const uint16_t *in = c->x + (size_t)m * K;
    float result[32];
    for (int l = 0; l < 32; ++l) result[l] = 0.0f;
    for (uint32_t k = 0; k < K; k += 512) {
      for (uint32_t lane = 0; lane < 32; ++lane) {
        const uint32_t input_base = k + lane * 16;
        float xt[16];
        float input_sum = 0.0f;
        for (uint32_t i = 0; i < 16; i += 4) {
          const float x0 = orc_bf2f(in[input_base + i + 0]);
          const float x1 = orc_bf2f(in[input_base + i + 1]);
          const float x2 = orc_bf2f(in[input_base + i + 2]);
          const float x3 = orc_bf2f(in[input_base + i + 3]);
          input_sum += x0 + x1 + x2 + x3;
          xt[i + 0] = x0;
          xt[i + 1] = x1 / 16.0f;
          xt[i + 2] = x2 / 256.0f;
          xt[i + 3] = x3 / 4096.0f;
        }
        const uint32_t k_byte_offset = k / 2 + lane * 8;
        const uint32_t group_index = k / 64 + lane / 4;
        float quant_acc = 0.0f;
        for (uint32_t pi = 0; pi < 4; ++pi) {
          const uint8_t *pb = wb + k_byte_offset + 2 * pi;
          const uint16_t packed = (uint16_t)(pb[0] | ((uint16_t)pb[1] << 8));
          const uint32_t xb = pi * 4;
          quant_acc += (float)(packed & 0x000f) * xt[xb + 0];
          quant_acc += (float)(packed & 0x00f0) * xt[xb + 1];
          quant_acc += (float)(packed & 0x0f00) * xt[xb + 2];
          quant_acc += (float)(packed & 0xf000) * xt[xb + 3];
        }
        const size_t meta = (size_t)n * group_count + group_index;
        result[lane] += orc_bf2f(c->s[meta]) * quant_acc + orc_bf2f(c->b[meta]) * input_sum;
      }
    }
    c->dots[(size_t)m * c->N + n] = simd_sum32(result);
  }
}

static void dots_range(void *ctx, size_t b, size_t e) {
  for (size_t n = b; n < e; ++n) dots_row((const dots_ctx *)ctx, (uint32_t)n);
}

void orc_q4_dots(const uint16_t *x, uint32_t M, const uint32_t *w, const uint16_t *s,
                 const uint16_t *b, float *dots, uint32_t N, uint32_t K) {
  dots_ctx c = {x, M, w, s, b, dots, N, K};
  parallel_for(N, dots_range, &c);
}

/* -------------------------------------------------------- A3-A7 ---------- */
void orc_q4_gemv_bf16(const uint16_t *x, const uint32_t *w, const uint16_t *s,
                      const uint16_t *b, uint16_t *y, uint32_t M, uint32_t N, uint32_t K) {
  float *d = (float *)malloc(sizeof(float) * (size_t)M * N);
  orc_q4_dots(x, M, w, s, b, d, N, K);
  for (size_t i = 0; i < (size_t)M * N; ++i) y[i] = orc_f2bf(d[i]);
  free(d);
}

void orc_q4_gemv_residual_add_bf16(const uint16_t *x, const uint32_t *w, const uint16_t *s,
                                   const uint16_t *b, const uint16_t *res, uint16_t *out,
                                   uint32_t M, uint32_t N, uint32_t K) {
  float *d = (float *)malloc(sizeof(float) * (size_t)M * N);
  orc_q4_dots(x, M, w, s, b, d, N, K);
  /* linear_decode.metal:188-189: rounded_dot = bfloat(result);
   * output = bfloat(float(rounded_dot) + float(residual)). */
  for (size_t i = 0; i < (size_t)M * N; ++i) out[i] = orc_f2bf(rbf(d[i]) + orc_bf2f(res[i]));
  free(d);
}

void orc_q4_gemv_silu_gate_bf16(const uint16_t *x, const uint32_t *gw, const uint16_t *gs,
                                const uint16_t *gb, const uint32_t *uw, const uint16_t *us,
                                const uint16_t *ub, uint16_t *out, uint32_t M, uint32_t N,
                                uint32_t K) {
  float *g = (float *)malloc(sizeof(float) * (size_t)M * N);
  float *u = (float *)malloc(sizeof(float) * (size_t)M * N);
  orc_q4_dots(x, M, gw, gs, gb, g, N, K);
  orc_q4_dots(x, M, uw, us, ub, u, N, K);
  /* linear_decode.metal:350-353 */
  for (size_t i = 0; i < (size_t)M * N; ++i) {
    const float gate = rbf(g[i]);
    const float up = rbf(u[i]);
    const float silu = gate / (1.0f + expf(-gate));
    out[i] = orc_f2bf(silu * up);
  }
  free(g);
  free(u);
}

void orc_q4_gemv_argmax_partial_bf16(const uint16_t *x, const uint32_t *w, const uint16_t *s,
                                     const uint16_t *b, float *pval, uint32_t *pidx,
                                     uint32_t M, uint32_t N, uint32_t K) {
  float *d = (float *)malloc(sizeof(float) * (size_t)M * N);
  orc_q4_dots(x, M, w, s, b, d, N, K);
  /* linear.metal:228-254: slots 0..7 hold bfloat-rounded logits of rows
   * out_base..out_base+7 in row order; first strict max wins. */
  const uint32_t P = N / 8;
  for (uint32_t m = 0; m < M; ++m)
    for (uint32_t p = 0; p < P; ++p) {
      const float *row = d + (size_t)m * N + (size_t)p * 8;
      float best = rbf(row[0]);
      uint32_t bi = p * 8;
      for (uint32_t slot = 1; slot < 8; ++slot) {
        const float v = rbf(row[slot]);
        if (v > best) {
          best = v;
          bi = p * 8 + slot;
        }
      }
      pval[(size_t)m * P + p] = best;
      pidx[(size_t)m * P + p] = bi;
    }
  free(d);
}

/* shaders/argmax.metal:6-43, simulated thread by thread (256 threads). */
uint32_t orc_argmax_pairs_f32_u32(const float *values, const uint32_t *indices, uint32_t n) {
  float bv[256];
  uint32_t bi[256];
  for (uint32_t tid = 0; tid < 256; ++tid) {
    float best_value = -INFINITY;
    uint32_t best_index = 0;
    for (uint32_t p = tid; p < n; p += 256) {
      const float v = values[p];
      if (v > best_value) {
        best_value = v;
        best_index = indices[p];
      }
    }
    bv[tid] = best_value;
    bi[tid] = best_index;
  }
  for (uint32_t stride = 128; stride > 0; stride /= 2)
    for (uint32_t tid = 0; tid < stride; ++tid)
      if (bv[tid + stride] > bv[tid]) {
        bv[tid] = bv[tid + stride];
        bi[tid] = bi[tid + stride];
      }
  return bi[0];
}
