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

/* ---------------------------------------------------------- A16 norms ---- */
/* rmsnorm_threadgroup_impl (shaders/rmsnorm.metal:80-116) with the host's
 * 512 threads (src/model/dims.zig:6): thread t sums col = t, t+512, ...;
 * tree over partial_sums with stride 256..1; scale = rsqrt(sum/hidden + eps);
 * out = T(float(x) * scale * float(w)). rsqrt restated as 1/sqrtf. */
#define ORC_NORM_THREADS 512
static float tree_sum(float *partial, int n) {
  for (int stride = n >> 1; stride > 0; stride >>= 1)
    for (int t = 0; t < stride; ++t) partial[t] += partial[t + stride];
  return partial[0];
}

static float rms_scale_ref(const float *v, uint32_t hidden, float eps) {
  float partial[ORC_NORM_THREADS];
  for (int t = 0; t < ORC_NORM_THREADS; ++t) {
    float sum = 0.0f;
    for (uint32_t col = (uint32_t)t; col < hidden; col += ORC_NORM_THREADS) sum += v[col] * v[col];
    partial[t] = sum;
  }
  const float total = tree_sum(partial, ORC_NORM_THREADS);
  return 1.0f / sqrtf(total / (float)hidden + eps);
}

void orc_rmsnorm_bf16(const uint16_t *x, const uint16_t *w, uint16_t *out, uint32_t hidden,
                      uint32_t rows, float eps) {
  float *v = (float *)malloc(sizeof(float) * hidden);
  for (uint32_t r = 0; r < rows; ++r) {
    const uint16_t *xr = x + (size_t)r * hidden;
    for (uint32_t i = 0; i < hidden; ++i) v[i] = orc_bf2f(xr[i]);
    const float scale = rms_scale_ref(v, hidden, eps);
    for (uint32_t i = 0; i < hidden; ++i) out[(size_t)r * hidden + i] = orc_f2bf(v[i] * scale * orc_bf2f(w[i]));
  }
  free(v);
}

/* add_rmsnorm_threadgroup_impl (shaders/rmsnorm.metal:178-220): the residual
 * is rounded to bf16 first and the rounded value is normalised. */
void orc_add_rmsnorm_bf16(const uint16_t *lhs, const uint16_t *rhs, const uint16_t *w,
                          uint16_t *residual_out, uint16_t *norm_out, uint32_t hidden,
                          uint32_t rows, float eps) {
  float *v = (float *)malloc(sizeof(float) * hidden);
  for (uint32_t r = 0; r < rows; ++r) {
    const size_t o = (size_t)r * hidden;
    for (uint32_t i = 0; i < hidden; ++i) {
      residual_out[o + i] = orc_f2bf(orc_bf2f(lhs[o + i]) + orc_bf2f(rhs[o + i]));
      v[i] = orc_bf2f(residual_out[o + i]);
    }
    const float scale = rms_scale_ref(v, hidden, eps);
    for (uint32_t i = 0; i < hidden; ++i) norm_out[o + i] = orc_f2bf(v[i] * scale * orc_bf2f(w[i]));
  }
  free(v);
}

/* ------------------------------------------------------ A18 embedding ---- */
/* q4_embedding_gather_bf16 (shaders/embedding.metal:55-71) */
void orc_q4_embedding_gather_bf16(const uint32_t *w, const uint16_t *s, const uint16_t *b,
                                  uint16_t *out, uint32_t token, uint32_t hidden) {
  const size_t words = hidden / 8, groups = hidden / 64;
  for (uint32_t h = 0; h < hidden; ++h) {
    const uint32_t q = (w[(size_t)token * words + (h >> 3)] >> ((h & 7) * 4)) & 0xF;
    const uint32_t g = h >> 6;
    out[h] = orc_f2bf(orc_bf2f(s[(size_t)token * groups + g]) * (float)q + orc_bf2f(b[(size_t)token * groups + g]));
  }
}

/* ---------------------------------------------------------- A8 conv ------ */
/* conv1d_silu_decode_bf16 (shaders/conv1d.metal:40-62); state f32 [K-1, C]. */
void orc_conv1d_silu_decode_bf16(float *state, const uint16_t *qkv, const uint16_t *w,
                                 uint16_t *out, uint32_t conv_dim, uint32_t kernel_size) {
  const uint32_t km1 = kernel_size - 1;
  for (uint32_t c = 0; c < conv_dim; ++c) {
    const float xnew = orc_bf2f(qkv[c]);
    float acc = 0.0f;
    for (uint32_t j = 0; j < km1; ++j) acc += orc_bf2f(w[c * kernel_size + j]) * state[j * conv_dim + c];
    acc += orc_bf2f(w[c * kernel_size + km1]) * xnew;
    out[c] = orc_f2bf(acc / (1.0f + expf(-acc)));
    for (uint32_t j = 0; j + 1 < km1; ++j) state[j * conv_dim + c] = state[(j + 1) * conv_dim + c];
    if (km1 > 0) state[(km1 - 1) * conv_dim + c] = xnew;
  }
}

/* ------------------------------------------------------------ A9 GDN ----- */
/* gated_delta_decode_h128_fused_bf16 (shaders/gated_delta.metal:147-261):
 * lane L holds dk = L + 32*chunk (chunk 0..3); per-lane sums over chunks in
 * order, then simd_sum. Dk must be 128. */
void orc_gated_delta_decode_bf16(float *state, const uint16_t *conv_out, const uint16_t *a,
                                 const uint16_t *b, const float *A_log, const uint16_t *dt_bias,
                                 uint16_t *y, uint32_t Hk, uint32_t Hv, uint32_t Dk, uint32_t Dv,
                                 uint32_t has_previous_state) {
  const uint32_t key_dim = Hk * Dk;
  for (uint32_t hv = 0; hv < Hv; ++hv) {
    const uint32_t hk = hv / (Hv / Hk);
    const float gate_x = orc_bf2f(a[hv]) + orc_bf2f(dt_bias[hv]);
    const float softplus = fmaxf(gate_x, 0.0f) + logf(1.0f + expf(-fabsf(gate_x)));
    const float decay = expf(-expf(A_log[hv]) * softplus);
    const float beta = 1.0f / (1.0f + expf(-orc_bf2f(b[hv])));
    float qraw[32][4], kraw[32][4], qss[32], kss[32];
    for (int l = 0; l < 32; ++l) {
      qss[l] = kss[l] = 0.0f;
      for (int ch = 0; ch < 4; ++ch) {
        const uint32_t dk = l + ch * 32;
        qraw[l][ch] = orc_bf2f(conv_out[hk * Dk + dk]);
        kraw[l][ch] = orc_bf2f(conv_out[key_dim + hk * Dk + dk]);
        qss[l] += qraw[l][ch] * qraw[l][ch];
        kss[l] += kraw[l][ch] * kraw[l][ch];
      }
    }
    const float q_inv = (1.0f / sqrtf(simd_sum32(qss) + 1.0e-6f)) * (1.0f / sqrtf((float)Dk));
    const float k_inv = 1.0f / sqrtf(simd_sum32(kss) + 1.0e-6f);
    float key[32][4], query[32][4], kql[32];
    for (int l = 0; l < 32; ++l) {
      kql[l] = 0.0f;
      for (int ch = 0; ch < 4; ++ch) {
        query[l][ch] = qraw[l][ch] * q_inv;
        key[l][ch] = kraw[l][ch] * k_inv;
        kql[l] += key[l][ch] * query[l][ch];
      }
    }
    const float kq = simd_sum32(kql);
    for (uint32_t dv = 0; dv < Dv; ++dv) {
      float *row = state + ((size_t)hv * Dv + dv) * Dk;
      float dec[32][4], kvl[32], obl[32];
      for (int l = 0; l < 32; ++l) {
        kvl[l] = obl[l] = 0.0f;
        for (int ch = 0; ch < 4; ++ch) {
          const float s = has_previous_state ? row[l + ch * 32] : 0.0f;
          dec[l][ch] = s * decay;
          kvl[l] += dec[l][ch] * key[l][ch];
          obl[l] += dec[l][ch] * query[l][ch];
        }
      }
      const float kv_mem = simd_sum32(kvl);
      const float ob = simd_sum32(obl);
      const float delta = (orc_bf2f(conv_out[2 * key_dim + hv * Dv + dv]) - kv_mem) * beta;
      for (int l = 0; l < 32; ++l)
        for (int ch = 0; ch < 4; ++ch) row[l + ch * 32] = dec[l][ch] + key[l][ch] * delta;
      y[hv * Dv + dv] = orc_f2bf(ob + delta * kq);
    }
  }
}

/* ----------------------------------------------------- A10 gated norm ---- */
/* rmsnorm_gated_bf16 (shaders/gated_norm.metal:163-189): one serial thread per
 * row. */
void orc_rmsnorm_gated_bf16(const uint16_t *x, const uint16_t *w, const uint16_t *gate,
                            uint16_t *out, uint32_t dim, float eps, uint32_t rows) {
  for (uint32_t r = 0; r < rows; ++r) {
    const uint16_t *xr = x + (size_t)r * dim, *gr = gate + (size_t)r * dim;
    float ss = 0.0f;
    for (uint32_t i = 0; i < dim; ++i) {
      const float v = orc_bf2f(xr[i]);
      ss += v * v;
    }
    const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    for (uint32_t i = 0; i < dim; ++i) {
      const float n = orc_bf2f(xr[i]) * scale * orc_bf2f(w[i]);
      const float gg = orc_bf2f(gr[i]);
      out[(size_t)r * dim + i] = orc_f2bf(n * (gg / (1.0f + expf(-gg))));
    }
  }
}

/* -------------------------------------------------- A12 attn prepare ----- */
/* qwen35_q_gate_prepare_kv_append_pair_head_major_value_dim_major_bf16
 * (shaders/attention.metal:327-421), threads_per_threadgroup = 256
 * (block_attn.zig:35), one value per thread, tree over 256. */
void orc_attn_decode_prepare_bf16(const uint16_t *packed_q, const uint16_t *q_weight,
                                  uint16_t *q_out, uint16_t *gate, const uint16_t *k_in,
                                  const uint16_t *v_in, const uint16_t *k_weight,
                                  uint16_t *key_dst, uint16_t *value_dst, uint32_t num_heads,
                                  uint32_t num_kv_heads, uint32_t head_dim, uint32_t rotary_dim,
                                  uint32_t position_offset, float theta, uint32_t stride,
                                  uint32_t dst) {
  float partial[256];
  for (uint32_t tg = 0; tg < num_heads + num_kv_heads; ++tg) {
    const int use_q = tg < num_heads;
    const uint32_t head = use_q ? tg : tg - num_heads;
    const size_t row_base = (size_t)head * head_dim, packed_base = (size_t)head * 2 * head_dim;
    const uint16_t *w = use_q ? q_weight : k_weight;
    for (uint32_t t = 0; t < 256; ++t) {
      float sum = 0.0f;
      for (uint32_t col = t; col < head_dim; col += 256) {
        const float v = orc_bf2f(use_q ? packed_q[packed_base + col] : k_in[row_base + col]);
        sum += v * v;
        if (use_q) gate[row_base + col] = packed_q[packed_base + head_dim + col];
        else value_dst[(row_base + col) * stride + dst] = v_in[row_base + col];
      }
      partial[t] = sum;
    }
    const float inv_rms = 1.0f / sqrtf(tree_sum(partial, 256) / (float)head_dim + 1.0e-6f);
    const uint32_t half = rotary_dim / 2;
    for (uint32_t p = 0; p < half; ++p) {
      const float s1 = orc_bf2f(use_q ? packed_q[packed_base + p] : k_in[row_base + p]);
      const float s2 = orc_bf2f(use_q ? packed_q[packed_base + p + half] : k_in[row_base + p + half]);
      const float x1 = rbf(s1 * inv_rms * orc_bf2f(w[p]));
      const float x2 = rbf(s2 * inv_rms * orc_bf2f(w[p + half]));
      const float inv_freq = powf(theta, -(2.0f * (float)p) / (float)rotary_dim);
      const float angle = (float)position_offset * inv_freq;
      const float c = cosf(angle), s = sinf(angle);
      const uint16_t r1 = orc_f2bf(x1 * c - x2 * s), r2 = orc_f2bf(x2 * c + x1 * s);
      if (use_q) {
        q_out[row_base + p] = r1;
        q_out[row_base + p + half] = r2;
      } else {
        const size_t kb = ((size_t)head * stride + dst) * head_dim;
        key_dst[kb + p] = r1;
        key_dst[kb + p + half] = r2;
      }
    }
    for (uint32_t col = rotary_dim; col < head_dim; ++col) {
      const float sv = orc_bf2f(use_q ? packed_q[packed_base + col] : k_in[row_base + col]);
      const uint16_t nv = orc_f2bf(sv * inv_rms * orc_bf2f(w[col]));
      if (use_q) q_out[row_base + col] = nv;
      else key_dst[((size_t)head * stride + dst) * head_dim + col] = nv;
    }
  }
}

/* -------------------------------------------- A13/A14 attention decode --- */
/* sdpa_decode_prefix_flash_partials_bf16 (shaders/attention_decode.metal:24-210)
 * with the non-prefix binding (prefix = local cache, prefix_len = 0,
 * block_attn.zig:340-343), then ..._reduce_gated_bf16 (:215-243).
 * 1024-token chunks per kv head; 8 simdgroups take 64-token tiles sg, sg+8..;
 * lane L holds dims 4L..4L+3 and 128+4L..; online softmax per tile; the
 * simdgroup partials are merged in order, then the chunk partials. */
#define ATT_D 256
#define ATT_G 4
typedef struct {
  const uint16_t *q, *K, *V, *gate;
  uint16_t *out;
  uint32_t num_q, num_kv, stride, seq_len, chunk_count;
  float scale;
  float *partials;
} att_ctx;

static void att_partial_one(const att_ctx *c, uint32_t kvh, uint32_t chunk) {
  const uint32_t t_begin = chunk * 1024, t_end = (t_begin + 1024 < c->seq_len) ? t_begin + 1024 : c->seq_len;
  float q[ATT_G][ATT_D];
  for (int g = 0; g < ATT_G; ++g)
    for (int d = 0; d < ATT_D; ++d) q[g][d] = orc_bf2f(c->q[(size_t)(kvh * ATT_G + g) * ATT_D + d]);
  const uint16_t *kb = c->K + (size_t)kvh * c->stride * ATT_D;
  const uint16_t *vb = c->V + (size_t)kvh * ATT_D * c->stride;
  float sg_m[8][ATT_G], sg_den[8][ATT_G];
  static __thread float sg_acc[8][ATT_G][ATT_D];
  for (int sg = 0; sg < 8; ++sg) {
    float m[ATT_G], den[ATT_G];
    for (int g = 0; g < ATT_G; ++g) {
      m[g] = -INFINITY;
      den[g] = 0.0f;
      for (int d = 0; d < ATT_D; ++d) sg_acc[sg][g][d] = 0.0f;
    }
    for (uint32_t tile = (uint32_t)sg; tile < 16; tile += 8) {
      const uint32_t tile_base = t_begin + tile * 64;
      if (tile_base >= t_end) break;
      const uint32_t valid = (t_end - tile_base < 64) ? t_end - tile_base : 64;
      float s[64][ATT_G];
      for (uint32_t tt = 0; tt < 64; ++tt) {
        for (int g = 0; g < ATT_G; ++g) s[tt][g] = -INFINITY;
        if (tt >= valid) continue;
        const uint16_t *kt = kb + (size_t)(tile_base + tt) * ATT_D;
        for (int g = 0; g < ATT_G; ++g) {
          float lanev[32];
          for (int l = 0; l < 32; ++l) {
            float p[4];
            for (int i = 0; i < 4; ++i)
              p[i] = q[g][4 * l + i] * orc_bf2f(kt[4 * l + i]) + q[g][128 + 4 * l + i] * orc_bf2f(kt[128 + 4 * l + i]);
            lanev[l] = p[0] + p[1] + p[2] + p[3];
          }
          s[tt][g] = simd_sum32(lanev) * c->scale;
        }
      }
      float w_t[64][ATT_G];
      for (int g = 0; g < ATT_G; ++g) {
        float tile_max = -INFINITY;
        for (int l = 0; l < 32; ++l) {
          const float a = s[l][g], b2 = s[32 + l][g];
          tile_max = fmaxf(tile_max, fmaxf(a, b2));
        }
        const float m_new = fmaxf(m[g], tile_max);
        const float corr = (m[g] == -INFINITY) ? 0.0f : expf(m[g] - m_new);
        float lw[32];
        for (int l = 0; l < 32; ++l) {
          const float wa = (s[l][g] == -INFINITY) ? 0.0f : expf(s[l][g] - m_new);
          const float wb = (s[32 + l][g] == -INFINITY) ? 0.0f : expf(s[32 + l][g] - m_new);
          w_t[l][g] = wa;
          w_t[32 + l][g] = wb;
          lw[l] = wa + wb;
        }
        den[g] = den[g] * corr + simd_sum32(lw);
        m[g] = m_new;
        for (int d = 0; d < ATT_D; ++d) sg_acc[sg][g][d] *= corr;
      }
      for (int d = 0; d < ATT_D; ++d) {
        const uint16_t *vrow = vb + (size_t)d * c->stride + tile_base;
        float sum_g[ATT_G] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t tt = 0; tt < valid; ++tt) {
          const float vv = orc_bf2f(vrow[tt]);
          for (int g = 0; g < ATT_G; ++g) sum_g[g] += w_t[tt][g] * vv;
        }
        for (int g = 0; g < ATT_G; ++g) sg_acc[sg][g][d] += sum_g[g];
      }
    }
    for (int g = 0; g < ATT_G; ++g) {
      sg_m[sg][g] = m[g];
      sg_den[sg][g] = den[g];
    }
  }
  for (int g = 0; g < ATT_G; ++g) {
    float m_all = -INFINITY;
    for (int i = 0; i < 8; ++i) m_all = fmaxf(m_all, sg_m[i][g]);
    float den_all = 0.0f, outv[ATT_D];
    for (int d = 0; d < ATT_D; ++d) outv[d] = 0.0f;
    for (int i = 0; i < 8; ++i) {
      const float w = (sg_m[i][g] == -INFINITY) ? 0.0f : expf(sg_m[i][g] - m_all);
      den_all += sg_den[i][g] * w;
      for (int d = 0; d < ATT_D; ++d) outv[d] += sg_acc[i][g][d] * w;
    }
    float *dst = c->partials + ((size_t)(kvh * ATT_G + g) * c->chunk_count + chunk) * (ATT_D + 2);
    dst[0] = m_all;
    dst[1] = den_all;
    for (int d = 0; d < ATT_D; ++d) dst[2 + d] = outv[d];
  }
}

static void att_range(void *ctx, size_t b, size_t e) {
  const att_ctx *c = (const att_ctx *)ctx;
  for (size_t i = b; i < e; ++i) att_partial_one(c, (uint32_t)(i / c->chunk_count), (uint32_t)(i % c->chunk_count));
}

void orc_attn_decode_bf16(const uint16_t *q, const uint16_t *K, const uint16_t *V,
                          const uint16_t *gate, uint16_t *out, uint32_t num_q_heads,
                          uint32_t num_kv_heads, uint32_t stride, uint32_t seq_len, float scale) {
  const uint32_t chunk_count = (seq_len + 1023) / 1024;
  float *partials = (float *)malloc(sizeof(float) * num_q_heads * chunk_count * (ATT_D + 2));
  att_ctx c = {q, K, V, gate, out, num_q_heads, num_kv_heads, stride, seq_len, chunk_count, scale, partials};
  parallel_for((size_t)num_kv_heads * chunk_count, att_range, &c);
  for (uint32_t h = 0; h < num_q_heads; ++h)
    for (uint32_t d = 0; d < ATT_D; ++d) {
      const float *base = partials + (size_t)h * chunk_count * (ATT_D + 2);
      float m_all = -INFINITY;
      for (uint32_t ch = 0; ch < chunk_count; ++ch) m_all = fmaxf(m_all, base[ch * (ATT_D + 2)]);
      float den = 0.0f, acc = 0.0f;
      for (uint32_t ch = 0; ch < chunk_count; ++ch) {
        const float *pc = base + ch * (ATT_D + 2);
        const float w = (pc[0] == -INFINITY) ? 0.0f : expf(pc[0] - m_all);
        den += pc[1] * w;
        acc += pc[2 + d] * w;
      }
      const size_t i = (size_t)h * ATT_D + d;
      const float sig = 1.0f / (1.0f + expf(-orc_bf2f(gate[i])));
      out[i] = orc_f2bf((acc / den) * sig);
    }
  free(partials);
}

/* =================================================================== */
/*                         prompt (prefill) path                       */
/* =================================================================== */

/* ------------------------------------------------------- A22 QMM -------- */
/* q4_affine_group64_qmm_nt_bf16_tile_impl (shaders/linear.metal:780-941) and
 * the prepared-dense route it shares semantics with (q4_dequantize_bf16,
 * linear.metal:422-444, then an MLX bf16 NT GEMM): each weight is rounded to
 * bf16 as bf16(s*q + b) before the product; products accumulate in f32 (here
 * in natural k order, the hardware MMA order being unobservable); the output
 * is bf16(acc), and the residual variant (:932-937) stores
 * bf16(float(bf16(acc)) + float(res)). */
typedef struct {
  const uint16_t *x, *residual;
  const uint32_t *w;
  const uint16_t *s, *b;
  uint16_t *out;
  uint32_t M, N, K;
} qmm_ctx;

static void qmm_rows(void *ctx, size_t nb, size_t ne) {
  const qmm_ctx *c = (const qmm_ctx *)ctx;
  const uint32_t words = c->K / 8, groups = c->K / 64;
  float *wrow = (float *)malloc(sizeof(float) * c->K);
  for (size_t n = nb; n < ne; ++n) {
    for (uint32_t k = 0; k < c->K; ++k) {
      const uint32_t q = (c->w[n * words + k / 8] >> ((k & 7u) * 4u)) & 0x0fu;
      const size_t meta = n * groups + k / 64;
      wrow[k] = rbf(orc_bf2f(c->s[meta]) * (float)q + orc_bf2f(c->b[meta]));
    }
    for (uint32_t m = 0; m < c->M; ++m) {
      const uint16_t *xr = c->x + (size_t)m * c->K;
      float acc = 0.0f;
      for (uint32_t k = 0; k < c->K; ++k) acc += orc_bf2f(xr[k]) * wrow[k];
      const size_t o = (size_t)m * c->N + n;
      c->out[o] = c->residual ? orc_f2bf(rbf(acc) + orc_bf2f(c->residual[o])) : orc_f2bf(acc);
    }
  }
  free(wrow);
}

void orc_q4_qmm_bf16(const uint16_t *x, uint32_t M, const uint32_t *w, const uint16_t *s,
                     const uint16_t *b, const uint16_t *residual, uint16_t *out, uint32_t N,
                     uint32_t K) {
  qmm_ctx c = {x, residual, w, s, b, out, M, N, K};
  parallel_for(N, qmm_rows, &c);
}

/* silu_mul_pair_inplace_bf16 (shaders/elementwise.metal:64-73):
 * gate = bf16(silu(gate) * up), silu(g) = g / (1 + exp(-g)). */
void orc_silu_mul_pair_bf16(uint16_t *gate, const uint16_t *up, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float g = orc_bf2f(gate[i]);
    gate[i] = orc_f2bf((g / (1.0f + expf(-g))) * orc_bf2f(up[i]));
  }
}

/* sigmoid_mul_pair_inplace_bf16 (shaders/elementwise.metal:88-99):
 * x = bf16(x * 1/(1 + exp(-gate))). */
void orc_sigmoid_mul_pair_bf16(uint16_t *x, const uint16_t *gate, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float sg = 1.0f / (1.0f + expf(-orc_bf2f(gate[i])));
    x[i] = orc_f2bf(orc_bf2f(x[i]) * sg);
  }
}

/* q4_embedding_gather_many_bf16 (shaders/embedding.metal:73-96). */
void orc_q4_embedding_gather_many_bf16(const uint32_t *w, const uint16_t *s, const uint16_t *b,
                                       const uint32_t *tokens, uint32_t T, uint16_t *out,
                                       uint32_t hidden) {
  for (uint32_t t = 0; t < T; ++t) orc_q4_embedding_gather_bf16(w, s, b, out + (size_t)t * hidden, tokens[t], hidden);
}

/* ------------------------------------------- A23 attention prefill ------ */
/* split_qg_many_bf16 (shaders/layout.metal:68-89): qp [T, H, 2*D] holds
 * q ‖ gate per head. */
void orc_split_qg_many_bf16(const uint16_t *qp, uint16_t *q, uint16_t *gate, uint32_t head_dim,
                            uint32_t heads, uint32_t T) {
  for (uint32_t t = 0; t < T; ++t)
    for (uint32_t h = 0; h < heads; ++h)
      for (uint32_t d = 0; d < head_dim; ++d) {
        const size_t src = ((size_t)t * heads + h) * 2 * head_dim, dst = ((size_t)t * heads + h) * head_dim + d;
        q[dst] = qp[src + d];
        gate[dst] = qp[src + head_dim + d];
      }
}

/* qwen35_qk_norm_rope_append_many_bf16 (shaders/attention.metal:146-220).
 * One 256-thread group per row (q rows then k rows); thread t sums x^2 over
 * d = t, t+256, ..., then a halving tree. The normed value stays f32 through
 * RoPE (unlike the decode prepare, which rounds it to bf16 first). q is
 * rewritten in place; K rows go to cache_k[h, stride, D] at
 * start_cache + t; V rows to cache_v[h, D, stride]. */
void orc_qk_norm_rope_append_many_bf16(uint16_t *q, const uint16_t *q_weight, const uint16_t *k,
                                       const uint16_t *k_weight, const uint16_t *v,
                                       uint16_t *cache_k, uint16_t *cache_v, uint32_t start_rope,
                                       uint32_t T, uint32_t start_cache, uint32_t stride,
                                       uint32_t num_q, uint32_t num_kv, uint32_t head_dim,
                                       uint32_t rotary_dim, float theta) {
  float partial[256];
  const uint32_t q_rows = T * num_q, kv_rows = T * num_kv;
  for (uint32_t rg = 0; rg < q_rows + kv_rows; ++rg) {
    const int is_q = rg < q_rows;
    const uint32_t lr = is_q ? rg : rg - q_rows;
    const uint32_t heads = is_q ? num_q : num_kv;
    const uint32_t t = lr / heads, h = lr - t * heads;
    const uint16_t *src = (is_q ? q : k) + (size_t)lr * head_dim;
    const uint16_t *wt = is_q ? q_weight : k_weight;
    for (uint32_t th = 0; th < 256; ++th) {
      float ss = 0.0f;
      for (uint32_t d = th; d < head_dim; d += 256) ss += orc_bf2f(src[d]) * orc_bf2f(src[d]);
      partial[th] = ss;
    }
    const float scale = 1.0f / sqrtf(tree_sum(partial, 256) / (float)head_dim + 1.0e-6f);
    const uint32_t pos = start_rope + t;
    float x[512];
    for (uint32_t d = 0; d < head_dim; ++d) x[d] = orc_bf2f(src[d]);
    uint16_t *dst = is_q ? q + (size_t)lr * head_dim
                         : cache_k + ((size_t)h * stride + (start_cache + t)) * head_dim;
    const uint32_t half = rotary_dim / 2;
    for (uint32_t i = 0; i < half; ++i) {
      const float a = x[i] * scale * orc_bf2f(wt[i]);
      const float bb = x[i + half] * scale * orc_bf2f(wt[i + half]);
      const float inv_freq = powf(theta, -(2.0f * (float)i) / (float)rotary_dim);
      const float ang = (float)pos * inv_freq;
      const float cs = cosf(ang), sn = sinf(ang);
      dst[i] = orc_f2bf(a * cs - bb * sn);
      dst[i + half] = orc_f2bf(bb * cs + a * sn);
    }
    for (uint32_t d = rotary_dim; d < head_dim; ++d) dst[d] = orc_f2bf(x[d] * scale * orc_bf2f(wt[d]));
    if (!is_q) {
      const uint16_t *vs = v + (size_t)lr * head_dim;
      for (uint32_t d = 0; d < head_dim; ++d)
        cache_v[((size_t)h * head_dim + d) * stride + (start_cache + t)] = vs[d];
    }
  }
}

/* Materialised causal prefill attention (src/model/block_attn.zig:500-631).
 * Per kv head g, rows r = j*T + t (j = q head within the group):
 *   score[r][c] = bf16(sum_d q[t, g*G + j, d] * K[g, c, d])   (MLX NT GEMM,
 *                 f32 accumulation; block_attn.zig:75-109)
 *   prefill_softmax_scaled_masked_bf16 (shaders/attention.metal:1463-1523):
 *     visible iff c <= prefix + t; value = float(score) * scale; 256 threads
 *     stride the row for max and for sum of exp2((v - max) * log2e); each
 *     reduced by a halving tree; p = bf16(exp2(...) / denom) (0 if masked;
 *     denom 0 -> 1)
 *   out[t, g*G + j, d] = bf16(sum_c p[r][c] * V[g, d, c])   (MLX NT GEMM)
 * The gate sigmoid (orc_sigmoid_mul_pair_bf16) is a separate step, as in the
 * reference (block_attn.zig:475-490). */
typedef struct {
  const uint16_t *q, *K, *V;
  uint16_t *out;
  uint32_t T, prefix, stride, num_q, num_kv, D;
  float scale;
} attp_ctx;

static void attp_rows(void *ctx, size_t rb, size_t re) {
  const attp_ctx *c = (const attp_ctx *)ctx;
  const uint32_t G = c->num_q / c->num_kv, L = c->prefix + c->T;
  float *s = (float *)malloc(sizeof(float) * L);
  float *p = (float *)malloc(sizeof(float) * L);
  float partial[256];
  const float log2e = 1.4426950408889634f;
  for (size_t idx = rb; idx < re; ++idx) {
    const uint32_t g = (uint32_t)(idx / ((size_t)G * c->T));
    const uint32_t r = (uint32_t)(idx % ((size_t)G * c->T));
    const uint32_t j = r / c->T, t = r % c->T, hq = g * G + j;
    const uint16_t *qr = c->q + ((size_t)t * c->num_q + hq) * c->D;
    for (uint32_t col = 0; col < L; ++col) {
      const uint16_t *kr = c->K + ((size_t)g * c->stride + col) * c->D;
      float acc = 0.0f;
      for (uint32_t d = 0; d < c->D; ++d) acc += orc_bf2f(qr[d]) * orc_bf2f(kr[d]);
      s[col] = rbf(acc);
    }
    const uint32_t vis = c->prefix + t;
    for (int th = 0; th < 256; ++th) {
      float m = -INFINITY;
      for (uint32_t col = (uint32_t)th; col < L; col += 256) {
        const float v = (col > vis) ? -INFINITY : s[col] * c->scale;
        m = fmaxf(m, v);
      }
      partial[th] = m;
    }
    for (int stride = 128; stride > 0; stride >>= 1)
      for (int th = 0; th < stride; ++th) partial[th] = fmaxf(partial[th], partial[th + stride]);
    const float row_max = partial[0];
    for (int th = 0; th < 256; ++th) {
      float sum = 0.0f;
      for (uint32_t col = (uint32_t)th; col < L; col += 256)
        if (col <= vis) sum += exp2f((s[col] * c->scale - row_max) * log2e);
      partial[th] = sum;
    }
    const float total = tree_sum(partial, 256);
    const float denom = total == 0.0f ? 1.0f : total;
    for (uint32_t col = 0; col < L; ++col)
      p[col] = (col > vis) ? 0.0f : rbf(exp2f((s[col] * c->scale - row_max) * log2e) / denom);
    for (uint32_t d = 0; d < c->D; ++d) {
      const uint16_t *vr = c->V + ((size_t)g * c->D + d) * c->stride;
      float acc = 0.0f;
      for (uint32_t col = 0; col < L; ++col) acc += p[col] * orc_bf2f(vr[col]);
      c->out[((size_t)t * c->num_q + hq) * c->D + d] = orc_f2bf(acc);
    }
  }
  free(s);
  free(p);
}

void orc_attn_prefill_bf16(const uint16_t *q, const uint16_t *cache_k, const uint16_t *cache_v,
                           uint16_t *out, uint32_t T, uint32_t prefix, uint32_t stride,
                           uint32_t num_q, uint32_t num_kv, uint32_t head_dim, float scale) {
  attp_ctx c = {q, cache_k, cache_v, out, T, prefix, stride, num_q, num_kv, head_dim, scale};
  parallel_for((size_t)num_q * T, attp_rows, &c);
}

/* ---------------------------------------------- A24 GDN prefill --------- */
/* conv1d_silu_prefill_vec4_bf16 + conv1d_silu_prefill_state_bf16
 * (shaders/conv1d.metal:136-198). Source index u = t + j over the virtual
 * sequence [state rows 0..K-2 ‖ inputs]; state rows count only when
 * has_previous_state; acc += w[c, j] * x in j order; out = bf16(silu(acc)).
 * The state is then rewritten with the last K-1 entries of that sequence. */
void orc_conv1d_silu_prefill_bf16(float *state, const uint16_t *qkv, const uint16_t *w,
                                  uint16_t *out, uint32_t T, uint32_t conv_dim,
                                  uint32_t kernel_size, uint32_t has_previous_state) {
  const uint32_t km1 = kernel_size - 1;
  for (uint32_t c = 0; c < conv_dim; ++c) {
    for (uint32_t t = 0; t < T; ++t) {
      float acc = 0.0f;
      for (uint32_t j = 0; j < kernel_size; ++j) {
        const uint32_t u = t + j;
        float x = 0.0f;
        if (u < km1) {
          if (has_previous_state) x = state[(size_t)u * conv_dim + c];
        } else if (u - km1 < T) {
          x = orc_bf2f(qkv[(size_t)(u - km1) * conv_dim + c]);
        }
        acc += orc_bf2f(w[(size_t)c * kernel_size + j]) * x;
      }
      out[(size_t)t * conv_dim + c] = orc_f2bf(acc / (1.0f + expf(-acc)));
    }
    float hist[8];
    for (uint32_t j = 0; j < km1; ++j) {
      const uint32_t u = T + j;
      float x = 0.0f;
      if (u < km1) {
        if (has_previous_state) x = state[(size_t)u * conv_dim + c];
      } else if (u - km1 < T) {
        x = orc_bf2f(qkv[(size_t)(u - km1) * conv_dim + c]);
      }
      hist[j] = x;
    }
    for (uint32_t j = 0; j < km1; ++j) state[(size_t)j * conv_dim + c] = hist[j];
  }
}

/* qk_l2norm_prefill_bf16 (shaders/gated_norm.metal:191-245), 128 threads per
 * (token, k-head) row; thread t sums dk = t, t+128, ..., halving tree.
 * q = x * rsqrt(sum q^2 + 1e-6) * rsqrt(Dk); k = x * rsqrt(sum k^2 + 1e-6). */
void orc_qk_l2norm_prefill_bf16(const uint16_t *conv_out, float *qn, float *kn, uint32_t T,
                                uint32_t Hk, uint32_t Dk, uint32_t conv_dim) {
  float qp[128], kp[128];
  const uint32_t key_dim = Hk * Dk;
  for (uint32_t row = 0; row < T * Hk; ++row) {
    const uint32_t t = row / Hk, h = row - t * Hk;
    const uint16_t *qs = conv_out + (size_t)t * conv_dim + (size_t)h * Dk;
    const uint16_t *ks = qs + key_dim;
    for (uint32_t th = 0; th < 128; ++th) {
      float a = 0.0f, b = 0.0f;
      for (uint32_t d = th; d < Dk; d += 128) {
        a += orc_bf2f(qs[d]) * orc_bf2f(qs[d]);
        b += orc_bf2f(ks[d]) * orc_bf2f(ks[d]);
      }
      qp[th] = a;
      kp[th] = b;
    }
    const float qi = 1.0f / sqrtf(tree_sum(qp, 128) + 1.0e-6f);
    const float ki = 1.0f / sqrtf(tree_sum(kp, 128) + 1.0e-6f);
    const float qscale = 1.0f / sqrtf((float)Dk);
    for (uint32_t d = 0; d < Dk; ++d) {
      qn[(size_t)row * Dk + d] = orc_bf2f(qs[d]) * qi * qscale;
      kn[(size_t)row * Dk + d] = orc_bf2f(ks[d]) * ki;
    }
  }
}

/* gating_many_bf16 (shaders/gated_norm.metal:247-268). */
void orc_gating_many_bf16(const float *A_log, const uint16_t *a, const uint16_t *dt_bias,
                          const uint16_t *b, float *g, float *beta, uint32_t Hv, uint32_t T) {
  for (uint32_t t = 0; t < T; ++t)
    for (uint32_t h = 0; h < Hv; ++h) {
      const size_t o = (size_t)t * Hv + h;
      const float x = orc_bf2f(a[o]) + orc_bf2f(dt_bias[h]);
      const float softplus = fmaxf(x, 0.0f) + logf(1.0f + expf(-fabsf(x)));
      g[o] = expf(-expf(A_log[h]) * softplus);
      beta[o] = 1.0f / (1.0f + expf(-orc_bf2f(b[o])));
    }
}

/* gated_delta_prefill_h128_norm_prepared_value_major_r8_bf16
 * (shaders/gated_delta.metal:35-138). Per (hv, dv) row over t = 0..T-1 with
 * prepared f32 q/k [T, Hk, Dk] and gates [T, Hv]; lane L of 32 holds
 * dk = L + 32*chunk; per-lane chunk sums then simd_sum:
 *   kq = sum k*q; d = S*decay; kv = sum d*k; ob = sum d*q;
 *   delta = (v - kv) * beta; S = d + k*delta; y = bf16(ob + delta*kq). */
typedef struct {
  float *state;
  const float *q, *k, *g, *beta;
  const uint16_t *conv_out;
  uint16_t *y;
  uint32_t T, Hk, Hv, Dk, Dv, conv_dim, has_state;
} gdnp_ctx;

static void gdnp_rows(void *ctx, size_t rb, size_t re) {
  const gdnp_ctx *c = (const gdnp_ctx *)ctx;
  const uint32_t key_dim = c->Hk * c->Dk;
  float lanes[32];
  for (size_t idx = rb; idx < re; ++idx) {
    const uint32_t hv = (uint32_t)(idx / c->Dv), dv = (uint32_t)(idx % c->Dv);
    const uint32_t hk = hv / (c->Hv / c->Hk);
    float *srow = c->state + ((size_t)hv * c->Dv + dv) * c->Dk;
    float S[32][4];
    for (int l = 0; l < 32; ++l)
      for (int ch = 0; ch < 4; ++ch) S[l][ch] = c->has_state ? srow[l + 32 * ch] : 0.0f;
    for (uint32_t t = 0; t < c->T; ++t) {
      const float *qk = c->q + ((size_t)t * c->Hk + hk) * c->Dk;
      const float *kk = c->k + ((size_t)t * c->Hk + hk) * c->Dk;
      const float decay = c->g[(size_t)t * c->Hv + hv], beta = c->beta[(size_t)t * c->Hv + hv];
      for (int l = 0; l < 32; ++l) {
        float s = 0.0f;
        for (int ch = 0; ch < 4; ++ch) s += kk[l + 32 * ch] * qk[l + 32 * ch];
        lanes[l] = s;
      }
      const float kq = simd_sum32(lanes);
      float d[32][4], kvl[32], obl[32];
      for (int l = 0; l < 32; ++l) {
        float a = 0.0f, o = 0.0f;
        for (int ch = 0; ch < 4; ++ch) {
          d[l][ch] = S[l][ch] * decay;
          a += d[l][ch] * kk[l + 32 * ch];
          o += d[l][ch] * qk[l + 32 * ch];
        }
        kvl[l] = a;
        obl[l] = o;
      }
      const float kv = simd_sum32(kvl), ob = simd_sum32(obl);
      const float v = orc_bf2f(c->conv_out[(size_t)t * c->conv_dim + 2 * (size_t)key_dim + (size_t)hv * c->Dv + dv]);
      const float delta = (v - kv) * beta;
      for (int l = 0; l < 32; ++l)
        for (int ch = 0; ch < 4; ++ch) S[l][ch] = d[l][ch] + kk[l + 32 * ch] * delta;
      c->y[(size_t)t * c->Hv * c->Dv + (size_t)hv * c->Dv + dv] = orc_f2bf(ob + delta * kq);
    }
    for (int l = 0; l < 32; ++l)
      for (int ch = 0; ch < 4; ++ch) srow[l + 32 * ch] = S[l][ch];
  }
}

void orc_gated_delta_prefill_bf16(float *state, const float *q, const float *k,
                                  const uint16_t *conv_out, const float *g, const float *beta,
                                  uint16_t *y, uint32_t T, uint32_t Hk, uint32_t Hv, uint32_t Dk,
                                  uint32_t Dv, uint32_t conv_dim, uint32_t has_previous_state) {
  gdnp_ctx c = {state, q, k, g, beta, conv_out, y, T, Hk, Hv, Dk, Dv, conv_dim, has_previous_state};
  parallel_for((size_t)Hv * Dv, gdnp_rows, &c);
}
