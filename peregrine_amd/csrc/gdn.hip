// Gated DeltaNet decode: conv1d+SiLU, the delta-rule recurrence, gated RMSNorm.
//
// Reference semantics:
//   conv1d_silu_decode_bf16            shaders/conv1d.metal:40-62
//   gated_delta_decode_h128_fused_bf16 shaders/gated_delta.metal:147-261
//   rmsnorm_gated_bf16                 shaders/gated_norm.metal:163-189
//   composition                        src/model/block_linear.zig:199-263
//
// Recurrence per v-head hv (k/q head hk = hv / (Hv/Hk)), state S[hv] f32
// [Dv, Dk] row-major (row = dv):
//   decay = exp(-exp(A_log) * softplus(a + dt_bias)),  beta = sigmoid(b)
//   q = q_raw * rsqrt(|q_raw|^2 + 1e-6) * rsqrt(Dk),  k = k_raw * rsqrt(|k_raw|^2 + 1e-6)
//   per row: d = S*decay; kv = d.k; ob = d.q; delta = (v - kv)*beta;
//            S = d + k*delta; y = bf16(ob + delta*(k.q))
//
// gfx950 layout: lane j of a half-wave (32 lanes) holds dk = 4j..4j+3 of a
// state row as a float4, so one wave load moves two 512-byte state rows; dot
// products reduce over the 32 lanes of a half-wave. Each block recomputes the
// head's gates and q/k norms (256 values) and updates RPH rows per half-wave.
//   * Unfused (the decode model): 256-thread blocks of 16 rows, 8 blocks per
//     head, 256 blocks in all, so the 4 MiB state stream is spread over the
//     whole chip; block b takes head b mod 32 (one XCD per head). The gated
//     RMSNorm then runs in the out_proj GEMV prologue. In the model each
//     block also computes the head's gate inputs a and b (the in_proj_a /
//     in_proj_b rows of block_linear.zig:229-231) from the in_proj GEMV's
//     normalised row, so that GEMV carries only the qkv and z rows.
//   * Fused gated norm: one 512-thread block per head (16 half-waves x 8 rows)
//     holds all 128 outputs of its head and normalises them in place.
#include "gdn.hpp"
#include "norm.hpp"
#include "q4_gemv.hpp"

namespace {

using namespace prg;

constexpr int kGdnFusedThreads = 512;  // fused gated norm: 16 half-waves x 8 rows = one head
constexpr int kGdnSplitThreads = 256;  // unfused: 8 half-waves x 2 rows = 16 rows per block

__device__ inline float hsum32(float v) { return half_sum32(v); }

// The per-token math, shared by the one- and two-token kernels. Every
// multiply-add is an explicit __fmaf_rn / __fmul_rn / __fadd_rn, so both
// kernels round identically (the two-token verify must equal two single
// steps bit for bit).
//
// A token's inputs are loaded together, before any arithmetic and on
// straight-line code, so the block pays one memory round trip for them (in
// parallel with its state rows) instead of one per dependent step.
template <int RPH>
struct GdnIn {
  uint16_t a, b, dt;  // per-head gate inputs (bf16 bits)
  float alog;
  uint2 q, k;         // this lane's 4 dk of the head's q and k
  uint16_t v[RPH];    // the half-wave's rows of v
};
// GATES: a / b come from gdn_gate_proj instead of memory.
template <int RPH, bool GATES = false>
__device__ inline GdnIn<RPH> gdn_load(const uint16_t* conv_out, const uint16_t* a, const uint16_t* bgate,
                                      const float* A_log, const uint16_t* dt_bias, uint32_t hv, uint32_t hk,
                                      int j, uint32_t row0) {
  GdnIn<RPH> in;
  if constexpr (!GATES) {
    in.a = a[hv];
    in.b = bgate[hv];
  }
  in.dt = dt_bias[hv];
  in.alog = A_log[hv];
  in.q = *reinterpret_cast<const uint2*>(conv_out + hk * kGdnDk + 4 * j);
  in.k = *reinterpret_cast<const uint2*>(conv_out + kGdnKeyDim + hk * kGdnDk + 4 * j);
  const uint16_t* vsrc = conv_out + 2 * kGdnKeyDim + hv * kGdnDv + row0;
#pragma unroll
  for (int r = 0; r < RPH; ++r) in.v[r] = vsrc[r];
  return in;
}

// ---- gate projections in the kernel (GdnGateProj), over a 256-thread
// block: thread t takes a quarter (16 values) of quantisation group t / 4
// of head hv's a and b rows (threads past K / 64 groups load the last group
// and add 0), with the Q4 GEMV's arithmetic: the nibbles unpacked as bf16
// 128 + q, dot2 against the activation pairs in the image's order. The four
// quarters are summed with quad DPP (all four lanes then hold the same bits),
// each group adds s * sum(q x) + b * sum(x), the wave sums go through LDS
// and the block total is (w0 + w1) + (w2 + w3), rounded to bf16 as the GEMV's
// output. One barrier; every block of the head gets the same bits.
constexpr int kGateThreads = 256;
struct GdnGateW {
  uint2 wa, wb;  // 16 nibbles of each row
  uint16_t sa, ba, sb, bb;
};
struct GdnGateX {
  uint4 x[2];  // 16 activation values (image order)
};
__device__ inline uint32_t gdn_gate_group(const GdnGateProj& g, int tid) {
  return min(static_cast<uint32_t>(tid) / 4u, g.K / 64 - 1);
}
__device__ inline GdnGateW gdn_gate_load_w(const GdnGateProj& g, uint32_t hv, int tid) {
  const uint32_t gl = gdn_gate_group(g, tid);
  const size_t meta = static_cast<size_t>(hv) * (g.K / 64) + gl;
  const size_t word = static_cast<size_t>(hv) * (g.K / 8) + 8 * gl + 2 * (tid & 3);
  GdnGateW w;
  w.wa = *reinterpret_cast<const uint2*>(g.wa + word);
  w.wb = *reinterpret_cast<const uint2*>(g.wb + word);
  w.sa = g.sa[meta];
  w.ba = g.ba[meta];
  w.sb = g.sb[meta];
  w.bb = g.bb[meta];
  return w;
}
__device__ inline GdnGateX gdn_gate_load_x(const GdnGateProj& g, uint32_t row, int tid) {
  const uint4* xp = reinterpret_cast<const uint4*>(g.x_image + static_cast<size_t>(row) * (g.K / 2)) +
                    8 * gdn_gate_group(g, tid) + 2 * (tid & 3);
  GdnGateX x;
  x.x[0] = xp[0];
  x.x[1] = xp[1];
  return x;
}
__device__ inline float quad_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  return v;
}
__device__ inline float gdn_gate_qx(uint2 w, const GdnGateX& x, float xsum_part) {
  float aq[2] = {-128.0f * xsum_part, 0.0f};  // removes the 128 offset of the unpacked nibbles
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    uint32_t t[4];
    unpack_q4_word(j == 0 ? w.x : w.y, t);
    const uint32_t xd[4] = {x.x[j].x, x.x[j].y, x.x[j].z, x.x[j].w};
#pragma unroll
    for (int c = 0; c < 4; ++c) aq[c & 1] = dot2_bf16(t[c], xd[c], aq[c & 1]);
  }
  return aq[0] + aq[1];
}
// The wave's share of row r's a and b, into red[r][0..1][wave]; the totals
// are read by gdn_gate_total after a barrier.
__device__ inline void gdn_gate_partial(const GdnGateProj& g, const GdnGateW& w, const GdnGateX& x, int tid,
                                        float (*red)[kGateThreads / kWave]) {
  constexpr uint32_t kOnes = 0x3F803F80u;  // bf16 pair (1, 1)
  float s[2] = {0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t xd[4] = {x.x[j].x, x.x[j].y, x.x[j].z, x.x[j].w};
#pragma unroll
    for (int c = 0; c < 4; ++c) s[c & 1] = dot2_bf16(kOnes, xd[c], s[c & 1]);
  }
  const float xs_part = s[0] + s[1];
  const float xs = quad_sum(xs_part);
  const float qa = quad_sum(gdn_gate_qx(w.wa, x, xs_part));
  const float qb = quad_sum(gdn_gate_qx(w.wb, x, xs_part));
  const bool lead = (tid & 3) == 0 && static_cast<uint32_t>(tid) / 4u < g.K / 64;
  const float va = lead ? __fmaf_rn(bf_lo(w.ba), xs, __fmul_rn(bf_lo(w.sa), qa)) : 0.0f;
  const float vb = lead ? __fmaf_rn(bf_lo(w.bb), xs, __fmul_rn(bf_lo(w.sb), qb)) : 0.0f;
  const float ta = wave_sum_uniform(va), tb = wave_sum_uniform(vb);
  if ((tid & (kWave - 1)) == 0) {
    red[0][tid / kWave] = ta;
    red[1][tid / kWave] = tb;
  }
}
__device__ inline void gdn_gate_total(const float (*red)[kGateThreads / kWave], uint16_t& a, uint16_t& b) {
  a = f2bf((red[0][0] + red[0][1]) + (red[0][2] + red[0][3]));
  b = f2bf((red[1][0] + red[1][1]) + (red[1][2] + red[1][3]));
}

struct GdnGates {
  float decay, beta;
};
// gating_many_bf16 math (shaders/gated_norm.metal:247-268).
template <int RPH>
__device__ inline GdnGates gdn_gates(const GdnIn<RPH>& in) {
  const float gx = __fadd_rn(bf2f(in.a), bf2f(in.dt));
  const float softplus = __fadd_rn(fmaxf(gx, 0.0f), logf(__fadd_rn(1.0f, expf(-fabsf(gx)))));
  return GdnGates{expf(-__fmul_rn(expf(in.alog), softplus)), 1.0f / __fadd_rn(1.0f, expf(-bf2f(in.b)))};
}

// q/k L2 norms (qk_l2norm_prefill_bf16 math, shaders/gated_norm.metal:191-245)
// for lane j of a half-wave (dk = 4j..4j+3), and k.q over the head.
struct GdnQK {
  float qn[4], kn[4], kq;
};
__device__ inline GdnQK gdn_qk(uint2 qv, uint2 kv) {
  const float q[4] = {bf_lo(qv.x), bf_hi(qv.x), bf_lo(qv.y), bf_hi(qv.y)};
  const float k[4] = {bf_lo(kv.x), bf_hi(kv.x), bf_lo(kv.y), bf_hi(kv.y)};
  float qss = 0.f, kss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qss = __fmaf_rn(q[i], q[i], qss);
    kss = __fmaf_rn(k[i], k[i], kss);
  }
  const float q_inv = __fmul_rn(rsqrtf(__fadd_rn(hsum32(qss), 1.0e-6f)), rsqrtf(static_cast<float>(kGdnDk)));
  const float k_inv = rsqrtf(__fadd_rn(hsum32(kss), 1.0e-6f));
  GdnQK r;
  float kq = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r.qn[i] = __fmul_rn(q[i], q_inv);
    r.kn[i] = __fmul_rn(k[i], k_inv);
    kq = __fmaf_rn(r.kn[i], r.qn[i], kq);
  }
  r.kq = hsum32(kq);
  return r;
}

// S & keep bit for bit: keep = 0 gives +0.0 (a fresh sequence), ~0 leaves S.
__device__ inline float4 gdn_mask(float4 S, uint32_t keep) {
  return make_float4(__uint_as_float(__float_as_uint(S.x) & keep), __uint_as_float(__float_as_uint(S.y) & keep),
                     __uint_as_float(__float_as_uint(S.z) & keep), __uint_as_float(__float_as_uint(S.w) & keep));
}

// One state row (this lane's 4 of its 128 dk): d = S*decay; kv = d.k;
// ob = d.q; delta = (v - kv)*beta; S <- d + k*delta; returns bf16(ob + delta*(k.q)).
__device__ inline uint16_t gdn_row(float4& S, const GdnQK& qk, const GdnGates& g, float v) {
  const float d[4] = {__fmul_rn(S.x, g.decay), __fmul_rn(S.y, g.decay), __fmul_rn(S.z, g.decay),
                      __fmul_rn(S.w, g.decay)};
  float kvm = 0.f, ob = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kvm = __fmaf_rn(d[i], qk.kn[i], kvm);
    ob = __fmaf_rn(d[i], qk.qn[i], ob);
  }
  kvm = hsum32(kvm);
  ob = hsum32(ob);
  const float delta = __fmul_rn(__fsub_rn(v, kvm), g.beta);
  S = make_float4(__fmaf_rn(qk.kn[0], delta, d[0]), __fmaf_rn(qk.kn[1], delta, d[1]),
                  __fmaf_rn(qk.kn[2], delta, d[2]), __fmaf_rn(qk.kn[3], delta, d[3]));
  return f2bf(__fmaf_rn(delta, qk.kq, ob));
}

// IN_PLACE: state_out is state (each thread reads its rows before writing
// them); otherwise the two buffers are distinct. NT threads, RPH rows per
// half-wave; FUSE_NORM needs the whole head in one block. GATES: a / b are
// computed from `gp` (GdnGateProj) instead of read.
template <bool IN_PLACE, int NT, int RPH, bool FUSE_NORM, bool GATES>
__global__ __launch_bounds__(NT) void gdn_decode_kernel(
    float* __restrict__ state, const uint16_t* __restrict__ conv_out, const uint16_t* __restrict__ a,
    const uint16_t* __restrict__ bgate, const float* __restrict__ A_log,
    const uint16_t* __restrict__ dt_bias, uint16_t* __restrict__ y_out,
    const StepScalars* __restrict__ step, uint32_t has_state_host,
    const uint16_t* __restrict__ norm_w, const uint16_t* __restrict__ z, float eps, float* __restrict__ state_out,
    const GdnGateProj gp) {
  constexpr int kRowsPerBlock = (NT / 32) * RPH;
  constexpr int kBlocksPerHead = kGdnDv / kRowsPerBlock;
  static_assert(!FUSE_NORM || kBlocksPerHead == 1, "the fused norm needs a whole head per block");
  __shared__ float ysh[kGdnDv];
  __shared__ float red[NT / kWave];

  // Block b takes head b mod 32 and row slice b / 32: the workgroup
  // dispatcher deals blocks to the 8 XCDs round-robin, so every slice of a
  // head runs on the same XCD and its gate weights are fetched into one L2.
  const uint32_t hv = blockIdx.x % kGdnHv;
  const uint32_t hk = hv / (kGdnHv / kGdnHk);
  const int tid = threadIdx.x;
  const int hw = tid >> 5;   // half-wave
  const int j = tid & 31;    // lane in half-wave
  const uint32_t row0 = (blockIdx.x / kGdnHv) * kRowsPerBlock + hw * RPH;  // first dv row
  // State rows for this half-wave, issued first and unconditionally: the
  // step scalars decide only afterwards whether they are used, so the state
  // loads do not wait for the step block's load.
  float4 S[RPH];
  const size_t row_off = (static_cast<size_t>(hv) * kGdnDv + row0) * kGdnDk;
  const float4* srow = reinterpret_cast<const float4*>(state + row_off) + j;
  float4* sout = reinterpret_cast<float4*>((IN_PLACE ? state : state_out) + row_off) + j;
#pragma unroll
  for (int r = 0; r < RPH; ++r) S[r] = srow[r * (kGdnDk / 4)];
  GdnIn<RPH> in = gdn_load<RPH, GATES>(conv_out, a, bgate, A_log, dt_bias, hv, hk, j, row0);
  GdnGateW gw;
  GdnGateX gx;
  __shared__ float gred[GATES ? 2 : 1][kGateThreads / kWave];
  if constexpr (GATES) {
    static_assert(!GATES || NT == kGateThreads, "gate projections need 256-thread blocks");
    gw = gdn_gate_load_w(gp, hv, tid);
    gx = gdn_gate_load_x(gp, 0, tid);
  }
  // A fresh sequence ignores the stored state (it may hold anything): a mask,
  // not a branch, so no wait for the state rows is forced here.
  const bool has_state = step ? (step->rope_pos != 0) : (has_state_host != 0);
  const uint32_t keep = has_state ? 0xffffffffu : 0u;

  if constexpr (GATES) {
    gdn_gate_partial(gp, gw, gx, tid, gred);
    __syncthreads();
    gdn_gate_total(gred, in.a, in.b);
  }
  const GdnGates gates = gdn_gates(in);
  const GdnQK qk = gdn_qk(in.q, in.k);
#pragma unroll
  for (int r = 0; r < RPH; ++r) {
    S[r] = gdn_mask(S[r], keep);
    const uint16_t yb = gdn_row(S[r], qk, gates, bf2f(in.v[r]));
    sout[r * (kGdnDk / 4)] = S[r];
    if (j == 0) {
      if constexpr (FUSE_NORM)
        ysh[row0 + r] = bf2f(yb);
      else
        y_out[hv * kGdnDv + row0 + r] = yb;
    }
  }
  if constexpr (!FUSE_NORM) return;

  // Gated RMSNorm over the head's 128 outputs (shaders/gated_norm.metal:163-189):
  // out = bf16(y * rsqrt(mean(y^2) + eps) * w * silu(z)).
  __syncthreads();
  const float yv = tid < static_cast<int>(kGdnDv) ? ysh[tid] : 0.0f;
  const float ss = block_sum<NT>(yv * yv, red);
  const float scale = rsqrtf(ss / static_cast<float>(kGdnDv) + eps);
  if (tid < static_cast<int>(kGdnDv)) {
    const float n = yv * scale * bf2f(norm_w[tid]);
    const float g = bf2f(z[hv * kGdnDv + tid]);
    y_out[hv * kGdnDv + tid] = f2bf(n * (g / (1.0f + expf(-g))));
  }
}

// Two consecutive tokens (the verify rows) in one launch: token 0 updates the
// state read from `state` and writes it to `snap`, token 1 continues from
// it in registers and writes `state_out` (may equal state). Inputs per token
// r: conv_out + r*8192, a / b + r*32, y_out + r*4096, step[r]. The per-token
// math is the single-token kernel's (gdn_gates, gdn_qk, gdn_row).
template <int NT, int RPH, bool GATES>
__global__ __launch_bounds__(NT) void gdn_decode2_kernel(
    const float* state, float* __restrict__ snap, float* state_out, const uint16_t* __restrict__ conv_out,
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ bgate, const float* __restrict__ A_log,
    const uint16_t* __restrict__ dt_bias, uint16_t* __restrict__ y_out, const StepScalars* __restrict__ step,
    const GdnGateProj gp) {
  constexpr int kRowsPerBlock = (NT / 32) * RPH;
  static_assert(kGdnDv % kRowsPerBlock == 0, "whole row slices per head");
  // Block b takes head b mod 32 and row slice b / 32: the workgroup
  // dispatcher deals blocks to the 8 XCDs round-robin, so every slice of a
  // head runs on the same XCD and its gate weights are fetched into one L2.
  const uint32_t hv = blockIdx.x % kGdnHv;
  const uint32_t hk = hv / (kGdnHv / kGdnHk);
  const int tid = threadIdx.x;
  const int hw = tid >> 5;
  const int j = tid & 31;
  const uint32_t row0 = (blockIdx.x / kGdnHv) * kRowsPerBlock + hw * RPH;
  const size_t row_off = (static_cast<size_t>(hv) * kGdnDv + row0) * kGdnDk;
  float4 S[RPH];
#pragma unroll
  for (int r = 0; r < RPH; ++r) S[r] = reinterpret_cast<const float4*>(state + row_off)[j + r * (kGdnDk / 4)];
  GdnIn<RPH> in[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
    in[t] = gdn_load<RPH, GATES>(conv_out + t * kGdnConvDim, a + t * kGdnHv, bgate + t * kGdnHv, A_log, dt_bias, hv,
                                 hk, j, row0);
  GdnGateW gw;
  GdnGateX gx[2];
  __shared__ float gred[GATES ? 2 : 1][2][kGateThreads / kWave];
  if constexpr (GATES) {
    static_assert(!GATES || NT == kGateThreads, "gate projections need 256-thread blocks");
    gw = gdn_gate_load_w(gp, hv, tid);
#pragma unroll
    for (int t = 0; t < 2; ++t) gx[t] = gdn_gate_load_x(gp, t, tid);
#pragma unroll
    for (int t = 0; t < 2; ++t) gdn_gate_partial(gp, gw, gx[t], tid, gred[t]);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 2; ++t) gdn_gate_total(gred[t], in[t].a, in[t].b);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    // a fresh sequence: the incoming state is ignored (mask, no branch)
    const uint32_t keep = step[t].rope_pos != 0 ? 0xffffffffu : 0u;
    const GdnGates gates = gdn_gates(in[t]);
    const GdnQK qk = gdn_qk(in[t].q, in[t].k);
    float4* dst = reinterpret_cast<float4*>((t == 0 ? snap : state_out) + row_off) + j;
#pragma unroll
    for (int r = 0; r < RPH; ++r) {
      S[r] = gdn_mask(S[r], keep);
      const uint16_t yb = gdn_row(S[r], qk, gates, bf2f(in[t].v[r]));
      dst[r * (kGdnDk / 4)] = S[r];
      if (j == 0) y_out[t * kGdnValDim + hv * kGdnDv + row0 + r] = yb;
    }
  }
}

__global__ void conv1d_decode_kernel(float* __restrict__ state, const uint16_t* __restrict__ qkv,
                                     const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                     uint32_t conv_dim) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= conv_dim) return;
  out[c] = conv1d_silu_step(state, state, w, conv_dim, c, bf2f(qkv[c]));
}

__global__ void rmsnorm_gated_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                     const uint16_t* __restrict__ gate, uint16_t* __restrict__ out,
                                     uint32_t dim, float eps) {
  __shared__ float red[kGdnDv / kWave];
  const size_t off = static_cast<size_t>(blockIdx.x) * dim;
  const uint32_t i = threadIdx.x;
  const float v = i < dim ? bf2f(x[off + i]) : 0.0f;
  const float ss = block_sum<kGdnDv>(v * v, red);
  const float scale = rsqrtf(ss / static_cast<float>(dim) + eps);
  if (i < dim) {
    const float n = v * scale * bf2f(w[i]);
    const float g = bf2f(gate[off + i]);
    out[off + i] = f2bf(n * (g / (1.0f + expf(-g))));
  }
}

// dim == 128: 16 lanes per row (8 values each, 16-byte loads), 16 rows per
// 256-thread block; the sum of squares and the per-value formula are those of
// the out_proj GEMV's gated-norm prologue (8 values per lane in order, then
// the 16-lane DPP row sum), so a row gets the prologue's bits.
__global__ __launch_bounds__(256) void rmsnorm_gated128_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ w,
                                                               const uint16_t* __restrict__ gate,
                                                               uint16_t* __restrict__ out, uint32_t rows, float eps) {
  const uint32_t row = blockIdx.x * 16 + threadIdx.x / 16, j = threadIdx.x % 16;
  if (row >= rows) return;  // a whole DPP row
  const size_t off = static_cast<size_t>(row) * kGdnDv + 8 * j;
  const uint4 v = *reinterpret_cast<const uint4*>(x + off);
  const uint4 wv = *reinterpret_cast<const uint4*>(w + 8 * j);
  const uint4 gv = *reinterpret_cast<const uint4*>(gate + off);
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = bf_lo(d[i]), b = bf_hi(d[i]);
    ss = __fmaf_rn(a, a, ss);
    ss = __fmaf_rn(b, b, ss);
  }
  const float scale = rsqrtf(__fadd_rn(__fmul_rn(row16_sum(ss), 1.0f / kGdnDv), eps));
  const float4 z0 = make_float4(silu(bf_lo(gv.x)), silu(bf_hi(gv.x)), silu(bf_lo(gv.y)), silu(bf_hi(gv.y)));
  const float4 z1 = make_float4(silu(bf_lo(gv.z)), silu(bf_hi(gv.z)), silu(bf_lo(gv.w)), silu(bf_hi(gv.w)));
  *reinterpret_cast<uint4*>(out + off) = gated_rms_apply(v, wv, z0, z1, scale);
}

}  // namespace

namespace prg {

// Checks a GdnGateProj for the in-kernel gate projections.
static int check_gates(const GdnGateProj* g, const char* name) {
  if (!(g->x_image && g->wa && g->sa && g->ba && g->wb && g->sb && g->bb))
    return set_error(PRG_ERR_INVALID_ARG, "%s: gate projections need the activation image and both matrices", name);
  if (g->K == 0 || g->K % 64 != 0 || g->K > kGdnGateProjMaxK)
    return set_error(PRG_ERR_INVALID_ARG, "%s: gate projections need K a multiple of 64 and <= %u (K = %u)", name,
                     kGdnGateProjMaxK, g->K);
  return PRG_OK;
}

int launch_gdn_decode(hipStream_t s, float* state, const uint16_t* conv_out, const uint16_t* a,
                      const uint16_t* b, const float* A_log, const uint16_t* dt_bias,
                      uint16_t* y_out, const StepScalars* step_dev, uint32_t has_state_host,
                      const uint16_t* norm_w, const uint16_t* z, float eps, float* state_out,
                      const GdnGateProj* gates) {
  const bool in_place = !(state_out && state_out != state);
  const GdnGateProj gp = gates ? *gates : GdnGateProj{};
  if (norm_w) {
    if (gates) return set_error(PRG_ERR_INVALID_ARG, "gated_delta_decode: gate projections need the unfused form");
    constexpr int kRph = 8;
    const dim3 grid(kGdnHv);
    if (in_place)
      hipLaunchKernelGGL((gdn_decode_kernel<true, kGdnFusedThreads, kRph, true, false>), grid, dim3(kGdnFusedThreads),
                         0, s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev, has_state_host, norm_w, z, eps,
                         nullptr, gp);
    else
      hipLaunchKernelGGL((gdn_decode_kernel<false, kGdnFusedThreads, kRph, true, false>), grid,
                         dim3(kGdnFusedThreads), 0, s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev,
                         has_state_host, norm_w, z, eps, state_out, gp);
  } else {
    constexpr int kRph = 2;
    const dim3 grid(kGdnHv * (kGdnDv / ((kGdnSplitThreads / 32) * kRph)));
    float* out = in_place ? nullptr : state_out;
    if (gates) {
      if (int rc = check_gates(gates, "gated_delta_decode")) return rc;
      if (in_place)
        hipLaunchKernelGGL((gdn_decode_kernel<true, kGdnSplitThreads, kRph, false, true>), grid,
                           dim3(kGdnSplitThreads), 0, s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev,
                           has_state_host, nullptr, nullptr, 0.0f, out, gp);
      else
        hipLaunchKernelGGL((gdn_decode_kernel<false, kGdnSplitThreads, kRph, false, true>), grid,
                           dim3(kGdnSplitThreads), 0, s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev,
                           has_state_host, nullptr, nullptr, 0.0f, out, gp);
    } else {
      if (in_place)
        hipLaunchKernelGGL((gdn_decode_kernel<true, kGdnSplitThreads, kRph, false, false>), grid,
                           dim3(kGdnSplitThreads), 0, s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev,
                           has_state_host, nullptr, nullptr, 0.0f, out, gp);
      else
        hipLaunchKernelGGL((gdn_decode_kernel<false, kGdnSplitThreads, kRph, false, false>), grid,
                           dim3(kGdnSplitThreads), 0, s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev,
                           has_state_host, nullptr, nullptr, 0.0f, out, gp);
    }
  }
  PRG_CHECK_LAUNCH("gated_delta_decode");
  return PRG_OK;
}

int launch_gdn_decode2(hipStream_t s, const float* state, float* snap, float* state_out, const uint16_t* conv_out,
                       const uint16_t* a, const uint16_t* b, const float* A_log, const uint16_t* dt_bias,
                       uint16_t* y_out, const StepScalars* step_dev, const GdnGateProj* gates) {
  if (!state || !snap || !state_out || !step_dev || snap == state || snap == state_out)
    return set_error(PRG_ERR_INVALID_ARG, "gated_delta_decode2: needs state, a distinct snapshot and step scalars");
  constexpr int kRph = 2;
  const dim3 grid(kGdnHv * (kGdnDv / ((kGdnSplitThreads / 32) * kRph)));
  if (gates) {
    if (int rc = check_gates(gates, "gated_delta_decode2")) return rc;
    hipLaunchKernelGGL((gdn_decode2_kernel<kGdnSplitThreads, kRph, true>), grid, dim3(kGdnSplitThreads), 0, s, state,
                       snap, state_out, conv_out, a, b, A_log, dt_bias, y_out, step_dev, *gates);
  } else {
    hipLaunchKernelGGL((gdn_decode2_kernel<kGdnSplitThreads, kRph, false>), grid, dim3(kGdnSplitThreads), 0, s, state,
                       snap, state_out, conv_out, a, b, A_log, dt_bias, y_out, step_dev, GdnGateProj{});
  }
  PRG_CHECK_LAUNCH("gated_delta_decode2");
  return PRG_OK;
}

}  // namespace prg

extern "C" {

int prg_conv1d_silu_decode_bf16(void* stream, float* state, const uint16_t* qkv,
                                const uint16_t* weight, uint16_t* out, uint32_t conv_dim,
                                uint32_t kernel_size) {
  PRG_CHECK_ARG(state && qkv && weight && out, "prg_conv1d_silu_decode_bf16: null pointer");
  PRG_CHECK_ARG(kernel_size == prg::kGdnConvK, "prg_conv1d_silu_decode_bf16: kernel_size %u != 4", kernel_size);
  PRG_CHECK_ARG(conv_dim > 0, "prg_conv1d_silu_decode_bf16: conv_dim == 0");
  hipLaunchKernelGGL(conv1d_decode_kernel, dim3((conv_dim + 255) / 256), dim3(256), 0,
                     prg::as_stream(stream), state, qkv, weight, out, conv_dim);
  PRG_CHECK_LAUNCH("prg_conv1d_silu_decode_bf16");
  return PRG_OK;
}

int prg_gated_delta_decode_bf16(void* stream, float* state, const uint16_t* conv_out,
                                const uint16_t* a, const uint16_t* b, const float* A_log,
                                const uint16_t* dt_bias, uint16_t* y, uint32_t Hk, uint32_t Hv,
                                uint32_t Dk, uint32_t Dv, uint32_t conv_dim,
                                uint32_t has_previous_state) {
  PRG_CHECK_ARG(state && conv_out && a && b && A_log && dt_bias && y, "prg_gated_delta_decode_bf16: null pointer");
  PRG_CHECK_ARG(Hk == prg::kGdnHk && Hv == prg::kGdnHv && Dk == prg::kGdnDk && Dv == prg::kGdnDv,
                "prg_gated_delta_decode_bf16: only the Qwen3.5 shape Hk=16 Hv=32 Dk=Dv=128 is built");
  PRG_CHECK_ARG(conv_dim >= 2 * Hk * Dk + Hv * Dv, "prg_gated_delta_decode_bf16: conv_dim too small");
  return prg::launch_gdn_decode(prg::as_stream(stream), state, conv_out, a, b, A_log, dt_bias, y, nullptr,
                                has_previous_state, nullptr, nullptr, 0.0f);
}

int prg_gated_delta_decode_norm_bf16(void* stream, float* state, const uint16_t* conv_out,
                                     const uint16_t* a, const uint16_t* b, const float* A_log,
                                     const uint16_t* dt_bias, const uint16_t* norm_weight,
                                     const uint16_t* z, uint16_t* out, float eps,
                                     uint32_t has_previous_state) {
  PRG_CHECK_ARG(state && conv_out && a && b && A_log && dt_bias && norm_weight && z && out,
                "prg_gated_delta_decode_norm_bf16: null pointer");
  return prg::launch_gdn_decode(prg::as_stream(stream), state, conv_out, a, b, A_log, dt_bias, out, nullptr,
                                has_previous_state, norm_weight, z, eps);
}

int prg_rmsnorm_gated_bf16(void* stream, const uint16_t* x, const uint16_t* weight,
                           const uint16_t* gate, uint16_t* out, uint32_t dim, float eps,
                           uint32_t rows) {
  PRG_CHECK_ARG(x && weight && gate && out, "prg_rmsnorm_gated_bf16: null pointer");
  PRG_CHECK_ARG(dim > 0 && dim <= prg::kGdnDv, "prg_rmsnorm_gated_bf16: dim %u must be in (0, 128]", dim);
  PRG_CHECK_ARG(rows > 0, "prg_rmsnorm_gated_bf16: rows == 0");
  // 16 lanes per row with 16-byte accesses when every pointer allows them
  const bool aligned16 = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                           reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
  if (dim == prg::kGdnDv && aligned16)
    hipLaunchKernelGGL(rmsnorm_gated128_kernel, dim3((rows + 15) / 16), dim3(256), 0, prg::as_stream(stream), x,
                       weight, gate, out, rows, eps);
  else
    hipLaunchKernelGGL(rmsnorm_gated_kernel, dim3(rows), dim3(prg::kGdnDv), 0, prg::as_stream(stream), x, weight,
                       gate, out, dim, eps);
  PRG_CHECK_LAUNCH("prg_rmsnorm_gated_bf16");
  return PRG_OK;
}

}  // extern "C"
