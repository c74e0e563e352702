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
//     whole chip. The gated RMSNorm then runs in the out_proj GEMV prologue.
//   * Fused gated norm: one 512-thread block per head (16 half-waves x 8 rows)
//     holds all 128 outputs of its head and normalises them in place.
#include "gdn.hpp"

namespace {

using namespace prg;

constexpr int kGdnFusedThreads = 512;  // fused gated norm: 16 half-waves x 8 rows = one head
constexpr int kGdnSplitThreads = 256;  // unfused: 8 half-waves x 2 rows = 16 rows per block

__device__ inline float hsum32(float v) { return group_sum<32>(v); }

// IN_PLACE: state_out is state (each thread reads its rows before writing
// them); otherwise the two buffers are distinct. NT threads, RPH rows per
// half-wave; FUSE_NORM needs the whole head in one block.
template <bool IN_PLACE, int NT, int RPH, bool FUSE_NORM>
__global__ __launch_bounds__(NT) void gdn_decode_kernel(
    float* __restrict__ state, const uint16_t* __restrict__ conv_out, const uint16_t* __restrict__ a,
    const uint16_t* __restrict__ bgate, const float* __restrict__ A_log,
    const uint16_t* __restrict__ dt_bias, uint16_t* __restrict__ y_out,
    const StepScalars* __restrict__ step, uint32_t has_state_host,
    const uint16_t* __restrict__ norm_w, const uint16_t* __restrict__ z, float eps, float* __restrict__ state_out) {
  constexpr int kRowsPerBlock = (NT / 32) * RPH;
  constexpr int kBlocksPerHead = kGdnDv / kRowsPerBlock;
  static_assert(!FUSE_NORM || kBlocksPerHead == 1, "the fused norm needs a whole head per block");
  __shared__ float ysh[kGdnDv];
  __shared__ float red[NT / kWave];

  const uint32_t hv = blockIdx.x / kBlocksPerHead;
  const uint32_t hk = hv / (kGdnHv / kGdnHk);
  const int tid = threadIdx.x;
  const int hw = tid >> 5;   // half-wave
  const int j = tid & 31;    // lane in half-wave
  const uint32_t row0 = (blockIdx.x % kBlocksPerHead) * kRowsPerBlock + hw * RPH;  // first dv row
  // State rows for this half-wave, issued first and unconditionally: the
  // step scalars decide only afterwards whether they are used, so the state
  // loads do not wait for the step block's load.
  float4 S[RPH];
  const size_t row_off = (static_cast<size_t>(hv) * kGdnDv + row0) * kGdnDk;
  const float4* srow = reinterpret_cast<const float4*>(state + row_off) + j;
  float4* sout = reinterpret_cast<float4*>((IN_PLACE ? state : state_out) + row_off) + j;
#pragma unroll
  for (int r = 0; r < RPH; ++r) S[r] = srow[r * (kGdnDk / 4)];
  const bool has_state = step ? (step->rope_pos != 0) : (has_state_host != 0);
  if (!has_state) {  // a fresh sequence: the stored state is ignored (may hold anything)
#pragma unroll
    for (int r = 0; r < RPH; ++r) S[r] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // Gates (gating_many_bf16 math, shaders/gated_norm.metal:247-268).
  const float gx = bf2f(a[hv]) + bf2f(dt_bias[hv]);
  const float softplus = fmaxf(gx, 0.0f) + logf(1.0f + expf(-fabsf(gx)));
  const float decay = expf(-expf(A_log[hv]) * softplus);
  const float beta = 1.0f / (1.0f + expf(-bf2f(bgate[hv])));

  // q/k L2 norms (qk_l2norm_prefill_bf16 math, shaders/gated_norm.metal:191-245).
  const uint2 qv = *reinterpret_cast<const uint2*>(conv_out + hk * kGdnDk + 4 * j);
  const uint2 kv = *reinterpret_cast<const uint2*>(conv_out + kGdnKeyDim + hk * kGdnDk + 4 * j);
  const float q[4] = {bf_lo(qv.x), bf_hi(qv.x), bf_lo(qv.y), bf_hi(qv.y)};
  const float k[4] = {bf_lo(kv.x), bf_hi(kv.x), bf_lo(kv.y), bf_hi(kv.y)};
  float qss = 0.f, kss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qss += q[i] * q[i];
    kss += k[i] * k[i];
  }
  const float q_inv = rsqrtf(hsum32(qss) + 1.0e-6f) * rsqrtf(static_cast<float>(kGdnDk));
  const float k_inv = rsqrtf(hsum32(kss) + 1.0e-6f);
  float qn[4], kn[4], kq = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qn[i] = q[i] * q_inv;
    kn[i] = k[i] * k_inv;
    kq += kn[i] * qn[i];
  }
  kq = hsum32(kq);

  const uint16_t* vsrc = conv_out + 2 * kGdnKeyDim + hv * kGdnDv + row0;
#pragma unroll
  for (int r = 0; r < RPH; ++r) {
    const float d[4] = {S[r].x * decay, S[r].y * decay, S[r].z * decay, S[r].w * decay};
    float kvm = 0.f, ob = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kvm += d[i] * kn[i];
      ob += d[i] * qn[i];
    }
    kvm = hsum32(kvm);
    ob = hsum32(ob);
    const float delta = (bf2f(vsrc[r]) - kvm) * beta;
    sout[r * (kGdnDk / 4)] = make_float4(d[0] + kn[0] * delta, d[1] + kn[1] * delta,
                                         d[2] + kn[2] * delta, d[3] + kn[3] * delta);
    const uint16_t yb = f2bf(ob + delta * kq);
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

}  // namespace

namespace prg {

int launch_gdn_decode(hipStream_t s, float* state, const uint16_t* conv_out, const uint16_t* a,
                      const uint16_t* b, const float* A_log, const uint16_t* dt_bias,
                      uint16_t* y_out, const StepScalars* step_dev, uint32_t has_state_host,
                      const uint16_t* norm_w, const uint16_t* z, float eps, float* state_out) {
  const bool in_place = !(state_out && state_out != state);
  if (norm_w) {
    constexpr int kRph = 8;
    const dim3 grid(kGdnHv);
    if (in_place)
      hipLaunchKernelGGL((gdn_decode_kernel<true, kGdnFusedThreads, kRph, true>), grid, dim3(kGdnFusedThreads), 0, s,
                         state, conv_out, a, b, A_log, dt_bias, y_out, step_dev, has_state_host, norm_w, z, eps,
                         nullptr);
    else
      hipLaunchKernelGGL((gdn_decode_kernel<false, kGdnFusedThreads, kRph, true>), grid, dim3(kGdnFusedThreads), 0,
                         s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev, has_state_host, norm_w, z, eps,
                         state_out);
  } else {
    constexpr int kRph = 2;
    const dim3 grid(kGdnHv * (kGdnDv / ((kGdnSplitThreads / 32) * kRph)));
    if (in_place)
      hipLaunchKernelGGL((gdn_decode_kernel<true, kGdnSplitThreads, kRph, false>), grid, dim3(kGdnSplitThreads), 0,
                         s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev, has_state_host, nullptr, nullptr,
                         0.0f, nullptr);
    else
      hipLaunchKernelGGL((gdn_decode_kernel<false, kGdnSplitThreads, kRph, false>), grid, dim3(kGdnSplitThreads), 0,
                         s, state, conv_out, a, b, A_log, dt_bias, y_out, step_dev, has_state_host, nullptr, nullptr,
                         0.0f, state_out);
  }
  PRG_CHECK_LAUNCH("gated_delta_decode");
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
  hipLaunchKernelGGL(rmsnorm_gated_kernel, dim3(rows), dim3(prg::kGdnDv), 0, prg::as_stream(stream), x, weight,
                     gate, out, dim, eps);
  PRG_CHECK_LAUNCH("prg_rmsnorm_gated_bf16");
  return PRG_OK;
}

}  // extern "C"
