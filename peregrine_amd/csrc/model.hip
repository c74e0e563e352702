// Decode model layer: weights, per-sequence state, the per-token kernel
// sequence, and the device-resident greedy token loop.
//
// Mirrors the reference's composition (file:line in the reference tree):
//   DeviceModel.encodeStackBf16 / encodeNextTokenBf16     src/model/model.zig:686-809
//   DecoderLayer.decodeStepBf16                           src/model/decoder_layer.zig:461-566, 756-781
//   LinearAttentionBlock.decodeStepBf16                   src/model/block_linear.zig:199-263
//   FullAttentionBlock.decodeStepBf16                     src/model/block_attn.zig:261-359
//   MlpBlock.decodeResidualBf16 / decodeResidual2Bf16     src/model/block_mlp.zig:260-311
//   encodeArgmaxFromHiddenBf16 (final norm, lm_head, argmax) src/model/model.zig:1346-1388
//   ModelState (GDN conv/recurrent state, bf16 KV caches)  src/model/state.zig:11-118
//   decodeFromPrefixCache                                 src/server/decode_loop.zig:96-160
//
// Where the reference runs a separate dispatch for a norm, a residual add or
// the conv, this layer fuses it into the neighbouring kernel with the same
// rounding points:
//   input_layernorm / post_attention_layernorm / final norm -> GEMV prologue
//   conv1d_silu_decode -> in_proj_qkv GEMV epilogue
//   add_rmsnorm's add (bf16(x + bf16(attn))) -> out_proj / o_proj residual epilogue
//   rmsnorm_gated -> out_proj GEMV prologue (per-head norm x silu(z))
// giving 5 launches per GDN layer, 7 per attention layer and 3 for embed + tail.
// One token's launches are captured once into a HIP graph; the token, positions
// and sequence length live in device memory (DecodeCtl) and are advanced by the
// argmax kernel, so replaying the graph runs the greedy loop with no host sync.
// The prompt path lives in model_prefill.hip, the MTP drafter and speculative
// loop in model_spec.hip.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "model.hpp"
#include "q4_gemv_t16.hpp"

namespace prg {
namespace {

// ------------------------------------------------------------------ RNG ----
__device__ __host__ inline uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
__device__ inline float u01(uint64_t h) { return static_cast<float>(h >> 40) * (1.0f / 16777216.0f); }
__device__ inline float normal01(uint64_t key, uint64_t i) {
  const float u1 = fmaxf(u01(mix64(key ^ (2 * i))), 1.0e-7f);
  const float u2 = u01(mix64(key ^ (2 * i + 1)));
  return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

enum FillKind : int { kFillBits = 0, kFillUniform = 1, kFillNormal = 2, kFillQ4Bias = 3 };

// Fill `n` elements. bits: u32 words; uniform/normal: bf16 (or f32 when f32);
// q4 bias: bf16(-7.5 * scale[i] + N(0, std)).
__global__ void fill_kernel(void* dst, size_t n, uint64_t key, int kind, float a, float b, int f32,
                            const uint16_t* scale) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (kind == kFillBits) {
    static_cast<uint32_t*>(dst)[i] = static_cast<uint32_t>(mix64(key ^ i));
    return;
  }
  float v;
  if (kind == kFillUniform)
    v = a + (b - a) * u01(mix64(key ^ i));
  else if (kind == kFillNormal)
    v = a + b * normal01(key, i);
  else
    v = -7.5f * bf2f(scale[i]) + b * normal01(key, i);
  if (f32)
    static_cast<float*>(dst)[i] = v;
  else
    static_cast<uint16_t*>(dst)[i] = f2bf(v);
}

// ------------------------------------------------------------ builders -----
struct Builder {
  PrgModel* m;
  uint64_t seed;
  uint64_t tensor_id = 0;
  size_t offset = 0;
  bool sizing = true;
  struct Fill {
    void* dst;
    size_t n;
    int kind;
    float a, b;
    int f32;
    const uint16_t* scale;
    uint64_t key;
  };
  std::vector<Fill> fills;

  void* take(const std::string& name, size_t bytes, const char* dtype, std::vector<uint64_t> shape) {
    const size_t off = offset;
    offset = align_up(offset + bytes, kAlign);
    if (sizing) return nullptr;
    void* p = m->arena + off;
    m->tensors[name] = TensorRef{p, bytes};
    m->specs[name] = TensorSpec{dtype, std::move(shape)};
    return p;
  }
  uint64_t next_key() { return mix64(seed ^ mix64(++tensor_id * 0x632be59bd9b4e019ull)); }

  Q4Linear q4(const std::string& base, uint32_t out_dim, uint32_t in_dim) {
    Q4Linear l;
    l.out_dim = out_dim;
    l.in_dim = in_dim;
    const size_t nw = static_cast<size_t>(out_dim) * in_dim / 8, ng = static_cast<size_t>(out_dim) * in_dim / 64;
    // checkpoint shapes: weight u32 [out, in/8], scales / biases bf16 [out, in/64]
    l.weight = static_cast<uint32_t*>(take(base + ".weight", nw * 4, "U32", {out_dim, in_dim / 8u}));
    l.scales = static_cast<uint16_t*>(take(base + ".scales", ng * 2, "BF16", {out_dim, in_dim / 64u}));
    l.biases = static_cast<uint16_t*>(take(base + ".biases", ng * 2, "BF16", {out_dim, in_dim / 64u}));
    const uint64_t k0 = next_key(), k1 = next_key(), k2 = next_key();
    if (!sizing) {
      fills.push_back({l.weight, nw, kFillBits, 0, 0, 0, nullptr, k0});
      fills.push_back({l.scales, ng, kFillUniform, 0.002f, 0.02f, 0, nullptr, k1});
      fills.push_back({l.biases, ng, kFillQ4Bias, 0.0f, 0.01f, 0, l.scales, k2});
    }
    return l;
  }
  uint16_t* bf16(const std::string& name, size_t n, float mean, float stddev, std::vector<uint64_t> shape = {}) {
    if (shape.empty()) shape = {n};
    auto* p = static_cast<uint16_t*>(take(name, n * 2, "BF16", std::move(shape)));
    const uint64_t k = next_key();
    if (!sizing) fills.push_back({p, n, kFillNormal, mean, stddev, 0, nullptr, k});
    return p;
  }
  float* f32(const std::string& name, size_t n, float mean, float stddev) {
    auto* p = static_cast<float*>(take(name, n * 4, "F32", {n}));
    const uint64_t k = next_key();
    if (!sizing) fills.push_back({p, n, kFillNormal, mean, stddev, 1, nullptr, k});
    return p;
  }
};

}  // namespace

bool is_linear_layer(const PrgModelConfig& c, uint32_t i) {  // decoder_layer.zig:29-31
  return (i + 1) % c.full_attention_interval != 0;
}

uint32_t cache_stride_for(uint32_t max_seq) {  // state.zig:25-32
  const uint32_t a = max_seq >= 16000 ? 64u : 256u;
  return (max_seq + a - 1) / a * a;
}

namespace {

// Full-attention decoder layer weights under `p` (decoder_layer.zig:376-412).
void build_full_attention_layer(Builder& b, DecoderLayer& L, const std::string& p, const PrgModelConfig& c) {
  L.linear = false;
  L.input_norm = b.bf16(p + ".input_layernorm.weight", c.hidden, 1.0f, 0.1f);
  L.post_norm = b.bf16(p + ".post_attention_layernorm.weight", c.hidden, 1.0f, 0.1f);
  const std::string a = p + ".self_attn";
  L.full.q_proj = b.q4(a + ".q_proj", 2 * kAttnQHeads * kAttnHeadDim, c.hidden);
  L.full.k_proj = b.q4(a + ".k_proj", kAttnKvHeads * kAttnHeadDim, c.hidden);
  L.full.v_proj = b.q4(a + ".v_proj", kAttnKvHeads * kAttnHeadDim, c.hidden);
  L.full.o_proj = b.q4(a + ".o_proj", c.hidden, kAttnQHeads * kAttnHeadDim);
  L.full.q_norm = b.bf16(a + ".q_norm.weight", kAttnHeadDim, 1.0f, 0.1f);
  L.full.k_norm = b.bf16(a + ".k_norm.weight", kAttnHeadDim, 1.0f, 0.1f);
}

void build_mlp(Builder& b, DecoderLayer& L, const std::string& p, const PrgModelConfig& c) {
  const std::string mp = p + ".mlp";
  L.mlp.gate_proj = b.q4(mp + ".gate_proj", c.intermediate, c.hidden);
  L.mlp.up_proj = b.q4(mp + ".up_proj", c.intermediate, c.hidden);
  L.mlp.down_proj = b.q4(mp + ".down_proj", c.hidden, c.intermediate);
}

void build_model(Builder& b) {
  PrgModel* m = b.m;
  const PrgModelConfig& c = m->cfg;
  const std::string root = "language_model.model";
  m->embed = b.q4(root + ".embed_tokens", c.vocab, c.hidden);
  m->layers.assign(c.num_layers, DecoderLayer{});
  for (uint32_t i = 0; i < c.num_layers; ++i) {
    DecoderLayer& L = m->layers[i];
    const std::string p = root + ".layers." + std::to_string(i);
    if (is_linear_layer(c, i)) {
      L.linear = true;
      L.input_norm = b.bf16(p + ".input_layernorm.weight", c.hidden, 1.0f, 0.1f);
      L.post_norm = b.bf16(p + ".post_attention_layernorm.weight", c.hidden, 1.0f, 0.1f);
      const std::string a = p + ".linear_attn";
      L.lin.in_qkv = b.q4(a + ".in_proj_qkv", kGdnConvDim, c.hidden);
      L.lin.in_z = b.q4(a + ".in_proj_z", kGdnValDim, c.hidden);
      L.lin.in_a = b.q4(a + ".in_proj_a", kGdnHv, c.hidden);
      L.lin.in_b = b.q4(a + ".in_proj_b", kGdnHv, c.hidden);
      L.lin.out_proj = b.q4(a + ".out_proj", c.hidden, kGdnValDim);
      // MLX Conv1d layout [channels, kernel, in_channels / groups]
      L.lin.conv_weight = b.bf16(a + ".conv1d.weight", static_cast<size_t>(kGdnConvDim) * kGdnConvK, 0.0f, 0.5f,
                                 {kGdnConvDim, kGdnConvK, 1});
      L.lin.a_log = b.f32(a + ".A_log", kGdnHv, 0.0f, 0.5f);
      L.lin.dt_bias = b.bf16(a + ".dt_bias", kGdnHv, 0.0f, 0.5f);
      L.lin.norm_weight = b.bf16(a + ".norm.weight", kGdnDv, 1.0f, 0.1f);
    } else {
      build_full_attention_layer(b, L, p, c);
    }
    build_mlp(b, L, p, c);
  }
  m->final_norm = b.bf16(root + ".norm.weight", c.hidden, 1.0f, 0.1f);
  m->lm_head = b.q4("language_model.lm_head", c.vocab, c.hidden);
  if (c.mtp_layers) {  // mtp.zig:72-116 (tensor names under the "mtp." root)
    MtpWeights& t = m->mtp;
    t.present = true;
    t.pre_fc_norm_embedding = b.bf16("mtp.pre_fc_norm_embedding.weight", c.hidden, 1.0f, 0.1f);
    t.pre_fc_norm_hidden = b.bf16("mtp.pre_fc_norm_hidden.weight", c.hidden, 1.0f, 0.1f);
    t.fc = b.q4("mtp.fc", c.hidden, 2 * c.hidden);
    build_full_attention_layer(b, t.layer, "mtp.layers.0", c);
    build_mlp(b, t.layer, "mtp.layers.0", c);
    t.norm = b.bf16("mtp.norm.weight", c.hidden, 1.0f, 0.1f);
  }
}

}  // namespace

int layout_model(PrgModel* m) {
  Builder sizing{m, 0};
  build_model(sizing);
  m->arena_bytes = sizing.offset;
  const hipError_t e = hipMalloc(reinterpret_cast<void**>(&m->arena), m->arena_bytes);
  if (e != hipSuccess) {
    m->arena = nullptr;
    return set_error(PRG_ERR_OOM, "model weights: hipMalloc(%zu): %s", sizing.offset, hipGetErrorString(e));
  }
  Builder b{m, 0};
  b.sizing = false;
  build_model(b);
  return PRG_OK;
}

namespace {

int validate_config(const PrgModelConfig& c) {
  PRG_CHECK_ARG(c.mtp_layers <= 1, "config: mtp_layers %u (0 or 1)", c.mtp_layers);
  PRG_CHECK_ARG(c.num_layers >= 1 && c.num_layers <= 256, "config: num_layers %u", c.num_layers);
  PRG_CHECK_ARG(c.hidden >= 512 && c.hidden % 512 == 0 && c.hidden <= 16384, "config: hidden %u", c.hidden);
  PRG_CHECK_ARG(c.intermediate >= 512 && c.intermediate % 512 == 0 && c.intermediate <= 16384,
                "config: intermediate %u", c.intermediate);
  PRG_CHECK_ARG(c.vocab >= 8 && c.vocab % 8 == 0, "config: vocab %u must be a multiple of 8", c.vocab);
  PRG_CHECK_ARG(c.full_attention_interval >= 1, "config: full_attention_interval 0");
  PRG_CHECK_ARG(c.rms_eps > 0.0f, "config: rms_eps");
  return PRG_OK;
}

}  // namespace

int validate_model_config(const PrgModelConfig& c) { return validate_config(c); }

// ------------------------------------------------------- per-token chain ---
GemvParams gemv_params(const uint16_t* x, uint32_t K) {
  GemvParams p{};
  p.x[0] = x;
  p.K = K;
  return p;
}

void add_seg(GemvParams& p, const Q4Linear& l, uint16_t* out) {
  GemvSeg& s = p.seg[p.nseg++];
  s.w[0] = l.weight;
  s.s[0] = l.scales;
  s.b[0] = l.biases;
  s.tw[0] = l.t16_w;
  s.ts[0] = l.t16_s;
  s.tb[0] = l.t16_b;
  s.out[0] = out;
  s.rows = l.out_dim;
}

namespace {
uint32_t total_rows(const GemvParams& p) {
  uint32_t r = 0;
  for (uint32_t i = 0; i < p.nseg; ++i) r += p.seg[i].rows;
  return r;
}
}  // namespace

// Launches whose segments all carry decode-layout copies run on the
// matrix-core GEMV; the rest (and every launch of a model without copies) on
// q4_gemv_kernel.
int run_gemv(hipStream_t s, GemvParams& p, int epi, int norm, const char* name) {
  int M = p.x[1] ? 2 : 1;
  if (t16_usable(p, M, epi, norm)) return launch_q4_gemv_t16(s, p, M, epi, norm, name);
  const int rows = gemv_rows_per_wave(total_rows(p), p.K, epi, M);
  return launch_q4_gemv(s, p, M, rows, epi, norm, name);
}

int run_argmax_gemv(hipStream_t s, GemvParams& p, int M, int norm, const char* name) {
  if (t16_usable(p, M, kEpiArgmax, norm)) return launch_q4_gemv_t16(s, p, M, kEpiArgmax, norm, name);
  return launch_q4_gemv(s, p, M, 8, kEpiArgmax, norm, name);
}

// GDN layer: norm+in_proj(+conv) -> recurrence -> gated norm+out_proj + residual.
// The GDN gate projections (in_proj_a / in_proj_b, 32 rows each) run inside
// the recurrence kernel when the hidden size allows it (one quantisation
// group per lane): the in_proj GEMV then has 8192 + 4096 rows, four per wave
// of its grid, instead of a fifth round for 64 rows.
static bool gates_in_gdn(const PrgModelConfig& c) { return c.hidden <= kGdnGateProjMaxK && c.hidden % 64 == 0; }
static GdnGateProj gate_proj(PrgModelState* st, const LinearAttentionBlock& b, uint32_t hidden) {
  return GdnGateProj{st->ximg,          b.in_a.weight, b.in_a.scales, b.in_a.biases,
                     b.in_b.weight,     b.in_b.scales, b.in_b.biases, hidden};
}

int encode_linear_attention(PrgModel* m, PrgModelState* st, const DecoderLayer& L, const GdnIO& io,
                            const uint16_t* x, uint16_t* h, const StepScalars* step) {
  const LinearAttentionBlock& b = L.lin;
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  GemvParams p = gemv_params(x, c.hidden);
  p.norm_w = L.input_norm;
  p.eps = c.rms_eps;
  add_seg(p, b.in_qkv, st->conv_out);
  p.seg[0].conv_state = io.conv_in;
  p.seg[0].conv_state_out = io.conv_out;
  p.seg[0].conv_w = b.conv_weight;
  p.seg[0].conv_dim = kGdnConvDim;
  add_seg(p, b.in_z, nullptr);
  p.seg[1].silu_out[0] = st->zsilu;
  const GdnGateProj gp = gate_proj(st, b, c.hidden);
  if (gates_in_gdn(c)) {
    p.x_image[0] = st->ximg;
  } else {
    add_seg(p, b.in_a, st->abuf);
    add_seg(p, b.in_b, st->bbuf);
  }
  if (int rc = run_gemv(s, p, kEpiPlain, kNormRms, "linear_attn.in_proj")) return rc;
  // Recurrence -> raw y (bf16); the gated RMSNorm runs in the out_proj
  // GEMV's prologue (per 128-wide head, gate z from in_proj).
  if (!st->gemv_only)
    if (int rc = launch_gdn_decode(s, io.recur_in, st->conv_out, st->abuf, st->bbuf, b.a_log, b.dt_bias, st->gated,
                                   step, 0, nullptr, nullptr, 0.0f, io.recur_out, gates_in_gdn(c) ? &gp : nullptr))
      return rc;
  GemvParams o = gemv_params(st->gated, kGdnValDim);
  o.norm_w = b.norm_weight;
  o.eps = c.rms_eps;
  o.gz[0] = st->zsilu;
  add_seg(o, b.out_proj, h);
  o.seg[0].res[0] = x;
  return run_gemv(s, o, kEpiResidual, kNormGated, "linear_attn.out_proj");
}

// Two consecutive tokens through one GDN layer (the verify rows, positions in
// step[0] / step[1]): the normed in_proj for both rows in one M = 2 GEMV whose
// epilogue runs both conv steps per channel (row 0's rolled conv state to
// io.conv_out, row 1's back to io.conv_in), both recurrence steps in one
// launch (row 0: io.recur_in -> io.recur_out, row 1: on to io.recur_in),
// and the gated-norm out_proj for both rows in one M = 2 GEMV. Every per-row
// number equals two single-token layers: the M = 2 GEMVs do the M = 1
// per-row arithmetic, and the conv epilogue repeats the single-step order.
int encode_linear_attention2(PrgModel* m, PrgModelState* st, const DecoderLayer& L, const GdnIO& io,
                             const uint16_t* const* x, uint16_t* const* h, const StepScalars* step) {
  const LinearAttentionBlock& b = L.lin;
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  uint16_t* conv_out[2] = {st->conv_out, st->conv_out + kGdnConvDim};
  float* zsilu[2] = {st->zsilu, st->zsilu + kGdnValDim};
  uint16_t* abuf[2] = {st->abuf, st->abuf + kGdnHv};
  uint16_t* bbuf[2] = {st->bbuf, st->bbuf + kGdnHv};
  uint16_t* gated[2] = {st->gated, st->gated + kGdnValDim};
  GemvParams p = gemv_params(x[0], c.hidden);
  p.x[1] = x[1];
  p.norm_w = L.input_norm;
  p.eps = c.rms_eps;
  add_seg(p, b.in_qkv, conv_out[0]);
  p.seg[0].out[1] = conv_out[1];
  p.seg[0].conv_state = io.conv_in;
  p.seg[0].conv_state_out = io.conv_out;
  p.seg[0].conv_w = b.conv_weight;
  p.seg[0].conv_dim = kGdnConvDim;
  add_seg(p, b.in_z, nullptr);
  p.seg[1].silu_out[0] = zsilu[0];
  p.seg[1].silu_out[1] = zsilu[1];
  const GdnGateProj gp = gate_proj(st, b, c.hidden);
  if (gates_in_gdn(c)) {
    p.x_image[0] = st->ximg;
    p.x_image[1] = st->ximg + c.hidden / 2;
  } else {
    add_seg(p, b.in_a, abuf[0]);
    p.seg[2].out[1] = abuf[1];
    add_seg(p, b.in_b, bbuf[0]);
    p.seg[3].out[1] = bbuf[1];
  }
  if (int rc = run_gemv(s, p, kEpiPlain, kNormRms, "linear_attn.in_proj2")) return rc;
  // both recurrence steps in one launch: row 0's state to io.recur_out (the
  // snapshot), row 1's back to io.recur_in
  if (int rc = launch_gdn_decode2(s, io.recur_in, io.recur_out, io.recur_in, conv_out[0], abuf[0], bbuf[0], b.a_log,
                                  b.dt_bias, gated[0], step, gates_in_gdn(c) ? &gp : nullptr))
    return rc;
  GemvParams o = gemv_params(gated[0], kGdnValDim);
  o.x[1] = gated[1];
  o.norm_w = b.norm_weight;
  o.eps = c.rms_eps;
  o.gz[0] = zsilu[0];
  o.gz[1] = zsilu[1];
  add_seg(o, b.out_proj, h[0]);
  o.seg[0].out[1] = h[1];
  o.seg[0].res[0] = x[0];
  o.seg[0].res[1] = x[1];
  return run_gemv(s, o, kEpiResidual, kNormGated, "linear_attn.out_proj2");
}

// Decode-step attention over a layer's cache: split partials over the cached
// tokens (q normalised and rotated in the kernel), then the gated merge that
// adds the new token(s) and appends their K / V (prepare, partials and merge
// of FullAttentionBlock.decodeStepBf16, block_attn.zig:321-358, in two launches).
static AttnDecodeArgs attn_step_args(PrgModelState* st, const FullAttentionBlock& b, LayerState& ls, const uint16_t* qp,
                              const uint16_t* k, const uint16_t* v, uint16_t* ctx, const StepScalars* step) {
  AttnDecodeArgs da{};
  da.q = st->qbuf;
  da.key_cache = ls.cache_k;
  da.value_cache = ls.cache_v;
  da.gate = nullptr;
  da.out = ctx;
  da.partials = st->partials;
  da.stride = st->stride;
  da.nsplit = st->nsplit;
  da.split_tokens = st->split_tokens;
  da.step = step;
  da.scale = kAttnScale;
  da.packed_q = qp;
  da.q_norm = b.q_norm;
  da.k_in = k;
  da.v_in = v;
  da.k_norm = b.k_norm;
  da.key_cache_w = ls.cache_k;
  da.value_cache_w = ls.cache_v;
  return da;
}

// Two consecutive tokens through one attention layer: q/k/v for both rows in
// one M = 2 GEMV, one split decode over the cached tokens for both rows plus
// one merge (row 1 also attends to row 0's new token), and o_proj for both
// rows in one M = 2 GEMV.
int encode_full_attention2(PrgModel* m, PrgModelState* st, const DecoderLayer& L, LayerState& ls,
                           const uint16_t* const* x, uint16_t* const* h, const StepScalars* step) {
  const FullAttentionBlock& b = L.full;
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  constexpr uint32_t kQp = 2 * kAttnQHeads * kAttnHeadDim, kKv = kAttnKvHeads * kAttnHeadDim;
  constexpr uint32_t kCtx = kAttnQHeads * kAttnHeadDim;
  uint16_t* qp[2] = {st->qp, st->qp + kQp};
  uint16_t* kb[2] = {st->kbuf, st->kbuf + kKv};
  uint16_t* vb[2] = {st->vbuf, st->vbuf + kKv};
  uint16_t* ctx[2] = {st->ctx, st->ctx + kCtx};
  GemvParams p = gemv_params(x[0], c.hidden);
  p.x[1] = x[1];
  p.norm_w = L.input_norm;
  p.eps = c.rms_eps;
  add_seg(p, b.q_proj, qp[0]);
  p.seg[0].out[1] = qp[1];
  add_seg(p, b.k_proj, kb[0]);
  p.seg[1].out[1] = kb[1];
  add_seg(p, b.v_proj, vb[0]);
  p.seg[2].out[1] = vb[1];
  if (int rc = run_gemv(s, p, kEpiPlain, kNormRms, "self_attn.qkv_proj2")) return rc;
  // Both rows attend over the cached tokens [0, pos); the merge adds row 0's
  // new token to both rows and row 1's to row 1 only, and appends both.
  AttnDecodeArgs da = attn_step_args(st, b, ls, qp[0], kb[0], vb[0], ctx[0], step);
  da.rows = 2;
  if (int rc = launch_attn_decode(s, da)) return rc;
  GemvParams o = gemv_params(ctx[0], kCtx);
  o.x[1] = ctx[1];
  add_seg(o, b.o_proj, h[0]);
  o.seg[0].out[1] = h[1];
  o.seg[0].res[0] = x[0];
  o.seg[0].res[1] = x[1];
  return run_gemv(s, o, kEpiResidual, kNormNone, "self_attn.o_proj2");
}

// Attention layer: norm+q/k/v -> prepare/append -> flash decode -> o_proj + residual.
int encode_full_attention(PrgModel* m, PrgModelState* st, const DecoderLayer& L, LayerState& ls, const uint16_t* x,
                          uint16_t* h, const StepScalars* step) {
  const FullAttentionBlock& b = L.full;
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  GemvParams p = gemv_params(x, c.hidden);
  p.norm_w = L.input_norm;
  p.eps = c.rms_eps;
  add_seg(p, b.q_proj, st->qp);
  add_seg(p, b.k_proj, st->kbuf);
  add_seg(p, b.v_proj, st->vbuf);
  if (int rc = run_gemv(s, p, kEpiPlain, kNormRms, "self_attn.qkv_proj")) return rc;
  AttnDecodeArgs da = attn_step_args(st, b, ls, st->qp, st->kbuf, st->vbuf, st->ctx, step);
  if (!st->gemv_only)
    if (int rc = launch_attn_decode(s, da)) return rc;
  GemvParams o = gemv_params(st->ctx, kAttnQHeads * kAttnHeadDim);
  add_seg(o, b.o_proj, h);
  o.seg[0].res[0] = x;
  return run_gemv(s, o, kEpiResidual, kNormNone, "self_attn.o_proj");
}

// MLP for M rows: post_attention_layernorm + gate/up SiLU -> down + residual.
int encode_mlp(PrgModel* m, PrgModelState* st, const DecoderLayer& L, int M, const uint16_t* const* h,
               uint16_t* const* inter, uint16_t* const* out) {
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  GemvParams p = gemv_params(h[0], c.hidden);
  p.norm_w = L.post_norm;
  p.eps = c.rms_eps;
  add_seg(p, L.mlp.gate_proj, inter[0]);
  p.seg[0].w[1] = L.mlp.up_proj.weight;
  p.seg[0].s[1] = L.mlp.up_proj.scales;
  p.seg[0].b[1] = L.mlp.up_proj.biases;
  p.seg[0].tw[1] = L.mlp.up_proj.t16_w;
  p.seg[0].ts[1] = L.mlp.up_proj.t16_s;
  p.seg[0].tb[1] = L.mlp.up_proj.t16_b;
  if (M == 2) {
    p.x[1] = h[1];
    p.seg[0].out[1] = inter[1];
  }
  if (int rc = run_gemv(s, p, kEpiSiluGate, kNormRms, "mlp.gate_up")) return rc;
  GemvParams d = gemv_params(inter[0], c.intermediate);
  add_seg(d, L.mlp.down_proj, out[0]);
  d.seg[0].res[0] = h[0];
  if (M == 2) {
    d.x[1] = inter[1];
    d.seg[0].out[1] = out[1];
    d.seg[0].res[1] = h[1];
  }
  return run_gemv(s, d, kEpiResidual, kNormNone, "mlp.down_proj");
}

namespace {

// One token: embed(ctl.token) -> layers -> (lm_head argmax | forced) + advance.
int encode_token(PrgModel* m, PrgModelState* st, bool with_head) {
  hipStream_t s = st->stream;
  const StepScalars* step = &st->ctl->s;
  if (!st->gemv_only)
    if (int rc = launch_embedding(s, m->embed.weight, m->embed.scales, m->embed.biases, st->hA, &st->ctl->s.token,
                                  0, 1, m->cfg.hidden))
      return rc;
  for (size_t i = 0; i < m->layers.size(); ++i) {
    const DecoderLayer& L = m->layers[i];
    LayerState& ls = st->layers[i];
    int rc = L.linear ? encode_linear_attention(m, st, L, GdnIO{ls.conv, nullptr, ls.recur, nullptr}, st->hA, st->hB,
                                                step)
                      : encode_full_attention(m, st, L, ls, st->hA, st->hB, step);
    if (rc) return rc;
    const uint16_t* h[1] = {st->hB};
    uint16_t* inter[1] = {st->inter};
    uint16_t* out[1] = {st->hA};
    if ((rc = encode_mlp(m, st, L, 1, h, inter, out))) return rc;
  }
  if (!with_head) return launch_advance_forced(s, st->ctl, st->prompt);
  GemvParams p = gemv_params(st->hA, m->cfg.hidden);
  p.norm_w = m->final_norm;
  p.eps = m->cfg.rms_eps;
  add_seg(p, m->lm_head, nullptr);
  p.seg[0].pval[0] = st->pval;
  p.seg[0].pidx[0] = st->pidx;
  p.argmax_waves = st->argmax_waves;
  if (int rc = run_argmax_gemv(s, p, 1, kNormRms, "lm_head.argmax")) return rc;
  if (st->gemv_only) return PRG_OK;
  return launch_argmax_waves_advance(s, st->pval, st->pidx, st->argmax_waves, st->ctl, st->prompt, st->predictions);
}

int capture(PrgModel* m, PrgModelState* st, bool with_head, hipGraphExec_t* out) {
  hipGraph_t g = nullptr;
  PRG_HIP(hipStreamBeginCapture(st->stream, hipStreamCaptureModeThreadLocal));
  const int rc = encode_token(m, st, with_head);
  hipError_t e = hipStreamEndCapture(st->stream, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return set_error(PRG_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
  e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return set_error(PRG_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  return PRG_OK;
}

int ensure_graphs(PrgModelState* st) {
  if (st->eager) return PRG_OK;
  if (!st->graph_decode)
    if (int rc = capture(st->model, st, true, &st->graph_decode)) return rc;
  if (!st->graph_prompt)
    if (int rc = capture(st->model, st, false, &st->graph_prompt)) return rc;
  return PRG_OK;
}

// One token step: graph replay, or the same launches issued eagerly.
int run_step(PrgModelState* st, bool with_head) {
  if (st->eager) return encode_token(st->model, st, with_head);
  PRG_HIP(hipGraphLaunch(with_head ? st->graph_decode : st->graph_prompt, st->stream));
  return PRG_OK;
}

}  // namespace

// Every GEMV weight that has a decode-layout shape: the layers' projections
// and MLPs, the lm_head, and the MTP drafter's fc and layer.
static std::vector<Q4Linear*> t16_linears(PrgModel* m) {
  std::vector<Q4Linear*> lins;
  auto add = [&](Q4Linear* q) {
    if (q->weight && t16_shape_ok(q->out_dim, q->in_dim)) lins.push_back(q);
  };
  auto add_layer = [&](DecoderLayer& L) {
    if (L.linear) {
      for (Q4Linear* q : {&L.lin.in_qkv, &L.lin.in_z, &L.lin.in_a, &L.lin.in_b, &L.lin.out_proj}) add(q);
    } else {
      for (Q4Linear* q : {&L.full.q_proj, &L.full.k_proj, &L.full.v_proj, &L.full.o_proj}) add(q);
    }
    for (Q4Linear* q : {&L.mlp.gate_proj, &L.mlp.up_proj, &L.mlp.down_proj}) add(q);
  };
  for (DecoderLayer& L : m->layers) add_layer(L);
  add(&m->lm_head);
  if (m->mtp.present) {
    add(&m->mtp.fc);
    add_layer(m->mtp.layer);
  }
  return lins;
}

int prepare_t16(PrgModel* m) {
  if (!m->t16_enabled) return PRG_OK;
  const std::vector<Q4Linear*> lins = t16_linears(m);
  auto wbytes = [](const Q4Linear* q) { return align_up(static_cast<size_t>(q->out_dim) * q->in_dim / 2, kAlign); };
  auto mbytes = [](const Q4Linear* q) { return align_up(static_cast<size_t>(q->out_dim) * (q->in_dim / 64) * 2, kAlign); };
  size_t total = 0;
  for (const Q4Linear* q : lins) total += wbytes(q) + 2 * mbytes(q);
  if (!m->t16_arena && total > 0) {
    void* p = nullptr;
    if (hipMalloc(&p, total) != hipSuccess) return set_error(PRG_ERR_OOM, "decode-layout weights: %zu bytes", total);
    m->t16_arena = static_cast<uint8_t*>(p);
    m->t16_bytes = total;
  }
  size_t off = 0;
  for (Q4Linear* q : lins) {
    q->t16_w = reinterpret_cast<uint32_t*>(m->t16_arena + off);
    off += wbytes(q);
    q->t16_s = reinterpret_cast<uint16_t*>(m->t16_arena + off);
    off += mbytes(q);
    q->t16_b = reinterpret_cast<uint16_t*>(m->t16_arena + off);
    off += mbytes(q);
    if (int rc = launch_t16_repack(nullptr, q->weight, q->scales, q->biases, q->t16_w, q->t16_s, q->t16_b,
                                   q->out_dim, q->in_dim))
      return rc;
  }
  PRG_HIP(hipDeviceSynchronize());
  m->t16_dirty = false;
  return PRG_OK;
}

int ensure_t16(PrgModel* m) { return m->t16_dirty ? prepare_t16(m) : PRG_OK; }

}  // namespace prg

using namespace prg;

extern "C" {

void prg_model_default_config(PrgModelConfig* cfg) {
  if (!cfg) return;
  cfg->num_layers = 32;
  cfg->hidden = 4096;
  cfg->intermediate = 12288;
  cfg->vocab = 248320;
  cfg->full_attention_interval = 4;
  cfg->rms_eps = 1e-6f;
  cfg->mtp_layers = 0;
}

int prg_model_create_random(const PrgModelConfig* cfg, uint64_t seed, PrgModel** out) {
  PRG_CHECK_ARG(cfg && out, "prg_model_create_random: null argument");
  *out = nullptr;
  if (int rc = validate_config(*cfg)) return rc;
  auto* m = new PrgModel();
  m->cfg = *cfg;
  if (const char* e = getenv("PEREGRINE_T16")) m->t16_enabled = e[0] != '0';
  Builder sizing{m, seed};
  build_model(sizing);
  m->arena_bytes = sizing.offset;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&m->arena), m->arena_bytes);
  if (e != hipSuccess) {
    delete m;
    return set_error(PRG_ERR_OOM, "model weights: hipMalloc(%zu): %s", sizing.offset, hipGetErrorString(e));
  }
  Builder b{m, seed};
  b.sizing = false;
  build_model(b);
  for (const auto& f : b.fills) {
    const uint32_t blocks = static_cast<uint32_t>((f.n + 255) / 256);
    hipLaunchKernelGGL(fill_kernel, dim3(blocks), dim3(256), 0, nullptr, f.dst, f.n, f.key, f.kind, f.a, f.b,
                       f.f32, f.scale);
  }
  e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(m->arena);
    delete m;
    return set_error(PRG_ERR_HIP, "model init: %s", hipGetErrorString(e));
  }
  if (int rc = prepare_t16(m)) {
    prg_model_destroy(m);
    return rc;
  }
  *out = m;
  return PRG_OK;
}

void prg_model_destroy(PrgModel* model) {
  if (!model) return;
  (void)hipFree(model->arena);
  (void)hipFree(model->dense_arena);
  (void)hipFree(model->t16_arena);
  delete model;
}

int prg_model_prepare_decode(PrgModel* model) {
  PRG_CHECK_ARG(model, "prg_model_prepare_decode: null model");
  return prepare_t16(model);
}

size_t prg_model_decode_layout_bytes(const PrgModel* model) { return model ? model->t16_bytes : 0; }

// The reference's prepared dense RHS for the prompt path
// (block_attn.zig:143-215, linear_q4.denseRhsBf16ByteLen): every Q4 matrix
// the prompt GEMMs read, dequantised once into bf16 [out, in].
int prg_model_prepare_dense(PrgModel* model) {
  PRG_CHECK_ARG(model, "prg_model_prepare_dense: null model");
  std::vector<Q4Linear*> lins;
  auto add_layer = [&](DecoderLayer& L) {
    if (L.linear) {
      for (Q4Linear* q : {&L.lin.in_qkv, &L.lin.in_z, &L.lin.in_a, &L.lin.in_b, &L.lin.out_proj}) lins.push_back(q);
    } else {
      for (Q4Linear* q : {&L.full.q_proj, &L.full.k_proj, &L.full.v_proj, &L.full.o_proj}) lins.push_back(q);
    }
    for (Q4Linear* q : {&L.mlp.gate_proj, &L.mlp.up_proj, &L.mlp.down_proj}) lins.push_back(q);
  };
  for (DecoderLayer& L : model->layers) add_layer(L);
  if (model->mtp.present) {
    lins.push_back(&model->mtp.fc);
    add_layer(model->mtp.layer);
  }
  size_t total = 0;
  for (const Q4Linear* q : lins) total += align_up(static_cast<size_t>(q->out_dim) * q->in_dim * 2, kAlign);
  if (!model->dense_arena) {
    void* p = nullptr;
    if (hipMalloc(&p, total) != hipSuccess)
      return set_error(PRG_ERR_OOM, "prg_model_prepare_dense: %zu bytes", total);
    model->dense_arena = static_cast<uint8_t*>(p);
    model->dense_bytes = total;
  }
  size_t off = 0;
  for (Q4Linear* q : lins) {
    q->dense = reinterpret_cast<uint16_t*>(model->dense_arena + off);
    if (int rc = launch_dequant_dense(nullptr, q->weight, q->scales, q->biases, q->dense, q->out_dim, q->in_dim,
                                      "prg_model_prepare_dense"))
      return rc;
    off += align_up(static_cast<size_t>(q->out_dim) * q->in_dim * 2, kAlign);
  }
  PRG_HIP(hipDeviceSynchronize());
  return PRG_OK;
}

size_t prg_model_dense_bytes(const PrgModel* model) { return model ? model->dense_bytes : 0; }

size_t prg_model_weight_bytes(const PrgModel* model) { return model ? model->arena_bytes : 0; }

uint32_t prg_model_tensor_count(const PrgModel* model) {
  return model ? static_cast<uint32_t>(model->tensors.size()) : 0u;
}

int prg_model_tensor_name(const PrgModel* model, uint32_t index, char* buf, size_t len) {
  PRG_CHECK_ARG(model && buf && len, "prg_model_tensor_name: null argument");
  PRG_CHECK_ARG(index < model->tensors.size(), "prg_model_tensor_name: index %u of %zu", index,
                model->tensors.size());
  const std::string& n = std::next(model->tensors.begin(), index)->first;
  PRG_CHECK_ARG(n.size() < len, "prg_model_tensor_name: buffer of %zu bytes too small", len);
  memcpy(buf, n.c_str(), n.size() + 1);
  return PRG_OK;
}

int prg_model_tensor_info(const PrgModel* model, const char* name, char* dtype, size_t dtype_len, uint64_t* shape,
                          uint32_t max_dims, uint32_t* ndim) {
  PRG_CHECK_ARG(model && name && ndim, "prg_model_tensor_info: null argument");
  auto it = model->specs.find(name);
  if (it == model->specs.end()) return set_error(PRG_ERR_INVALID_ARG, "prg_model_tensor_info: no tensor '%s'", name);
  const TensorSpec& sp = it->second;
  *ndim = static_cast<uint32_t>(sp.shape.size());
  if (shape) {
    PRG_CHECK_ARG(sp.shape.size() <= max_dims, "prg_model_tensor_info: %zu dims > %u", sp.shape.size(), max_dims);
    for (size_t k = 0; k < sp.shape.size(); ++k) shape[k] = sp.shape[k];
  }
  if (dtype) {
    PRG_CHECK_ARG(sp.dtype.size() < dtype_len, "prg_model_tensor_info: dtype buffer too small");
    memcpy(dtype, sp.dtype.c_str(), sp.dtype.size() + 1);
  }
  return PRG_OK;
}

int prg_model_tensor(const PrgModel* model, const char* name, void** ptr, size_t* bytes) {
  PRG_CHECK_ARG(model && name && ptr && bytes, "prg_model_tensor: null argument");
  auto it = model->tensors.find(name);
  if (it == model->tensors.end()) return set_error(PRG_ERR_INVALID_ARG, "prg_model_tensor: no tensor '%s'", name);
  *ptr = it->second.ptr;
  *bytes = it->second.bytes;
  // the caller may write the weights through ptr: rewrite the decode-layout
  // copies before the next run
  model->t16_dirty = model->t16_arena != nullptr;
  return PRG_OK;
}

int prg_model_state_create(PrgModel* model, uint32_t max_seq, PrgModelState** out) {
  PRG_CHECK_ARG(model && out, "prg_model_state_create: null argument");
  PRG_CHECK_ARG(max_seq >= 1 && max_seq <= 65536, "prg_model_state_create: max_seq %u outside [1, 65536]", max_seq);
  *out = nullptr;
  auto* st = new PrgModelState();
  st->model = model;
  st->max_seq = max_seq;
  st->stride = cache_stride_for(max_seq);
  st->nsplit = attn_num_splits(st->stride);
  st->split_tokens = attn_split_tokens(st->stride, st->nsplit);
  if (const char* e = getenv("PEREGRINE_EAGER")) st->eager = (e[0] == '1');
  const PrgModelConfig& c = model->cfg;

  // Two passes over the same layout: size, then carve the arena.
  struct Item {
    std::string name;
    size_t bytes;
    void** slot;
  };
  std::vector<Item> items;
  st->layers.assign(c.num_layers, LayerState{});
  // GDN states first, as one contiguous block.
  for (uint32_t i = 0; i < c.num_layers; ++i) {
    const std::string p = "layers." + std::to_string(i);
    if (model->layers[i].linear) {
      items.push_back({p + ".conv", sizeof(float) * (kGdnConvK - 1) * kGdnConvDim, reinterpret_cast<void**>(&st->layers[i].conv)});
      items.push_back({p + ".recur", sizeof(float) * kGdnHv * kGdnDv * kGdnDk, reinterpret_cast<void**>(&st->layers[i].recur)});
    }
  }
  const size_t gdn_items = items.size();
  for (uint32_t i = 0; i < c.num_layers; ++i) {
    const std::string p = "layers." + std::to_string(i);
    if (!model->layers[i].linear) {
      const size_t kv = sizeof(uint16_t) * kAttnKvHeads * static_cast<size_t>(st->stride) * kAttnHeadDim;
      items.push_back({p + ".cache_k", kv, reinterpret_cast<void**>(&st->layers[i].cache_k)});
      items.push_back({p + ".cache_v", kv, reinterpret_cast<void**>(&st->layers[i].cache_v)});
    }
  }
  const size_t bf = sizeof(uint16_t);
  const size_t state_items = items.size();
  items.push_back({"ws.hA", bf * c.hidden, reinterpret_cast<void**>(&st->hA)});
  items.push_back({"ws.hB", bf * c.hidden, reinterpret_cast<void**>(&st->hB)});
  items.push_back({"ws.conv_out", 2 * bf * kGdnConvDim, reinterpret_cast<void**>(&st->conv_out)});
  items.push_back({"ws.z_silu", 2 * sizeof(float) * kGdnValDim, reinterpret_cast<void**>(&st->zsilu)});
  items.push_back({"ws.a", 2 * bf * kGdnHv, reinterpret_cast<void**>(&st->abuf)});
  items.push_back({"ws.ximg", 2 * bf * c.hidden, reinterpret_cast<void**>(&st->ximg)});
  items.push_back({"ws.b", 2 * bf * kGdnHv, reinterpret_cast<void**>(&st->bbuf)});
  items.push_back({"ws.gated", 2 * bf * kGdnValDim, reinterpret_cast<void**>(&st->gated)});
  items.push_back({"ws.qp", 2 * bf * 2 * kAttnQHeads * kAttnHeadDim, reinterpret_cast<void**>(&st->qp)});
  items.push_back({"ws.k", 2 * bf * kAttnKvHeads * kAttnHeadDim, reinterpret_cast<void**>(&st->kbuf)});
  items.push_back({"ws.v", 2 * bf * kAttnKvHeads * kAttnHeadDim, reinterpret_cast<void**>(&st->vbuf)});
  items.push_back({"ws.q", 2 * bf * kAttnQHeads * kAttnHeadDim, reinterpret_cast<void**>(&st->qbuf)});
  items.push_back({"ws.gate", 2 * bf * kAttnQHeads * kAttnHeadDim, reinterpret_cast<void**>(&st->gatebuf)});
  items.push_back({"ws.ctx", 2 * bf * kAttnQHeads * kAttnHeadDim, reinterpret_cast<void**>(&st->ctx)});
  items.push_back({"ws.partials", 2 * sizeof(float) * kAttnQHeads * st->nsplit * kAttnPartialStride,
                   reinterpret_cast<void**>(&st->partials)});
  items.push_back({"ws.inter", bf * c.intermediate, reinterpret_cast<void**>(&st->inter)});
  items.push_back({"ws.pval", sizeof(float) * kArgmaxMaxWaves, reinterpret_cast<void**>(&st->pval)});
  items.push_back({"ws.pidx", sizeof(uint32_t) * kArgmaxMaxWaves, reinterpret_cast<void**>(&st->pidx)});
  items.push_back({"ws.argmax_waves", sizeof(uint32_t), reinterpret_cast<void**>(&st->argmax_waves)});
  items.push_back({"ws.ctl", sizeof(DecodeCtl), reinterpret_cast<void**>(&st->ctl)});
  items.push_back({"ws.prompt", sizeof(uint32_t) * st->stride, reinterpret_cast<void**>(&st->prompt)});
  items.push_back({"ws.predictions", sizeof(uint32_t) * st->stride, reinterpret_cast<void**>(&st->predictions)});
  size_t total = 0;
  for (auto& it : items) total = align_up(total + it.bytes, kAlign);
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&st->arena), total);
  if (e != hipSuccess) {
    delete st;
    return set_error(PRG_ERR_OOM, "model state: hipMalloc(%zu): %s", total, hipGetErrorString(e));
  }
  st->arena_bytes = total;
  size_t off = 0;
  for (size_t i = 0; i < items.size(); ++i) {
    const Item& it = items[i];
    *it.slot = st->arena + off;
    st->tensors[it.name] = TensorRef{st->arena + off, it.bytes};
    off = align_up(off + it.bytes, kAlign);
    if (i + 1 == gdn_items) st->gdn_bytes = off;
  }
  st->gdn_base = st->arena;
  (void)state_items;
  // Everything starts at zero (GDN states, caches, workspace).
  if ((e = hipMemset(st->arena, 0, total)) != hipSuccess ||
      (e = hipStreamCreateWithFlags(&st->stream, hipStreamNonBlocking)) != hipSuccess ||
      (e = hipEventCreate(&st->ev0)) != hipSuccess || (e = hipEventCreate(&st->ev1)) != hipSuccess ||
      (e = hipDeviceSynchronize()) != hipSuccess) {
    prg_model_state_destroy(st);
    return set_error(PRG_ERR_HIP, "model state init: %s", hipGetErrorString(e));
  }
  *out = st;
  return PRG_OK;
}

void prg_model_state_destroy(PrgModelState* st) {
  if (!st) return;
  if (st->graph_decode) (void)hipGraphExecDestroy(st->graph_decode);
  if (st->graph_prompt) (void)hipGraphExecDestroy(st->graph_prompt);
  if (st->ev0) (void)hipEventDestroy(st->ev0);
  if (st->ev1) (void)hipEventDestroy(st->ev1);
  if (st->graph_spec) (void)hipGraphExecDestroy(st->graph_spec);
  if (st->stream) (void)hipStreamDestroy(st->stream);
  (void)hipFree(st->arena);
  if (st->pf.arena) (void)hipFree(st->pf.arena);
  if (st->spec_arena) (void)hipFree(st->spec_arena);
  delete st;
}

int prg_model_state_reset(PrgModelState* st) {
  PRG_CHECK_ARG(st, "prg_model_state_reset: null state");
  for (auto& l : st->layers) {
    if (l.conv) PRG_HIP(hipMemsetAsync(l.conv, 0, sizeof(float) * (kGdnConvK - 1) * kGdnConvDim, st->stream));
    if (l.recur) PRG_HIP(hipMemsetAsync(l.recur, 0, sizeof(float) * kGdnHv * kGdnDv * kGdnDk, st->stream));
  }
  PRG_HIP(hipStreamSynchronize(st->stream));
  return PRG_OK;
}

int prg_model_state_tensor(const PrgModelState* st, const char* name, void** ptr, size_t* bytes) {
  PRG_CHECK_ARG(st && name && ptr && bytes, "prg_model_state_tensor: null argument");
  auto it = st->tensors.find(name);
  if (it == st->tensors.end()) return set_error(PRG_ERR_INVALID_ARG, "prg_model_state_tensor: no tensor '%s'", name);
  *ptr = it->second.ptr;
  *bytes = it->second.bytes;
  return PRG_OK;
}

uint32_t prg_model_state_stride(const PrgModelState* st) { return st ? st->stride : 0; }

int prg_model_forward_next_token(PrgModel* model, PrgModelState* st, uint32_t token, uint32_t cache_pos,
                                 uint32_t rope_pos, uint32_t seq_len, uint32_t* next_token) {
  PRG_CHECK_ARG(model && st && next_token && st->model == model, "prg_model_forward_next_token: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  if (cache_pos >= st->max_seq)  // model.zig:805
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "cache_pos %u >= max_seq %u", cache_pos, st->max_seq);
  if (token >= model->cfg.vocab)  // model.zig:806
    return set_error(PRG_ERR_INVALID_TOKEN, "token %u >= vocab %u", token, model->cfg.vocab);
  if (seq_len != cache_pos + 1)
    return set_error(PRG_ERR_INVALID_ARG, "seq_len %u != cache_pos + 1 (prefix caches are not supported)", seq_len);
  if (int rc = ensure_graphs(st)) return rc;
  // Step n = cache_pos: the argmax records predictions[cache_pos] and leaves
  // the loop at cache_pos + 1 with the prediction as its input, so a later
  // prg_model_decode continues from here.
  DecodeCtl ctl{};
  ctl.s = StepScalars{token, cache_pos, rope_pos, seq_len};
  ctl.n = cache_pos;
  ctl.rope_off = rope_pos - cache_pos;  // later steps keep the caller's RoPE offset
  ctl.prompt_len = 0;
  ctl.capacity = st->max_seq;
  PRG_HIP(hipMemcpyAsync(st->ctl, &ctl, sizeof(ctl), hipMemcpyHostToDevice, st->stream));
  if (int rc = run_step(st, true)) return rc;
  PRG_HIP(hipMemcpyAsync(next_token, st->predictions + cache_pos, sizeof(uint32_t), hipMemcpyDeviceToHost,
                         st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  return PRG_OK;
}

int prg_model_forward_next_token_prefixed(PrgModel* model, PrgModelState* st, uint32_t token, uint32_t cache_pos,
                                          uint32_t rope_pos, uint32_t seq_len, uint32_t prefix_len,
                                          uint32_t* next_token) {
  PRG_CHECK_ARG(model && st && next_token && st->model == model, "prg_model_forward_next_token_prefixed: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  const uint64_t slot = static_cast<uint64_t>(prefix_len) + cache_pos;
  if (slot >= st->max_seq)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix_len %u + cache_pos %u >= max_seq %u", prefix_len, cache_pos,
                     st->max_seq);
  if (static_cast<uint64_t>(seq_len) != slot + 1)
    return set_error(PRG_ERR_INVALID_ARG, "seq_len %u != prefix_len %u + cache_pos %u + 1", seq_len, prefix_len,
                     cache_pos);
  return prg_model_forward_next_token(model, st, token, static_cast<uint32_t>(slot), rope_pos, seq_len, next_token);
}

int prg_model_decode(PrgModel* model, PrgModelState* st, uint32_t n_steps, uint32_t* tokens_out, float* gpu_ms) {
  PRG_CHECK_ARG(model && st && tokens_out && st->model == model, "prg_model_decode: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  PRG_CHECK_ARG(n_steps >= 1, "prg_model_decode: n_steps == 0");
  if (int rc = ensure_graphs(st)) return rc;
  DecodeCtl ctl{};
  PRG_HIP(hipMemcpyAsync(&ctl, st->ctl, sizeof(ctl), hipMemcpyDeviceToHost, st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  if (ctl.overflow)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "the state is at max_seq %u; nothing left to decode", st->max_seq);
  if (ctl.n + n_steps > st->max_seq)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "position %u + %u steps exceeds max_seq %u", ctl.n, n_steps,
                     st->max_seq);
  PRG_HIP(hipEventRecord(st->ev0, st->stream));
  for (uint32_t i = 0; i < n_steps; ++i)
    if (int rc = run_step(st, true)) return rc;
  PRG_HIP(hipEventRecord(st->ev1, st->stream));
  PRG_HIP(hipMemcpyAsync(tokens_out, st->predictions + ctl.n, sizeof(uint32_t) * n_steps, hipMemcpyDeviceToHost,
                         st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  if (gpu_ms) PRG_HIP(hipEventElapsedTime(gpu_ms, st->ev0, st->ev1));
  return PRG_OK;
}

// Measurement only: one decode token's GEMV launches (all 129 of them, with
// the model's weights, fused norms and epilogues) captured as a graph and
// replayed `replays` times between two events; the other kernels are left
// out. The GEMVs write the state's activations and conv states, which stay
// undefined until the next prefill from position 0.
int prg_model_time_token_gemvs(PrgModel* model, PrgModelState* st, uint32_t replays, float* us_per_token) {
  PRG_CHECK_ARG(model && st && us_per_token && st->model == model, "prg_model_time_token_gemvs: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  PRG_CHECK_ARG(replays >= 1, "prg_model_time_token_gemvs: replays == 0");
  hipGraphExec_t ge = nullptr;
  st->gemv_only = true;
  const int rc = capture(model, st, true, &ge);
  st->gemv_only = false;
  if (rc) return rc;
  hipError_t e = hipSuccess;
  for (int i = 0; i < 2 && e == hipSuccess; ++i) e = hipGraphLaunch(ge, st->stream);
  if (e == hipSuccess) e = hipEventRecord(st->ev0, st->stream);
  for (uint32_t i = 0; i < replays && e == hipSuccess; ++i) e = hipGraphLaunch(ge, st->stream);
  if (e == hipSuccess) e = hipEventRecord(st->ev1, st->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(st->stream);
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, st->ev0, st->ev1);
  (void)hipGraphExecDestroy(ge);  // cleanup: its own error does not change the result
  if (e != hipSuccess) return set_error(PRG_ERR_HIP, "prg_model_time_token_gemvs: %s", hipGetErrorString(e));
  *us_per_token = ms * 1000.0f / static_cast<float>(replays);
  return PRG_OK;
}

int prg_model_generate(PrgModel* model, PrgModelState* st, const uint32_t* prompt, uint32_t prompt_len,
                       uint32_t n_new, int teacher_force, uint32_t* predictions, float* decode_ms) {
  PRG_CHECK_ARG(model && st && prompt && predictions && st->model == model, "prg_model_generate: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  PRG_CHECK_ARG(prompt_len >= 1, "prg_model_generate: empty prompt");
  if (teacher_force) PRG_CHECK_ARG(n_new == 0, "prg_model_generate: teacher forcing takes n_new == 0");
  else PRG_CHECK_ARG(n_new >= 1, "prg_model_generate: n_new == 0");
  const uint32_t steps = teacher_force ? prompt_len : prompt_len - 1 + n_new;
  if (steps > st->max_seq)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "%u steps exceed max_seq %u", steps, st->max_seq);
  for (uint32_t i = 0; i < prompt_len; ++i)
    if (prompt[i] >= model->cfg.vocab)
      return set_error(PRG_ERR_INVALID_TOKEN, "prompt[%u] = %u >= vocab %u", i, prompt[i], model->cfg.vocab);
  if (int rc = ensure_graphs(st)) return rc;
  if (int rc = prg_model_state_reset(st)) return rc;

  DecodeCtl ctl{};
  ctl.s = StepScalars{prompt[0], 0, 0, 1};
  ctl.n = 0;
  ctl.prompt_len = prompt_len;
  ctl.capacity = st->max_seq;
  PRG_HIP(hipMemcpyAsync(st->prompt, prompt, sizeof(uint32_t) * prompt_len, hipMemcpyHostToDevice, st->stream));
  PRG_HIP(hipMemsetAsync(st->predictions, 0xFF, sizeof(uint32_t) * st->stride, st->stream));
  PRG_HIP(hipMemcpyAsync(st->ctl, &ctl, sizeof(ctl), hipMemcpyHostToDevice, st->stream));
  const uint32_t head_from = teacher_force ? 0 : prompt_len - 1;
  for (uint32_t n = 0; n < head_from; ++n)
    if (int rc = run_step(st, false)) return rc;
  PRG_HIP(hipEventRecord(st->ev0, st->stream));
  for (uint32_t n = head_from; n < steps; ++n)
    if (int rc = run_step(st, true)) return rc;
  PRG_HIP(hipEventRecord(st->ev1, st->stream));
  PRG_HIP(hipMemcpyAsync(predictions, st->predictions, sizeof(uint32_t) * steps, hipMemcpyDeviceToHost, st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  if (decode_ms) PRG_HIP(hipEventElapsedTime(decode_ms, st->ev0, st->ev1));
  return PRG_OK;
}

}  // extern "C"
