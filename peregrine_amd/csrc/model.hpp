// Model internals shared by model.hip (weights, state, single-token decode),
// model_prefill.hip (the prompt path) and model_spec.hip (MTP drafter,
// two-token verify, speculative loop).
//
// Reference structures (file:line in the reference tree):
//   Q4Linear                      src/model/linear_q4.zig:17-25
//   LinearAttentionBlock          src/model/block_linear.zig:143-184
//   FullAttentionBlock            src/model/block_attn.zig:227-255
//   MlpBlock                      src/model/block_mlp.zig:110-130
//   DecoderLayer                  src/model/decoder_layer.zig:360-412
//   Drafter (MTP)                 src/model/mtp.zig:72-84
//   ModelState / LayerState       src/model/state.zig:11-118
#pragma once

#include <stddef.h>

#include <map>
#include <string>
#include <vector>

#include "attention.hpp"
#include "gdn.hpp"
#include "gemm.hpp"
#include "norm.hpp"
#include "peregrine_model.h"
#include "prefill.hpp"
#include "q4_gemv.hpp"

namespace prg {

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Q4Linear {
  uint32_t* weight = nullptr;
  uint16_t* scales = nullptr;
  uint16_t* biases = nullptr;
  uint32_t out_dim = 0, in_dim = 0;
  // Prepared bf16 [out_dim, in_dim] copy for the prompt GEMMs (inside
  // PrgModel::dense_arena; null until prg_model_prepare_dense).
  uint16_t* dense = nullptr;
  // Decode-layout copy for the matrix-core GEMVs (q4_gemv_t16.hpp; inside
  // PrgModel::t16_arena; null when the shape has none or copies are off).
  uint32_t* t16_w = nullptr;
  uint16_t* t16_s = nullptr;
  uint16_t* t16_b = nullptr;
};

struct LinearAttentionBlock {
  Q4Linear in_qkv, in_z, in_a, in_b, out_proj;
  uint16_t* conv_weight = nullptr;  // bf16 [8192, 4]
  float* a_log = nullptr;           // f32 [32]
  uint16_t* dt_bias = nullptr;      // bf16 [32]
  uint16_t* norm_weight = nullptr;  // bf16 [128]
};

struct FullAttentionBlock {
  Q4Linear q_proj, k_proj, v_proj, o_proj;
  uint16_t* q_norm = nullptr;  // bf16 [256]
  uint16_t* k_norm = nullptr;
};

struct MlpBlock {
  Q4Linear gate_proj, up_proj, down_proj;
};

struct DecoderLayer {
  bool linear = true;
  uint16_t* input_norm = nullptr;
  uint16_t* post_norm = nullptr;
  LinearAttentionBlock lin;
  FullAttentionBlock full;
  MlpBlock mlp;
};

// Multi-token-prediction drafter: pre-fc norms of the token embedding and of
// the target's normalised hidden, fc [hidden, 2*hidden], one full-attention
// decoder layer and a final norm; embedding and lm_head are the target's.
struct MtpWeights {
  bool present = false;
  uint16_t* pre_fc_norm_embedding = nullptr;
  uint16_t* pre_fc_norm_hidden = nullptr;
  Q4Linear fc;
  DecoderLayer layer;
  uint16_t* norm = nullptr;
};

struct TensorRef {
  void* ptr;
  size_t bytes;
};

// How a tensor is stored in a checkpoint: safetensors dtype and shape.
struct TensorSpec {
  std::string dtype;
  std::vector<uint64_t> shape;
};

struct LayerState {
  float* conv = nullptr;        // f32 [3, 8192]
  float* recur = nullptr;       // f32 [32, 128, 128]
  uint16_t* cache_k = nullptr;  // bf16 [4, stride, 256]
  uint16_t* cache_v = nullptr;  // bf16 [4, 256, stride]
};

// Prompt-path workspace, allocated on the first prefill ([rows, dim] bf16
// unless noted).
struct PrefillWs {
  uint8_t* arena = nullptr;
  uint32_t rows = 0;        // tokens per chunk the buffers hold
  size_t scores_elems = 0;  // bf16 attention score capacity
  uint16_t *h0 = nullptr, *h1 = nullptr, *normed = nullptr, *attn = nullptr, *resid = nullptr, *inter = nullptr;
  uint16_t *qkv = nullptr, *conv_out = nullptr, *z = nullptr, *a = nullptr, *b = nullptr, *y = nullptr,
           *gated = nullptr;
  float *qn = nullptr, *kn = nullptr, *g = nullptr, *beta = nullptr, *kq = nullptr;  // f32
  uint16_t *qp = nullptr, *k = nullptr, *v = nullptr, *q = nullptr, *gate = nullptr, *ctx = nullptr,
           *scores = nullptr;
  uint16_t* fc_in = nullptr;  // [rows, 2*hidden] drafter input
};

constexpr uint32_t kPrefillChunk = 2048;
constexpr size_t kPrefillScoresBytes = size_t(512) << 20;

// Device control block of the speculative loop (decode_loop.zig:163-293).
// The current token sits at position pos; one step drafts its successor with
// the MTP layer, verifies both with the target, and advances by 1 or 2.
struct SpecCtl {
  StepScalars v0;      // verify row 0: current token at pos
  StepScalars v1;      // verify row 1: the draft at pos + 1 (token written by the drafter)
  StepScalars d0;      // drafter step for the current token, at pos - 1
  StepScalars d1;      // drafter step for the draft, at pos (run after the verify)
  uint32_t pos;        // position of the current token
  uint32_t n;          // tokens emitted so far
  uint32_t verify;     // target argmax after row 0
  uint32_t bonus;      // target argmax after row 1
  uint32_t reject;     // this step rejected its draft: GDN states roll back
  uint32_t accepted, attempted;
  uint32_t capacity;   // positions must stay below it
  uint32_t stop;       // set when the next step would pass capacity or `target` tokens are out
  uint32_t target;     // tokens the loop was asked for
};
// The two verify rows' steps are read as an array (&v0)[0..1].
static_assert(offsetof(SpecCtl, v1) == offsetof(SpecCtl, v0) + sizeof(StepScalars), "v1 must follow v0");

bool is_linear_layer(const PrgModelConfig& c, uint32_t i);
int validate_model_config(const PrgModelConfig& c);
// Lay out every tensor of m->cfg in one device arena: m->tensors and m->specs
// filled, contents undefined. Returns a PRG_ERR_* code.
int layout_model(PrgModel* m);
uint32_t cache_stride_for(uint32_t max_seq);
// Write the decode-layout copies (allocating them on first use); ensure_t16
// does it only when a tensor pointer was handed out since the last write.
int prepare_t16(PrgModel* m);
int ensure_t16(PrgModel* m);

}  // namespace prg

struct PrgModel {
  PrgModelConfig cfg{};
  uint8_t* arena = nullptr;
  size_t arena_bytes = 0;
  std::map<std::string, prg::TensorRef> tensors;
  std::map<std::string, prg::TensorSpec> specs;
  prg::Q4Linear embed;
  std::vector<prg::DecoderLayer> layers;
  uint16_t* final_norm = nullptr;
  prg::Q4Linear lm_head;
  prg::MtpWeights mtp;
  // Prepared bf16 copies of the prompt GEMMs' weights (prg_model_prepare_dense).
  uint8_t* dense_arena = nullptr;
  size_t dense_bytes = 0;
  // Decode-layout copies of the GEMV weights, written at creation and again
  // before the next run once a tensor pointer has been handed out
  // (prg_model_tensor: the caller may write the Q4 weights through it).
  // PEREGRINE_T16=0 at creation: no copies, every GEMV on q4_gemv_kernel.
  uint8_t* t16_arena = nullptr;
  size_t t16_bytes = 0;
  bool t16_enabled = true;
  mutable bool t16_dirty = false;
};

struct PrgModelState {
  PrgModel* model = nullptr;
  uint32_t max_seq = 0, stride = 0;
  uint8_t* arena = nullptr;
  size_t arena_bytes = 0;
  std::map<std::string, prg::TensorRef> tensors;
  std::vector<prg::LayerState> layers;
  // All GDN conv/recurrent states lie in [gdn_base, gdn_base + gdn_bytes) of
  // the arena (the speculative loop snapshots and restores them as one block).
  uint8_t* gdn_base = nullptr;
  size_t gdn_bytes = 0;
  // decode workspace
  uint16_t *hA = nullptr, *hB = nullptr;
  uint16_t *conv_out = nullptr, *abuf = nullptr, *bbuf = nullptr, *gated = nullptr;
  uint32_t* ximg = nullptr;  // [2][hidden / 2]: the GDN in_proj's normalised rows for the gate projections
  float* zsilu = nullptr;  // silu(z) of the GDN gate, f32 (feeds the gated norm)
  uint16_t *qp = nullptr, *kbuf = nullptr, *vbuf = nullptr, *qbuf = nullptr, *gatebuf = nullptr, *ctx = nullptr;
  float* partials = nullptr;
  uint16_t* inter = nullptr;
  float* pval = nullptr;      // lm_head argmax: per-wave entries (kArgmaxMaxWaves)
  uint32_t* pidx = nullptr;
  uint32_t* argmax_waves = nullptr;  // entry count written by the lm_head GEMV
  prg::DecodeCtl* ctl = nullptr;
  uint32_t* prompt = nullptr;
  uint32_t* predictions = nullptr;
  uint32_t nsplit = 0, split_tokens = 0;
  // execution
  hipStream_t stream = nullptr;
  hipGraphExec_t graph_decode = nullptr;  // layers + lm_head argmax + advance
  hipGraphExec_t graph_prompt = nullptr;  // layers + forced advance
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  // PEREGRINE_EAGER=1: launch each token's kernels directly instead of
  // replaying the captured graph (same kernels and arguments; for tools such as
  // kernel tracers that do not follow graph launches).
  bool eager = false;
  bool gemv_only = false;  // measurement capture: only the token's GEMV launches
  prg::PrefillWs pf;
  // speculative decode (allocated on first use; the drafter state only when
  // the model has MTP weights)
  uint8_t* spec_arena = nullptr;
  prg::LayerState mtp;            // drafter KV cache
  uint8_t* gdn_snap = nullptr;    // GDN states after verify row 0
  uint16_t *h2a = nullptr, *h2b = nullptr, *inter2 = nullptr, *hnorm2 = nullptr;  // [2, dim]
  uint16_t *cur_hidden = nullptr, *fc_in = nullptr, *mtp_x = nullptr, *mtp_h = nullptr;
  float* pval2 = nullptr;
  uint32_t* pidx2 = nullptr;
  uint32_t* spec_out = nullptr;   // emitted tokens
  uint32_t* drafts = nullptr;     // draft token of each attempt
  prg::SpecCtl* spec = nullptr;
  hipGraphExec_t graph_spec = nullptr;
};

namespace prg {

// ------------------------------------------------- single-token encoders ---
GemvParams gemv_params(const uint16_t* x, uint32_t K);
void add_seg(GemvParams& p, const Q4Linear& l, uint16_t* out);
int run_gemv(hipStream_t s, GemvParams& p, int epi, int norm, const char* name);
// The lm_head argmax GEMV (one segment, per-block or per-wave entries in
// pval / pidx and their count in p.argmax_waves) for M rows.
int run_argmax_gemv(hipStream_t s, GemvParams& p, int M, int norm, const char* name);

// Where a layer's GDN state is read and written for one token (in == out for
// the ordinary in-place update).
struct GdnIO {
  float* conv_in;
  float* conv_out;
  float* recur_in;
  float* recur_out;
};

// h = x + attn(norm(x)) for one token (decoder_layer.zig:461-566).
int encode_linear_attention(PrgModel* m, PrgModelState* st, const DecoderLayer& L, const GdnIO& io,
                            const uint16_t* x, uint16_t* h, const StepScalars* step);
int encode_full_attention(PrgModel* m, PrgModelState* st, const DecoderLayer& L, LayerState& ls, const uint16_t* x,
                          uint16_t* h, const StepScalars* step);
// Two consecutive tokens through one layer with M = 2 projections; step[0]
// and step[1] hold the two rows' positions (decoder_layer.zig:485-516).
int encode_linear_attention2(PrgModel* m, PrgModelState* st, const DecoderLayer& L, const GdnIO& io,
                             const uint16_t* const* x, uint16_t* const* h, const StepScalars* step);
int encode_full_attention2(PrgModel* m, PrgModelState* st, const DecoderLayer& L, LayerState& ls,
                           const uint16_t* const* x, uint16_t* const* h, const StepScalars* step);
// out_r = h_r + mlp(norm(h_r)) for M = 1 or 2 rows (block_mlp.zig:260-311).
int encode_mlp(PrgModel* m, PrgModelState* st, const DecoderLayer& L, int M, const uint16_t* const* h,
               uint16_t* const* inter, uint16_t* const* out);

// ------------------------------------------------------------ prompt path ---
int ensure_prefill_ws(PrgModelState* st);
// Tokens of the next prefill chunk at `start`: at most the workspace rows, and
// halved until the attention score block of the chunk fits the workspace.
uint32_t prefill_chunk_tokens(const PrgModelState* st, uint32_t start, uint32_t remaining);
int prefill_layer(PrgModel* m, PrgModelState* st, const DecoderLayer& L, LayerState& ls, const uint16_t* x,
                  uint16_t* out, uint32_t T, uint32_t start);
// Ingest st->prompt[from, len) on top of positions [0, from); with_mtp also
// seeds the drafter's KV cache and leaves the last prompt row's normalised
// hidden in st->cur_hidden. hidden_out (with_mtp only, may be null) receives
// the final-normed hidden row of every ingested position p at row p.
int run_prefill(PrgModel* m, PrgModelState* st, uint32_t from, uint32_t len, bool with_mtp,
                uint16_t* hidden_out = nullptr);

// ------------------------------------------------------ state transfers ---
// ModelState.copyFullAttentionRangeFrom / copyLinearStateFrom
// (state.zig:124-180) between two states of one model, ordered after the
// source's pending work and complete on return.
int copy_attention_range(PrgModelState* dst, uint32_t dst_start, const PrgModelState* src, uint32_t src_start,
                         uint32_t count);
int copy_linear_state(PrgModelState* dst, const PrgModelState* src);

// ------------------------------------------------------ speculative path ---
int ensure_spec_ws(PrgModelState* st);
// Drafter prefill over rows [0, T): tokens (device) and the target's
// normalised hidden rows, at drafter positions start.. (mtp.zig:137-185).
int mtp_prefill_rows(PrgModel* m, PrgModelState* st, const uint32_t* tokens_dev, const uint16_t* hidden_rows,
                     uint32_t T, uint32_t start);

}  // namespace prg
