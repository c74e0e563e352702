// Prompt path of the model: layer-major chunked prefill
// (DeviceModel.prefillLayerMajor*, src/model/model.zig:940-1060;
// DecoderLayer.prefillStepBf16, src/model/decoder_layer.zig:644-760): every
// projection is an MFMA QMM over the chunk, attention is causal over the cache
// written so far, and the GDN recurrence runs token-sequentially inside one
// kernel per layer. Also the drafter's prompt seeding (src/model/mtp.zig:137-185).
#include <stdlib.h>

#include <algorithm>
#include <initializer_list>
#include <utility>

#include "model.hpp"

namespace prg {

int ensure_prefill_ws(PrgModelState* st) {
  PrefillWs& w = st->pf;
  if (w.arena) return PRG_OK;
  const PrgModelConfig& c = st->model->cfg;
  size_t R = std::min(kPrefillChunk, st->max_seq);
  // PEREGRINE_PREFILL_CHUNK=n caps the chunk (tests of chunk boundaries).
  if (const char* e = getenv("PEREGRINE_PREFILL_CHUNK")) {
    const long v = atol(e);
    if (v >= 1) R = std::min<size_t>(R, static_cast<size_t>(v));
  }
  w.rows = static_cast<uint32_t>(R);
  w.scores_elems = std::min<size_t>(static_cast<size_t>(kAttnQHeads) * R * align_up(st->max_seq, 64),
                                    kPrefillScoresBytes / sizeof(uint16_t));
  const size_t bf = sizeof(uint16_t), f4 = sizeof(float);
  struct Item {
    void** slot;
    size_t bytes;
  };
  const Item items[] = {
      {reinterpret_cast<void**>(&w.h0), bf * R * c.hidden},
      {reinterpret_cast<void**>(&w.h1), bf * R * c.hidden},
      {reinterpret_cast<void**>(&w.normed), bf * R * c.hidden},
      {reinterpret_cast<void**>(&w.attn), bf * R * c.hidden},
      {reinterpret_cast<void**>(&w.resid), bf * R * c.hidden},
      {reinterpret_cast<void**>(&w.inter), bf * R * c.intermediate},
      {reinterpret_cast<void**>(&w.qkv), bf * R * kGdnConvDim},
      {reinterpret_cast<void**>(&w.conv_out), bf * R * kGdnConvDim},
      {reinterpret_cast<void**>(&w.z), bf * R * kGdnValDim},
      {reinterpret_cast<void**>(&w.a), bf * R * kGdnHv},
      {reinterpret_cast<void**>(&w.b), bf * R * kGdnHv},
      {reinterpret_cast<void**>(&w.y), bf * R * kGdnValDim},
      {reinterpret_cast<void**>(&w.gated), bf * R * kGdnValDim},
      {reinterpret_cast<void**>(&w.qn), f4 * R * kGdnKeyDim},
      {reinterpret_cast<void**>(&w.kn), f4 * R * kGdnKeyDim},
      {reinterpret_cast<void**>(&w.g), f4 * R * kGdnHv},
      {reinterpret_cast<void**>(&w.beta), f4 * R * kGdnHv},
      {reinterpret_cast<void**>(&w.kq), f4 * R * kGdnHk},
      {reinterpret_cast<void**>(&w.qp), bf * R * 2 * kAttnQHeads * kAttnHeadDim},
      {reinterpret_cast<void**>(&w.k), bf * R * kAttnKvHeads * kAttnHeadDim},
      {reinterpret_cast<void**>(&w.v), bf * R * kAttnKvHeads * kAttnHeadDim},
      {reinterpret_cast<void**>(&w.q), bf * R * kAttnQHeads * kAttnHeadDim},
      {reinterpret_cast<void**>(&w.gate), bf * R * kAttnQHeads * kAttnHeadDim},
      {reinterpret_cast<void**>(&w.ctx), bf * R * kAttnQHeads * kAttnHeadDim},
      {reinterpret_cast<void**>(&w.scores), bf * w.scores_elems},
      {reinterpret_cast<void**>(&w.fc_in), bf * R * 2 * c.hidden},
  };
  size_t total = 0;
  for (const Item& it : items) total = align_up(total + it.bytes, kAlign);
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&w.arena), total);
  if (e != hipSuccess) {
    w.arena = nullptr;
    return set_error(PRG_ERR_OOM, "prefill workspace: hipMalloc(%zu): %s", total, hipGetErrorString(e));
  }
  size_t off = 0;
  for (const Item& it : items) {
    *it.slot = w.arena + off;
    off = align_up(off + it.bytes, kAlign);
  }
  return PRG_OK;
}

// Largest chunk (<= the workspace rows) whose attention scores fit.
uint32_t prefill_chunk_tokens(const PrgModelState* st, uint32_t start, uint32_t remaining) {
  uint32_t T = std::min(remaining, st->pf.rows);
  while (T > 1 && attn_prefill_scores_elems(T, start) > st->pf.scores_elems) T = (T + 1) / 2;
  return T;
}

namespace {

// x [T, in] -> out [T, out_dim] on the matrix cores (Q4Linear.encodePrefillQmm*,
// linear_q4.zig:197-233). `up` selects the gate/up SiLU pair.
int qmm(hipStream_t s, const uint16_t* x, const Q4Linear& l, uint16_t* out, uint32_t T, int epi,
        const uint16_t* res, const Q4Linear* up, const char* name) {
  GemmArgs g;
  g.a = x;
  g.lda = l.in_dim;
  g.q[0] = GemmQ4{l.weight, l.scales, l.biases, out, l.out_dim, 0, l.dense};
  g.nq = 1;
  if (up) {
    g.q[1] = GemmQ4{up->weight, up->scales, up->biases, nullptr, up->out_dim, 0, up->dense};
    g.nq = 2;
  }
  g.res = res;
  g.M = T;
  g.K = l.in_dim;
  return launch_gemm_q4(s, g, epi, name);
}

// Several projections of the same activations in one launch (each keeps its
// own output buffer); the reference encodes them one after another.
int qmm_multi(hipStream_t s, const uint16_t* x, uint32_t K, uint32_t T, std::initializer_list<std::pair<const Q4Linear*, uint16_t*>> segs,
              const char* name) {
  GemmArgs g;
  g.a = x;
  g.lda = K;
  for (const auto& sg : segs) {
    const Q4Linear& l = *sg.first;
    g.q[g.nq++] = GemmQ4{l.weight, l.scales, l.biases, sg.second, l.out_dim, 0, l.dense};
  }
  g.M = T;
  g.K = K;
  return launch_gemm_q4(s, g, kGemmStore, name);
}

}  // namespace

// DecoderLayer.prefillStepBf16 (decoder_layer.zig:644-760) for T tokens at
// positions start.. : x -> out.
int prefill_layer(PrgModel* m, PrgModelState* st, const DecoderLayer& L, LayerState& ls, const uint16_t* x,
                  uint16_t* out, uint32_t T, uint32_t start) {
  PrefillWs& w = st->pf;
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  if (int rc = launch_rmsnorm(s, x, L.input_norm, w.normed, c.hidden, T, c.rms_eps)) return rc;
  if (L.linear) {  // block_linear.zig:265-361
    const LinearAttentionBlock& b = L.lin;
    const uint32_t has_state = start != 0;  // decoder_layer.zig:635
    if (int rc = qmm_multi(s, w.normed, c.hidden, T,
                           {{&b.in_qkv, w.qkv}, {&b.in_z, w.z}, {&b.in_a, w.a}, {&b.in_b, w.b}},
                           "prefill.in_proj"))
      return rc;
    if (int rc = launch_conv1d_prefill(s, ls.conv, w.qkv, b.conv_weight, w.conv_out, T, has_state)) return rc;
    if (int rc = launch_gdn_prefill_prepare(s, w.conv_out, w.a, w.b, b.a_log, b.dt_bias, w.qn, w.kn, w.g, w.beta,
                                            w.kq, T))
      return rc;
    if (int rc = launch_gdn_prefill(s, ls.recur, w.qn, w.kn, w.conv_out, w.g, w.beta, w.kq, w.y, T, has_state))
      return rc;
    if (int rc = prg_rmsnorm_gated_bf16(s, w.y, b.norm_weight, w.z, w.gated, kGdnDv, c.rms_eps, T * kGdnHv))
      return rc;
    if (int rc = qmm(s, w.gated, b.out_proj, w.attn, T, kGemmStore, nullptr, nullptr, "prefill.out_proj")) return rc;
  } else {  // block_attn.zig:361-498
    const FullAttentionBlock& b = L.full;
    if (int rc = qmm_multi(s, w.normed, c.hidden, T, {{&b.q_proj, w.qp}, {&b.k_proj, w.k}, {&b.v_proj, w.v}},
                           "prefill.qkv_proj"))
      return rc;
    if (int rc = launch_attn_prefill_prepare(s, w.qp, b.q_norm, w.k, b.k_norm, w.v, w.q, w.gate, ls.cache_k,
                                             ls.cache_v, T, start, start, st->stride))
      return rc;
    if (int rc = launch_attn_prefill(s, w.q, ls.cache_k, ls.cache_v, w.gate, w.ctx, w.scores, w.scores_elems, T,
                                     start, st->stride, kAttnScale))
      return rc;
    if (int rc = qmm(s, w.ctx, b.o_proj, w.attn, T, kGemmStore, nullptr, nullptr, "prefill.o_proj")) return rc;
  }
  // decoder_layer.zig:717-735: add + post norm, then the MLP (block_mlp.zig:155-258)
  if (int rc = prg_add_rmsnorm_bf16(s, x, w.attn, L.post_norm, w.resid, w.normed, c.hidden, T, c.rms_eps)) return rc;
  if (int rc = qmm(s, w.normed, L.mlp.gate_proj, w.inter, T, kGemmSiluPair, nullptr, &L.mlp.up_proj,
                   "prefill.mlp.gate_up"))
    return rc;
  return qmm(s, w.inter, L.mlp.down_proj, out, T, kGemmResidual, w.resid, nullptr, "prefill.mlp.down_proj");
}

// Ingest st->prompt[from, len) in chunks on top of a state that holds
// positions [0, from), then the argmax tail on the last row
// (encodePrefillArgmaxTailBf16, model.zig:1307-1324). The caller has set ctl
// to step len-1 of a len-token prompt; the argmax kernel records the
// prediction and advances ctl to position len. With the drafter, each chunk's
// final-normed hidden rows also seed its KV cache (server.zig:1286-1325: the
// drafter consumes hidden[t] with token[t+1]) and the last row is kept in
// st->cur_hidden for the speculative loop.
int run_prefill(PrgModel* m, PrgModelState* st, uint32_t from, uint32_t len, bool with_mtp, uint16_t* hidden_out) {
  if (int rc = ensure_prefill_ws(st)) return rc;
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  PrefillWs& w = st->pf;
  const uint16_t* last = nullptr;
  uint32_t T = 0, tail_rows = 0, tail_start = 0;
  for (uint32_t start = from; start < len; start += T) {
    T = prefill_chunk_tokens(st, start, len - start);
    if (int rc = launch_embedding(s, m->embed.weight, m->embed.scales, m->embed.biases, w.h0, st->prompt + start, 0,
                                  T, c.hidden))
      return rc;
    uint16_t *x = w.h0, *y = w.h1;
    for (uint32_t li = 0; li < c.num_layers; ++li) {
      if (int rc = prefill_layer(m, st, m->layers[li], st->layers[li], x, y, T, start)) return rc;
      std::swap(x, y);
    }
    last = x + static_cast<size_t>(T - 1) * c.hidden;
    if (!with_mtp) continue;
    // normalised hidden rows of this chunk (model.zig:1049-1058)
    if (int rc = launch_rmsnorm(s, x, m->final_norm, w.resid, c.hidden, T, c.rms_eps)) return rc;
    if (hidden_out)
      PRG_HIP(hipMemcpyAsync(hidden_out + static_cast<size_t>(start) * c.hidden, w.resid,
                             sizeof(uint16_t) * T * c.hidden, hipMemcpyDeviceToDevice, s));
    if (start + T < len) {
      // every row has its successor token; the drafter reuses h0/h1 (x is done)
      if (int rc = mtp_prefill_rows(m, st, st->prompt + start + 1, w.resid, T, start)) return rc;
    } else {
      PRG_HIP(hipMemcpyAsync(st->cur_hidden, w.resid + static_cast<size_t>(T - 1) * c.hidden,
                             sizeof(uint16_t) * c.hidden, hipMemcpyDeviceToDevice, s));
      tail_rows = T - 1;  // the last row has no successor in the prompt
      tail_start = start;
    }
  }
  GemvParams p = gemv_params(last, c.hidden);
  p.norm_w = m->final_norm;
  p.eps = c.rms_eps;
  add_seg(p, m->lm_head, nullptr);
  p.seg[0].pval[0] = st->pval;
  p.seg[0].pidx[0] = st->pidx;
  p.argmax_waves = st->argmax_waves;
  if (int rc = run_argmax_gemv(s, p, 1, kNormRms, "lm_head.argmax")) return rc;
  if (int rc = launch_argmax_waves_advance(s, st->pval, st->pidx, st->argmax_waves, st->ctl, st->prompt,
                                           st->predictions))
    return rc;
  if (tail_rows > 0)  // after the tail: the drafter overwrites the rows `last` points into
    return mtp_prefill_rows(m, st, st->prompt + tail_start + 1, w.resid, tail_rows, tail_start);
  return PRG_OK;
}

// Drafter.forwardPrefill (mtp.zig:137-185) over T rows.
int mtp_prefill_rows(PrgModel* m, PrgModelState* st, const uint32_t* tokens_dev, const uint16_t* hidden_rows,
                     uint32_t T, uint32_t start) {
  if (int rc = ensure_prefill_ws(st)) return rc;
  const PrgModelConfig& c = m->cfg;
  const MtpWeights& t = m->mtp;
  hipStream_t s = st->stream;
  PrefillWs& w = st->pf;
  PRG_CHECK_ARG(T <= w.rows, "drafter prefill: %u rows exceed the chunk workspace (%u)", T, w.rows);
  // encodePreFcRows (mtp.zig:244-280): norm(embed) ‖ norm(hidden) -> fc
  if (int rc = launch_embedding(s, m->embed.weight, m->embed.scales, m->embed.biases, w.h0, tokens_dev, 0, T,
                                c.hidden))
    return rc;
  if (int rc = launch_rmsnorm(s, w.h0, t.pre_fc_norm_embedding, w.normed, c.hidden, T, c.rms_eps)) return rc;
  if (int rc = launch_rmsnorm(s, hidden_rows, t.pre_fc_norm_hidden, w.attn, c.hidden, T, c.rms_eps)) return rc;
  if (int rc = launch_concat_rows(s, w.normed, w.attn, w.fc_in, T, c.hidden)) return rc;
  if (int rc = qmm(s, w.fc_in, t.fc, w.h1, T, kGemmStore, nullptr, nullptr, "mtp.fc")) return rc;
  return prefill_layer(m, st, t.layer, st->mtp, w.h1, w.h0, T, start);
}

}  // namespace prg

using namespace prg;

extern "C" {

int prg_model_prefill(PrgModel* model, PrgModelState* st, const uint32_t* prompt, uint32_t prompt_len,
                      uint32_t* next_token) {
  PRG_CHECK_ARG(model && st && prompt && next_token && st->model == model, "prg_model_prefill: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  PRG_CHECK_ARG(prompt_len >= 1, "prg_model_prefill: empty prompt");
  if (prompt_len > st->max_seq)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prompt of %u tokens exceeds max_seq %u", prompt_len, st->max_seq);
  for (uint32_t i = 0; i < prompt_len; ++i)
    if (prompt[i] >= model->cfg.vocab)
      return set_error(PRG_ERR_INVALID_TOKEN, "prompt[%u] = %u >= vocab %u", i, prompt[i], model->cfg.vocab);
  if (int rc = prg_model_state_reset(st)) return rc;
  // Control block as if step prompt_len-1 were running: the argmax tail
  // records predictions[prompt_len-1] and moves the decode loop to prompt_len.
  DecodeCtl ctl{};
  ctl.s = StepScalars{prompt[prompt_len - 1], prompt_len - 1, prompt_len - 1, prompt_len};
  ctl.n = prompt_len - 1;
  ctl.prompt_len = prompt_len;
  ctl.capacity = st->max_seq;
  PRG_HIP(hipMemcpyAsync(st->prompt, prompt, sizeof(uint32_t) * prompt_len, hipMemcpyHostToDevice, st->stream));
  PRG_HIP(hipMemcpyAsync(st->ctl, &ctl, sizeof(ctl), hipMemcpyHostToDevice, st->stream));
  if (int rc = run_prefill(model, st, 0, prompt_len, false)) return rc;
  PRG_HIP(hipMemcpyAsync(next_token, st->predictions + (prompt_len - 1), sizeof(uint32_t), hipMemcpyDeviceToHost,
                         st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  return PRG_OK;
}

}  // extern "C"
