// MTP drafter, two-token verify, and the device-resident speculative loop.
//
// Reference (file:line in the reference tree):
//   Drafter.forwardDraftTokenProfiled       src/model/mtp.zig:187-242
//   Drafter.encodePreFcRows                 src/model/mtp.zig:244-280
//   Drafter.forwardPrefill                  src/model/mtp.zig:137-185
//   forwardTwoTokenDecodeVerifierBf16...    src/model/model.zig:1627-1659
//   encodeStack2Bf16 / decodeStep2Bf16      src/model/model.zig:719-760,
//                                           src/model/decoder_layer.zig:485-516, 784-819
//   encodeArgmaxFromTwoHiddenBf16           src/model/model.zig:1390-1446
//   decodeSpeculativeFromPrefixCache        src/server/decode_loop.zig:163-293
//   prepareVerifierState                    src/server/decode_loop.zig:295-311
//
// The reference verifies on a second ModelState, swaps states on accept and,
// on reject, recomputes the current token on the committed state before
// copying its GDN state and KV range back into the verifier. Here the verify
// runs on the committed state itself:
//   * K/V of both rows go to their cache slots; a rejected draft's slot is the
//     next step's first slot and is simply overwritten;
//   * each GDN layer's row-0 update is written out of place to a snapshot
//     block and row 1 reads it from there, so after a reject one gated copy
//     restores exactly the state a one-token step would have left; the
//     recompute disappears (row 0's argmax and normalised hidden are the
//     same numbers the recompute would produce: every per-row kernel is the
//     single-token kernel, and the M = 2 GEMVs do per-row arithmetic identical
//     to M = 1).
// One step (draft, verify, drafter advance, decide, restore) is one captured
// HIP graph whose positions live in SpecCtl, so the loop replays with no host
// synchronisation until the requested number of tokens has been emitted.
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "model.hpp"

namespace prg {
namespace {

// Accept or reject the draft and advance the control block
// (decode_loop.zig:186-284). Thread 0 owns SpecCtl; the block then copies the
// next drafter hidden (row 1 on accept, row 0 on reject) into cur_hidden.
__global__ void spec_decide_kernel(SpecCtl* __restrict__ c, uint32_t* __restrict__ out,
                                   uint32_t* __restrict__ drafts, const uint4* __restrict__ hnorm2,
                                   uint4* __restrict__ cur_hidden, uint32_t w8) {
  __shared__ uint32_t acc_s;
  if (threadIdx.x == 0) {
    uint32_t accept = 0;
    if (!c->stop) {
      const uint32_t draft = c->v1.token;
      accept = draft == c->verify ? 1u : 0u;
      const uint32_t n = c->n, pos = c->pos;
      drafts[c->attempted] = draft;
      out[n] = c->v0.token;
      if (accept) out[n + 1] = draft;
      const uint32_t cur = accept ? c->bonus : c->verify;
      const uint32_t np = pos + 1 + accept;
      c->reject = accept ? 0u : 1u;
      c->accepted += accept;
      c->attempted += 1;
      c->n = n + 1 + accept;
      c->pos = np;
      c->v0 = StepScalars{cur, np, np, np + 1};
      c->v1 = StepScalars{0u, np + 1, np + 1, np + 2};
      c->d0 = StepScalars{cur, np - 1, np - 1, np};
      c->d1 = StepScalars{0u, np, np, np + 1};
      if (np + 2 > c->capacity || c->n >= c->target) c->stop = 1;
    } else {
      c->reject = 0;
    }
    acc_s = accept;
  }
  __syncthreads();
  const uint4* src = hnorm2 + (acc_s ? w8 : 0);
  for (uint32_t i = threadIdx.x; i < w8; i += blockDim.x) cur_hidden[i] = src[i];
}

// After a rejected draft: GDN states <- the snapshot taken after row 0.
__global__ void spec_restore_kernel(const SpecCtl* __restrict__ c, const uint4* __restrict__ snap,
                                    uint4* __restrict__ live, size_t n16) {
  if (!c->reject) return;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    live[i] = snap[i];
}

template <typename T>
T* snap_of(const PrgModelState* st, T* live) {
  return reinterpret_cast<T*>(st->gdn_snap + (reinterpret_cast<uint8_t*>(live) - st->gdn_base));
}

// Drafter.forwardDraftTokenProfiled (mtp.zig:187-242) for the token at
// token_dev with the target's normalised hidden `hidden`; the draft goes to
// out_token.
int encode_mtp_step(PrgModel* m, PrgModelState* st, const uint32_t* token_dev, const uint16_t* hidden,
                    const StepScalars* step, uint32_t* out_token) {
  // out_token == nullptr: the step only advances the drafter's KV cache, so
  // the final norm and the lm_head argmax are skipped.
  const MtpWeights& t = m->mtp;
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  const uint32_t H = c.hidden;
  // encodePreFcRows: norm(embed(token)) ‖ norm(hidden) -> fc (one launch)
  if (int rc = launch_embed_norm_pair(s, m->embed.weight, m->embed.scales, m->embed.biases, token_dev,
                                     t.pre_fc_norm_embedding, hidden, t.pre_fc_norm_hidden, st->fc_in, H, c.rms_eps))
    return rc;
  GemvParams f = gemv_params(st->fc_in, 2 * H);
  add_seg(f, t.fc, st->mtp_h);
  if (int rc = run_gemv(s, f, kEpiPlain, kNormNone, "mtp.fc")) return rc;
  // the drafter's decoder layer on its own KV cache
  if (int rc = encode_full_attention(m, st, t.layer, st->mtp, st->mtp_h, st->mtp_x, step)) return rc;
  const uint16_t* h[1] = {st->mtp_x};
  uint16_t* inter[1] = {st->inter};
  uint16_t* out[1] = {st->mtp_h};
  if (int rc = encode_mlp(m, st, t.layer, 1, h, inter, out)) return rc;
  if (out_token == nullptr) return PRG_OK;
  // final norm, shared lm_head argmax (mtp.zig:230-233)
  GemvParams p = gemv_params(st->mtp_h, H);
  p.norm_w = t.norm;
  p.eps = c.rms_eps;
  add_seg(p, m->lm_head, nullptr);
  p.seg[0].pval[0] = st->pval;
  p.seg[0].pidx[0] = st->pidx;
  p.argmax_waves = st->argmax_waves;
  if (int rc = run_argmax_gemv(s, p, 1, kNormRms, "mtp.lm_head.argmax")) return rc;
  const float* vals[1] = {st->pval};
  const uint32_t* rows[1] = {st->pidx};
  uint32_t* outs[1] = {out_token};
  return launch_argmax_waves(s, 1, vals, rows, st->argmax_waves, outs);
}

// Two tokens through the target (tokens and positions in spec->v0 / v1):
// per layer row 0 then row 1 through attention / GDN, both rows through the
// MLP at M = 2; then the two final norms, the M = 2 lm_head argmax, verify and
// bonus tokens, and the normalised hidden rows in hnorm2.
int encode_verify(PrgModel* m, PrgModelState* st) {
  const PrgModelConfig& c = m->cfg;
  hipStream_t s = st->stream;
  const uint32_t H = c.hidden;
  SpecCtl* sc = st->spec;
  uint16_t* xa[2] = {st->h2a, st->h2a + H};
  uint16_t* xb[2] = {st->h2b, st->h2b + H};
  uint16_t* inter[2] = {st->inter2, st->inter2 + c.intermediate};
  // both rows' tokens in one launch (v0 and v1 are consecutive StepScalars; xa[1] = xa[0] + H)
  static_assert(sizeof(StepScalars) % sizeof(uint32_t) == 0, "token stride");
  if (int rc = launch_embedding(s, m->embed.weight, m->embed.scales, m->embed.biases, xa[0], &sc->v0.token, 0, 2, H,
                                sizeof(StepScalars) / sizeof(uint32_t)))
    return rc;
  for (size_t i = 0; i < m->layers.size(); ++i) {
    const DecoderLayer& L = m->layers[i];
    LayerState& ls = st->layers[i];
    int rc;
    // v0 and v1 are consecutive in SpecCtl: &sc->v0 is the two rows' steps.
    const uint16_t* xin[2] = {xa[0], xa[1]};
    if (L.linear) {
      // row 0's GDN update goes to the snapshot, row 1 continues from it
      if ((rc = encode_linear_attention2(m, st, L,
                                         GdnIO{ls.conv, snap_of(st, ls.conv), ls.recur, snap_of(st, ls.recur)}, xin,
                                         xb, &sc->v0)))
        return rc;
    } else {
      if ((rc = encode_full_attention2(m, st, L, ls, xin, xb, &sc->v0))) return rc;
    }
    const uint16_t* hin[2] = {xb[0], xb[1]};
    if ((rc = encode_mlp(m, st, L, 2, hin, inter, xa))) return rc;
  }
  if (int rc = launch_rmsnorm(s, st->h2a, m->final_norm, st->hnorm2, H, 2, c.rms_eps)) return rc;
  GemvParams p = gemv_params(st->hnorm2, H);
  p.x[1] = st->hnorm2 + H;
  add_seg(p, m->lm_head, nullptr);
  p.seg[0].pval[0] = st->pval;
  p.seg[0].pidx[0] = st->pidx;
  p.seg[0].pval[1] = st->pval2;
  p.seg[0].pidx[1] = st->pidx2;
  p.argmax_waves = st->argmax_waves;
  // The norm stays a launch of its own. Fused into the decode-layout M = 2
  // prologue, with block 0 writing the normalised rows, the speculative step
  // measured 1.784-1.786 ms against 1.774-1.778 ms with this launch.
  if (int rc = run_argmax_gemv(s, p, 2, kNormNone, "lm_head.argmax2")) return rc;
  const float* vals[2] = {st->pval, st->pval2};
  const uint32_t* rows[2] = {st->pidx, st->pidx2};
  uint32_t* outs[2] = {&sc->verify, &sc->bonus};
  return launch_argmax_waves(s, 2, vals, rows, st->argmax_waves, outs);
}

// One speculative step (decode_loop.zig:173-284).
int encode_spec_step(PrgModel* m, PrgModelState* st) {
  hipStream_t s = st->stream;
  SpecCtl* sc = st->spec;
  if (int rc = encode_mtp_step(m, st, &sc->v0.token, st->cur_hidden, &sc->d0, &sc->v1.token)) return rc;
  if (int rc = encode_verify(m, st)) return rc;
  // the drafter consumes (draft, hidden after the current token) whether or not
  // the draft is accepted: on a reject the next draft step rewrites that slot.
  // Only its KV cache matters here, so no lm_head.
  if (int rc = encode_mtp_step(m, st, &sc->v1.token, st->hnorm2, &sc->d1, nullptr)) return rc;
  const uint32_t w8 = m->cfg.hidden / 8;
  hipLaunchKernelGGL(spec_decide_kernel, dim3(1), dim3(256), 0, s, sc, st->spec_out, st->drafts,
                     reinterpret_cast<const uint4*>(st->hnorm2), reinterpret_cast<uint4*>(st->cur_hidden), w8);
  PRG_CHECK_LAUNCH("spec_decide");
  hipLaunchKernelGGL(spec_restore_kernel, dim3(1024), dim3(256), 0, s, sc,
                     reinterpret_cast<const uint4*>(st->gdn_snap), reinterpret_cast<uint4*>(st->gdn_base),
                     st->gdn_bytes / 16);
  PRG_CHECK_LAUNCH("spec_restore");
  return PRG_OK;
}

int run_spec_step(PrgModel* m, PrgModelState* st) {
  if (st->eager) return encode_spec_step(m, st);
  if (!st->graph_spec) {
    hipGraph_t g = nullptr;
    PRG_HIP(hipStreamBeginCapture(st->stream, hipStreamCaptureModeThreadLocal));
    const int rc = encode_spec_step(m, st);
    hipError_t e = hipStreamEndCapture(st->stream, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return set_error(PRG_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(&st->graph_spec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return set_error(PRG_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  }
  PRG_HIP(hipGraphLaunch(st->graph_spec, st->stream));
  return PRG_OK;
}

int check_tokens(const PrgModel* m, const uint32_t* t, uint32_t n) {
  for (uint32_t i = 0; i < n; ++i)
    if (t[i] >= m->cfg.vocab) return set_error(PRG_ERR_INVALID_TOKEN, "token[%u] = %u >= vocab %u", i, t[i], m->cfg.vocab);
  return PRG_OK;
}

}  // namespace

int ensure_spec_ws(PrgModelState* st) {
  if (st->spec_arena) return PRG_OK;
  const PrgModel* m = st->model;
  const PrgModelConfig& c = m->cfg;
  const size_t bf = sizeof(uint16_t), H = c.hidden, I = c.intermediate, S = st->stride;
  const size_t kv = bf * kAttnKvHeads * S * kAttnHeadDim;
  struct Item {
    void** slot;
    size_t bytes;
  };
  const Item items[] = {
      {reinterpret_cast<void**>(&st->mtp.cache_k), m->mtp.present ? kv : 0},
      {reinterpret_cast<void**>(&st->mtp.cache_v), m->mtp.present ? kv : 0},
      {reinterpret_cast<void**>(&st->gdn_snap), st->gdn_bytes},
      {reinterpret_cast<void**>(&st->h2a), bf * 2 * H},
      {reinterpret_cast<void**>(&st->h2b), bf * 2 * H},
      {reinterpret_cast<void**>(&st->inter2), bf * 2 * I},
      {reinterpret_cast<void**>(&st->hnorm2), bf * 2 * H},
      {reinterpret_cast<void**>(&st->cur_hidden), bf * H},
      {reinterpret_cast<void**>(&st->fc_in), bf * 2 * H},
      {reinterpret_cast<void**>(&st->mtp_x), bf * H},
      {reinterpret_cast<void**>(&st->mtp_h), bf * H},
      {reinterpret_cast<void**>(&st->pval2), sizeof(float) * kArgmaxMaxWaves},
      {reinterpret_cast<void**>(&st->pidx2), sizeof(uint32_t) * kArgmaxMaxWaves},
      {reinterpret_cast<void**>(&st->spec_out), sizeof(uint32_t) * (S + 4)},
      {reinterpret_cast<void**>(&st->drafts), sizeof(uint32_t) * (S + 4)},
      {reinterpret_cast<void**>(&st->spec), sizeof(SpecCtl)},
  };
  size_t total = 0;
  for (const Item& it : items) total = align_up(total + it.bytes, kAlign);
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&st->spec_arena), total);
  if (e != hipSuccess) {
    st->spec_arena = nullptr;
    return set_error(PRG_ERR_OOM, "speculative workspace: hipMalloc(%zu): %s", total, hipGetErrorString(e));
  }
  size_t off = 0;
  for (const Item& it : items) {
    *it.slot = it.bytes ? st->spec_arena + off : nullptr;
    off = align_up(off + it.bytes, kAlign);
  }
  if ((e = hipMemsetAsync(st->spec_arena, 0, total, st->stream)) != hipSuccess)
    return set_error(PRG_ERR_HIP, "speculative workspace: %s", hipGetErrorString(e));
  if (m->mtp.present) {  // the drafter's KV cache, readable by name like the target's
    st->tensors["mtp.cache_k"] = TensorRef{reinterpret_cast<uint8_t*>(st->mtp.cache_k), kv};
    st->tensors["mtp.cache_v"] = TensorRef{reinterpret_cast<uint8_t*>(st->mtp.cache_v), kv};
  }
  return PRG_OK;
}

}  // namespace prg

using namespace prg;

extern "C" {

int prg_model_forward_two_tokens(PrgModel* model, PrgModelState* st, uint32_t token0, uint32_t token1,
                                 uint32_t cache_pos, uint32_t rope_pos, uint32_t seq_len,
                                 uint32_t* verify_token, uint32_t* bonus_token, uint16_t* hidden_out) {
  PRG_CHECK_ARG(model && st && verify_token && bonus_token && st->model == model,
                "prg_model_forward_two_tokens: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  if (static_cast<uint64_t>(cache_pos) + 2 > st->max_seq)  // model.zig:1645-1646
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "cache_pos %u + 2 > max_seq %u", cache_pos, st->max_seq);
  const uint32_t toks[2] = {token0, token1};
  if (int rc = check_tokens(model, toks, 2)) return rc;
  if (seq_len != cache_pos + 1)
    return set_error(PRG_ERR_INVALID_ARG, "seq_len %u != cache_pos + 1 (prefix caches are not supported)", seq_len);
  if (int rc = ensure_spec_ws(st)) return rc;
  SpecCtl c{};
  c.v0 = StepScalars{token0, cache_pos, rope_pos, seq_len};
  c.v1 = StepScalars{token1, cache_pos + 1, rope_pos + 1, seq_len + 1};
  c.capacity = st->max_seq;
  PRG_HIP(hipMemcpyAsync(st->spec, &c, sizeof(c), hipMemcpyHostToDevice, st->stream));
  if (int rc = encode_verify(model, st)) return rc;
  PRG_HIP(hipMemcpyAsync(&c, st->spec, sizeof(c), hipMemcpyDeviceToHost, st->stream));
  if (hidden_out)
    PRG_HIP(hipMemcpyAsync(hidden_out, st->hnorm2, sizeof(uint16_t) * 2 * model->cfg.hidden,
                           hipMemcpyDeviceToDevice, st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  *verify_token = c.verify;
  *bonus_token = c.bonus;
  // Both tokens are now in the state: a later prg_model_decode continues at
  // cache_pos + 2 with the bonus token, as after two single steps.
  const uint32_t preds[2] = {c.verify, c.bonus};
  DecodeCtl ctl{};
  ctl.s = StepScalars{c.bonus, cache_pos + 2, rope_pos + 2, cache_pos + 3};
  ctl.n = cache_pos + 2;
  ctl.rope_off = rope_pos - cache_pos;
  ctl.capacity = st->max_seq;
  ctl.overflow = cache_pos + 2 >= st->max_seq;
  PRG_HIP(hipMemcpyAsync(st->predictions + cache_pos, preds, sizeof(preds), hipMemcpyHostToDevice, st->stream));
  PRG_HIP(hipMemcpyAsync(st->ctl, &ctl, sizeof(ctl), hipMemcpyHostToDevice, st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  return PRG_OK;
}

int prg_model_mtp_draft(PrgModel* model, PrgModelState* st, uint32_t token, const uint16_t* hidden,
                        uint32_t cache_pos, uint32_t rope_pos, uint32_t seq_len, uint32_t* draft_token) {
  PRG_CHECK_ARG(model && st && hidden && draft_token && st->model == model, "prg_model_mtp_draft: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  PRG_CHECK_ARG(model->mtp.present, "prg_model_mtp_draft: the model has no MTP drafter");
  if (cache_pos >= st->max_seq)  // mtp.zig:202
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "cache_pos %u >= max_seq %u", cache_pos, st->max_seq);
  if (int rc = check_tokens(model, &token, 1)) return rc;
  if (seq_len != cache_pos + 1)
    return set_error(PRG_ERR_INVALID_ARG, "seq_len %u != cache_pos + 1", seq_len);
  if (int rc = ensure_spec_ws(st)) return rc;
  SpecCtl c{};
  c.v0.token = token;
  c.d0 = StepScalars{token, cache_pos, rope_pos, seq_len};
  c.capacity = st->max_seq;
  PRG_HIP(hipMemcpyAsync(st->spec, &c, sizeof(c), hipMemcpyHostToDevice, st->stream));
  PRG_HIP(hipMemcpyAsync(st->cur_hidden, hidden, sizeof(uint16_t) * model->cfg.hidden, hipMemcpyDeviceToDevice,
                         st->stream));
  if (int rc = encode_mtp_step(model, st, &st->spec->v0.token, st->cur_hidden, &st->spec->d0, &st->spec->v1.token))
    return rc;
  PRG_HIP(hipMemcpyAsync(&c, st->spec, sizeof(c), hipMemcpyDeviceToHost, st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  *draft_token = c.v1.token;
  return PRG_OK;
}

int prg_model_mtp_prefill(PrgModel* model, PrgModelState* st, const uint32_t* tokens, uint32_t token_count,
                          const uint16_t* hidden_rows, uint32_t start_pos) {
  PRG_CHECK_ARG(model && st && tokens && hidden_rows && st->model == model, "prg_model_mtp_prefill: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  PRG_CHECK_ARG(model->mtp.present, "prg_model_mtp_prefill: the model has no MTP drafter");
  if (token_count == 0) return PRG_OK;  // mtp.zig:148
  if (static_cast<uint64_t>(start_pos) + token_count > st->max_seq)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "%u + %u tokens exceed max_seq %u", start_pos, token_count,
                     st->max_seq);
  if (int rc = check_tokens(model, tokens, token_count)) return rc;
  if (int rc = ensure_spec_ws(st)) return rc;
  if (int rc = ensure_prefill_ws(st)) return rc;
  // the device copy of the tokens is staged in spec_out (sized for the cache)
  PRG_HIP(hipMemcpyAsync(st->spec_out, tokens, sizeof(uint32_t) * token_count, hipMemcpyHostToDevice, st->stream));
  const size_t H = model->cfg.hidden;
  for (uint32_t off = 0; off < token_count;) {
    const uint32_t T = prefill_chunk_tokens(st, start_pos + off, token_count - off);
    if (int rc = mtp_prefill_rows(model, st, st->spec_out + off, hidden_rows + off * H, T, start_pos + off)) return rc;
    off += T;
  }
  PRG_HIP(hipStreamSynchronize(st->stream));
  return PRG_OK;
}

}  // extern "C"

namespace {

// Shared body of the two speculative entry points. prefix_len == 0: reset and
// prefill the whole prompt. prefix_len > 0: the state already holds
// prompt[0, prefix_len); the drafter is seeded from prefix_hidden for those
// positions (seedMtpDrafter, server.zig:1240-1330), then the rest of the
// prompt is prefilled as usual.
int generate_speculative(PrgModel* model, PrgModelState* st, const uint32_t* prompt, uint32_t prompt_len,
                         uint32_t prefix_len, const uint16_t* prefix_hidden, uint16_t* hidden_out, uint32_t n_new,
                         uint32_t* tokens_out, uint32_t* accepted, uint32_t* attempted, float* decode_ms) {
  PRG_CHECK_ARG(model && st && prompt && tokens_out && st->model == model,
                "prg_model_generate_speculative: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  PRG_CHECK_ARG(model->mtp.present, "prg_model_generate_speculative: the model has no MTP drafter");
  PRG_CHECK_ARG(prompt_len >= 1 && n_new >= 1, "prg_model_generate_speculative: empty prompt or n_new == 0");
  PRG_CHECK_ARG(prefix_len < prompt_len, "prg_model_generate_speculative: prefix_len %u must be below prompt_len %u",
                prefix_len, prompt_len);
  PRG_CHECK_ARG(prefix_len == 0 || prefix_hidden != nullptr,
                "prg_model_generate_speculative: a cached prefix needs its hidden rows");
  if (static_cast<uint64_t>(prompt_len) + n_new + 2 > st->max_seq)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prompt %u + %u new tokens (+2 verify slots) exceed max_seq %u",
                     prompt_len, n_new, st->max_seq);
  if (int rc = check_tokens(model, prompt, prompt_len)) return rc;
  if (int rc = ensure_spec_ws(st)) return rc;
  if (prefix_len == 0)
    if (int rc = prg_model_state_reset(st)) return rc;
  // prompt: target prefill + drafter seeding; next token -> predictions[len-1]
  DecodeCtl ctl{};
  ctl.s = StepScalars{prompt[prompt_len - 1], prompt_len - 1, prompt_len - 1, prompt_len};
  ctl.n = prompt_len - 1;
  ctl.prompt_len = prompt_len;
  ctl.capacity = st->max_seq;
  PRG_HIP(hipMemcpyAsync(st->prompt, prompt, sizeof(uint32_t) * prompt_len, hipMemcpyHostToDevice, st->stream));
  PRG_HIP(hipMemcpyAsync(st->ctl, &ctl, sizeof(ctl), hipMemcpyHostToDevice, st->stream));
  if (prefix_len > 0) {
    // drafter rows t < prefix_len pair hidden[t] with prompt[t + 1]; they go
    // first, since the suffix rows attend to them
    if (int rc = ensure_prefill_ws(st)) return rc;
    const size_t H = model->cfg.hidden;
    for (uint32_t t = 0; t < prefix_len;) {
      const uint32_t T = prefill_chunk_tokens(st, t, prefix_len - t);
      if (int rc = mtp_prefill_rows(model, st, st->prompt + t + 1, prefix_hidden + t * H, T, t)) return rc;
      t += T;
    }
    if (hidden_out)
      PRG_HIP(hipMemcpyAsync(hidden_out, prefix_hidden, sizeof(uint16_t) * prefix_len * H, hipMemcpyDeviceToDevice,
                             st->stream));
  }
  if (int rc = run_prefill(model, st, prefix_len, prompt_len, true, hidden_out)) return rc;
  uint32_t first = 0;
  PRG_HIP(hipMemcpyAsync(&first, st->predictions + (prompt_len - 1), sizeof(uint32_t), hipMemcpyDeviceToHost,
                         st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  // decode_loop.zig:163-171: the current token sits at position prompt_len
  const uint32_t L = prompt_len;
  SpecCtl c{};
  c.v0 = StepScalars{first, L, L, L + 1};
  c.v1 = StepScalars{0u, L + 1, L + 1, L + 2};
  c.d0 = StepScalars{first, L - 1, L - 1, L};
  c.d1 = StepScalars{0u, L, L, L + 1};
  c.pos = L;
  c.capacity = st->max_seq;
  c.target = n_new;
  PRG_HIP(hipMemcpyAsync(st->spec, &c, sizeof(c), hipMemcpyHostToDevice, st->stream));
  PRG_HIP(hipEventRecord(st->ev0, st->stream));
  uint32_t n = 0;
  while (n < n_new) {
    // Each step emits 1 or 2 tokens, so ceil(remaining / 2) steps never run
    // past the request: at most n_new + 1 tokens, and no step after the one
    // that reaches n_new (the decide kernel also stops there).
    const uint32_t batch = std::min<uint32_t>(8, (n_new - n + 1) / 2);
    for (uint32_t i = 0; i < batch; ++i)
      if (int rc = run_spec_step(model, st)) return rc;
    PRG_HIP(hipMemcpyAsync(&c, st->spec, sizeof(c), hipMemcpyDeviceToHost, st->stream));
    PRG_HIP(hipStreamSynchronize(st->stream));
    if (c.n == n && c.stop) return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "speculative loop reached max_seq");
    n = c.n;
  }
  PRG_HIP(hipEventRecord(st->ev1, st->stream));
  PRG_HIP(hipMemcpyAsync(tokens_out, st->spec_out, sizeof(uint32_t) * n_new, hipMemcpyDeviceToHost, st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  if (decode_ms) PRG_HIP(hipEventElapsedTime(decode_ms, st->ev0, st->ev1));
  if (accepted) *accepted = c.accepted;
  if (attempted) *attempted = c.attempted;
  return PRG_OK;
}

}  // namespace

extern "C" {

int prg_model_generate_speculative(PrgModel* model, PrgModelState* st, const uint32_t* prompt, uint32_t prompt_len,
                                   uint32_t n_new, uint32_t* tokens_out, uint32_t* accepted, uint32_t* attempted,
                                   float* decode_ms) {
  return generate_speculative(model, st, prompt, prompt_len, 0, nullptr, nullptr, n_new, tokens_out, accepted,
                              attempted, decode_ms);
}

int prg_model_generate_speculative_from(PrgModel* model, PrgModelState* st, const uint32_t* prompt,
                                        uint32_t prompt_len, uint32_t prefix_len, const uint16_t* prefix_hidden,
                                        uint16_t* hidden_out, uint32_t n_new, uint32_t* tokens_out,
                                        uint32_t* accepted, uint32_t* attempted, float* decode_ms) {
  return generate_speculative(model, st, prompt, prompt_len, prefix_len, prefix_hidden, hidden_out, n_new,
                              tokens_out, accepted, attempted, decode_ms);
}

}  // extern "C"
