// Prefix reuse on the model side: copies between ModelStates of one model and
// prefill on top of a restored prefix.
//
// Reference: ModelState.copyPrefixFrom / copyLinearStateFrom /
// copyFullAttentionRangeFrom (src/model/state.zig:124-180,
// copyFullAttentionKeyRange / ValueRange :182-240); the prefix-hit prefill
// (DeviceModel.prefillLayerMajor* with a PrefixState, model.zig:940-1060).
//
// The reference decodes on top of a cached prefix by binding two KV sources in
// its attention kernels (prefix cache + local cache, block_attn.zig:340-348).
// Here the prefix state is copied device-to-device into the working state
// (K rows of 512 B per token and head, V columns per (head, dim); about
// 0.2 ms for a 16k-token prefix at the 9B shape), after which positions are
// absolute and the decode and prefill kernels keep a single KV source.
#include "model.hpp"

namespace prg {

int copy_attention_range(PrgModelState* dst, uint32_t dst_start, const PrgModelState* src, uint32_t src_start,
                         uint32_t count) {
  PRG_CHECK_ARG(dst && src && dst->model == src->model, "state copy: states of different models");
  if (dst_start > dst->max_seq || count > dst->max_seq - dst_start)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "state copy: [%u, +%u) past destination capacity %u", dst_start,
                     count, dst->max_seq);
  if (src_start > src->max_seq || count > src->max_seq - src_start)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "state copy: [%u, +%u) past source capacity %u", src_start, count,
                     src->max_seq);
  if (count == 0) return PRG_OK;
  PRG_HIP(hipStreamSynchronize(src->stream));
  const size_t row = sizeof(uint16_t) * kAttnHeadDim;
  for (size_t i = 0; i < dst->layers.size(); ++i) {
    const LayerState& s = src->layers[i];
    LayerState& d = dst->layers[i];
    if (!d.cache_k) continue;
    // K [4, stride, 256]: per head, `count` contiguous 512-byte rows
    PRG_HIP(hipMemcpy2DAsync(d.cache_k + static_cast<size_t>(dst_start) * kAttnHeadDim, dst->stride * row,
                             s.cache_k + static_cast<size_t>(src_start) * kAttnHeadDim, src->stride * row,
                             count * row, kAttnKvHeads, hipMemcpyDeviceToDevice, dst->stream));
    // V [4, 256, stride]: per (head, dim), `count` contiguous values
    PRG_HIP(hipMemcpy2DAsync(d.cache_v + dst_start, dst->stride * sizeof(uint16_t), s.cache_v + src_start,
                             src->stride * sizeof(uint16_t), count * sizeof(uint16_t), kAttnKvHeads * kAttnHeadDim,
                             hipMemcpyDeviceToDevice, dst->stream));
  }
  PRG_HIP(hipStreamSynchronize(dst->stream));
  return PRG_OK;
}

int copy_linear_state(PrgModelState* dst, const PrgModelState* src) {
  PRG_CHECK_ARG(dst && src && dst->model == src->model, "state copy: states of different models");
  if (dst == src || dst->gdn_bytes == 0) return PRG_OK;
  PRG_CHECK_ARG(dst->gdn_bytes == src->gdn_bytes, "state copy: GDN blocks differ in size");
  PRG_HIP(hipStreamSynchronize(src->stream));
  PRG_HIP(hipMemcpyAsync(dst->gdn_base, src->gdn_base, dst->gdn_bytes, hipMemcpyDeviceToDevice, dst->stream));
  PRG_HIP(hipStreamSynchronize(dst->stream));
  return PRG_OK;
}

}  // namespace prg

using namespace prg;

extern "C" {

int prg_model_state_copy_range(PrgModelState* dst, uint32_t dst_start, const PrgModelState* src, uint32_t src_start,
                               uint32_t token_count) {
  return copy_attention_range(dst, dst_start, src, src_start, token_count);
}

int prg_model_state_copy_linear(PrgModelState* dst, const PrgModelState* src) { return copy_linear_state(dst, src); }

int prg_model_state_copy_prefix(PrgModelState* dst, const PrgModelState* src, uint32_t token_count) {
  PRG_CHECK_ARG(dst && src, "prg_model_state_copy_prefix: null state");
  if (token_count > dst->max_seq || token_count > src->max_seq)  // state.zig:124-125
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "copy prefix: %u tokens, capacities %u / %u", token_count,
                     dst->max_seq, src->max_seq);
  if (int rc = copy_attention_range(dst, 0, src, 0, token_count)) return rc;
  return copy_linear_state(dst, src);
}

int prg_model_prefill_from(PrgModel* model, PrgModelState* st, const uint32_t* prompt, uint32_t prompt_len,
                           uint32_t prefix_len, uint32_t* next_token) {
  PRG_CHECK_ARG(model && st && prompt && next_token && st->model == model, "prg_model_prefill_from: bad argument");
  if (int rc = ensure_t16(model)) return rc;
  PRG_CHECK_ARG(prefix_len >= 1 && prefix_len < prompt_len,
                "prg_model_prefill_from: prefix_len %u must be in [1, prompt_len %u)", prefix_len, prompt_len);
  if (prompt_len > st->max_seq)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prompt of %u tokens exceeds max_seq %u", prompt_len, st->max_seq);
  for (uint32_t i = 0; i < prompt_len; ++i)
    if (prompt[i] >= model->cfg.vocab)
      return set_error(PRG_ERR_INVALID_TOKEN, "prompt[%u] = %u >= vocab %u", i, prompt[i], model->cfg.vocab);
  DecodeCtl ctl{};
  ctl.s = StepScalars{prompt[prompt_len - 1], prompt_len - 1, prompt_len - 1, prompt_len};
  ctl.n = prompt_len - 1;
  ctl.prompt_len = prompt_len;
  ctl.capacity = st->max_seq;
  PRG_HIP(hipMemcpyAsync(st->prompt, prompt, sizeof(uint32_t) * prompt_len, hipMemcpyHostToDevice, st->stream));
  PRG_HIP(hipMemcpyAsync(st->ctl, &ctl, sizeof(ctl), hipMemcpyHostToDevice, st->stream));
  if (int rc = run_prefill(model, st, prefix_len, prompt_len, false)) return rc;
  PRG_HIP(hipMemcpyAsync(next_token, st->predictions + (prompt_len - 1), sizeof(uint32_t), hipMemcpyDeviceToHost,
                         st->stream));
  PRG_HIP(hipStreamSynchronize(st->stream));
  return PRG_OK;
}

}  // extern "C"
