/*
 * peregrine_model.h — C ABI of the decode model layer in libperegrine_hip.so.
 *
 * Replaces the reference's Zig model composition for the single-stream Q4
 * token loop:
 *   DeviceModel            src/model/model.zig:538-790, 1326-1460, 1564-1662
 *   ModelState             src/model/state.zig:45-180
 *   DecoderLayer           src/model/decoder_layer.zig:461-566, 756-819
 *   LinearAttentionBlock   src/model/block_linear.zig:199-263
 *   FullAttentionBlock     src/model/block_attn.zig:261-359
 *   MlpBlock               src/model/block_mlp.zig:260-311
 *   decodeFromPrefixCache  src/server/decode_loop.zig:96-160 (no prefix)
 *   Repository (safetensors) src/model/safetensors.zig:17-220
 *   verifyFingerprint      src/model/config.zig:34-73, src/model/mtp.zig:318-345
 * Models are either loaded from an MLX safetensors checkpoint
 * (prg_model_load) or random-initialised on the GPU from a seed; both use the
 * reference's tensor layout and names.
 * All functions return 0 or a PRG_ERR_* code (see peregrine_hip.h).
 */
#ifndef PEREGRINE_MODEL_H
#define PEREGRINE_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct PrgModel PrgModel;
typedef struct PrgModelState PrgModelState;

/* Model shape. The attention / GDN head geometry is fixed by the kernels
 * (16 q / 4 kv heads x 256; GDN 16 k / 32 v heads x 128, conv 4). */
typedef struct PrgModelConfig {
  uint32_t num_layers;              /* 32 */
  uint32_t hidden;                  /* 4096, multiple of 512 */
  uint32_t intermediate;            /* 12288, multiple of 512 */
  uint32_t vocab;                   /* 248320, multiple of 8 */
  uint32_t full_attention_interval; /* 4: layer i is full attention iff (i+1) % 4 == 0 */
  float rms_eps;                    /* 1e-6 */
  uint32_t mtp_layers;              /* 0, or 1: the MTP drafter (src/model/mtp.zig) */
} PrgModelConfig;

/* Qwen3.5-9B shape (src/model/config.zig:58-72, dims.zig:3-7). */
void prg_model_default_config(PrgModelConfig *cfg);

/* Allocate and randomly initialise a model on the current device.
 * Q4 weights: nibbles uniform 0..15, scales ~U(0.002, 0.02), biases
 * -7.5*scale + N(0, 0.01) (zero-mean dequantised weights); norm weights
 * 1 + N(0, 0.1); conv weights N(0, 0.5); A_log, dt_bias N(0, 0.5).
 * Replaces DeviceModel.upload (model.zig:580-658). */
int prg_model_create_random(const PrgModelConfig *cfg, uint64_t seed, PrgModel **out);
void prg_model_destroy(PrgModel *model);
/* Total bytes of device weights. */
size_t prg_model_weight_bytes(const PrgModel *model);
/* Prepared dense weights for the prompt path: every Q4 matrix the prefill
 * GEMMs read (projections and MLP of every layer and of the drafter) is
 * dequantised once into a bf16 [out, in] copy (4x its Q4 bytes: ~14 GB for
 * the 9B shape), and the prefill GEMMs then stage those values instead of
 * dequantising each tile; prefill results are identical bit for bit, decode
 * keeps reading the Q4 weights. Call again after changing weights through
 * prg_model_tensor. Replaces the prepared dense RHS buffers
 * (src/model/block_attn.zig:143-215, linear_q4.denseRhsBf16ByteLen). */
int prg_model_prepare_dense(PrgModel *model);
/* Bytes of the prepared dense copies (0 before prg_model_prepare_dense). */
size_t prg_model_dense_bytes(const PrgModel *model);

/* Decode-layout copies (prg_q4_repack_t16) of every GEMV weight whose shape
 * has one (rows % 16 == 0, in_dim % 1024 == 0), read by the matrix-core
 * GEMVs of the token loop, the two-token verify and the drafter. Written by
 * model creation and loading, and again before the next run once
 * prg_model_tensor has handed out a pointer; call this after writing weights
 * through a pointer kept from earlier. PEREGRINE_T16=0 at creation turns the
 * copies (and the matrix-core GEMVs) off. No counterpart in the reference:
 * its Metal kernels read the MLX layout. */
int prg_model_prepare_decode(PrgModel *model);
/* Bytes of the decode-layout copies (0 when off). */
size_t prg_model_decode_layout_bytes(const PrgModel *model);
/* Device pointer and byte size of a named tensor, e.g.
 * "language_model.model.layers.3.self_attn.q_proj.weight" (names as the
 * reference's checkpoint, decoder_layer.zig:376-412). */
int prg_model_tensor(const PrgModel *model, const char *name, void **ptr, size_t *bytes);
/* The model's tensors in name order: count, name of entry `index`, and the
 * checkpoint dtype ("U32", "BF16", "F32") and shape each is stored with (Q4
 * weight [out, in/8] u32, scales / biases [out, in/64] bf16;
 * linear_q4.zig:261-268). */
uint32_t prg_model_tensor_count(const PrgModel *model);
int prg_model_tensor_name(const PrgModel *model, uint32_t index, char *buf, size_t len);
int prg_model_tensor_info(const PrgModel *model, const char *name, char *dtype, size_t dtype_len,
                          uint64_t *shape, uint32_t max_dims, uint32_t *ndim);

/* ======================================================================
 * Prefix reuse: state copies and prefill on top of a restored prefix.
 * ====================================================================== */

/* ModelState.copyPrefixFrom (state.zig:124-128): K/V of positions
 * [0, token_count) of every attention layer and all GDN conv / recurrent
 * states, from src to dst (same model; strides may differ). Ordered after
 * src's pending work; complete on return. */
int prg_model_state_copy_prefix(PrgModelState *dst, const PrgModelState *src, uint32_t token_count);
/* copyFullAttentionRangeFrom (state.zig:144-180): K/V positions
 * [src_start, +token_count) of src to [dst_start, ...) of dst. */
int prg_model_state_copy_range(PrgModelState *dst, uint32_t dst_start, const PrgModelState *src,
                               uint32_t src_start, uint32_t token_count);
/* copyLinearStateFrom (state.zig:130-142): the GDN conv / recurrent states. */
int prg_model_state_copy_linear(PrgModelState *dst, const PrgModelState *src);

/* Prefill prompt[prefix_len, prompt_len) on top of a state that already holds
 * prompt[0, prefix_len) (restored from a prefix cache entry, or left by an
 * earlier prefill), then the greedy argmax tail; the state is positioned to
 * decode from prompt_len as after prg_model_prefill. 1 <= prefix_len <
 * prompt_len. Replaces the prefix-hit prefill (model.zig:940-1060 with a
 * PrefixState). The prefix is copied into the working state instead of being
 * bound as a second KV source, so positions are absolute. */
int prg_model_prefill_from(PrgModel *model, PrgModelState *state, const uint32_t *prompt, uint32_t prompt_len,
                           uint32_t prefix_len, uint32_t *next_token);

/* ======================================================================
 * Prompt-prefix cache (src/server/prefix_state_cache.zig:21-795) and its
 * PRGPFXS1 v3 file (src/server/prefix_persist.zig:31-412).
 * ====================================================================== */

typedef struct PrgPrefixCache PrgPrefixCache;
/* Cache.Match: entry index and matched length (len 0 = no match). Indexes
 * shift when entries are removed; use the match a mutator returns. */
typedef struct PrgPrefixMatch {
  uint32_t index;
  uint32_t len;
} PrgPrefixMatch;
/* Cache.Stats (prefix_state_cache.zig:343-366) plus resident_tokens. */
typedef struct PrgPrefixCacheStats {
  uint64_t hits, misses, hit_tokens, computed_tokens;
  uint64_t reserved_tokens, resident_tokens, max_tokens, entry_count, evictions;
} PrgPrefixCacheStats;

/* Cache.init(max_cache_tokens, prefill_chunk_tokens). Entries own a state of
 * max(tokens, min(max_cache_tokens, prefill_chunk_tokens)) positions; the sum
 * of those capacities stays within max_cache_tokens by evicting the least
 * recently used unpinned entry. model may be NULL: the cache then keeps tokens
 * and accounting only (store takes a NULL work state; restore, save and load
 * need a model). */
int prg_prefix_cache_create(PrgModel *model, uint32_t max_cache_tokens, uint32_t prefill_chunk_tokens,
                            PrgPrefixCache **out);
void prg_prefix_cache_destroy(PrgPrefixCache *cache);
int prg_prefix_cache_clear(PrgPrefixCache *cache);                 /* clearAll */
uint32_t prg_prefix_cache_entry_count(const PrgPrefixCache *cache);
uint32_t prg_prefix_cache_pinned_count(const PrgPrefixCache *cache);
uint32_t prg_prefix_cache_active_tokens(const PrgPrefixCache *cache);
int prg_prefix_cache_stats(const PrgPrefixCache *cache, PrgPrefixCacheStats *stats);
void prg_prefix_cache_record_hit(PrgPrefixCache *cache, uint32_t reused_tokens);
void prg_prefix_cache_record_miss(PrgPrefixCache *cache);
void prg_prefix_cache_record_computed(PrgPrefixCache *cache, uint32_t token_count);
/* findPrefix: the longest cached entry that is a prefix of prompt. */
int prg_prefix_cache_find(const PrgPrefixCache *cache, const uint32_t *prompt, uint32_t prompt_len,
                          PrgPrefixMatch *match);
/* containsPromptPrefix: 1 when prompt[0, prefix_len) is an entry, else 0. */
int prg_prefix_cache_contains(const PrgPrefixCache *cache, const uint32_t *prompt, uint32_t prompt_len,
                              uint32_t prefix_len);
int prg_prefix_cache_touch(PrgPrefixCache *cache, PrgPrefixMatch match);
int prg_prefix_cache_remove(PrgPrefixCache *cache, uint32_t index);  /* removeEntry */
int prg_prefix_cache_entry_info(const PrgPrefixCache *cache, uint32_t index, uint32_t *token_count,
                                uint32_t *capacity, int *pinned, uint64_t *hits);
int prg_prefix_cache_entry_tokens(const PrgPrefixCache *cache, uint32_t index, uint32_t *tokens, uint32_t capacity);
/* entryStateMut: the entry's state (prefill into it after start_direct). */
int prg_prefix_cache_entry_state(PrgPrefixCache *cache, uint32_t index, PrgModelState **state);
int prg_prefix_cache_cached_next_token(const PrgPrefixCache *cache, PrgPrefixMatch match, uint32_t *token,
                                       int *valid);
/* startDirectEntry / finishDirectEntry: reserve (or reuse) the entry for ids,
 * reset its state for a direct prefill, then record its next token. */
int prg_prefix_cache_start_direct(PrgPrefixCache *cache, const uint32_t *ids, uint32_t n, int pinned,
                                  PrgPrefixMatch *out);
int prg_prefix_cache_finish_direct(PrgPrefixCache *cache, PrgPrefixMatch match, uint32_t next_token);
/* storePrefixFromWork: cache ids[0, n) from a working state that holds those
 * positions. With `reuse` (a match the work state was restored from) that
 * entry is re-keyed to the longer prefix and takes positions [reuse->len, n)
 * plus the GDN state; otherwise positions [0, n) are copied. work_hidden
 * (device bf16 rows, may be NULL) feeds the hidden rows when tracking is on;
 * next_token (host, may be NULL) is the cached greedy successor. */
int prg_prefix_cache_store(PrgPrefixCache *cache, const uint32_t *ids, uint32_t n, const PrgPrefixMatch *reuse,
                           const PrgModelState *work, const uint16_t *work_hidden, uint32_t work_hidden_base_rows,
                           const uint32_t *next_token, int pinned, PrgPrefixMatch *out);
/* Copy a full-entry match into a working state (positions [0, match.len) and
 * the GDN states); continue with prg_model_prefill_from. */
int prg_prefix_cache_restore(const PrgPrefixCache *cache, PrgPrefixMatch match, PrgModelState *work);
/* Normalised hidden rows per entry (MTP drafter seeding):
 * enableHiddenTracking, entryHidden / entryHiddenValid, setEntryHidden. */
int prg_prefix_cache_enable_hidden(PrgPrefixCache *cache);
int prg_prefix_cache_entry_hidden(const PrgPrefixCache *cache, PrgPrefixMatch match, uint16_t **rows, int *valid);
int prg_prefix_cache_set_entry_hidden(PrgPrefixCache *cache, PrgPrefixMatch match, const uint16_t *rows);

/* PRGPFXS1 v3: 48-byte header {magic u64, version u32 = 3, dtype u32 = 0
 * (bf16), model_fingerprint u64, token_count u64, next_token u32,
 * next_token_valid u32, hidden_valid u32, pad}, the token ids u32, then per
 * layer in order the GDN conv f32 [3, 8192] and recurrent f32 [32, 128, 128],
 * or K [4][T][256] and V [4][256][T] bf16 compacted to the T cached tokens,
 * then the hidden rows bf16 [T, hidden] (zeros unless hidden_valid). Little
 * endian (prefix_persist.zig:36-80, 253-328). */
/* save: atomically (temp file + rename) write the active entry, else the most
 * recently used one. EMPTY_INPUT when nothing is cached. */
int prg_prefix_cache_save(const PrgPrefixCache *cache, const char *path, uint64_t model_fingerprint);
/* load: validate magic, version, dtype, fingerprint, next token < vocab,
 * flags, token count within the budget and the exact file length; a missing
 * or invalid file leaves the cache unchanged and sets *loaded_tokens = 0
 * (prg_last_error() says why). A valid file replaces the cache's contents with
 * one pinned, active entry. Errors only for failures while reading, after
 * which the cache is empty. */
int prg_prefix_cache_load(PrgPrefixCache *cache, const char *path, uint64_t model_fingerprint,
                          uint32_t *loaded_tokens);
/* Byte length of a PRGPFXS1 file of token_count tokens for this topology
 * (expectedFileBytes, prefix_persist.zig:71-80). */
int prg_prefix_state_file_bytes(const PrgModelConfig *cfg, uint64_t token_count, uint64_t *bytes);
/* $HOME/.cache/peregrine/qwen35-9b-q4-prefix-state.bin (resolveDefaultPath). */
int prg_prefix_state_default_path(char *buf, size_t len);
/* modelFingerprint (prefix_persist.zig:149-190): Wyhash seeded with
 * MAGIC ^ VERSION over config.json, then each *.safetensors file in bytewise
 * name order (name, then content). */
int prg_model_fingerprint(const char *model_dir, uint64_t *out);
/* The Wyhash used above (std.hash.Wyhash: final-v4 rounds, original secret). */
int prg_wyhash(const void *data, size_t len, uint64_t seed, uint64_t *out);

/* ======================================================================
 * Checkpoints (host code; no GPU needed except for prg_model_load).
 * ====================================================================== */

/* A directory of safetensors shards named by model.safetensors.index.json.
 * Replaces safetensors.Repository.open / deinit (safetensors.zig:25-87):
 * shards are the index's unique weight_map values, sorted; each header is
 * parsed into the tensor table. Errors: NOT_FOUND (no index or shard),
 * MALFORMED (TruncatedHeader, MalformedHeader, MalformedIndex, NoShardsFound). */
typedef struct PrgSafetensors PrgSafetensors;
int prg_safetensors_open(const char *dir, PrgSafetensors **out);
void prg_safetensors_close(PrgSafetensors *st);
uint32_t prg_safetensors_shard_count(const PrgSafetensors *st);
int prg_safetensors_shard_name(const PrgSafetensors *st, uint32_t index, char *buf, size_t len);
/* Tensors in name order. */
uint32_t prg_safetensors_tensor_count(const PrgSafetensors *st);
int prg_safetensors_tensor_name(const PrgSafetensors *st, uint32_t index, char *buf, size_t len);
/* Repository.get + tensorByteLen (safetensors.zig:98-104, 123-141): dtype
 * string, shape (up to max_dims), byte length and shard index (each output
 * may be NULL except ndim and bytes). NOT_FOUND for an unknown name. */
int prg_safetensors_tensor_info(const PrgSafetensors *st, const char *name, char *dtype, size_t dtype_len,
                                uint64_t *shape, uint32_t max_dims, uint32_t *ndim, uint64_t *bytes,
                                uint32_t *shard);
/* Repository.readInto (safetensors.zig:89-100): the tensor's bytes into host
 * memory `dst` of exactly `bytes` (InvalidTensorBuffer otherwise). */
int prg_safetensors_read(const PrgSafetensors *st, const char *name, void *dst, uint64_t bytes);

/* config.verifyFingerprint (config.zig:34-73): the exact Qwen3.5-9B MLX
 * affine 4-bit group-64 checkpoint, else UNSUPPORTED with the reference's
 * error name in prg_last_error(). */
int prg_checkpoint_verify_config(const char *dir);
/* mtp.verifyFingerprint (mtp.zig:318-345) for the MTP sidecar directory. */
int prg_checkpoint_verify_mtp_config(const char *dir);
/* config.json -> PrgModelConfig (layers, widths, vocab, attention interval,
 * rms_norm_eps). Applies verifyFingerprint's generic checks, then requires
 * the head geometry the kernels implement; depth and widths are free. */
int prg_checkpoint_read_config(const char *dir, PrgModelConfig *cfg);

/* Allocate a model of shape *cfg and fill every tensor from the checkpoint
 * in target_dir (and, with cfg->mtp_layers == 1, the drafter from mtp_dir,
 * whose tensor root is detected as in mtp.zig:347-355). Each tensor must be
 * present with the dtype and shape prg_model_tensor_info reports (A_log may
 * also be stored as bf16; it is widened to f32). Bytes go file -> pinned
 * staging -> device, double-buffered. Replaces DeviceModel.upload
 * (model.zig:580-658), DecoderLayer.upload (decoder_layer.zig:376-412),
 * Q4Linear.upload (linear_q4.zig:28-63), Drafter.upload (mtp.zig:86-116) and
 * upload.tensorPrivate (upload.zig:6-21). */
int prg_model_load(const PrgModelConfig *cfg, const char *target_dir, const char *mtp_dir, PrgModel **out);

/* Per-sequence state for up to max_seq tokens: GDN conv f32 [3, 8192] and
 * recurrent f32 [32, 128, 128] per linear layer, bf16 K [4, stride, 256] and
 * V [4, 256, stride] per full-attention layer (stride = max_seq aligned to 256,
 * or 64 when max_seq >= 16000, state.zig:25-32), plus the decode workspace.
 * Replaces ModelState.initBf16FullCaches (state.zig:52-90). */
int prg_model_state_create(PrgModel *model, uint32_t max_seq, PrgModelState **out);
void prg_model_state_destroy(PrgModelState *state);
/* Zero the GDN states (ModelState.resetForNewSequence, state.zig:110-118). */
int prg_model_state_reset(PrgModelState *state);
/* Device pointer of a state tensor: "layers.<i>.conv", "layers.<i>.recur",
 * "layers.<i>.cache_k", "layers.<i>.cache_v", the drafter's "mtp.cache_k" /
 * "mtp.cache_v" (once a drafter call has run); or of a workspace buffer. */
int prg_model_state_tensor(const PrgModelState *state, const char *name, void **ptr, size_t *bytes);
uint32_t prg_model_state_stride(const PrgModelState *state);

/* One token through the whole stack and the greedy argmax tail, synchronous.
 * cache_pos: KV slot written; rope_pos: RoPE position (GDN state is used iff
 * rope_pos != 0); seq_len: tokens attended (must be cache_pos + 1; for a
 * cached prefix see prg_model_forward_next_token_prefixed). Afterwards
 * prg_model_decode continues at cache_pos + 1 with *next_token as its input;
 * its positions keep this call's offset rope_pos - cache_pos. Errors:
 * SEQUENCE_TOO_LONG, INVALID_TOKEN.
 * Replaces DeviceModel.forwardNextTokenBf16WithPrefix (model.zig:1564-1578)
 * with prefix == null. */
int prg_model_forward_next_token(PrgModel *model, PrgModelState *state, uint32_t token,
                                 uint32_t cache_pos, uint32_t rope_pos, uint32_t seq_len,
                                 uint32_t *next_token);

/* The same step with the reference's prefix bookkeeping
 * (decode_loop.zig:96-160): cache_pos = logical_pos - prefix_len is the
 * slot after the prefix, rope_pos = logical_pos, seq_len = logical_pos + 1
 * (must equal prefix_len + cache_pos + 1). The reference binds the prefix
 * entry's K/V as a second attention source; here the state must already hold
 * the prefix's tokens in its slots [0, prefix_len) (prg_prefix_cache_restore,
 * then prg_model_prefill_from for the rest of the prompt), and the step writes
 * slot prefix_len + cache_pos. Errors: SEQUENCE_TOO_LONG, INVALID_TOKEN,
 * INVALID_ARG (seq_len mismatch).
 * Replaces DeviceModel.forwardNextTokenBf16WithPrefix (model.zig:1564-1578)
 * with prefix = {entry state, prefix_len}. */
int prg_model_forward_next_token_prefixed(PrgModel *model, PrgModelState *state, uint32_t token,
                                          uint32_t cache_pos, uint32_t rope_pos, uint32_t seq_len,
                                          uint32_t prefix_len, uint32_t *next_token);

/* Reset the state and ingest prompt[0..prompt_len) at positions 0.. layer-major
 * in chunks of up to 2048 tokens (MFMA QMMs, causal prefill attention, GDN
 * prefill recurrence); the lm_head runs only on the last prompt token.
 * *next_token receives the greedy token that follows the prompt; the state is
 * then positioned to decode it (prg_model_decode continues from there).
 * Replaces DeviceModel's layer-major prefill + argmax tail
 * (model.zig:940-1060, 1307-1324; DecoderLayer.prefillStepBf16,
 * decoder_layer.zig:644-760). */
int prg_model_prefill(PrgModel *model, PrgModelState *state, const uint32_t *prompt,
                      uint32_t prompt_len, uint32_t *next_token);

/* Continue the greedy loop for n_steps tokens from the current state (after
 * prg_model_prefill, prg_model_generate, prg_model_forward_next_token,
 * prg_model_forward_two_tokens or an earlier prg_model_decode),
 * device-resident (graph replay, no host sync between tokens). tokens_out (host,
 * n_steps) receives the greedy token produced by each step; gpu_ms (optional)
 * the GPU time of the n_steps steps from HIP events on the decode stream.
 * Replaces decode_loop.decodeFromPrefixCache (decode_loop.zig:96-160). */
int prg_model_decode(PrgModel *model, PrgModelState *state, uint32_t n_steps, uint32_t *tokens_out,
                     float *gpu_ms);

/* Measurement entry point, no counterpart in the reference: one decode token's
 * GEMV launches only (the model's weights, fused norms and epilogues; no
 * embedding, GDN recurrence, attention or argmax) captured as a graph and
 * replayed `replays` times; *us_per_token receives the average GPU time of one
 * replay. For the token-loop GEMV bandwidth of the benchmark. The state's
 * activations and conv states are undefined afterwards until the next
 * prg_model_prefill. */
int prg_model_time_token_gemvs(PrgModel *model, PrgModelState *state, uint32_t replays,
                               float *us_per_token);

/* Greedy generation from an empty state, the whole loop device-resident (one
 * captured HIP graph per token, no host sync between tokens). Step n consumes
 * the token at position n.
 *   teacher_force == 0: steps n = 0 .. prompt_len + n_new - 2. The inputs are
 *     prompt[n] while n < prompt_len, then the previous step's greedy token.
 *     Steps before prompt_len - 1 skip the lm_head (prompt ingestion).
 *     predictions (host, prompt_len - 1 + n_new entries) receives the greedy
 *     token after position n for every step that ran the lm_head (others are
 *     0xFFFFFFFF); the generated tokens are predictions[prompt_len - 1 ..].
 *   teacher_force != 0: n_new must be 0; steps n = 0 .. prompt_len - 1 all take
 *     prompt[n] as input and all run the lm_head (predictions: prompt_len).
 * decode_ms (optional): GPU time of the steps that ran the lm_head after the
 * prompt (the n_new generation steps), from HIP events on the decode stream.
 * Replaces decode_loop.decodeFromPrefixCache (decode_loop.zig:96-160) for an
 * empty prefix. */
int prg_model_generate(PrgModel *model, PrgModelState *state, const uint32_t *prompt,
                       uint32_t prompt_len, uint32_t n_new, int teacher_force,
                       uint32_t *predictions, float *decode_ms);

/* ======================================================================
 * Multi-token prediction (needs cfg.mtp_layers == 1).
 * ====================================================================== */

/* Two tokens through the target at cache slots cache_pos, cache_pos + 1
 * (rope_pos, rope_pos + 1; seq_len must be cache_pos + 1): the state advances
 * by both. verify_token = argmax after token0, bonus_token = argmax after
 * token1; hidden_out (device bf16 [2, hidden], may be NULL) receives the two
 * final-normed hidden rows. Afterwards prg_model_decode continues at
 * cache_pos + 2 (RoPE position rope_pos + 2, keeping the offset) with
 * bonus_token as its input. Errors: SEQUENCE_TOO_LONG, INVALID_TOKEN.
 * Replaces DeviceModel.forwardTwoTokenDecodeVerifierBf16WithPrefixProfiled
 * (model.zig:1627-1659; encodeStack2Bf16 :719-760, decodeStep2Bf16
 * decoder_layer.zig:485-516). */
int prg_model_forward_two_tokens(PrgModel *model, PrgModelState *state, uint32_t token0, uint32_t token1,
                                 uint32_t cache_pos, uint32_t rope_pos, uint32_t seq_len,
                                 uint32_t *verify_token, uint32_t *bonus_token, uint16_t *hidden_out);

/* One drafter step: norm(embed(token)) ‖ norm(hidden) -> fc -> the drafter's
 * decoder layer at its own cache slot cache_pos -> norm -> lm_head argmax.
 * hidden: device bf16 [hidden], the target's final-normed hidden of the
 * previous position. Replaces Drafter.forwardDraftTokenProfiled
 * (src/model/mtp.zig:187-242). */
int prg_model_mtp_draft(PrgModel *model, PrgModelState *state, uint32_t token, const uint16_t *hidden,
                        uint32_t cache_pos, uint32_t rope_pos, uint32_t seq_len, uint32_t *draft_token);

/* Drafter prefill of token_count rows (tokens: host u32; hidden_rows: device
 * bf16 [token_count, hidden]) at drafter slots start_pos.. . Replaces
 * Drafter.forwardPrefill (src/model/mtp.zig:137-185). */
int prg_model_mtp_prefill(PrgModel *model, PrgModelState *state, const uint32_t *tokens, uint32_t token_count,
                          const uint16_t *hidden_rows, uint32_t start_pos);

/* Greedy generation with MTP speculation: reset, prefill the prompt (seeding
 * the drafter), then draft / verify / accept-or-reject until n_new tokens are
 * emitted into tokens_out (the first is the token after the prompt). The
 * tokens equal prg_model_prefill + prg_model_decode's greedy tokens.
 * accepted / attempted: drafts accepted / verified (may be NULL). decode_ms:
 * GPU time of the loop (may be NULL). The whole step runs as one replayed HIP
 * graph with positions in device memory. Requires prompt_len + n_new + 2 <=
 * max_seq. Replaces decodeSpeculativeFromPrefixCache
 * (src/server/decode_loop.zig:163-293) without its per-token host sync and
 * without the reject-path recompute. */
int prg_model_generate_speculative(PrgModel *model, PrgModelState *state, const uint32_t *prompt,
                                   uint32_t prompt_len, uint32_t n_new, uint32_t *tokens_out,
                                   uint32_t *accepted, uint32_t *attempted, float *decode_ms);

/* The same loop continuing from a prefix-cache hit: the state already holds
 * prompt[0, prefix_len) (prg_prefix_cache_restore), and prefix_hidden (device
 * bf16 [prefix_len, hidden], e.g. prg_prefix_cache_entry_hidden) holds the
 * final-normed hidden rows of those positions. The drafter is seeded from
 * them (row t with prompt[t + 1]), prompt[prefix_len, prompt_len) is
 * prefilled (seeding the drafter from the new rows), and the draft / verify
 * loop runs as above; the tokens equal the greedy continuation of the whole
 * prompt. hidden_out (device bf16 [prompt_len, hidden], may be NULL) receives
 * the prompt's hidden rows (the prefix rows copied, the rest computed), ready
 * for prg_prefix_cache_store. prefix_len = 0 (prefix_hidden unused) is
 * prg_model_generate_speculative with the hidden rows captured. Replaces
 * decodeSpeculativeFromPrefixCache with prefix_len > 0
 * (src/server/decode_loop.zig:163-293) and seedMtpDrafter
 * (src/server.zig:1240-1330). */
int prg_model_generate_speculative_from(PrgModel *model, PrgModelState *state, const uint32_t *prompt,
                                        uint32_t prompt_len, uint32_t prefix_len, const uint16_t *prefix_hidden,
                                        uint16_t *hidden_out, uint32_t n_new, uint32_t *tokens_out,
                                        uint32_t *accepted, uint32_t *attempted, float *decode_ms);

#ifdef __cplusplus
}
#endif

#endif
