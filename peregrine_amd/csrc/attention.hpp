// GQA decode attention for the Qwen3.5 full-attention layers — declarations.
#pragma once

#include "common.hpp"

namespace prg {

// reference src/model/block_attn.zig:21-28, shaders/attention.metal:43-48
constexpr uint32_t kAttnQHeads = 16;
constexpr uint32_t kAttnKvHeads = 4;
constexpr uint32_t kAttnGroup = kAttnQHeads / kAttnKvHeads;  // 4
constexpr uint32_t kAttnHeadDim = 256;
constexpr uint32_t kAttnRotary = 64;
constexpr float kAttnTheta = 1.0e7f;
constexpr float kAttnEps = 1.0e-6f;
constexpr float kAttnScale = 1.0f / 16.0f;
constexpr uint32_t kAttnPartialStride = kAttnHeadDim + 2;  // [m, denom, acc[256]]

// Look up the device address of the allocation-free decode attention's
// partials on the current device (once per device; later calls are free).
int attn_noalloc_setup();

// Split-context count for a cache of `capacity` tokens: every kv head is split
// into this many contiguous token ranges (one block each), fixed per cache so a
// captured graph stays valid as seq_len grows.
uint32_t attn_num_splits(uint32_t capacity);
// Largest per-split token range (rounded to 64) for a cache of `capacity`.
uint32_t attn_split_tokens(uint32_t capacity, uint32_t nsplit);

struct AttnPrepareArgs {
  const uint16_t* packed_q;  // [16, 512] = q(256) | gate(256) per head
  const uint16_t* q_norm;    // [256]
  const uint16_t* k_in;      // [4, 256]
  const uint16_t* v_in;      // [4, 256]
  const uint16_t* k_norm;    // [256]
  uint16_t* q_out;           // [16, 256]
  uint16_t* gate_out;        // [16, 256]
  uint16_t* key_cache;       // [4, stride, 256]
  uint16_t* value_cache;     // [4, 256, stride]
  uint32_t stride;           // cache capacity in tokens
  uint32_t cache_pos_host;   // used when step == nullptr
  uint32_t rope_pos_host;
  const StepScalars* step;   // device scalars (graph replay) or nullptr
  // Consecutive tokens handled by one launch (1 or 2; 2 needs step). Token r
  // reads and writes the row-r slices (packed_q + r*8192, k_in / v_in +
  // r*1024, q_out / gate_out + r*4096) and uses step[r].
  uint32_t rows = 1;
};

int launch_attn_prepare(hipStream_t s, const AttnPrepareArgs& a);

struct AttnDecodeArgs {
  const uint16_t* q;          // [16, 256] prepared queries
  const uint16_t* key_cache;  // [4, stride, 256]
  const uint16_t* value_cache;  // [4, 256, stride]
  const uint16_t* gate;       // [16, 256]
  uint16_t* out;              // [16, 256]
  float* partials;            // [16, nsplit, 258]
  uint32_t stride;
  uint32_t nsplit;
  uint32_t split_tokens;      // LDS sizing bound (>= ceil(seq_len/nsplit) rounded to 32)
  uint32_t seq_len_host;      // used when step == nullptr
  const StepScalars* step;
  float scale;
  // Consecutive tokens handled by one launch (1 or 2; 2 needs step). Query r
  // uses q / gate / out + r*4096, partials + r*16*nsplit*258 and step[r].
  uint32_t rows = 1;
  // Decode-step form (packed_q != nullptr): the inputs are the raw q | gate,
  // k and v projections of the `rows` new tokens, not yet in the cache. Row r
  // covers its cached tokens [0, step[r].seq_len - 1), split exactly as a
  // one-token step at its position splits them, and normalises + rotates q
  // itself; the split holding row r's last cached token (split 0 on an empty
  // cache) also prepares the new tokens' k / v, attends to row r's own new
  // token as an extra token, and appends it at step[r].cache_pos. Row 1's last
  // cached token is row 0's new token: its k / v come from that preparation,
  // not from the cache slot row 0's block is writing. The merge takes the
  // gate from packed_q. Without packed_q, q and gate are prepared and the
  // cache already holds all seq_len tokens.
  const uint16_t* packed_q = nullptr;  // [rows][16][512]
  const uint16_t* q_norm = nullptr;    // [256]
  const uint16_t* k_in = nullptr;      // [rows][4][256]
  const uint16_t* v_in = nullptr;      // [rows][4][256]
  const uint16_t* k_norm = nullptr;    // [256]
  uint16_t* key_cache_w = nullptr;     // writable views of the caches for the append
  uint16_t* value_cache_w = nullptr;
  uint32_t cache_pos_host = 0;         // row 0's slot and RoPE position when step == nullptr
  uint32_t rope_pos_host = 0;
};

int launch_attn_decode(hipStream_t s, const AttnDecodeArgs& a);

}  // namespace prg
