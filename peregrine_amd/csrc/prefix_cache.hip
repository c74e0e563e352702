// Prompt-prefix state cache and its PRGPFXS1 v3 persistence file (host code;
// the device work is copies between ModelStates).
//
// Reference:
//   PrefixIndex, Entry, Cache   src/server/prefix_state_cache.zig:21-795
//   save / load / fingerprint   src/server/prefix_persist.zig:31-412
//
// Entries own a PrgModelState sized to their tokens (at least the prefill
// chunk), keyed in a token trie; the reserved-token budget evicts the least
// recently used unpinned entry. A working state reuses a cached prefix by
// copying it in (prg_prefix_cache_restore), so positions stay absolute (see
// model_prefix.hip). Created without a model, the cache keeps tokens and
// accounting only (no device state), which is all the index needs.
#include <dirent.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <string>
#include <vector>

#include "model.hpp"

namespace prg {

// ------------------------------------------------------------- wyhash -------
// Wyhash ("final v4" round structure with the original 64-bit secret), the
// hash behind std.hash.Wyhash that prefix_persist.zig:149-190 streams the
// checkpoint through. Streaming: 48-byte blocks are mixed only once a later
// byte is known to follow, and the final 16 bytes of the whole stream are
// kept, which makes update() over any split equal to the one-shot hash.
class Wyhash {
 public:
  explicit Wyhash(uint64_t seed) {
    s0_ = seed ^ mix(seed ^ kSecret[0], kSecret[1]);
    s1_ = s2_ = s0_;
  }

  void update(const void* data, size_t n) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    total_ += n;
    keep_tail(p, n);
    while (n > 0) {
      if (len_ == 48) {  // more input follows: the block is not the last
        round(buf_);
        len_ = 0;
      }
      const size_t take = std::min<size_t>(48 - len_, n);
      memcpy(buf_ + len_, p, take);
      len_ += take;
      p += take;
      n -= take;
    }
  }

  uint64_t final() const {
    uint64_t a, b, seed = s0_;
    if (total_ <= 16) {
      const uint8_t* p = buf_;
      const size_t len = static_cast<size_t>(total_);
      if (len >= 4) {
        a = (r4(p) << 32) | r4(p + ((len >> 3) << 2));
        b = (r4(p + len - 4) << 32) | r4(p + len - 4 - ((len >> 3) << 2));
      } else if (len > 0) {
        a = (static_cast<uint64_t>(p[0]) << 16) | (static_cast<uint64_t>(p[len >> 1]) << 8) | p[len - 1];
        b = 0;
      } else {
        a = b = 0;
      }
    } else {
      seed ^= s1_ ^ s2_;
      const uint8_t* p = buf_;
      size_t i = len_;
      while (i > 16) {
        seed = mix(r8(p) ^ kSecret[1], r8(p + 8) ^ seed);
        i -= 16;
        p += 16;
      }
      a = r8(tail_);
      b = r8(tail_ + 8);
    }
    a ^= kSecret[1];
    b ^= seed;
    mum(&a, &b);
    return mix(a ^ kSecret[0] ^ total_, b ^ kSecret[1]);
  }

 private:
  static constexpr uint64_t kSecret[4] = {0xa0761d6478bd642full, 0xe7037ed1a0b428dbull, 0x8ebc6af09c88c6e3ull,
                                          0x589965cc75374cc3ull};
  uint64_t s0_, s1_, s2_;
  uint64_t total_ = 0;
  uint8_t buf_[48];
  size_t len_ = 0;
  uint8_t tail_[16] = {0};  // last 16 bytes of the stream

  static void mum(uint64_t* a, uint64_t* b) {
    const __uint128_t r = static_cast<__uint128_t>(*a) * *b;
    *a = static_cast<uint64_t>(r);
    *b = static_cast<uint64_t>(r >> 64);
  }
  static uint64_t mix(uint64_t a, uint64_t b) {
    mum(&a, &b);
    return a ^ b;
  }
  static uint64_t r8(const uint8_t* p) {
    uint64_t v;
    memcpy(&v, p, 8);
    return v;
  }
  static uint64_t r4(const uint8_t* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
  }
  void round(const uint8_t* p) {
    s0_ = mix(r8(p) ^ kSecret[1], r8(p + 8) ^ s0_);
    s1_ = mix(r8(p + 16) ^ kSecret[2], r8(p + 24) ^ s1_);
    s2_ = mix(r8(p + 32) ^ kSecret[3], r8(p + 40) ^ s2_);
  }
  void keep_tail(const uint8_t* p, size_t n) {
    if (n >= 16) {
      memcpy(tail_, p + n - 16, 16);
    } else {
      memmove(tail_, tail_ + n, 16 - n);
      memcpy(tail_ + 16 - n, p, n);
    }
  }
};
constexpr uint64_t Wyhash::kSecret[4];

// ------------------------------------------------------------ the index -----
// Token trie: node 0 is the root; an entry is registered at the node of its
// full token sequence (prefix_state_cache.zig:21-210).
class PrefixIndex {
 public:
  void clear() {
    nodes_.clear();
    free_.clear();
  }

  void insert(const uint32_t* t, size_t n, int entry) {
    if (n == 0) return;
    if (nodes_.empty()) nodes_.push_back(root());
    int node = 0;
    for (size_t i = 0; i < n; ++i) {
      int c = child(node, t[i]);
      if (c < 0) {
        c = alloc(node, t[i]);
        nodes_[node].children.push_back({t[i], c});
      }
      node = c;
    }
    nodes_[node].entry = entry;
  }

  void remove(const uint32_t* t, size_t n) {
    const int node = find_node(t, n);
    if (node < 0) return;
    nodes_[node].entry = -1;
    prune(node);
  }

  // Longest registered prefix of p: entry index and length, or false.
  bool find_longest(const uint32_t* p, size_t n, int* entry, size_t* len) const {
    if (nodes_.empty()) return false;
    int node = 0;
    bool found = false;
    for (size_t i = 0; i < n; ++i) {
      node = child(node, p[i]);
      if (node < 0) break;
      if (nodes_[node].entry >= 0) {
        *entry = nodes_[node].entry;
        *len = i + 1;
        found = true;
      }
    }
    return found;
  }

  int find_exact(const uint32_t* t, size_t n) const {
    const int node = find_node(t, n);
    return node < 0 ? -1 : nodes_[node].entry;
  }

  bool contains_prefix(const uint32_t* p, size_t n, size_t prefix_len) const {
    if (prefix_len == 0) return true;
    if (prefix_len > n || nodes_.empty()) return false;
    const int node = find_node(p, prefix_len);
    return node >= 0 && nodes_[node].entry >= 0;
  }

  // Entry `removed` left the entry list: later indexes shift down by one.
  void decrement_after(int removed) {
    for (Node& nd : nodes_) {
      if (!nd.alive || nd.entry < 0) continue;
      if (nd.entry == removed)
        nd.entry = -1;
      else if (nd.entry > removed)
        nd.entry -= 1;
    }
  }

 private:
  struct Node {
    int parent = -1;
    uint32_t parent_token = 0;
    std::vector<std::pair<uint32_t, int>> children;
    int entry = -1;
    bool alive = false;
  };
  std::vector<Node> nodes_;
  std::vector<int> free_;

  static Node root() {
    Node r;
    r.alive = true;
    return r;
  }
  int alloc(int parent, uint32_t token) {
    Node nd;
    nd.parent = parent;
    nd.parent_token = token;
    nd.alive = true;
    if (!free_.empty()) {
      const int i = free_.back();
      free_.pop_back();
      nodes_[i] = std::move(nd);
      return i;
    }
    nodes_.push_back(std::move(nd));
    return static_cast<int>(nodes_.size()) - 1;
  }
  int child(int node, uint32_t token) const {
    const Node& nd = nodes_[node];
    if (!nd.alive) return -1;
    for (const auto& c : nd.children)
      if (c.first == token) return c.second;
    return -1;
  }
  int find_node(const uint32_t* t, size_t n) const {
    if (nodes_.empty()) return -1;
    int node = 0;
    for (size_t i = 0; i < n && node >= 0; ++i) node = child(node, t[i]);
    return node;
  }
  // Drop childless nodes without an entry, walking up towards the root.
  void prune(int node) {
    while (node != 0) {
      Node& nd = nodes_[node];
      if (nd.entry >= 0 || !nd.children.empty()) return;
      const int parent = nd.parent;
      auto& sib = nodes_[parent].children;
      for (size_t k = 0; k < sib.size(); ++k) {
        if (sib[k].first == nd.parent_token && sib[k].second == node) {
          sib.erase(sib.begin() + static_cast<long>(k));
          break;
        }
      }
      nd = Node{};
      free_.push_back(node);
      node = parent;
    }
  }
};

struct PrefixEntry {
  PrgModelState* state = nullptr;  // nullptr without a model
  uint32_t capacity = 0;           // token capacity of `state` (the reserved tokens)
  uint16_t* hidden = nullptr;      // device bf16 [hidden_rows, hidden] when tracking
  uint32_t hidden_rows = 0;
  bool hidden_valid = false;
  uint32_t next_token = 0;
  bool next_valid = false;
  std::vector<uint32_t> tokens;
  bool pinned = false;
  uint64_t last_access = 0;
  uint64_t hits = 0;
};

}  // namespace prg

struct PrgPrefixCache {
  PrgModel* model = nullptr;
  std::vector<prg::PrefixEntry> entries;
  prg::PrefixIndex index;
  uint64_t max_tokens = 0, initial_state_tokens = 0;
  uint64_t resident_tokens = 0, reserved_tokens = 0;
  int active = -1;
  uint64_t clock = 0;
  uint64_t hits = 0, misses = 0, hit_tokens = 0, computed_tokens = 0, evictions = 0;
  bool track_hidden = false;
  hipStream_t stream = nullptr;  // hidden-row copies
};

namespace prg {
namespace {

using Cache = PrgPrefixCache;

size_t hidden_row_bytes(const Cache* c) { return sizeof(uint16_t) * c->model->cfg.hidden; }

void free_entry(PrefixEntry& e) {
  if (e.state) prg_model_state_destroy(e.state);
  if (e.hidden) hipFree(e.hidden);
  e.state = nullptr;
  e.hidden = nullptr;
}

int new_entry(Cache* c, uint32_t capacity, bool pinned, PrefixEntry* out) {
  PrefixEntry e;
  e.capacity = capacity;
  e.pinned = pinned;
  if (c->model) {
    if (int rc = prg_model_state_create(c->model, capacity, &e.state)) return rc;
  }
  *out = std::move(e);
  return PRG_OK;
}

uint64_t next_access(Cache* c) { return ++c->clock; }

void clear_all(Cache* c) {
  for (PrefixEntry& e : c->entries) free_entry(e);
  c->entries.clear();
  c->index.clear();
  c->resident_tokens = c->reserved_tokens = 0;
  c->active = -1;
}

void remove_entry(Cache* c, size_t i) {
  if (i >= c->entries.size()) return;
  PrefixEntry& e = c->entries[i];
  c->index.remove(e.tokens.data(), e.tokens.size());
  c->resident_tokens -= std::min<uint64_t>(c->resident_tokens, e.tokens.size());
  c->reserved_tokens -= std::min<uint64_t>(c->reserved_tokens, e.capacity);
  free_entry(e);
  c->entries.erase(c->entries.begin() + static_cast<long>(i));
  c->index.decrement_after(static_cast<int>(i));
  if (c->active == static_cast<int>(i))
    c->active = -1;
  else if (c->active > static_cast<int>(i))
    c->active -= 1;
}

void touch(Cache* c, size_t i) {
  if (i >= c->entries.size()) return;
  c->entries[i].last_access = next_access(c);
  c->entries[i].hits += 1;
  c->active = static_cast<int>(i);
}

int evictable(const Cache* c, int preserve) {
  int victim = -1;
  for (size_t i = 0; i < c->entries.size(); ++i) {
    if (static_cast<int>(i) == preserve || c->entries[i].pinned) continue;
    if (victim < 0 || c->entries[i].last_access < c->entries[victim].last_access) victim = static_cast<int>(i);
  }
  return victim;
}

// ensureReservedTokenBudget (prefix_state_cache.zig:760-774).
int ensure_budget(Cache* c, int* preserve, uint64_t additional) {
  if (additional > c->max_tokens)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix cache: %llu tokens exceed the budget %llu",
                     (unsigned long long)additional, (unsigned long long)c->max_tokens);
  while (c->reserved_tokens + additional > c->max_tokens) {
    const int victim = evictable(c, *preserve);
    if (victim < 0)
      return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix cache: budget %llu exhausted by pinned entries",
                       (unsigned long long)c->max_tokens);
    remove_entry(c, static_cast<size_t>(victim));
    if (*preserve >= 0 && victim < *preserve) *preserve -= 1;
    c->evictions += 1;
  }
  return PRG_OK;
}

// Entry.ensureStateCapacity (prefix_state_cache.zig:246-258).
int ensure_state_capacity(Cache* c, PrefixEntry& e, uint32_t n) {
  if (n == 0 || n <= e.capacity) return PRG_OK;
  PrefixEntry grown;
  if (int rc = new_entry(c, n, e.pinned, &grown)) return rc;
  if (e.state && !e.tokens.empty()) {
    const uint32_t keep = static_cast<uint32_t>(e.tokens.size());
    int rc = copy_attention_range(grown.state, 0, e.state, 0, keep);
    if (rc == PRG_OK) rc = copy_linear_state(grown.state, e.state);
    if (rc) {
      free_entry(grown);
      return rc;
    }
  }
  if (e.state) prg_model_state_destroy(e.state);
  e.state = grown.state;
  e.capacity = n;
  return PRG_OK;
}

// Entry.ensureHiddenCapacity (prefix_state_cache.zig:262-290): the old rows
// are kept, new rows are zero.
int ensure_hidden_capacity(Cache* c, PrefixEntry& e, uint32_t n) {
  const uint32_t rows = std::max(n, e.capacity);
  if (e.hidden && e.hidden_rows >= rows) return PRG_OK;
  const size_t rb = hidden_row_bytes(c);
  uint16_t* buf = nullptr;
  PRG_HIP(hipMalloc(reinterpret_cast<void**>(&buf), rb * rows));
  hipError_t err = hipMemsetAsync(buf, 0, rb * rows, c->stream);
  if (err == hipSuccess && e.hidden) {
    const size_t keep = std::min<size_t>(e.tokens.size(), e.hidden_rows);
    if (keep) err = hipMemcpyAsync(buf, e.hidden, rb * keep, hipMemcpyDeviceToDevice, c->stream);
  }
  if (err == hipSuccess) err = hipStreamSynchronize(c->stream);
  if (err != hipSuccess) {
    hipFree(buf);
    return set_error(PRG_ERR_HIP, "prefix cache hidden rows: %s", hipGetErrorString(err));
  }
  if (e.hidden) hipFree(e.hidden);
  e.hidden = buf;
  e.hidden_rows = rows;
  return PRG_OK;
}

// replaceEntryPrefix (prefix_state_cache.zig:736-756).
int replace_entry_prefix(Cache* c, int* preserve, const uint32_t* ids, uint32_t n, bool pinned) {
  PrefixEntry* e = &c->entries[*preserve];
  const uint64_t old_len = e->tokens.size(), old_capacity = e->capacity;
  if (n > old_capacity)
    if (int rc = ensure_budget(c, preserve, n - old_capacity)) return rc;
  e = &c->entries[*preserve];
  if (int rc = ensure_state_capacity(c, *e, n)) return rc;
  c->reserved_tokens = c->reserved_tokens - old_capacity + e->capacity;
  e->tokens.assign(ids, ids + n);
  e->pinned = e->pinned || pinned;
  c->resident_tokens = c->resident_tokens - old_len + n;
  return PRG_OK;
}

// prepareEntry (prefix_state_cache.zig:693-734): the exact entry, the reused
// entry re-keyed to the longer prefix, or a new entry within the budget.
int prepare_entry(Cache* c, const uint32_t* ids, uint32_t n, int reuse, bool pinned, int* out) {
  if (n == 0 || n > c->max_tokens)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix cache: prefix of %u tokens (budget %llu)", n,
                     (unsigned long long)c->max_tokens);
  const int exact = c->index.find_exact(ids, n);
  if (exact >= 0) {
    int keep = exact;
    if (int rc = replace_entry_prefix(c, &keep, ids, n, pinned)) return rc;
    *out = keep;
    return PRG_OK;
  }
  if (reuse >= 0) {
    int keep = reuse;
    const std::vector<uint32_t> old_tokens = c->entries[keep].tokens;
    c->index.insert(ids, n, keep);
    if (int rc = replace_entry_prefix(c, &keep, ids, n, pinned)) {
      c->index.remove(ids, n);
      return rc;
    }
    c->index.remove(old_tokens.data(), old_tokens.size());
    *out = keep;
    return PRG_OK;
  }
  int none = -1;
  const uint32_t capacity = static_cast<uint32_t>(std::max<uint64_t>(n, c->initial_state_tokens));
  if (int rc = ensure_budget(c, &none, capacity)) return rc;
  PrefixEntry e;
  if (int rc = new_entry(c, capacity, pinned, &e)) return rc;
  e.tokens.assign(ids, ids + n);
  e.last_access = next_access(c);
  c->entries.push_back(std::move(e));
  const int idx = static_cast<int>(c->entries.size()) - 1;
  c->index.insert(ids, n, idx);
  c->resident_tokens += n;
  c->reserved_tokens += capacity;
  *out = idx;
  return PRG_OK;
}

int check_match(const Cache* c, const PrgPrefixMatch& m) {
  PRG_CHECK_ARG(m.index < c->entries.size(), "prefix cache: match index %u of %zu entries", m.index,
                c->entries.size());
  return PRG_OK;
}

// ------------------------------------------------------- persistence --------
constexpr uint64_t kMagic = 0x3153584650475250ull;  // "PRGPFXS1" little-endian
constexpr uint32_t kVersion = 3;
constexpr uint32_t kDtypeBf16 = 0;

// Fixed little-endian header; 44 bytes of fields padded to 48 (8-byte
// alignment), as the reference's extern struct (prefix_persist.zig:44-56).
struct FileHeader {
  uint64_t magic;
  uint32_t version;
  uint32_t dtype;
  uint64_t model_fingerprint;
  uint64_t token_count;
  uint32_t next_token;
  uint32_t next_token_valid;
  uint32_t hidden_valid;
  uint32_t pad;
};
static_assert(sizeof(FileHeader) == 48, "PRGPFXS1 header is 48 bytes");

constexpr uint64_t kConvBytes = sizeof(float) * (kGdnConvK - 1) * kGdnConvDim;
constexpr uint64_t kRecurBytes = sizeof(float) * kGdnHv * kGdnDv * kGdnDk;

// expectedFileBytes (prefix_persist.zig:71-80) for any layer topology.
uint64_t expected_file_bytes(const PrgModelConfig& cfg, uint64_t T) {
  uint64_t linear = 0, full = 0;
  for (uint32_t i = 0; i < cfg.num_layers; ++i) (is_linear_layer(cfg, i) ? linear : full) += 1;
  const uint64_t kv = kAttnKvHeads * T * kAttnHeadDim * sizeof(uint16_t);
  return sizeof(FileHeader) + T * sizeof(uint32_t) + linear * (kConvBytes + kRecurBytes) + full * 2 * kv +
         T * cfg.hidden * sizeof(uint16_t);
}

class File {
 public:
  ~File() {
    if (fd_ >= 0) close(fd_);
  }
  int open_read(const std::string& path, bool* missing) {
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    *missing = fd_ < 0 && errno == ENOENT;
    if (fd_ < 0 && !*missing) return set_error(PRG_ERR_IO, "open %s: %s", path.c_str(), strerror(errno));
    return PRG_OK;
  }
  int open_write(const std::string& path) {
    fd_ = ::open(path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (fd_ < 0) return set_error(PRG_ERR_IO, "create %s: %s", path.c_str(), strerror(errno));
    return PRG_OK;
  }
  uint64_t size() const {
    struct stat sb;
    return fstat(fd_, &sb) == 0 ? static_cast<uint64_t>(sb.st_size) : 0;
  }
  int read_all(void* dst, size_t n) {
    char* p = static_cast<char*>(dst);
    while (n) {
      const ssize_t r = ::read(fd_, p, n);
      if (r < 0 && errno == EINTR) continue;
      if (r <= 0) return set_error(PRG_ERR_IO, "EndOfStream: persisted prefix file ends early");
      p += r;
      n -= static_cast<size_t>(r);
    }
    return PRG_OK;
  }
  int write_all(const void* src, size_t n) {
    const char* p = static_cast<const char*>(src);
    while (n) {
      const ssize_t w = ::write(fd_, p, n);
      if (w < 0 && errno == EINTR) continue;
      if (w <= 0) return set_error(PRG_ERR_IO, "write failed: %s", strerror(errno));
      p += w;
      n -= static_cast<size_t>(w);
    }
    return PRG_OK;
  }
  int sync_close() {
    const int rc = fsync(fd_);
    const int cl = close(fd_);
    fd_ = -1;
    if (rc != 0 || cl != 0) return set_error(PRG_ERR_IO, "fsync/close failed: %s", strerror(errno));
    return PRG_OK;
  }

 private:
  int fd_ = -1;
};

int make_parent_dirs(const std::string& path) {
  for (size_t pos = path.find('/', 1); pos != std::string::npos; pos = path.find('/', pos + 1)) {
    const std::string dir = path.substr(0, pos);
    if (mkdir(dir.c_str(), 0755) != 0 && errno != EEXIST)
      return set_error(PRG_ERR_IO, "mkdir %s: %s", dir.c_str(), strerror(errno));
  }
  return PRG_OK;
}

// The entry a save persists: the active one, else the most recently used
// non-empty one (persistedEntryConst, prefix_state_cache.zig:380-391).
const PrefixEntry* persisted_entry(const Cache* c) {
  if (c->active >= 0 && c->active < static_cast<int>(c->entries.size())) return &c->entries[c->active];
  const PrefixEntry* best = nullptr;
  for (const PrefixEntry& e : c->entries)
    if (!e.tokens.empty() && (!best || e.last_access > best->last_access)) best = &e;
  return best;
}

// State sections of the file for T tokens: per layer in order, conv and
// recurrent f32 (linear) or the K rows [4][T][256] then the V runs [4][256][T]
// (full attention; FullCacheRunIterator, prefix_persist.zig:90-143).
int write_state(File& f, const PrgModelState* st, uint32_t T, std::vector<uint8_t>& host) {
  const size_t kv = static_cast<size_t>(kAttnKvHeads) * T * kAttnHeadDim * sizeof(uint16_t);
  for (const LayerState& l : st->layers) {
    if (l.conv) {
      host.resize(kConvBytes + kRecurBytes);
      PRG_HIP(hipMemcpy(host.data(), l.conv, kConvBytes, hipMemcpyDeviceToHost));
      PRG_HIP(hipMemcpy(host.data() + kConvBytes, l.recur, kRecurBytes, hipMemcpyDeviceToHost));
      if (int rc = f.write_all(host.data(), host.size())) return rc;
    } else if (l.cache_k) {
      host.resize(2 * kv);
      const size_t row = sizeof(uint16_t) * kAttnHeadDim;
      PRG_HIP(hipMemcpy2D(host.data(), T * row, l.cache_k, st->stride * row, T * row, kAttnKvHeads,
                          hipMemcpyDeviceToHost));
      PRG_HIP(hipMemcpy2D(host.data() + kv, T * sizeof(uint16_t), l.cache_v, st->stride * sizeof(uint16_t),
                          T * sizeof(uint16_t), kAttnKvHeads * kAttnHeadDim, hipMemcpyDeviceToHost));
      if (int rc = f.write_all(host.data(), host.size())) return rc;
    }
  }
  return PRG_OK;
}

int read_state(File& f, PrgModelState* st, uint32_t T, std::vector<uint8_t>& host) {
  const size_t kv = static_cast<size_t>(kAttnKvHeads) * T * kAttnHeadDim * sizeof(uint16_t);
  for (LayerState& l : st->layers) {
    if (l.conv) {
      host.resize(kConvBytes + kRecurBytes);
      if (int rc = f.read_all(host.data(), host.size())) return rc;
      PRG_HIP(hipMemcpy(l.conv, host.data(), kConvBytes, hipMemcpyHostToDevice));
      PRG_HIP(hipMemcpy(l.recur, host.data() + kConvBytes, kRecurBytes, hipMemcpyHostToDevice));
    } else if (l.cache_k) {
      host.resize(2 * kv);
      if (int rc = f.read_all(host.data(), host.size())) return rc;
      const size_t row = sizeof(uint16_t) * kAttnHeadDim;
      PRG_HIP(hipMemcpy2D(l.cache_k, st->stride * row, host.data(), T * row, T * row, kAttnKvHeads,
                          hipMemcpyHostToDevice));
      PRG_HIP(hipMemcpy2D(l.cache_v, st->stride * sizeof(uint16_t), host.data() + kv, T * sizeof(uint16_t),
                          T * sizeof(uint16_t), kAttnKvHeads * kAttnHeadDim, hipMemcpyHostToDevice));
    }
  }
  return PRG_OK;
}

}  // namespace
}  // namespace prg

using namespace prg;

extern "C" {

int prg_wyhash(const void* data, size_t len, uint64_t seed, uint64_t* out) {
  PRG_CHECK_ARG(out && (data || len == 0), "prg_wyhash: null argument");
  Wyhash h(seed);
  h.update(data, len);
  *out = h.final();
  return PRG_OK;
}

// modelFingerprint (prefix_persist.zig:149-190): config.json, then every
// *.safetensors file (regular or symlink) in bytewise name order, name then
// content, through one Wyhash seeded with MAGIC ^ VERSION.
int prg_model_fingerprint(const char* model_dir, uint64_t* out) {
  PRG_CHECK_ARG(model_dir && out, "prg_model_fingerprint: null argument");
  const std::string dir = model_dir;
  Wyhash h(kMagic ^ kVersion);
  std::vector<char> chunk(size_t(4) << 20);
  auto hash_file = [&](const std::string& path) -> int {
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
      if (errno == ENOENT) return set_error(PRG_ERR_NOT_FOUND, "FileNotFound: %s", path.c_str());
      return set_error(PRG_ERR_IO, "open %s: %s", path.c_str(), strerror(errno));
    }
    for (;;) {
      const ssize_t n = read(fd, chunk.data(), chunk.size());
      if (n < 0 && errno == EINTR) continue;
      if (n < 0) {
        close(fd);
        return set_error(PRG_ERR_IO, "read %s: %s", path.c_str(), strerror(errno));
      }
      if (n == 0) break;
      h.update(chunk.data(), static_cast<size_t>(n));
    }
    close(fd);
    return PRG_OK;
  };
  std::string config;
  {
    const std::string path = dir + "/config.json";
    struct stat sb;
    if (stat(path.c_str(), &sb) != 0) return set_error(PRG_ERR_NOT_FOUND, "FileNotFound: %s", path.c_str());
    if (sb.st_size > (4 << 20)) return set_error(PRG_ERR_MALFORMED, "StreamTooLong: %s", path.c_str());
    if (int rc = hash_file(path)) return rc;
  }
  DIR* d = opendir(dir.c_str());
  if (!d) return set_error(PRG_ERR_NOT_FOUND, "FileNotFound: %s", dir.c_str());
  std::vector<std::string> shards;
  const std::string suffix = ".safetensors";
  while (struct dirent* ent = readdir(d)) {
    const std::string name = ent->d_name;
    if (name.size() < suffix.size() || name.compare(name.size() - suffix.size(), suffix.size(), suffix) != 0)
      continue;
    unsigned char type = ent->d_type;
    if (type == DT_UNKNOWN) {
      struct stat sb;
      if (lstat((dir + "/" + name).c_str(), &sb) != 0) continue;
      type = S_ISREG(sb.st_mode) ? DT_REG : S_ISLNK(sb.st_mode) ? DT_LNK : DT_UNKNOWN;
    }
    if (type == DT_REG || type == DT_LNK) shards.push_back(name);
  }
  closedir(d);
  std::sort(shards.begin(), shards.end());
  for (const std::string& name : shards) {
    h.update(name.data(), name.size());
    if (int rc = hash_file(dir + "/" + name)) return rc;
  }
  *out = h.final();
  return PRG_OK;
}

int prg_prefix_state_file_bytes(const PrgModelConfig* cfg, uint64_t token_count, uint64_t* bytes) {
  PRG_CHECK_ARG(cfg && bytes && cfg->full_attention_interval >= 1, "prg_prefix_state_file_bytes: bad argument");
  *bytes = expected_file_bytes(*cfg, token_count);
  return PRG_OK;
}

int prg_prefix_state_default_path(char* buf, size_t len) {
  PRG_CHECK_ARG(buf && len, "prg_prefix_state_default_path: null argument");
  const char* home = getenv("HOME");
  if (!home || !*home) return set_error(PRG_ERR_NOT_FOUND, "HOME is not set");
  const int n = snprintf(buf, len, "%s/.cache/peregrine/qwen35-9b-q4-prefix-state.bin", home);
  PRG_CHECK_ARG(n > 0 && static_cast<size_t>(n) < len, "prg_prefix_state_default_path: buffer too small");
  return PRG_OK;
}

int prg_prefix_cache_create(PrgModel* model, uint32_t max_cache_tokens, uint32_t prefill_chunk_tokens,
                            PrgPrefixCache** out) {
  PRG_CHECK_ARG(out, "prg_prefix_cache_create: null argument");
  *out = nullptr;
  auto* c = new PrgPrefixCache();
  c->model = model;
  c->max_tokens = max_cache_tokens;
  c->initial_state_tokens = std::min(max_cache_tokens, prefill_chunk_tokens);
  if (model) {
    const hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete c;
      return set_error(PRG_ERR_HIP, "prefix cache stream: %s", hipGetErrorString(e));
    }
  }
  *out = c;
  return PRG_OK;
}

void prg_prefix_cache_destroy(PrgPrefixCache* c) {
  if (!c) return;
  clear_all(c);
  if (c->stream) hipStreamDestroy(c->stream);
  delete c;
}

int prg_prefix_cache_clear(PrgPrefixCache* c) {
  PRG_CHECK_ARG(c, "prg_prefix_cache_clear: null cache");
  clear_all(c);
  return PRG_OK;
}

uint32_t prg_prefix_cache_entry_count(const PrgPrefixCache* c) {
  return c ? static_cast<uint32_t>(c->entries.size()) : 0u;
}

uint32_t prg_prefix_cache_pinned_count(const PrgPrefixCache* c) {
  if (!c) return 0;
  uint32_t n = 0;
  for (const PrefixEntry& e : c->entries) n += e.pinned ? 1 : 0;
  return n;
}

uint32_t prg_prefix_cache_active_tokens(const PrgPrefixCache* c) {
  if (!c || c->active < 0 || c->active >= static_cast<int>(c->entries.size())) return 0;
  return static_cast<uint32_t>(c->entries[c->active].tokens.size());
}

int prg_prefix_cache_stats(const PrgPrefixCache* c, PrgPrefixCacheStats* s) {
  PRG_CHECK_ARG(c && s, "prg_prefix_cache_stats: null argument");
  s->hits = c->hits;
  s->misses = c->misses;
  s->hit_tokens = c->hit_tokens;
  s->computed_tokens = c->computed_tokens;
  s->reserved_tokens = c->reserved_tokens;
  s->resident_tokens = c->resident_tokens;
  s->max_tokens = c->max_tokens;
  s->entry_count = c->entries.size();
  s->evictions = c->evictions;
  return PRG_OK;
}

void prg_prefix_cache_record_hit(PrgPrefixCache* c, uint32_t reused_tokens) {
  if (!c) return;
  c->hits += 1;
  c->hit_tokens += reused_tokens;
}

void prg_prefix_cache_record_miss(PrgPrefixCache* c) {
  if (c) c->misses += 1;
}

void prg_prefix_cache_record_computed(PrgPrefixCache* c, uint32_t token_count) {
  if (c) c->computed_tokens += token_count;
}

int prg_prefix_cache_find(const PrgPrefixCache* c, const uint32_t* prompt, uint32_t prompt_len,
                          PrgPrefixMatch* match) {
  PRG_CHECK_ARG(c && match && (prompt || prompt_len == 0), "prg_prefix_cache_find: null argument");
  int entry = -1;
  size_t len = 0;
  if (c->index.find_longest(prompt, prompt_len, &entry, &len)) {
    match->index = static_cast<uint32_t>(entry);
    match->len = static_cast<uint32_t>(len);
  } else {
    match->index = 0;
    match->len = 0;
  }
  return PRG_OK;
}

int prg_prefix_cache_contains(const PrgPrefixCache* c, const uint32_t* prompt, uint32_t prompt_len,
                              uint32_t prefix_len) {
  if (!c || (!prompt && prompt_len)) return 0;
  return c->index.contains_prefix(prompt, prompt_len, prefix_len) ? 1 : 0;
}

int prg_prefix_cache_touch(PrgPrefixCache* c, PrgPrefixMatch match) {
  PRG_CHECK_ARG(c, "prg_prefix_cache_touch: null cache");
  if (int rc = check_match(c, match)) return rc;
  touch(c, match.index);
  return PRG_OK;
}

int prg_prefix_cache_remove(PrgPrefixCache* c, uint32_t index) {
  PRG_CHECK_ARG(c && index < c->entries.size(), "prg_prefix_cache_remove: bad index");
  remove_entry(c, index);
  return PRG_OK;
}

int prg_prefix_cache_entry_info(const PrgPrefixCache* c, uint32_t index, uint32_t* token_count, uint32_t* capacity,
                                int* pinned, uint64_t* hits) {
  PRG_CHECK_ARG(c && index < c->entries.size(), "prg_prefix_cache_entry_info: bad index");
  const PrefixEntry& e = c->entries[index];
  if (token_count) *token_count = static_cast<uint32_t>(e.tokens.size());
  if (capacity) *capacity = e.capacity;
  if (pinned) *pinned = e.pinned ? 1 : 0;
  if (hits) *hits = e.hits;
  return PRG_OK;
}

int prg_prefix_cache_entry_tokens(const PrgPrefixCache* c, uint32_t index, uint32_t* tokens, uint32_t capacity) {
  PRG_CHECK_ARG(c && tokens && index < c->entries.size(), "prg_prefix_cache_entry_tokens: bad argument");
  const PrefixEntry& e = c->entries[index];
  PRG_CHECK_ARG(capacity >= e.tokens.size(), "prg_prefix_cache_entry_tokens: buffer of %u < %zu", capacity,
                e.tokens.size());
  std::copy(e.tokens.begin(), e.tokens.end(), tokens);
  return PRG_OK;
}

int prg_prefix_cache_entry_state(PrgPrefixCache* c, uint32_t index, PrgModelState** state) {
  PRG_CHECK_ARG(c && state && index < c->entries.size(), "prg_prefix_cache_entry_state: bad argument");
  PRG_CHECK_ARG(c->model, "prg_prefix_cache_entry_state: the cache was created without a model");
  *state = c->entries[index].state;
  return PRG_OK;
}

int prg_prefix_cache_cached_next_token(const PrgPrefixCache* c, PrgPrefixMatch match, uint32_t* token, int* valid) {
  PRG_CHECK_ARG(c && token && valid, "prg_prefix_cache_cached_next_token: null argument");
  if (int rc = check_match(c, match)) return rc;
  *token = c->entries[match.index].next_token;
  *valid = c->entries[match.index].next_valid ? 1 : 0;
  return PRG_OK;
}

int prg_prefix_cache_start_direct(PrgPrefixCache* c, const uint32_t* ids, uint32_t n, int pinned,
                                  PrgPrefixMatch* out) {
  PRG_CHECK_ARG(c && out && (ids || n == 0), "prg_prefix_cache_start_direct: null argument");
  int idx = -1;
  if (int rc = prepare_entry(c, ids, n, -1, pinned != 0, &idx)) return rc;
  PrefixEntry& e = c->entries[idx];
  if (e.state)
    if (int rc = prg_model_state_reset(e.state)) return rc;
  e.next_valid = false;
  out->index = static_cast<uint32_t>(idx);
  out->len = n;
  return PRG_OK;
}

int prg_prefix_cache_finish_direct(PrgPrefixCache* c, PrgPrefixMatch match, uint32_t next_token) {
  PRG_CHECK_ARG(c, "prg_prefix_cache_finish_direct: null cache");
  if (int rc = check_match(c, match)) return rc;
  PrefixEntry& e = c->entries[match.index];
  e.next_token = next_token;
  e.next_valid = true;
  touch(c, match.index);
  return PRG_OK;
}

int prg_prefix_cache_store(PrgPrefixCache* c, const uint32_t* ids, uint32_t n, const PrgPrefixMatch* reuse,
                           const PrgModelState* work, const uint16_t* work_hidden, uint32_t work_hidden_base_rows,
                           const uint32_t* next_token, int pinned, PrgPrefixMatch* out) {
  PRG_CHECK_ARG(c && out && (ids || n == 0), "prg_prefix_cache_store: null argument");
  PRG_CHECK_ARG(!c->model || (work && work->model == c->model), "prg_prefix_cache_store: work state of another model");
  if (reuse)
    if (int rc = check_match(c, *reuse)) return rc;
  if (n == 0 || n > c->max_tokens)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix cache: prefix of %u tokens (budget %llu)", n,
                     (unsigned long long)c->max_tokens);
  if (work) PRG_CHECK_ARG(n <= work->max_seq, "prg_prefix_cache_store: %u tokens > work capacity %u", n, work->max_seq);
  const bool had_exact = c->index.find_exact(ids, n) >= 0;
  int idx = -1;
  if (int rc = prepare_entry(c, ids, n, reuse ? static_cast<int>(reuse->index) : -1, pinned != 0, &idx)) return rc;
  PrefixEntry& e = c->entries[idx];
  const uint32_t reuse_len = reuse ? std::min(reuse->len, n) : 0;
  // storePrefixFromWork (prefix_state_cache.zig:563-648). The working state
  // holds absolute positions [0, n) (the reused prefix was copied into it), so
  // a re-keyed entry takes positions [reuse_len, n) plus the GDN state.
  if (!had_exact && e.state) {
    int rc = copy_attention_range(e.state, reuse_len, work, reuse_len, n - reuse_len);
    if (rc == PRG_OK) rc = copy_linear_state(e.state, work);
    if (rc) return rc;
  }
  if (c->track_hidden && c->model) {
    const bool reuse_hidden_valid = reuse_len != 0 ? e.hidden_valid : false;
    if (int rc = ensure_hidden_capacity(c, e, n)) return rc;
    const uint32_t suffix = n - reuse_len;
    const size_t rb = hidden_row_bytes(c);
    if (suffix) {
      uint16_t* dst = e.hidden + static_cast<size_t>(reuse_len) * (rb / 2);
      if (work_hidden)
        PRG_HIP(hipMemcpyAsync(dst, work_hidden + static_cast<size_t>(work_hidden_base_rows) * (rb / 2), suffix * rb,
                               hipMemcpyDeviceToDevice, c->stream));
      else
        PRG_HIP(hipMemsetAsync(dst, 0, suffix * rb, c->stream));
      PRG_HIP(hipStreamSynchronize(c->stream));
    }
    e.hidden_valid = (reuse_len == 0 || reuse_hidden_valid) && (suffix == 0 || work_hidden != nullptr);
  }
  if (next_token) {
    e.next_token = *next_token;
    e.next_valid = true;
  } else {
    e.next_valid = false;
  }
  touch(c, idx);
  out->index = static_cast<uint32_t>(idx);
  out->len = n;
  return PRG_OK;
}

int prg_prefix_cache_restore(const PrgPrefixCache* c, PrgPrefixMatch match, PrgModelState* work) {
  PRG_CHECK_ARG(c && work, "prg_prefix_cache_restore: null argument");
  PRG_CHECK_ARG(c->model && work->model == c->model, "prg_prefix_cache_restore: work state of another model");
  if (int rc = check_match(c, match)) return rc;
  const PrefixEntry& e = c->entries[match.index];
  // The GDN state exists only after the entry's last token.
  PRG_CHECK_ARG(match.len == e.tokens.size(), "prg_prefix_cache_restore: match of %u tokens on an entry of %zu",
                match.len, e.tokens.size());
  if (match.len > work->max_seq)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "restore: %u tokens exceed max_seq %u", match.len, work->max_seq);
  if (int rc = copy_attention_range(work, 0, e.state, 0, match.len)) return rc;
  return copy_linear_state(work, e.state);
}

int prg_prefix_cache_enable_hidden(PrgPrefixCache* c) {
  PRG_CHECK_ARG(c, "prg_prefix_cache_enable_hidden: null cache");
  c->track_hidden = true;
  return PRG_OK;
}

int prg_prefix_cache_entry_hidden(const PrgPrefixCache* c, PrgPrefixMatch match, uint16_t** rows, int* valid) {
  PRG_CHECK_ARG(c && rows && valid, "prg_prefix_cache_entry_hidden: null argument");
  if (int rc = check_match(c, match)) return rc;
  *rows = c->entries[match.index].hidden;
  *valid = c->entries[match.index].hidden_valid ? 1 : 0;
  return PRG_OK;
}

int prg_prefix_cache_set_entry_hidden(PrgPrefixCache* c, PrgPrefixMatch match, const uint16_t* rows) {
  PRG_CHECK_ARG(c && rows && c->model, "prg_prefix_cache_set_entry_hidden: bad argument");
  if (int rc = check_match(c, match)) return rc;
  PrefixEntry& e = c->entries[match.index];
  if (int rc = ensure_hidden_capacity(c, e, match.len)) return rc;
  PRG_HIP(hipMemcpyAsync(e.hidden, rows, match.len * hidden_row_bytes(c), hipMemcpyDeviceToDevice, c->stream));
  PRG_HIP(hipStreamSynchronize(c->stream));
  e.hidden_valid = true;
  return PRG_OK;
}

// save (prefix_persist.zig:253-328): temp file + rename.
int prg_prefix_cache_save(const PrgPrefixCache* c, const char* path, uint64_t model_fingerprint) {
  PRG_CHECK_ARG(c && path && c->model, "prg_prefix_cache_save: bad argument");
  const PrefixEntry* e = persisted_entry(c);
  if (!e || e->tokens.empty()) return set_error(PRG_ERR_EMPTY_INPUT, "EmptyPrefix: nothing cached");
  const uint32_t T = static_cast<uint32_t>(e->tokens.size());
  if (T > e->capacity) return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "SequenceTooLong: %u > %u", T, e->capacity);
  const std::string final_path = path;
  if (int rc = make_parent_dirs(final_path)) return rc;
  const std::string tmp = final_path + ".tmp." + std::to_string(getpid());
  int rc = PRG_OK;
  {
    File f;
    if ((rc = f.open_write(tmp))) return rc;
    FileHeader h{};
    h.magic = kMagic;
    h.version = kVersion;
    h.dtype = kDtypeBf16;
    h.model_fingerprint = model_fingerprint;
    h.token_count = T;
    h.next_token = e->next_token;
    h.next_token_valid = e->next_valid ? 1 : 0;
    h.hidden_valid = (e->hidden && e->hidden_valid) ? 1 : 0;
    std::vector<uint8_t> host;
    if (!rc) rc = f.write_all(&h, sizeof(h));
    if (!rc) rc = f.write_all(e->tokens.data(), sizeof(uint32_t) * T);
    if (!rc) rc = write_state(f, e->state, T, host);
    if (!rc) {  // hidden section: real rows or zeros, always present
      const size_t hb = static_cast<size_t>(T) * hidden_row_bytes(c);
      host.assign(hb, 0);
      if (e->hidden) {
        const hipError_t err = hipMemcpy(host.data(), e->hidden, hb, hipMemcpyDeviceToHost);
        if (err != hipSuccess) rc = set_error(PRG_ERR_HIP, "hidden rows: %s", hipGetErrorString(err));
      }
      if (!rc) rc = f.write_all(host.data(), hb);
    }
    if (!rc) rc = f.sync_close();
  }
  if (!rc && rename(tmp.c_str(), final_path.c_str()) != 0)
    rc = set_error(PRG_ERR_IO, "rename %s: %s", final_path.c_str(), strerror(errno));
  if (rc) unlink(tmp.c_str());
  return rc;
}

// load (prefix_persist.zig:334-412). A missing or invalid file leaves the
// cache unchanged and reports *loaded_tokens = 0 (the reference returns null;
// prg_last_error() says why); a failure while reading clears the cache.
int prg_prefix_cache_load(PrgPrefixCache* c, const char* path, uint64_t model_fingerprint, uint32_t* loaded_tokens) {
  PRG_CHECK_ARG(c && path && loaded_tokens && c->model, "prg_prefix_cache_load: bad argument");
  *loaded_tokens = 0;
  File f;
  bool missing = false;
  if (int rc = f.open_read(path, &missing)) return rc;
  if (missing) {
    set_error(PRG_OK, "FileNotFound: %s", path);
    return PRG_OK;
  }
  FileHeader h{};
  const uint64_t size = f.size();
  auto ignore = [&](const char* why) {
    set_error(PRG_OK, "ignored persisted prefix state %s: %s", path, why);
    return PRG_OK;
  };
  if (size < sizeof(h) || f.read_all(&h, sizeof(h)) != PRG_OK) return ignore("short header");
  if (h.magic != kMagic || h.version != kVersion || h.dtype != kDtypeBf16) return ignore("magic / version / dtype");
  if (h.model_fingerprint != model_fingerprint) return ignore("model fingerprint differs");
  if (h.next_token_valid > 1 || (h.next_token_valid == 1 && h.next_token >= c->model->cfg.vocab))
    return ignore("cached next token outside the vocab");
  if (h.hidden_valid > 1) return ignore("hidden_valid flag");
  if (h.token_count == 0 || h.token_count > c->max_tokens || h.token_count > 65536)
    return ignore("token count outside the cache budget");
  const uint32_t T = static_cast<uint32_t>(h.token_count);
  if (size != expected_file_bytes(c->model->cfg, T)) return ignore("file length");

  // loadEntrySlot + finishLoadedEntry (prefix_state_cache.zig:663-690).
  clear_all(c);
  PrefixEntry e;
  int rc = new_entry(c, static_cast<uint32_t>(std::max<uint64_t>(T, c->initial_state_tokens)), true, &e);
  if (rc) return rc;
  e.tokens.resize(T);
  e.last_access = next_access(c);
  c->entries.push_back(std::move(e));
  PrefixEntry& ent = c->entries.back();
  c->resident_tokens = T;
  c->reserved_tokens = ent.capacity;
  c->active = static_cast<int>(c->entries.size()) - 1;
  if (c->track_hidden) rc = ensure_hidden_capacity(c, ent, T);
  std::vector<uint8_t> host;
  if (!rc) rc = f.read_all(ent.tokens.data(), sizeof(uint32_t) * T);
  if (!rc) {
    for (uint32_t t : ent.tokens)
      if (t >= c->model->cfg.vocab) rc = set_error(PRG_ERR_INVALID_TOKEN, "persisted token %u >= vocab", t);
  }
  if (!rc) c->index.insert(ent.tokens.data(), T, c->active);
  if (!rc) rc = read_state(f, ent.state, T, host);
  if (!rc) {
    ent.next_token = h.next_token;
    ent.next_valid = h.next_token_valid == 1;
    const size_t hb = static_cast<size_t>(T) * hidden_row_bytes(c);
    host.resize(hb);
    rc = f.read_all(host.data(), hb);
    if (!rc && ent.hidden) {
      const hipError_t err = hipMemcpy(ent.hidden, host.data(), hb, hipMemcpyHostToDevice);
      if (err != hipSuccess) rc = set_error(PRG_ERR_HIP, "hidden rows: %s", hipGetErrorString(err));
      ent.hidden_valid = h.hidden_valid == 1;
    }
  }
  if (rc) {
    clear_all(c);
    return rc;
  }
  *loaded_tokens = T;
  return PRG_OK;
}

}  // extern "C"
