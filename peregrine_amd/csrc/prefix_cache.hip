// Prompt-prefix state cache and its PRGPFXS1 v3 persistence file (host code;
// the device work is copies between ModelStates).
//
// Observable rules kept from the reference (src/server/prefix_state_cache.zig):
// an entry per exact token prefix; the longest cached prefix of a prompt is
// reused; storing a longer prefix that continues a reused entry re-keys that
// entry; every entry reserves max(tokens, prefill chunk) state slots and the
// reserved total stays within the token budget by evicting the least recently
// used unpinned entry; entries are numbered in creation order. The file format,
// its validation and the model fingerprint follow src/server/prefix_persist.zig:31-412.
//
// The store itself is this file's own: entries live in a table keyed by
// stable ids and are found through a hash of their whole token key with a
// per-length probe for the longest match (no trie), and the budget totals are
// summed from the entries when needed. A working state reuses a cached
// prefix by copying it in (prg_prefix_cache_restore), so positions stay
// absolute (see model_prefix.hip). Created without a model, the cache keeps
// tokens and accounting only (no device state).
#include <dirent.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <iterator>
#include <map>
#include <string>
#include <unordered_map>
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

// ------------------------------------------------------------ the store -----
// Cached prefixes live in a table keyed by a stable id that is never reused;
// ids grow with creation, so the table's order is creation order and the
// C ABI's entry index is an entry's rank in it. Lookups go through a hash of
// the whole token key (verified against the tokens, so a collision can only
// cost a comparison): the longest cached prefix of a prompt is found by
// hashing the prompt's prefixes once and probing only the key lengths that
// exist, longest first.
struct CachedPrefix {
  std::vector<uint32_t> tokens;    // the key
  uint64_t key_hash = 0;
  uint32_t reserved = 0;           // token capacity of `state`; counts against the budget
  PrgModelState* state = nullptr;  // nullptr for a cache without a model
  uint16_t* hidden = nullptr;      // device bf16 rows [reserved, hidden] once tracked
  bool hidden_valid = false;
  uint32_t next_token = 0;
  bool next_valid = false;
  bool pinned = false;
  uint64_t stamp = 0;  // last use (logical clock)
  uint64_t hits = 0;
};

// Polynomial hash of a token key, extended one token at a time.
inline uint64_t key_step(uint64_t h, uint32_t t) { return (h ^ (t + 0x9e3779b97f4a7c15ull)) * 0x100000001b3ull; }
inline uint64_t key_hash(const uint32_t* t, size_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; ++i) h = key_step(h, t[i]);
  return h;
}

class PrefixStore {
 public:
  using Table = std::map<uint64_t, CachedPrefix>;

  Table& table() { return table_; }
  const Table& table() const { return table_; }
  size_t size() const { return table_.size(); }

  CachedPrefix* get(uint64_t id) {
    auto it = table_.find(id);
    return it == table_.end() ? nullptr : &it->second;
  }
  const CachedPrefix* get(uint64_t id) const {
    auto it = table_.find(id);
    return it == table_.end() ? nullptr : &it->second;
  }
  // Id at C-ABI index `rank`, or 0.
  uint64_t id_at(size_t rank) const {
    if (rank >= table_.size()) return 0;
    return std::next(table_.begin(), static_cast<long>(rank))->first;
  }
  uint32_t rank_of(uint64_t id) const {
    return static_cast<uint32_t>(std::distance(table_.begin(), table_.find(id)));
  }

  uint64_t add(CachedPrefix&& e) {
    const uint64_t id = ++last_id_;
    e.key_hash = key_hash(e.tokens.data(), e.tokens.size());
    link(id, e);
    table_.emplace(id, std::move(e));
    return id;
  }
  // Re-key entry `id` to a new token sequence.
  void rekey(uint64_t id, const uint32_t* t, size_t n) {
    CachedPrefix& e = table_.at(id);
    unlink(id, e);
    e.tokens.assign(t, t + n);
    e.key_hash = key_hash(t, n);
    link(id, e);
  }
  // Remove entry `id` from the table; the caller releases its resources.
  CachedPrefix take(uint64_t id) {
    auto it = table_.find(id);
    unlink(id, it->second);
    CachedPrefix e = std::move(it->second);
    table_.erase(it);
    return e;
  }
  void reset() {
    table_.clear();
    by_hash_.clear();
    lengths_.clear();
  }

  uint64_t exact(const uint32_t* t, size_t n) const {
    if (n == 0 || lengths_.find(static_cast<uint32_t>(n)) == lengths_.end()) return 0;
    return probe(key_hash(t, n), t, n);
  }
  // Longest cached key that is a prefix of p[0, n): its id and length.
  uint64_t longest(const uint32_t* p, size_t n, size_t* len) const {
    if (lengths_.empty() || n == 0) return 0;
    const size_t top = std::min<size_t>(n, lengths_.rbegin()->first);
    std::vector<uint64_t> h(top + 1);
    h[0] = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < top; ++i) h[i + 1] = key_step(h[i], p[i]);
    for (auto it = lengths_.rbegin(); it != lengths_.rend(); ++it) {
      const size_t L = it->first;
      if (L > top) continue;
      if (const uint64_t id = probe(h[L], p, L)) {
        *len = L;
        return id;
      }
    }
    return 0;
  }

  uint64_t reserved_total() const {
    uint64_t s = 0;
    for (const auto& kv : table_) s += kv.second.reserved;
    return s;
  }
  uint64_t resident_total() const {
    uint64_t s = 0;
    for (const auto& kv : table_) s += kv.second.tokens.size();
    return s;
  }
  // The unpinned entry other than `keep` used longest ago, or 0.
  uint64_t coldest(uint64_t keep) const {
    uint64_t best = 0, best_stamp = 0;
    for (const auto& kv : table_) {
      if (kv.first == keep || kv.second.pinned) continue;
      if (best == 0 || kv.second.stamp < best_stamp) {
        best = kv.first;
        best_stamp = kv.second.stamp;
      }
    }
    return best;
  }

 private:
  Table table_;
  std::unordered_multimap<uint64_t, uint64_t> by_hash_;  // key hash -> id
  std::map<uint32_t, uint32_t> lengths_;                  // key length -> entries with it
  uint64_t last_id_ = 0;

  void link(uint64_t id, const CachedPrefix& e) {
    by_hash_.emplace(e.key_hash, id);
    lengths_[static_cast<uint32_t>(e.tokens.size())] += 1;
  }
  void unlink(uint64_t id, const CachedPrefix& e) {
    auto range = by_hash_.equal_range(e.key_hash);
    for (auto it = range.first; it != range.second; ++it)
      if (it->second == id) {
        by_hash_.erase(it);
        break;
      }
    auto l = lengths_.find(static_cast<uint32_t>(e.tokens.size()));
    if (l != lengths_.end() && --l->second == 0) lengths_.erase(l);
  }
  uint64_t probe(uint64_t h, const uint32_t* t, size_t n) const {
    auto range = by_hash_.equal_range(h);
    for (auto it = range.first; it != range.second; ++it) {
      const CachedPrefix& e = table_.at(it->second);
      if (e.tokens.size() == n && std::equal(e.tokens.begin(), e.tokens.end(), t)) return it->second;
    }
    return 0;
  }
};

}  // namespace prg

struct PrgPrefixCache {
  PrgModel* model = nullptr;
  prg::PrefixStore store;
  uint64_t max_tokens = 0, initial_state_tokens = 0;
  uint64_t active = 0;  // id of the entry last used, 0 = none
  uint64_t clock = 0;
  uint64_t hits = 0, misses = 0, hit_tokens = 0, computed_tokens = 0, evictions = 0;
  bool track_hidden = false;
  hipStream_t stream = nullptr;  // hidden-row copies
};

namespace prg {
namespace {

using Cache = PrgPrefixCache;

size_t hidden_row_bytes(const Cache* c) { return sizeof(uint16_t) * c->model->cfg.hidden; }

void release(CachedPrefix& e) {
  if (e.state) prg_model_state_destroy(e.state);
  if (e.hidden) (void)hipFree(e.hidden);
  e.state = nullptr;
  e.hidden = nullptr;
}

void drop(Cache* c, uint64_t id) {
  CachedPrefix e = c->store.take(id);
  release(e);
  if (c->active == id) c->active = 0;
}

void drop_all(Cache* c) {
  for (auto& kv : c->store.table()) release(kv.second);
  c->store.reset();
  c->active = 0;
}

void mark_used(Cache* c, uint64_t id) {
  CachedPrefix* e = c->store.get(id);
  if (!e) return;
  e->stamp = ++c->clock;
  e->hits += 1;
  c->active = id;
}

// Evict least recently used unpinned entries (never `keep`) until `extra`
// more reserved tokens fit the budget.
int make_room(Cache* c, uint64_t extra, uint64_t keep) {
  if (extra > c->max_tokens)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix cache: %llu tokens exceed the budget %llu",
                     (unsigned long long)extra, (unsigned long long)c->max_tokens);
  while (c->store.reserved_total() + extra > c->max_tokens) {
    const uint64_t victim = c->store.coldest(keep);
    if (victim == 0)
      return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix cache: budget %llu exhausted by pinned entries",
                       (unsigned long long)c->max_tokens);
    drop(c, victim);
    c->evictions += 1;
  }
  return PRG_OK;
}

// Device buffers of an entry with `capacity` token slots: a model state, and
// hidden rows when the cache tracks them. Existing contents (the entry's
// first `keep` positions and its GDN state, its first `keep` hidden rows)
// move into the new buffers.
int resize_buffers(Cache* c, CachedPrefix& e, uint32_t capacity, uint32_t keep) {
  if (!c->model) {
    e.reserved = capacity;
    return PRG_OK;
  }
  PrgModelState* st = nullptr;
  if (int rc = prg_model_state_create(c->model, capacity, &st)) return rc;
  if (e.state && keep) {
    int rc = copy_attention_range(st, 0, e.state, 0, keep);
    if (rc == PRG_OK) rc = copy_linear_state(st, e.state);
    if (rc) {
      prg_model_state_destroy(st);
      return rc;
    }
  }
  uint16_t* rows = nullptr;
  if (c->track_hidden || e.hidden) {
    const size_t rb = hidden_row_bytes(c);
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&rows), rb * capacity);
    if (err == hipSuccess) err = hipMemsetAsync(rows, 0, rb * capacity, c->stream);
    if (err == hipSuccess && e.hidden && keep)
      err = hipMemcpyAsync(rows, e.hidden, rb * keep, hipMemcpyDeviceToDevice, c->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(c->stream);
    if (err != hipSuccess) {
      if (rows) (void)hipFree(rows);
      prg_model_state_destroy(st);
      return set_error(PRG_ERR_HIP, "prefix cache hidden rows: %s", hipGetErrorString(err));
    }
  }
  if (e.state) prg_model_state_destroy(e.state);
  if (e.hidden) (void)hipFree(e.hidden);
  e.state = st;
  e.hidden = rows;
  e.reserved = capacity;
  return PRG_OK;
}

// Hidden rows for an entry created before tracking was switched on.
int ensure_hidden_rows(Cache* c, CachedPrefix& e) {
  if (e.hidden) return PRG_OK;
  const size_t rb = hidden_row_bytes(c);
  PRG_HIP(hipMalloc(reinterpret_cast<void**>(&e.hidden), rb * e.reserved));
  PRG_HIP(hipMemsetAsync(e.hidden, 0, rb * e.reserved, c->stream));
  PRG_HIP(hipStreamSynchronize(c->stream));
  return PRG_OK;
}

// Make the entry that will hold ids[0, n): the entry already keyed by exactly
// these tokens; else `reuse` re-keyed to them (a longer prefix continuing
// it); else a new entry of max(n, initial_state_tokens) slots. Growing an
// entry or adding one evicts least recently used unpinned entries first.
int admit(Cache* c, const uint32_t* ids, uint32_t n, uint64_t reuse, bool pinned, uint64_t* out) {
  if (n == 0 || n > c->max_tokens)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix cache: prefix of %u tokens (budget %llu)", n,
                     (unsigned long long)c->max_tokens);
  uint64_t id = c->store.exact(ids, n);
  if (id == 0) id = reuse;
  if (id != 0) {
    CachedPrefix& e = *c->store.get(id);
    if (n > e.reserved) {
      if (int rc = make_room(c, n - e.reserved, id)) return rc;
      CachedPrefix& grown = *c->store.get(id);
      if (int rc = resize_buffers(c, grown, n, static_cast<uint32_t>(grown.tokens.size()))) return rc;
    }
    CachedPrefix& ent = *c->store.get(id);
    if (ent.tokens.size() != n || !std::equal(ent.tokens.begin(), ent.tokens.end(), ids)) c->store.rekey(id, ids, n);
    ent.pinned = ent.pinned || pinned;
    *out = id;
    return PRG_OK;
  }
  const uint32_t capacity = static_cast<uint32_t>(std::max<uint64_t>(n, c->initial_state_tokens));
  if (int rc = make_room(c, capacity, 0)) return rc;
  CachedPrefix e;
  e.tokens.assign(ids, ids + n);
  e.pinned = pinned;
  e.stamp = ++c->clock;
  if (int rc = resize_buffers(c, e, capacity, 0)) {
    release(e);
    return rc;
  }
  *out = c->store.add(std::move(e));
  return PRG_OK;
}

int match_id(const Cache* c, const PrgPrefixMatch& m, uint64_t* id) {
  *id = c->store.id_at(m.index);
  PRG_CHECK_ARG(*id != 0, "prefix cache: match index %u of %zu entries", m.index, c->store.size());
  return PRG_OK;
}

PrgPrefixMatch match_of(const Cache* c, uint64_t id, uint32_t len) {
  PrgPrefixMatch m;
  m.index = c->store.rank_of(id);
  m.len = len;
  return m;
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

// The entry a save persists: the one last used, else the most recently used
// non-empty one (persistedEntryConst, prefix_state_cache.zig:380-391).
const CachedPrefix* persisted_entry(const Cache* c) {
  if (const CachedPrefix* e = c->store.get(c->active)) return e;
  const CachedPrefix* best = nullptr;
  for (const auto& kv : c->store.table())
    if (!kv.second.tokens.empty() && (!best || kv.second.stamp > best->stamp)) best = &kv.second;
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
  drop_all(c);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

int prg_prefix_cache_clear(PrgPrefixCache* c) {
  PRG_CHECK_ARG(c, "prg_prefix_cache_clear: null cache");
  drop_all(c);
  return PRG_OK;
}

uint32_t prg_prefix_cache_entry_count(const PrgPrefixCache* c) {
  return c ? static_cast<uint32_t>(c->store.size()) : 0u;
}

uint32_t prg_prefix_cache_pinned_count(const PrgPrefixCache* c) {
  if (!c) return 0;
  uint32_t n = 0;
  for (const auto& kv : c->store.table()) n += kv.second.pinned ? 1 : 0;
  return n;
}

uint32_t prg_prefix_cache_active_tokens(const PrgPrefixCache* c) {
  const CachedPrefix* e = c ? c->store.get(c->active) : nullptr;
  return e ? static_cast<uint32_t>(e->tokens.size()) : 0u;
}

int prg_prefix_cache_stats(const PrgPrefixCache* c, PrgPrefixCacheStats* s) {
  PRG_CHECK_ARG(c && s, "prg_prefix_cache_stats: null argument");
  s->hits = c->hits;
  s->misses = c->misses;
  s->hit_tokens = c->hit_tokens;
  s->computed_tokens = c->computed_tokens;
  s->reserved_tokens = c->store.reserved_total();
  s->resident_tokens = c->store.resident_total();
  s->max_tokens = c->max_tokens;
  s->entry_count = c->store.size();
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
  size_t len = 0;
  const uint64_t id = c->store.longest(prompt, prompt_len, &len);
  *match = id ? match_of(c, id, static_cast<uint32_t>(len)) : PrgPrefixMatch{0, 0};
  return PRG_OK;
}

int prg_prefix_cache_contains(const PrgPrefixCache* c, const uint32_t* prompt, uint32_t prompt_len,
                              uint32_t prefix_len) {
  if (!c || (!prompt && prompt_len)) return 0;
  if (prefix_len == 0) return 1;
  if (prefix_len > prompt_len) return 0;
  return c->store.exact(prompt, prefix_len) != 0 ? 1 : 0;
}

int prg_prefix_cache_touch(PrgPrefixCache* c, PrgPrefixMatch match) {
  PRG_CHECK_ARG(c, "prg_prefix_cache_touch: null cache");
  uint64_t id = 0;
  if (int rc = match_id(c, match, &id)) return rc;
  mark_used(c, id);
  return PRG_OK;
}

int prg_prefix_cache_remove(PrgPrefixCache* c, uint32_t index) {
  const uint64_t id = c ? c->store.id_at(index) : 0;
  PRG_CHECK_ARG(id != 0, "prg_prefix_cache_remove: bad index");
  drop(c, id);
  return PRG_OK;
}

int prg_prefix_cache_entry_info(const PrgPrefixCache* c, uint32_t index, uint32_t* token_count, uint32_t* capacity,
                                int* pinned, uint64_t* hits) {
  const CachedPrefix* e = c ? c->store.get(c->store.id_at(index)) : nullptr;
  PRG_CHECK_ARG(e, "prg_prefix_cache_entry_info: bad index");
  if (token_count) *token_count = static_cast<uint32_t>(e->tokens.size());
  if (capacity) *capacity = e->reserved;
  if (pinned) *pinned = e->pinned ? 1 : 0;
  if (hits) *hits = e->hits;
  return PRG_OK;
}

int prg_prefix_cache_entry_tokens(const PrgPrefixCache* c, uint32_t index, uint32_t* tokens, uint32_t capacity) {
  const CachedPrefix* e = c && tokens ? c->store.get(c->store.id_at(index)) : nullptr;
  PRG_CHECK_ARG(e, "prg_prefix_cache_entry_tokens: bad argument");
  PRG_CHECK_ARG(capacity >= e->tokens.size(), "prg_prefix_cache_entry_tokens: buffer of %u < %zu", capacity,
                e->tokens.size());
  std::copy(e->tokens.begin(), e->tokens.end(), tokens);
  return PRG_OK;
}

int prg_prefix_cache_entry_state(PrgPrefixCache* c, uint32_t index, PrgModelState** state) {
  const CachedPrefix* e = c && state ? c->store.get(c->store.id_at(index)) : nullptr;
  PRG_CHECK_ARG(e, "prg_prefix_cache_entry_state: bad argument");
  PRG_CHECK_ARG(c->model, "prg_prefix_cache_entry_state: the cache was created without a model");
  *state = e->state;
  return PRG_OK;
}

int prg_prefix_cache_cached_next_token(const PrgPrefixCache* c, PrgPrefixMatch match, uint32_t* token, int* valid) {
  PRG_CHECK_ARG(c && token && valid, "prg_prefix_cache_cached_next_token: null argument");
  uint64_t id = 0;
  if (int rc = match_id(c, match, &id)) return rc;
  const CachedPrefix& e = *c->store.get(id);
  *token = e.next_token;
  *valid = e.next_valid ? 1 : 0;
  return PRG_OK;
}

int prg_prefix_cache_start_direct(PrgPrefixCache* c, const uint32_t* ids, uint32_t n, int pinned,
                                  PrgPrefixMatch* out) {
  PRG_CHECK_ARG(c && out && (ids || n == 0), "prg_prefix_cache_start_direct: null argument");
  uint64_t id = 0;
  if (int rc = admit(c, ids, n, 0, pinned != 0, &id)) return rc;
  CachedPrefix& e = *c->store.get(id);
  if (e.state)
    if (int rc = prg_model_state_reset(e.state)) return rc;
  e.next_valid = false;
  *out = match_of(c, id, n);
  return PRG_OK;
}

int prg_prefix_cache_finish_direct(PrgPrefixCache* c, PrgPrefixMatch match, uint32_t next_token) {
  PRG_CHECK_ARG(c, "prg_prefix_cache_finish_direct: null cache");
  uint64_t id = 0;
  if (int rc = match_id(c, match, &id)) return rc;
  CachedPrefix& e = *c->store.get(id);
  e.next_token = next_token;
  e.next_valid = true;
  mark_used(c, id);
  return PRG_OK;
}

int prg_prefix_cache_store(PrgPrefixCache* c, const uint32_t* ids, uint32_t n, const PrgPrefixMatch* reuse,
                           const PrgModelState* work, const uint16_t* work_hidden, uint32_t work_hidden_base_rows,
                           const uint32_t* next_token, int pinned, PrgPrefixMatch* out) {
  PRG_CHECK_ARG(c && out && (ids || n == 0), "prg_prefix_cache_store: null argument");
  PRG_CHECK_ARG(!c->model || (work && work->model == c->model), "prg_prefix_cache_store: work state of another model");
  uint64_t reuse_id = 0;
  if (reuse)
    if (int rc = match_id(c, *reuse, &reuse_id)) return rc;
  if (n == 0 || n > c->max_tokens)
    return set_error(PRG_ERR_SEQUENCE_TOO_LONG, "prefix cache: prefix of %u tokens (budget %llu)", n,
                     (unsigned long long)c->max_tokens);
  if (work) PRG_CHECK_ARG(n <= work->max_seq, "prg_prefix_cache_store: %u tokens > work capacity %u", n, work->max_seq);
  const bool already_cached = c->store.exact(ids, n) != 0;
  uint64_t id = 0;
  if (int rc = admit(c, ids, n, reuse_id, pinned != 0, &id)) return rc;
  CachedPrefix& e = *c->store.get(id);
  // The working state holds absolute positions [0, n) (a reused prefix was
  // copied into it first), so an entry continuing `reuse` only needs
  // positions [reuse_len, n) and the GDN state after token n.
  const uint32_t reuse_len = reuse ? std::min(reuse->len, n) : 0;
  if (!already_cached && e.state) {
    int rc = copy_attention_range(e.state, reuse_len, work, reuse_len, n - reuse_len);
    if (rc == PRG_OK) rc = copy_linear_state(e.state, work);
    if (rc) return rc;
  }
  if (c->track_hidden && c->model) {
    // rows [0, reuse_len) stay; rows [reuse_len, n) come from work_hidden
    const bool prefix_rows_valid = reuse_len == 0 || e.hidden_valid;
    if (int rc = ensure_hidden_rows(c, e)) return rc;
    const uint32_t fresh = n - reuse_len;
    const size_t rb = hidden_row_bytes(c);
    if (fresh) {
      char* dst = reinterpret_cast<char*>(e.hidden) + static_cast<size_t>(reuse_len) * rb;
      if (work_hidden)
        PRG_HIP(hipMemcpyAsync(dst, reinterpret_cast<const char*>(work_hidden) + work_hidden_base_rows * rb,
                               fresh * rb, hipMemcpyDeviceToDevice, c->stream));
      else
        PRG_HIP(hipMemsetAsync(dst, 0, fresh * rb, c->stream));
      PRG_HIP(hipStreamSynchronize(c->stream));
    }
    e.hidden_valid = prefix_rows_valid && (fresh == 0 || work_hidden != nullptr);
  }
  e.next_valid = next_token != nullptr;
  if (next_token) e.next_token = *next_token;
  mark_used(c, id);
  *out = match_of(c, id, n);
  return PRG_OK;
}

int prg_prefix_cache_restore(const PrgPrefixCache* c, PrgPrefixMatch match, PrgModelState* work) {
  PRG_CHECK_ARG(c && work, "prg_prefix_cache_restore: null argument");
  PRG_CHECK_ARG(c->model && work->model == c->model, "prg_prefix_cache_restore: work state of another model");
  uint64_t id = 0;
  if (int rc = match_id(c, match, &id)) return rc;
  const CachedPrefix& e = *c->store.get(id);
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
  uint64_t id = 0;
  if (int rc = match_id(c, match, &id)) return rc;
  const CachedPrefix& e = *c->store.get(id);
  *rows = e.hidden;
  *valid = e.hidden_valid ? 1 : 0;
  return PRG_OK;
}

int prg_prefix_cache_set_entry_hidden(PrgPrefixCache* c, PrgPrefixMatch match, const uint16_t* rows) {
  PRG_CHECK_ARG(c && rows && c->model, "prg_prefix_cache_set_entry_hidden: bad argument");
  uint64_t id = 0;
  if (int rc = match_id(c, match, &id)) return rc;
  CachedPrefix& e = *c->store.get(id);
  PRG_CHECK_ARG(match.len <= e.reserved, "prg_prefix_cache_set_entry_hidden: %u rows > capacity %u", match.len,
                e.reserved);
  if (int rc = ensure_hidden_rows(c, e)) return rc;
  PRG_HIP(hipMemcpyAsync(e.hidden, rows, match.len * hidden_row_bytes(c), hipMemcpyDeviceToDevice, c->stream));
  PRG_HIP(hipStreamSynchronize(c->stream));
  e.hidden_valid = true;
  return PRG_OK;
}

// save (prefix_persist.zig:253-328): temp file + rename.
int prg_prefix_cache_save(const PrgPrefixCache* c, const char* path, uint64_t model_fingerprint) {
  PRG_CHECK_ARG(c && path && c->model, "prg_prefix_cache_save: bad argument");
  const CachedPrefix* e = persisted_entry(c);
  if (!e || e->tokens.empty()) return set_error(PRG_ERR_EMPTY_INPUT, "EmptyPrefix: nothing cached");
  const uint32_t T = static_cast<uint32_t>(e->tokens.size());
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

// load (prefix_persist.zig:334-412). A missing or invalid file (header,
// length or tokens) leaves the cache unchanged and reports *loaded_tokens = 0
// (the reference returns null; prg_last_error() says why); a failure while
// reading the state sections clears the cache.
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

  std::vector<uint32_t> tokens(T);
  if (f.read_all(tokens.data(), sizeof(uint32_t) * T) != PRG_OK) return ignore("short token list");
  for (uint32_t t : tokens)
    if (t >= c->model->cfg.vocab) return ignore("token outside the vocab");

  // The file replaces the cache's contents with one pinned entry
  // (prefix_state_cache.zig:663-690), which becomes the active one.
  drop_all(c);
  uint64_t id = 0;
  int rc = admit(c, tokens.data(), T, 0, true, &id);
  std::vector<uint8_t> host;
  if (!rc) rc = read_state(f, c->store.get(id)->state, T, host);
  if (!rc) {
    CachedPrefix& ent = *c->store.get(id);
    ent.next_token = h.next_token;
    ent.next_valid = h.next_token_valid == 1;
    const size_t hb = static_cast<size_t>(T) * hidden_row_bytes(c);
    host.resize(hb);
    rc = f.read_all(host.data(), hb);
    if (!rc && c->track_hidden) {
      rc = ensure_hidden_rows(c, ent);
      if (!rc) {
        const hipError_t err = hipMemcpy(ent.hidden, host.data(), hb, hipMemcpyHostToDevice);
        if (err != hipSuccess) rc = set_error(PRG_ERR_HIP, "hidden rows: %s", hipGetErrorString(err));
      }
      ent.hidden_valid = h.hidden_valid == 1;
    }
    c->active = id;
  }
  if (rc) {
    drop_all(c);
    return rc;
  }
  *loaded_tokens = T;
  return PRG_OK;
}

}  // extern "C"
