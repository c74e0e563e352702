// Safetensors repository and config.json checks (host code; no kernels).
//
// Error messages start with the reference's error name (TruncatedHeader,
// MalformedHeader, MalformedIndex, NoShardsFound, TensorNotFound,
// UnsupportedArchitecture, UnsupportedQuantization, InvalidConfig,
// NotQwen35_9B, ...) so callers can match them to the Zig error sets.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <set>

#include "checkpoint.hpp"
#include "common.hpp"
#include "json.hpp"

namespace prg {

StRepo::~StRepo() {
  for (int fd : fds)
    if (fd >= 0) close(fd);
}

const StTensor* StRepo::get(const std::string& name) const {
  auto it = tensors.find(name);
  return it == tensors.end() ? nullptr : &it->second;
}

int StRepo::range(const StTensor& t, uint64_t* file_off, uint64_t* len) const {
  if (t.shard >= fds.size()) return set_error(PRG_ERR_MALFORMED, "MalformedHeader: shard index %u", t.shard);
  if (t.begin > t.end) return set_error(PRG_ERR_MALFORMED, "MalformedHeader: data_offsets [%llu, %llu]",
                                        (unsigned long long)t.begin, (unsigned long long)t.end);
  const uint64_t size = shard_bytes[t.shard], start = data_start[t.shard];
  if (start > size || t.end > size - start)
    return set_error(PRG_ERR_MALFORMED, "MalformedHeader: tensor bytes [%llu, %llu) past the end of %s",
                     (unsigned long long)t.begin, (unsigned long long)t.end, shard_names[t.shard].c_str());
  *file_off = start + t.begin;
  *len = t.end - t.begin;
  return PRG_OK;
}

int StRepo::read(const StTensor& t, uint64_t off, void* dst, uint64_t len) const {
  uint64_t base = 0, total = 0;
  if (int rc = range(t, &base, &total)) return rc;
  if (off > total || len > total - off)
    return set_error(PRG_ERR_INVALID_ARG, "InvalidTensorBuffer: read [%llu, +%llu) of a %llu-byte tensor",
                     (unsigned long long)off, (unsigned long long)len, (unsigned long long)total);
  uint64_t done = 0;
  auto* p = static_cast<char*>(dst);
  while (done < len) {
    const size_t want = static_cast<size_t>(std::min<uint64_t>(len - done, uint64_t(1) << 30));
    const ssize_t n = pread(fds[t.shard], p + done, want, static_cast<off_t>(base + off + done));
    if (n < 0) {
      if (errno == EINTR) continue;
      return set_error(PRG_ERR_IO, "read %s: %s", shard_names[t.shard].c_str(), strerror(errno));
    }
    if (n == 0) return set_error(PRG_ERR_IO, "UnexpectedEof: %s", shard_names[t.shard].c_str());
    done += static_cast<uint64_t>(n);
  }
  return PRG_OK;
}

size_t st_dtype_size(const std::string& d) {
  if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E5M2" || d == "F8_E4M3") return 1;
  if (d == "I16" || d == "U16" || d == "F16" || d == "BF16") return 2;
  if (d == "I32" || d == "U32" || d == "F32") return 4;
  if (d == "I64" || d == "U64" || d == "F64") return 8;
  return 0;
}

int read_text_file(const std::string& path, size_t limit, std::string* out) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    if (errno == ENOENT) return set_error(PRG_ERR_NOT_FOUND, "FileNotFound: %s", path.c_str());
    return set_error(PRG_ERR_IO, "open %s: %s", path.c_str(), strerror(errno));
  }
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    close(fd);
    return set_error(PRG_ERR_IO, "stat %s: %s", path.c_str(), strerror(errno));
  }
  if (static_cast<uint64_t>(sb.st_size) > limit) {
    close(fd);
    return set_error(PRG_ERR_MALFORMED, "StreamTooLong: %s is %lld bytes (limit %zu)", path.c_str(),
                     (long long)sb.st_size, limit);
  }
  out->assign(static_cast<size_t>(sb.st_size), '\0');
  size_t done = 0;
  while (done < out->size()) {
    const ssize_t n = pread(fd, &(*out)[done], out->size() - done, static_cast<off_t>(done));
    if (n < 0 && errno == EINTR) continue;
    if (n <= 0) {
      close(fd);
      return set_error(PRG_ERR_IO, "read %s failed", path.c_str());
    }
    done += static_cast<size_t>(n);
  }
  close(fd);
  return PRG_OK;
}

namespace {

// discoverShards (safetensors.zig:144-177): the unique values of the index's
// weight_map, sorted bytewise.
int discover_shards(const std::string& dir, std::vector<std::string>* names) {
  std::string text;
  if (int rc = read_text_file(dir + "/model.safetensors.index.json", size_t(64) << 20, &text)) return rc;
  json::Value root;
  std::string err;
  if (!json::parse(text.data(), text.size(), root, err))
    return set_error(PRG_ERR_MALFORMED, "MalformedIndex: %s", err.c_str());
  const json::Value* wm = root.is_object() ? root.get("weight_map") : nullptr;
  if (!wm || !wm->is_object()) return set_error(PRG_ERR_MALFORMED, "MalformedIndex: no weight_map object");
  std::set<std::string> seen;
  for (const auto& kv : wm->obj) {
    if (!kv.second.is_string()) return set_error(PRG_ERR_MALFORMED, "MalformedIndex: weight_map value not a string");
    seen.insert(kv.second.s);
  }
  if (seen.empty()) return set_error(PRG_ERR_MALFORMED, "NoShardsFound: empty weight_map");
  names->assign(seen.begin(), seen.end());  // std::set orders bytewise
  for (const auto& n : *names)
    if (n.empty() || n.find('/') != std::string::npos || n == "." || n == "..")
      return set_error(PRG_ERR_MALFORMED, "MalformedIndex: shard name '%s'", n.c_str());
  return PRG_OK;
}

// parseHeader (safetensors.zig:189-220).
int parse_header(const std::string& header, uint32_t shard, const std::string& shard_name,
                 std::map<std::string, StTensor>* tensors) {
  json::Value root;
  std::string err;
  if (!json::parse(header.data(), header.size(), root, err))
    return set_error(PRG_ERR_MALFORMED, "MalformedHeader: %s: %s", shard_name.c_str(), err.c_str());
  if (!root.is_object()) return set_error(PRG_ERR_MALFORMED, "MalformedHeader: %s: not an object", shard_name.c_str());
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const json::Value& o = kv.second;
    const json::Value* shape = o.is_object() ? o.get("shape") : nullptr;
    const json::Value* offs = o.is_object() ? o.get("data_offsets") : nullptr;
    const json::Value* dtype = o.is_object() ? o.get("dtype") : nullptr;
    if (!shape || !shape->is_array() || !offs || !offs->is_array() || offs->arr.size() != 2)
      return set_error(PRG_ERR_MALFORMED, "MalformedHeader: %s: entry '%s'", shard_name.c_str(), kv.first.c_str());
    StTensor t;
    t.shard = shard;
    t.dtype = (dtype && dtype->is_string()) ? dtype->s : std::string();
    for (const auto& d : shape->arr) {
      uint64_t v = 0;
      if (!d.as_u64(&v))
        return set_error(PRG_ERR_MALFORMED, "MalformedHeader: %s: shape of '%s'", shard_name.c_str(), kv.first.c_str());
      t.shape.push_back(v);
    }
    if (!offs->arr[0].as_u64(&t.begin) || !offs->arr[1].as_u64(&t.end))
      return set_error(PRG_ERR_MALFORMED, "MalformedHeader: %s: data_offsets of '%s'", shard_name.c_str(),
                       kv.first.c_str());
    (*tensors)[kv.first] = std::move(t);
  }
  return PRG_OK;
}

}  // namespace

int st_open(const std::string& dir, std::unique_ptr<StRepo>* out) {
  auto repo = std::make_unique<StRepo>();
  if (int rc = discover_shards(dir, &repo->shard_names)) return rc;
  for (uint32_t s = 0; s < repo->shard_names.size(); ++s) {
    const std::string path = dir + "/" + repo->shard_names[s];
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
      if (errno == ENOENT) return set_error(PRG_ERR_NOT_FOUND, "FileNotFound: %s", path.c_str());
      return set_error(PRG_ERR_IO, "open %s: %s", path.c_str(), strerror(errno));
    }
    repo->fds.push_back(fd);
    struct stat sb;
    if (fstat(fd, &sb) != 0) return set_error(PRG_ERR_IO, "stat %s: %s", path.c_str(), strerror(errno));
    const uint64_t size = static_cast<uint64_t>(sb.st_size);
    repo->shard_bytes.push_back(size);
    if (size < 8) return set_error(PRG_ERR_MALFORMED, "TruncatedHeader: %s is %llu bytes", path.c_str(),
                                   (unsigned long long)size);
    uint8_t lenb[8];
    if (pread(fd, lenb, 8, 0) != 8) return set_error(PRG_ERR_IO, "read %s failed", path.c_str());
    uint64_t header_len = 0;
    for (int k = 7; k >= 0; --k) header_len = (header_len << 8) | lenb[k];  // little-endian u64
    if (header_len > size - 8)
      return set_error(PRG_ERR_MALFORMED, "TruncatedHeader: %s: header length %llu, file %llu bytes", path.c_str(),
                       (unsigned long long)header_len, (unsigned long long)size);
    if (header_len > (uint64_t(100) << 20))
      return set_error(PRG_ERR_MALFORMED, "MalformedHeader: %s: header length %llu exceeds 100 MiB", path.c_str(),
                       (unsigned long long)header_len);
    repo->data_start.push_back(8 + header_len);
    std::string header(static_cast<size_t>(header_len), '\0');
    size_t done = 0;
    while (done < header.size()) {
      const ssize_t n = pread(fd, &header[done], header.size() - done, static_cast<off_t>(8 + done));
      if (n < 0 && errno == EINTR) continue;
      if (n <= 0) return set_error(PRG_ERR_IO, "read %s failed", path.c_str());
      done += static_cast<size_t>(n);
    }
    if (int rc = parse_header(header, s, repo->shard_names[s], &repo->tensors)) return rc;
  }
  *out = std::move(repo);
  return PRG_OK;
}

namespace {

int load_config_json(const std::string& dir, json::Value* root) {
  std::string text;
  if (int rc = read_text_file(dir + "/config.json", size_t(4) << 20, &text)) return rc;
  std::string err;
  if (!json::parse(text.data(), text.size(), *root, err))
    return set_error(PRG_ERR_MALFORMED, "SyntaxError: config.json: %s", err.c_str());
  if (!root->is_object()) return set_error(PRG_ERR_MALFORMED, "UnexpectedToken: config.json is not an object");
  return PRG_OK;
}

// A u32 field as std.json parses it into a struct: required unless a default
// is given; negative, fractional or > u32 values are errors.
int u32_field(const json::Value& obj, const char* parent, const char* key, bool required, uint32_t* out) {
  const json::Value* v = obj.is_object() ? obj.get(key) : nullptr;
  if (!v) {
    if (required) return set_error(PRG_ERR_MALFORMED, "MissingField: %s.%s", parent, key);
    *out = 0;
    return PRG_OK;
  }
  uint64_t u = 0;
  if (!v->as_u64(&u) || u > 0xffffffffull)
    return set_error(PRG_ERR_MALFORMED, "InvalidNumber: %s.%s", parent, key);
  *out = static_cast<uint32_t>(u);
  return PRG_OK;
}

std::string str_field(const json::Value& obj, const char* key) {
  const json::Value* v = obj.is_object() ? obj.get(key) : nullptr;
  return (v && v->is_string()) ? v->s : std::string();
}

struct TextConfig {
  std::string model_type;
  uint32_t hidden_size, intermediate_size, num_hidden_layers, num_attention_heads, num_key_value_heads, head_dim,
      full_attention_interval, linear_num_key_heads, linear_num_value_heads, linear_key_head_dim,
      linear_value_head_dim, linear_conv_kernel_dim, vocab_size;
  double partial_rotary_factor = 0.25;
  double rms_norm_eps = 1e-6;
  double rope_theta = 0.0;  // 0 = absent
  std::string quant_mode;
  uint32_t quant_bits = 0, quant_group = 0;
};

// RawConfig of config.zig:6-31 (every text_config field required).
int parse_text_config(const json::Value& root, TextConfig* c) {
  const json::Value* tc = root.get("text_config");
  if (!tc || !tc->is_object()) return set_error(PRG_ERR_MALFORMED, "MissingField: text_config");
  const json::Value* q = root.get("quantization");
  if (!q || !q->is_object()) return set_error(PRG_ERR_MALFORMED, "MissingField: quantization");
  c->model_type = str_field(*tc, "model_type");
  struct F {
    const char* key;
    uint32_t* dst;
  } fields[] = {{"hidden_size", &c->hidden_size},
                {"intermediate_size", &c->intermediate_size},
                {"num_hidden_layers", &c->num_hidden_layers},
                {"num_attention_heads", &c->num_attention_heads},
                {"num_key_value_heads", &c->num_key_value_heads},
                {"head_dim", &c->head_dim},
                {"full_attention_interval", &c->full_attention_interval},
                {"linear_num_key_heads", &c->linear_num_key_heads},
                {"linear_num_value_heads", &c->linear_num_value_heads},
                {"linear_key_head_dim", &c->linear_key_head_dim},
                {"linear_value_head_dim", &c->linear_value_head_dim},
                {"linear_conv_kernel_dim", &c->linear_conv_kernel_dim},
                {"vocab_size", &c->vocab_size}};
  for (const F& f : fields)
    if (int rc = u32_field(*tc, "text_config", f.key, true, f.dst)) return rc;
  if (const json::Value* rp = tc->get("rope_parameters")) {
    if (rp->is_object()) {
      if (const json::Value* prf = rp->get("partial_rotary_factor")) {
        if (!prf->is_number()) return set_error(PRG_ERR_MALFORMED, "InvalidNumber: partial_rotary_factor");
        c->partial_rotary_factor = prf->as_double();
      }
      if (const json::Value* th = rp->get("rope_theta"))
        if (th->is_number()) c->rope_theta = th->as_double();
    }
  }
  if (const json::Value* eps = tc->get("rms_norm_eps"))
    if (eps->is_number()) c->rms_norm_eps = eps->as_double();
  c->quant_mode = str_field(*q, "mode");
  if (int rc = u32_field(*q, "quantization", "group_size", true, &c->quant_group)) return rc;
  if (int rc = u32_field(*q, "quantization", "bits", true, &c->quant_bits)) return rc;
  if (!q->get("mode") || !q->get("mode")->is_string()) return set_error(PRG_ERR_MALFORMED, "MissingField: quantization.mode");
  return PRG_OK;
}

// The generic checks of verifyFingerprint (config.zig:44-56), before the
// exact-shape test.
int check_text_config(const TextConfig& c, uint32_t* rotary_dim) {
  if (c.model_type != "qwen3_5_text")
    return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedArchitecture: model_type '%s'", c.model_type.c_str());
  if (c.quant_mode != "affine")
    return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedQuantization: mode '%s'", c.quant_mode.c_str());
  if (c.quant_bits != 4 || c.quant_group != 64)
    return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedQuantization: bits %u group_size %u", c.quant_bits,
                     c.quant_group);
  if (c.num_attention_heads == 0 || c.num_key_value_heads == 0)
    return set_error(PRG_ERR_UNSUPPORTED, "InvalidConfig: zero attention heads");
  if (c.num_attention_heads % c.num_key_value_heads != 0)
    return set_error(PRG_ERR_UNSUPPORTED, "InvalidConfig: %u heads over %u kv heads", c.num_attention_heads,
                     c.num_key_value_heads);
  if (c.full_attention_interval == 0) return set_error(PRG_ERR_UNSUPPORTED, "InvalidConfig: full_attention_interval 0");
  if (c.num_hidden_layers == 0) return set_error(PRG_ERR_UNSUPPORTED, "InvalidConfig: num_hidden_layers 0");
  if (c.head_dim == 0) return set_error(PRG_ERR_UNSUPPORTED, "InvalidConfig: head_dim 0");
  const double rd = std::round(c.partial_rotary_factor * static_cast<double>(c.head_dim));
  if (!(rd >= 1.0) || rd > static_cast<double>(c.head_dim))
    return set_error(PRG_ERR_UNSUPPORTED, "InvalidConfig: rotary dim %g of head_dim %u", rd, c.head_dim);
  *rotary_dim = static_cast<uint32_t>(rd);
  return PRG_OK;
}

}  // namespace

int verify_config(const std::string& dir) {
  json::Value root;
  if (int rc = load_config_json(dir, &root)) return rc;
  TextConfig c{};
  if (int rc = parse_text_config(root, &c)) return rc;
  uint32_t rot = 0;
  if (int rc = check_text_config(c, &rot)) return rc;
  const bool is_9b = c.hidden_size == 4096 && c.intermediate_size == 12288 && c.num_hidden_layers == 32 &&
                     c.num_attention_heads == 16 && c.num_key_value_heads == 4 && c.head_dim == 256 && rot == 64 &&
                     c.full_attention_interval == 4 && c.linear_num_key_heads == 16 &&
                     c.linear_num_value_heads == 32 && c.linear_key_head_dim == 128 &&
                     c.linear_value_head_dim == 128 && c.linear_conv_kernel_dim == 4 && c.vocab_size == 248320;
  if (!is_9b) return set_error(PRG_ERR_UNSUPPORTED, "NotQwen35_9B: config.json describes another shape");
  return PRG_OK;
}

int read_model_config(const std::string& dir, PrgModelConfig* cfg) {
  json::Value root;
  if (int rc = load_config_json(dir, &root)) return rc;
  TextConfig c{};
  if (int rc = parse_text_config(root, &c)) return rc;
  uint32_t rot = 0;
  if (int rc = check_text_config(c, &rot)) return rc;
  // The kernels implement one head geometry (attention 16 q / 4 kv heads of
  // 256 with RoPE on 64 dims, theta 1e7; GDN 16 k / 32 v heads of 128, conv 4).
  const bool heads_ok = c.num_attention_heads == 16 && c.num_key_value_heads == 4 && c.head_dim == 256 &&
                        rot == 64 && c.linear_num_key_heads == 16 && c.linear_num_value_heads == 32 &&
                        c.linear_key_head_dim == 128 && c.linear_value_head_dim == 128 &&
                        c.linear_conv_kernel_dim == 4 && (c.rope_theta == 0.0 || c.rope_theta == 1e7);
  if (!heads_ok)
    return set_error(PRG_ERR_UNSUPPORTED,
                     "UnsupportedArchitecture: head geometry differs from 16x256 (kv 4, rotary 64, theta 1e7) "
                     "attention and 16/32x128 GDN with conv 4");
  prg_model_default_config(cfg);
  cfg->num_layers = c.num_hidden_layers;
  cfg->hidden = c.hidden_size;
  cfg->intermediate = c.intermediate_size;
  cfg->vocab = c.vocab_size;
  cfg->full_attention_interval = c.full_attention_interval;
  cfg->rms_eps = static_cast<float>(c.rms_norm_eps);
  cfg->mtp_layers = 0;
  return PRG_OK;
}

// mtp.zig:318-345 (every field optional; quantization falls back to
// quantization_config when bits is 0).
int verify_mtp_config(const std::string& dir) {
  json::Value root;
  if (int rc = load_config_json(dir, &root)) return rc;
  const json::Value empty;
  const json::Value* tcp = root.get("text_config");
  const json::Value& tc = (tcp && tcp->is_object()) ? *tcp : empty;
  auto quant = [&](const char* key, std::string* mode, uint32_t* bits, uint32_t* group) -> int {
    const json::Value* q = root.get(key);
    const json::Value& qq = (q && q->is_object()) ? *q : empty;
    *mode = str_field(qq, "mode");
    if (int rc = u32_field(qq, key, "bits", false, bits)) return rc;
    return u32_field(qq, key, "group_size", false, group);
  };
  std::string mode;
  uint32_t bits = 0, group = 0;
  if (int rc = quant("quantization", &mode, &bits, &group)) return rc;
  if (bits == 0)
    if (int rc = quant("quantization_config", &mode, &bits, &group)) return rc;
  uint32_t hidden, inter, mtp_layers, heads, kv, head_dim, vocab;
  struct F {
    const char* key;
    uint32_t* dst;
  } fields[] = {{"hidden_size", &hidden}, {"intermediate_size", &inter}, {"mtp_num_hidden_layers", &mtp_layers},
                {"num_attention_heads", &heads}, {"num_key_value_heads", &kv}, {"head_dim", &head_dim},
                {"vocab_size", &vocab}};
  for (const F& f : fields)
    if (int rc = u32_field(tc, "text_config", f.key, false, f.dst)) return rc;
  if (str_field(root, "model_type") != "qwen3_5_mtp")
    return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedArchitecture: model_type '%s'", str_field(root, "model_type").c_str());
  if (str_field(tc, "model_type") != "qwen3_5_text")
    return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedArchitecture: text_config.model_type '%s'",
                     str_field(tc, "model_type").c_str());
  if (mtp_layers != 1) return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedArchitecture: mtp_num_hidden_layers %u", mtp_layers);
  if (mode != "affine") return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedQuantization: mode '%s'", mode.c_str());
  if (bits != 4 || group != 64)
    return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedQuantization: bits %u group_size %u", bits, group);
  if (hidden != 4096 || inter != 12288 || heads != 16 || kv != 4 || head_dim != 256 || vocab != 248320)
    return set_error(PRG_ERR_UNSUPPORTED, "NotQwen35_9B: MTP config describes another shape");
  return PRG_OK;
}

}  // namespace prg

struct PrgSafetensors {
  std::unique_ptr<prg::StRepo> repo;
  std::vector<std::string> names;  // sorted
};

using prg::set_error;

extern "C" {

int prg_safetensors_open(const char* dir, PrgSafetensors** out) {
  PRG_CHECK_ARG(dir && out, "prg_safetensors_open: null argument");
  *out = nullptr;
  std::unique_ptr<prg::StRepo> repo;
  if (int rc = prg::st_open(dir, &repo)) return rc;
  auto* h = new PrgSafetensors();
  h->repo = std::move(repo);
  for (const auto& kv : h->repo->tensors) h->names.push_back(kv.first);
  *out = h;
  return PRG_OK;
}

void prg_safetensors_close(PrgSafetensors* st) { delete st; }

uint32_t prg_safetensors_tensor_count(const PrgSafetensors* st) {
  return st ? static_cast<uint32_t>(st->names.size()) : 0u;
}

uint32_t prg_safetensors_shard_count(const PrgSafetensors* st) {
  return st ? static_cast<uint32_t>(st->repo->shard_names.size()) : 0u;
}

int prg_safetensors_shard_name(const PrgSafetensors* st, uint32_t index, char* buf, size_t len) {
  PRG_CHECK_ARG(st && buf && len, "prg_safetensors_shard_name: null argument");
  PRG_CHECK_ARG(index < st->repo->shard_names.size(), "prg_safetensors_shard_name: index %u", index);
  const std::string& n = st->repo->shard_names[index];
  PRG_CHECK_ARG(n.size() < len, "prg_safetensors_shard_name: buffer of %zu bytes too small", len);
  memcpy(buf, n.c_str(), n.size() + 1);
  return PRG_OK;
}

int prg_safetensors_tensor_name(const PrgSafetensors* st, uint32_t index, char* buf, size_t len) {
  PRG_CHECK_ARG(st && buf && len, "prg_safetensors_tensor_name: null argument");
  PRG_CHECK_ARG(index < st->names.size(), "prg_safetensors_tensor_name: index %u", index);
  const std::string& n = st->names[index];
  PRG_CHECK_ARG(n.size() < len, "prg_safetensors_tensor_name: buffer of %zu bytes too small", len);
  memcpy(buf, n.c_str(), n.size() + 1);
  return PRG_OK;
}

int prg_safetensors_tensor_info(const PrgSafetensors* st, const char* name, char* dtype, size_t dtype_len,
                                uint64_t* shape, uint32_t max_dims, uint32_t* ndim, uint64_t* bytes,
                                uint32_t* shard) {
  PRG_CHECK_ARG(st && name && ndim && bytes, "prg_safetensors_tensor_info: null argument");
  const prg::StTensor* t = st->repo->get(name);
  if (!t) return set_error(PRG_ERR_NOT_FOUND, "TensorNotFound: %s", name);
  uint64_t off = 0, len = 0;
  if (int rc = st->repo->range(*t, &off, &len)) return rc;
  *ndim = static_cast<uint32_t>(t->shape.size());
  *bytes = len;
  if (shard) *shard = t->shard;
  if (shape) {
    PRG_CHECK_ARG(t->shape.size() <= max_dims, "prg_safetensors_tensor_info: %zu dims > %u", t->shape.size(), max_dims);
    for (size_t k = 0; k < t->shape.size(); ++k) shape[k] = t->shape[k];
  }
  if (dtype) {
    PRG_CHECK_ARG(t->dtype.size() < dtype_len, "prg_safetensors_tensor_info: dtype buffer too small");
    memcpy(dtype, t->dtype.c_str(), t->dtype.size() + 1);
  }
  return PRG_OK;
}

int prg_safetensors_read(const PrgSafetensors* st, const char* name, void* dst, uint64_t bytes) {
  PRG_CHECK_ARG(st && name && dst, "prg_safetensors_read: null argument");
  const prg::StTensor* t = st->repo->get(name);
  if (!t) return set_error(PRG_ERR_NOT_FOUND, "TensorNotFound: %s", name);
  uint64_t off = 0, len = 0;
  if (int rc = st->repo->range(*t, &off, &len)) return rc;
  if (bytes != len)
    return set_error(PRG_ERR_INVALID_ARG, "InvalidTensorBuffer: %s is %llu bytes, buffer %llu", name,
                     (unsigned long long)len, (unsigned long long)bytes);
  return st->repo->read(*t, 0, dst, len);
}

int prg_checkpoint_verify_config(const char* dir) {
  PRG_CHECK_ARG(dir, "prg_checkpoint_verify_config: null argument");
  return prg::verify_config(dir);
}

int prg_checkpoint_verify_mtp_config(const char* dir) {
  PRG_CHECK_ARG(dir, "prg_checkpoint_verify_mtp_config: null argument");
  return prg::verify_mtp_config(dir);
}

int prg_checkpoint_read_config(const char* dir, PrgModelConfig* cfg) {
  PRG_CHECK_ARG(dir && cfg, "prg_checkpoint_read_config: null argument");
  return prg::read_model_config(dir, cfg);
}

}  // extern "C"
