// Model upload from an MLX safetensors checkpoint.
//
// Reference: DeviceModel.upload (src/model/model.zig:580-658),
// DecoderLayer.upload (src/model/decoder_layer.zig:376-412),
// LinearAttentionBlock.upload (src/model/block_linear.zig:155-186),
// FullAttentionBlock.upload (src/model/block_attn.zig:235-255),
// Q4Linear.upload (src/model/linear_q4.zig:28-63, shape check :261-268),
// Drafter.upload and detectRoot (src/model/mtp.zig:86-116, 347-355),
// upload.tensorPrivate (src/model/upload.zig:6-21).
//
// The reference preads each tensor into a shared staging buffer and blits it
// into a private buffer, one tensor at a time. Here the model's tensors are
// one device arena laid out exactly as for a random model; each tensor is read
// in chunks into two pinned staging buffers that alternate, so the pread of
// chunk i+1 overlaps the DMA of chunk i.
#include <stdlib.h>
#include <string.h>

#include <memory>

#include "checkpoint.hpp"
#include "model.hpp"

namespace prg {
namespace {

uint64_t elements(const std::vector<uint64_t>& shape) {
  uint64_t n = 1;
  for (uint64_t d : shape) {
    if (d != 0 && n > UINT64_MAX / d) return UINT64_MAX;
    n *= d;
  }
  return n;
}

std::string shape_str(const std::vector<uint64_t>& s) {
  std::string o = "[";
  for (size_t k = 0; k < s.size(); ++k) {
    if (k) o += ", ";
    o += std::to_string(s[k]);
  }
  return o + "]";
}

class Staging {
 public:
  static constexpr size_t kChunk = size_t(64) << 20;

  ~Staging() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (int k = 0; k < 2; ++k) {
      if (ev_[k]) (void)hipEventDestroy(ev_[k]);
      if (buf_[k]) (void)hipHostFree(buf_[k]);
    }
    if (stream_) (void)hipStreamDestroy(stream_);
  }

  int init() {
    PRG_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    for (int k = 0; k < 2; ++k) {
      PRG_HIP(hipHostMalloc(&buf_[k], kChunk, hipHostMallocDefault));
      PRG_HIP(hipEventCreateWithFlags(&ev_[k], hipEventDisableTiming));
    }
    return PRG_OK;
  }

  // File bytes of tensor t -> device dst.
  int file_to_device(const StRepo& repo, const StTensor& t, uint64_t len, void* dst) {
    for (uint64_t off = 0; off < len; off += kChunk) {
      const size_t n = static_cast<size_t>(std::min<uint64_t>(kChunk, len - off));
      if (int rc = acquire()) return rc;
      if (int rc = repo.read(t, off, buf_[cur_], n)) return rc;
      if (int rc = submit(static_cast<char*>(dst) + off, n)) return rc;
    }
    return PRG_OK;
  }

  // Host bytes -> device dst (small tensors converted on the host).
  int host_to_device(const void* src, size_t len, void* dst) {
    for (size_t off = 0; off < len; off += kChunk) {
      const size_t n = std::min(kChunk, len - off);
      if (int rc = acquire()) return rc;
      memcpy(buf_[cur_], static_cast<const char*>(src) + off, n);
      if (int rc = submit(static_cast<char*>(dst) + off, n)) return rc;
    }
    return PRG_OK;
  }

  int finish() {
    PRG_HIP(hipStreamSynchronize(stream_));
    return PRG_OK;
  }

 private:
  void* buf_[2] = {nullptr, nullptr};
  hipEvent_t ev_[2] = {nullptr, nullptr};
  bool pending_[2] = {false, false};
  hipStream_t stream_ = nullptr;
  int cur_ = 0;

  // Wait until the current buffer's previous copy has drained.
  int acquire() {
    if (pending_[cur_]) {
      PRG_HIP(hipEventSynchronize(ev_[cur_]));
      pending_[cur_] = false;
    }
    return PRG_OK;
  }
  int submit(void* dst, size_t n) {
    PRG_HIP(hipMemcpyAsync(dst, buf_[cur_], n, hipMemcpyHostToDevice, stream_));
    PRG_HIP(hipEventRecord(ev_[cur_], stream_));
    pending_[cur_] = true;
    cur_ ^= 1;
    return PRG_OK;
  }
};

// One tensor: presence, dtype, shape and byte-length checks, then upload.
int upload_tensor(Staging& stg, const StRepo& repo, const std::string& src_name, const std::string& name,
                  const TensorRef& ref, const TensorSpec& spec) {
  const StTensor* t = repo.get(src_name);
  if (!t) return set_error(PRG_ERR_NOT_FOUND, "TensorNotFound: %s", src_name.c_str());
  uint64_t off = 0, len = 0;
  if (int rc = repo.range(*t, &off, &len)) return rc;
  const bool q4_weight = spec.dtype == "U32";
  const bool widen = (name.size() >= 6 && name.compare(name.size() - 6, 6, ".A_log") == 0) && t->dtype == "BF16";
  if (q4_weight) {
    // q4WeightDims (linear_q4.zig:261-268) plus the model's expected shape;
    // the embedding's vocab comes from its row count (model.zig:98-104).
    if (t->shape.size() != 2 || t->shape[0] == 0 || t->shape[1] == 0)
      return set_error(PRG_ERR_UNSUPPORTED, "UnsupportedQuantization: %s has shape %s", src_name.c_str(),
                       shape_str(t->shape).c_str());
    if (t->shape != spec.shape)
      return set_error(PRG_ERR_MALFORMED, "InvalidTensorShape: %s is %s, the model expects %s", src_name.c_str(),
                       shape_str(t->shape).c_str(), shape_str(spec.shape).c_str());
  } else if (elements(t->shape) != elements(spec.shape)) {
    return set_error(PRG_ERR_MALFORMED, "InvalidTensorShape: %s is %s, the model expects %s", src_name.c_str(),
                     shape_str(t->shape).c_str(), shape_str(spec.shape).c_str());
  }
  if (t->dtype != spec.dtype && !widen)
    return set_error(PRG_ERR_MALFORMED, "InvalidTensorShape: %s has dtype %s, the model expects %s", src_name.c_str(),
                     t->dtype.c_str(), spec.dtype.c_str());
  const uint64_t want = elements(t->shape) * st_dtype_size(t->dtype);
  if (len != want)
    return set_error(PRG_ERR_MALFORMED, "MalformedHeader: %s spans %llu bytes, %s %s needs %llu", src_name.c_str(),
                     (unsigned long long)len, t->dtype.c_str(), shape_str(t->shape).c_str(),
                     (unsigned long long)want);
  if (widen) {  // bf16 A_log -> the f32 vector the GDN kernels read
    std::vector<uint16_t> raw(static_cast<size_t>(len / 2));
    if (int rc = repo.read(*t, 0, raw.data(), len)) return rc;
    std::vector<float> f(raw.size());
    for (size_t k = 0; k < raw.size(); ++k) {
      const uint32_t bits = static_cast<uint32_t>(raw[k]) << 16;
      memcpy(&f[k], &bits, sizeof(float));
    }
    if (f.size() * sizeof(float) != ref.bytes)
      return set_error(PRG_ERR_MALFORMED, "InvalidTensorShape: %s", src_name.c_str());
    return stg.host_to_device(f.data(), ref.bytes, ref.ptr);
  }
  if (len != ref.bytes)
    return set_error(PRG_ERR_MALFORMED, "InvalidTensorShape: %s is %llu bytes, the model expects %zu",
                     src_name.c_str(), (unsigned long long)len, ref.bytes);
  return stg.file_to_device(repo, *t, len, ref.ptr);
}

int upload_checkpoint(PrgModel* m, const char* target_dir, const char* mtp_dir) {
  std::unique_ptr<StRepo> target, mtp;
  if (int rc = st_open(target_dir, &target)) return rc;
  std::string root;
  if (m->cfg.mtp_layers) {
    if (int rc = st_open(mtp_dir, &mtp)) return rc;
    static const char* const kRoots[] = {"", "mtp.", "language_model.mtp.", "model.mtp."};
    bool found = false;
    for (const char* r : kRoots) {
      if (mtp->get(std::string(r) + "fc.weight")) {
        root = r;
        found = true;
        break;
      }
    }
    if (!found) return set_error(PRG_ERR_NOT_FOUND, "TensorNotFound: no MTP fc.weight under any known root in %s", mtp_dir);
  }
  Staging stg;
  if (int rc = stg.init()) return rc;
  for (const auto& kv : m->tensors) {
    const std::string& name = kv.first;
    const bool is_mtp = name.compare(0, 4, "mtp.") == 0;
    const StRepo& repo = is_mtp ? *mtp : *target;
    const std::string src = is_mtp ? root + name.substr(4) : name;
    if (int rc = upload_tensor(stg, repo, src, name, kv.second, m->specs.at(name))) return rc;
  }
  return stg.finish();
}

}  // namespace
}  // namespace prg

using namespace prg;

extern "C" int prg_model_load(const PrgModelConfig* cfg, const char* target_dir, const char* mtp_dir, PrgModel** out) {
  PRG_CHECK_ARG(cfg && target_dir && out, "prg_model_load: null argument");
  *out = nullptr;
  if (int rc = validate_model_config(*cfg)) return rc;
  PRG_CHECK_ARG((cfg->mtp_layers != 0) == (mtp_dir != nullptr),
                "prg_model_load: mtp_dir must be given exactly when cfg->mtp_layers is 1");
  auto* m = new PrgModel();
  m->cfg = *cfg;
  if (const char* e = getenv("PEREGRINE_T16")) m->t16_enabled = e[0] != '0';
  int rc = layout_model(m);
  if (rc == PRG_OK) rc = upload_checkpoint(m, target_dir, mtp_dir);
  if (rc == PRG_OK) rc = prepare_t16(m);
  if (rc != PRG_OK) {
    prg_model_destroy(m);
    return rc;
  }
  *out = m;
  return PRG_OK;
}
