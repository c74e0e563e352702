// Checkpoint reading on the host: the safetensors shard repository and the
// config.json checks of the reference.
//
//   StRepo            src/model/safetensors.zig:17-141 (Repository: open,
//                     get, tensorByteLen, readInto)
//   st_open           safetensors.zig:25-77, discoverShards :144-177,
//                     parseHeader :189-220
//   verify_config     src/model/config.zig:34-73 (verifyFingerprint)
//   verify_mtp_config src/model/mtp.zig:318-345 (verifyFingerprint)
//
// Shards are read with pread only (no mapping): the header is read once, and
// tensor bytes go straight from the file into the caller's buffer.
#pragma once

#include <stdint.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "peregrine_model.h"

namespace prg {

struct StTensor {
  std::string dtype;             // safetensors dtype string ("U32", "BF16", "F32", ...)
  std::vector<uint64_t> shape;
  uint32_t shard = 0;
  uint64_t begin = 0, end = 0;   // byte range within the shard's data blob
};

struct StRepo {
  std::vector<std::string> shard_names;  // sorted, unique
  std::vector<int> fds;
  std::vector<uint64_t> shard_bytes;     // file sizes
  std::vector<uint64_t> data_start;      // 8 + header length
  std::map<std::string, StTensor> tensors;

  StRepo() = default;
  StRepo(const StRepo&) = delete;
  StRepo& operator=(const StRepo&) = delete;
  ~StRepo();

  const StTensor* get(const std::string& name) const;
  // File offset and length of a tensor's bytes after the bounds checks of
  // tensorRange (safetensors.zig:123-141). Returns a PRG_ERR_* code.
  int range(const StTensor& t, uint64_t* file_off, uint64_t* len) const;
  // Bytes [off, off + len) of the tensor into dst.
  int read(const StTensor& t, uint64_t off, void* dst, uint64_t len) const;
};

// Open a checkpoint directory: shards named by model.safetensors.index.json,
// each header parsed into the tensor table. Returns a PRG_ERR_* code.
int st_open(const std::string& dir, std::unique_ptr<StRepo>* out);

// Bytes per element of a safetensors dtype string; 0 if unknown.
size_t st_dtype_size(const std::string& dtype);

// Whole file into *out (at most `limit` bytes, else an error).
int read_text_file(const std::string& path, size_t limit, std::string* out);

int verify_config(const std::string& dir);
int verify_mtp_config(const std::string& dir);
// config.json -> PrgModelConfig for any depth / width the kernels support.
int read_model_config(const std::string& dir, PrgModelConfig* cfg);

}  // namespace prg
