// GGUF v2/v3 reader (host).  Replaces candle's gguf_file::Content::read as used by the
// reference loader (src-tauri/src/engine/wgpu_loader.rs:105-109) and extract_meta
// (wgpu_loader.rs:305-406).  The file is mmapped; tensor data stay in place until upload.
#pragma once
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace tpt {

struct GgufValue {
  int type = -1;  // GGUF value type (0..12)
  uint64_t u = 0; // unsigned/bool payload
  int64_t i = 0;  // signed payload
  double f = 0;   // float payload
  std::string s;  // string payload
  bool is_array = false;
};

struct GgufTensor {
  std::string name;
  int type = 0;
  int n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  uint64_t offset = 0;  // relative to the aligned data section
  const uint8_t* data = nullptr;
  size_t bytes = 0;
};

struct GgufFile {
  std::string path;
  uint8_t* map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t data_offset = 0;
  std::map<std::string, GgufValue> meta;
  std::vector<GgufTensor> tensors;
  std::map<std::string, size_t> index;

  ~GgufFile();
  // Parses and validates.  Returns TPT_OK or a TPT_ERR_* code (message via set_error).
  int open(const std::string& path);
  const GgufTensor* find(const std::string& name) const;
  bool get_u64(const std::string& key, uint64_t* out) const;  // U32 or U64 (meta_u64)
  bool get_f32(const std::string& key, float* out) const;     // F32 or F64 (meta_f32)
  bool get_str(const std::string& key, std::string* out) const;
};

}  // namespace tpt
