// GGUF reader.  Format (ggml's gguf spec): magic "GGUF", u32 version, u64 tensor count,
// u64 metadata count, metadata (string key, u32 type, value), tensor infos (string name,
// u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset), then the data section aligned to
// general.alignment (default 32).  Note: the reference wgpu loader takes the data base as the
// unaligned cursor position after the infos (wgpu_loader.rs:109); the spec (and candle's
// tensor reads) use the aligned offset, which is what this reader does.
#include "gguf.h"

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "tpt_common.h"

namespace tpt {

namespace {

struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  bool bad = false;
  template <typename T>
  T get() {
    T v{};
    if (bad || (size_t)(end - p) < sizeof(T)) {
      bad = true;
      return v;
    }
    memcpy(&v, p, sizeof(T));
    p += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (bad || n > (uint64_t)(end - p)) {
      bad = true;
      return {};
    }
    std::string s((const char*)p, (size_t)n);
    p += n;
    return s;
  }
};

int scalar_bytes(int t) {
  switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
  }
  return -1;
}

bool read_value(Reader& r, int t, GgufValue* v, int depth) {
  if (depth > 2) return false;
  if (t == 8) {
    std::string s = r.str();
    if (v) v->s = std::move(s);
    return !r.bad;
  }
  if (t == 9) {
    const int et = (int)r.get<uint32_t>();
    const uint64_t n = r.get<uint64_t>();
    if (v) v->is_array = true;
    if (et != 8 && et != 9) {  // fixed-size elements: skip in one step
      const int eb = scalar_bytes(et);
      if (eb < 0 || n > (uint64_t)(r.end - r.p) / (uint64_t)eb) return false;
      r.p += n * (uint64_t)eb;
      return !r.bad;
    }
    for (uint64_t i = 0; i < n && !r.bad; i++)
      if (!read_value(r, et, nullptr, depth + 1)) return false;
    return !r.bad;
  }
  const int nb = scalar_bytes(t);
  if (nb < 0) return false;
  uint64_t raw = 0;
  if ((size_t)(r.end - r.p) < (size_t)nb) return false;
  memcpy(&raw, r.p, (size_t)nb);
  r.p += nb;
  if (v) {
    v->u = raw;
    switch (t) {
      case 1: v->i = (int8_t)raw; break;
      case 3: v->i = (int16_t)raw; break;
      case 5: v->i = (int32_t)raw; break;
      case 11: v->i = (int64_t)raw; break;
      default: v->i = (int64_t)raw;
    }
    if (t == 6) {
      float f;
      uint32_t b = (uint32_t)raw;
      memcpy(&f, &b, 4);
      v->f = f;
    } else if (t == 12) {
      memcpy(&v->f, &raw, 8);
    } else {
      v->f = (double)v->i;
    }
  }
  return true;
}

}  // namespace

GgufFile::~GgufFile() {
  if (map) munmap(map, size);
}

int GgufFile::open(const std::string& p) {
  path = p;
  const int fd = ::open(p.c_str(), O_RDONLY);
  if (fd < 0) return fail(TPT_ERR_IO, "opening " + p + ": " + strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return fail(TPT_ERR_IO, "stat " + p);
  }
  size = (size_t)st.st_size;
  void* m = size ? mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
  ::close(fd);
  if (m == MAP_FAILED) return fail(TPT_ERR_IO, "mmap " + p);
  map = (uint8_t*)m;
  Reader r{map, map + size};
  if (r.get<uint32_t>() != 0x46554747u) return fail(TPT_ERR_FORMAT, "not a GGUF file (bad magic): " + p);
  version = r.get<uint32_t>();
  if (version < 2 || version > 3) return fail(TPT_ERR_FORMAT, "unsupported GGUF version " + std::to_string(version));
  const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
  if (r.bad || nt > (1u << 20) || nkv > (1u << 20)) return fail(TPT_ERR_FORMAT, "GGUF header counts out of range");
  for (uint64_t i = 0; i < nkv; i++) {
    std::string key = r.str();
    GgufValue v;
    v.type = (int)r.get<uint32_t>();
    if (r.bad || !read_value(r, v.type, &v, 0)) return fail(TPT_ERR_FORMAT, "truncated GGUF metadata at key '" + key + "'");
    meta[key] = std::move(v);
  }
  tensors.resize(nt);
  for (uint64_t i = 0; i < nt; i++) {
    GgufTensor& t = tensors[i];
    t.name = r.str();
    t.n_dims = (int)r.get<uint32_t>();
    if (r.bad || t.n_dims < 1 || t.n_dims > 4) return fail(TPT_ERR_FORMAT, "bad tensor info for '" + t.name + "'");
    for (int d = 0; d < t.n_dims; d++) t.ne[d] = (int64_t)r.get<uint64_t>();
    t.type = (int)r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    if (r.bad) return fail(TPT_ERR_FORMAT, "truncated tensor info");
    index[t.name] = i;
  }
  uint64_t align = 32;
  uint64_t a;
  if (get_u64("general.alignment", &a) && a > 0 && (a & (a - 1)) == 0) align = a;
  const uint64_t pos = (uint64_t)(r.p - map);
  data_offset = (pos + align - 1) / align * align;
  if (data_offset > size) return fail(TPT_ERR_FORMAT, "GGUF data section starts past end of file");
  const uint64_t data_bytes = size - data_offset;
  for (GgufTensor& t : tensors) {
    // every extent in [0, 2^40) and the element count below 2^62: no product can overflow
    uint64_t n = 1;
    for (int d = 0; d < 4; d++) {
      if (t.ne[d] < 0 || t.ne[d] >= ((int64_t)1 << 40))
        return fail(TPT_ERR_FORMAT, "tensor '" + t.name + "' has an extent out of range");
      const uint64_t e = (uint64_t)t.ne[d];
      if (e && n > (((uint64_t)1 << 62) / e)) return fail(TPT_ERR_FORMAT, "tensor '" + t.name + "' has too many elements");
      n *= e;
    }
    const int bs = type_block(t.type), tb = type_bytes(t.type);
    if (tb == 0) continue;  // a dtype this path never reads: left unmapped, rejected if used
    if (n % (uint64_t)bs) return fail(TPT_ERR_FORMAT, "tensor '" + t.name + "' size is not a whole number of blocks");
    t.bytes = (size_t)(n / (uint64_t)bs) * (size_t)tb;
    // wgpu_loader.rs:130-132, written so that no sum can wrap
    if (t.offset > data_bytes || t.bytes > data_bytes - t.offset)
      return fail(TPT_ERR_FORMAT, "tensor '" + t.name + "' extends past end of file");
    t.data = map + data_offset + t.offset;
  }
  return TPT_OK;
}

const GgufTensor* GgufFile::find(const std::string& name) const {
  auto it = index.find(name);
  return it == index.end() ? nullptr : &tensors[it->second];
}

bool GgufFile::get_u64(const std::string& key, uint64_t* out) const {
  auto it = meta.find(key);
  if (it == meta.end() || it->second.is_array) return false;
  if (it->second.type != 4 && it->second.type != 10) return false;
  *out = it->second.u;
  return true;
}

bool GgufFile::get_f32(const std::string& key, float* out) const {
  auto it = meta.find(key);
  if (it == meta.end() || it->second.is_array) return false;
  if (it->second.type != 6 && it->second.type != 12) return false;
  *out = (float)it->second.f;
  return true;
}

bool GgufFile::get_str(const std::string& key, std::string* out) const {
  auto it = meta.find(key);
  if (it == meta.end() || it->second.type != 8) return false;
  *out = it->second.s;
  return true;
}

}  // namespace tpt
