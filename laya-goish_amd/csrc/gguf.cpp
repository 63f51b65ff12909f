// GGUF v3 reader, host side of the engine.  Accepts exactly what src/gguf.rs:95-179 accepts
// and reports the same messages, so a caller sees the reference's errors.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

#include "common.h"

namespace lg {

bool layout(uint32_t kind, uint64_t *block, uint64_t *bytes) {
  static const struct { uint32_t kind; uint64_t block, bytes; } table[] = {
      {LG_F32, 1, 4},    {LG_F16, 1, 2},     {LG_Q4_0, 32, 18},
      {LG_Q8_0, 32, 34}, {LG_Q4_K, 256, 144}, {LG_Q6_K, 256, 210},
  };
  for (const auto &t : table)
    if (t.kind == kind) {
      if (block) *block = t.block;
      if (bytes) *bytes = t.bytes;
      return true;
    }
  return false;
}

float half_to_float(uint16_t x) {
  const uint32_t sign = (uint32_t(x) & 0x8000u) << 16;
  const uint32_t exp = (x >> 10) & 0x1fu;
  const uint32_t man = x & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      // subnormal: man * 2^-24, exact in f32
      float v = float(man) * (1.0f / 16777216.0f);
      return sign ? -v : v;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

namespace {

struct Cursor {
  const uint8_t *b;
  uint64_t n, p = 0;

  const uint8_t *take(uint64_t k) {
    if (p + k < p) fail(LG_ERR_FORMAT, "GGUF length overflow");
    if (p + k > n) fail(LG_ERR_FORMAT, "truncated GGUF");
    const uint8_t *s = b + p;
    p += k;
    return s;
  }
  template <class T>
  T get() {
    T v;
    std::memcpy(&v, take(sizeof(T)), sizeof(T));
    return v;
  }
  std::string string() {
    uint64_t k = get<uint64_t>();
    if (k > 32ull * 1024 * 1024) fail(LG_ERR_FORMAT, "GGUF string too large");
    const uint8_t *s = take(k);
    if (!valid_utf8(s, k)) fail(LG_ERR_FORMAT, "invalid GGUF UTF-8");
    return std::string(reinterpret_cast<const char *>(s), k);
  }
  static bool valid_utf8(const uint8_t *s, uint64_t k) {
    uint64_t i = 0;
    while (i < k) {
      const uint8_t c = s[i];
      if (c < 0x80) {
        ++i;
        continue;
      }
      int extra;
      uint32_t cp, minimum;
      if ((c >> 5) == 0x6) { extra = 1; cp = c & 0x1f; minimum = 0x80; }
      else if ((c >> 4) == 0xe) { extra = 2; cp = c & 0x0f; minimum = 0x800; }
      else if ((c >> 3) == 0x1e) { extra = 3; cp = c & 0x07; minimum = 0x10000; }
      else return false;
      if (i + extra >= k) return false;  // continuation bytes run past the end
      for (int j = 1; j <= extra; ++j) {
        if ((s[i + j] & 0xc0) != 0x80) return false;
        cp = (cp << 6) | (s[i + j] & 0x3f);
      }
      if (cp < minimum || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return false;
      i += extra + 1;
    }
    return true;
  }
  // src/gguf.rs:48-79
  MetaValue value(uint32_t t, int depth) {
    if (depth > 4) fail(LG_ERR_FORMAT, "GGUF metadata nesting too deep");
    MetaValue v;
    v.type = t;
    switch (t) {
      case 0: v.num = get<uint8_t>(); break;
      case 1: v.num = get<int8_t>(); break;
      case 2: v.num = get<uint16_t>(); break;
      case 3: v.num = get<int16_t>(); break;
      case 4: v.num = get<uint32_t>(); break;
      case 5: v.num = get<int32_t>(); break;
      case 6: v.num = get<float>(); break;
      case 7: v.num = get<uint8_t>() != 0; break;
      case 8: v.str = string(); break;
      case 9: {
        uint32_t et = get<uint32_t>();
        uint64_t count = get<uint64_t>();
        if (count > 1000000) fail(LG_ERR_FORMAT, "GGUF array too large");
        for (uint64_t i = 0; i < count; ++i) {
          MetaValue e = value(et, depth + 1);
          if (et == 8) v.strs.push_back(std::move(e.str));  // kept: token lists name control tokens
        }
        v.count = count;
      } break;
      case 10: v.num = double(get<uint64_t>()); break;
      case 11: v.num = double(get<int64_t>()); break;
      case 12: v.num = get<double>(); break;
      default: fail(LG_ERR_FORMAT, "unsupported GGUF metadata type %u", t);
    }
    return v;
  }
};

}  // namespace

Gguf *Gguf::open_memory(const uint8_t *bytes, uint64_t len) {
  auto *g = new Gguf();
  g->bytes_ = bytes;
  g->len_ = len;
  try {
    g->parse();
  } catch (...) {
    delete g;
    throw;
  }
  return g;
}

Gguf *Gguf::open_file(const std::string &path) {
  if (path.find('\0') != std::string::npos) fail(LG_ERR_FORMAT, "NUL in path");
  int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) fail(LG_ERR_FORMAT, "open %s: errno %d", path.c_str(), errno);
  struct stat st;
  if (fstat(fd, &st) < 0 || st.st_size <= 0) {
    ::close(fd);
    fail(LG_ERR_FORMAT, "empty/unreadable model");
  }
  void *p = mmap(nullptr, size_t(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) fail(LG_ERR_FORMAT, "mmap failed");
  auto *g = new Gguf();
  g->map_ = p;
  g->bytes_ = static_cast<const uint8_t *>(p);
  g->len_ = uint64_t(st.st_size);
  try {
    g->parse();
  } catch (...) {
    delete g;
    throw;
  }
  return g;
}

Gguf::~Gguf() {
  if (map_) munmap(map_, size_t(len_));
}

void Gguf::parse() {
  Cursor r{bytes_, len_};
  if (std::memcmp(r.take(4), "GGUF", 4) != 0) fail(LG_ERR_FORMAT, "not a GGUF file");
  if (r.get<uint32_t>() != 3) fail(LG_ERR_FORMAT, "expected GGUF version 3");
  const uint64_t nt = r.get<uint64_t>();
  const uint64_t nk = r.get<uint64_t>();
  if (nt > 100000 || nk > 100000) fail(LG_ERR_FORMAT, "GGUF table too large");
  for (uint64_t i = 0; i < nk; ++i) {
    std::string key = r.string();
    uint32_t t = r.get<uint32_t>();
    MetaValue v = r.value(t, 0);
    if (!meta_.emplace(std::move(key), std::move(v)).second)
      fail(LG_ERR_FORMAT, "duplicate GGUF metadata key");
  }
  for (uint64_t i = 0; i < nt; ++i) {
    TensorInfo t;
    t.name = r.string();
    const uint32_t nd = r.get<uint32_t>();
    if (nd < 1 || nd > 4) fail(LG_ERR_FORMAT, "invalid tensor rank");
    uint64_t count = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      const uint64_t v = r.get<uint64_t>();
      if (v == 0) fail(LG_ERR_FORMAT, "empty tensor");
      if (count > UINT64_MAX / v) fail(LG_ERR_FORMAT, "tensor size overflow");
      count *= v;
      t.dims.push_back(v);
    }
    t.kind = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    uint64_t block, size;
    if (!layout(t.kind, &block, &size))
      fail(LG_ERR_FORMAT, "unsupported GGML tensor type %u; supported F32/F16/Q4_0/Q8_0/Q4_K/Q6_K",
           t.kind);
    if (t.dims[0] % block) fail(LG_ERR_FORMAT, "invalid quantized row alignment");
    if (count / block > UINT64_MAX / size) fail(LG_ERR_FORMAT, "tensor byte size overflow");
    t.len = count / block * size;
    if (index_.count(t.name)) fail(LG_ERR_FORMAT, "duplicate tensor");
    index_[t.name] = order_.size();
    order_.push_back(std::move(t));
  }
  // general.alignment as a number (a bool, string or array counts as 0), converted to an
  // integer the saturating way (NaN and negatives -> 0), default 32 (src/gguf.rs:158-165)
  const double av = num("general.alignment", 32);
  const uint64_t align = !(av > 0) ? 0 : av >= 18446744073709551616.0 ? UINT64_MAX : uint64_t(av);
  if (align == 0 || (align & (align - 1)) || align > 4096) fail(LG_ERR_FORMAT, "invalid GGUF alignment");
  const uint64_t base = (r.p + align - 1) & ~(align - 1);
  // relocation and bounds checks in name order, like the reference's BTreeMap walk
  for (const auto &kv : index_) {
    TensorInfo &t = order_[kv.second];
    if (t.offset % align) fail(LG_ERR_FORMAT, "unaligned GGUF tensor");
    if (t.offset + base < t.offset) fail(LG_ERR_FORMAT, "offset overflow");
    t.offset += base;
    if (t.offset + t.len < t.offset) fail(LG_ERR_FORMAT, "length overflow");
    if (t.offset + t.len > len_) fail(LG_ERR_FORMAT, "truncated tensor data");
  }
}

const MetaValue *Gguf::meta(const std::string &key) const {
  auto it = meta_.find(key);
  return it == meta_.end() ? nullptr : &it->second;
}

double Gguf::num(const std::string &key, double dflt) const {
  const MetaValue *v = meta(key);
  if (!v) return dflt;
  return (v->type == 7 || v->type == 8 || v->type == 9) ? 0.0 : v->num;  // J::num(): numbers only
}

std::string Gguf::str(const std::string &key) const {
  const MetaValue *v = meta(key);
  return v ? v->str : std::string();
}

const TensorInfo *Gguf::tensor(const std::string &name) const {
  auto it = index_.find(name);
  return it == index_.end() ? nullptr : &order_[it->second];
}

}  // namespace lg
