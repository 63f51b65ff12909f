// GGUF v3 reader for the engine (host side).  Restates the reference loader's accepted
// format and error behaviour, src/gguf.rs:22-199, over a read-only private mmap
// (src/io.rs:56-97) or caller-owned bytes.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace lg {

// src/gguf.rs:81-93
bool layout(uint32_t kind, uint64_t *block, uint64_t *bytes);
// src/gguf.rs:226-246
float half_to_float(uint16_t x);

struct MetaValue {
  uint32_t type = 0;  // GGUF metadata kind 0..12
  double num = 0;     // numeric kinds and bool
  std::string str;    // kind 8
  uint64_t count = 0; // kind 9: element count
  std::vector<std::string> strs;  // kind 9 over strings: the elements
};

struct TensorInfo {
  std::string name;
  std::vector<uint64_t> dims;  // dims[0] = row length
  uint32_t kind = 0;
  uint64_t offset = 0, len = 0;  // absolute offset in the file / image
  uint64_t rows() const {
    uint64_t r = 1;
    for (size_t i = 1; i < dims.size(); ++i) r *= dims[i];
    return r;
  }
  uint64_t cols() const { return dims.empty() ? 0 : dims[0]; }
};

class Gguf {
 public:
  // Throws lg::Error(LG_ERR_FORMAT, <reference message>) on malformed input.
  static Gguf *open_file(const std::string &path);
  static Gguf *open_memory(const uint8_t *bytes, uint64_t len);
  ~Gguf();

  const MetaValue *meta(const std::string &key) const;
  double num(const std::string &key, double dflt) const;
  std::string str(const std::string &key) const;
  const TensorInfo *tensor(const std::string &name) const;
  const uint8_t *data(const TensorInfo &t) const { return bytes_ + t.offset; }
  const std::vector<TensorInfo> &tensors() const { return order_; }

 private:
  Gguf() = default;
  void parse();
  const uint8_t *bytes_ = nullptr;
  uint64_t len_ = 0;
  void *map_ = nullptr;  // mmap base when owned
  std::map<std::string, MetaValue> meta_;
  std::vector<TensorInfo> order_;
  std::map<std::string, size_t> index_;
};

}  // namespace lg
