// Minimal JSON reader for model metadata (the openthai.config string of an OpenThai GGUF).
// Counterpart of the reference's json::parse as used at src/models/openthai/model.rs:97-126:
// get() on a missing key or a non-object yields null, num()/str() of another kind yield 0 / "".
#pragma once
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace lg {

struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double n = 0;
  std::string s;
  std::vector<Json> a;
  std::vector<std::pair<std::string, Json>> o;

  const Json &get(const std::string &key) const;  // object member or null
  const Json &at(size_t i) const;                 // array element or null
  double num() const { return kind == Num ? n : 0.0; }
  const std::string &str() const;
  size_t size() const { return kind == Arr ? a.size() : 0; }

  // Throws lg::Error(LG_ERR_FORMAT, "<what>: invalid JSON ...") on malformed text.
  static Json parse(const std::string &text, const char *what);
};

}  // namespace lg
