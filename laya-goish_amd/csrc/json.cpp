// Minimal recursive-descent JSON reader (RFC 8259 values; \u escapes decoded to UTF-8).
#include "json.h"

#include <cstdlib>

#include "common.h"

namespace lg {
namespace {

const Json kNull;
const std::string kEmpty;

struct Reader {
  const std::string &t;
  const char *what;
  size_t i = 0;
  [[noreturn]] void bad() { fail(LG_ERR_FORMAT, "%s: invalid JSON at byte %zu", what, i); }
  void ws() {
    while (i < t.size() && (t[i] == ' ' || t[i] == '\t' || t[i] == '\n' || t[i] == '\r')) ++i;
  }
  bool lit(const char *w) {
    size_t k = 0;
    while (w[k] && i + k < t.size() && t[i + k] == w[k]) ++k;
    if (w[k]) return false;
    i += k;
    return true;
  }
  void utf8(std::string &out, unsigned cp) {
    if (cp < 0x80) out += char(cp);
    else if (cp < 0x800) { out += char(0xc0 | (cp >> 6)); out += char(0x80 | (cp & 63)); }
    else if (cp < 0x10000) {
      out += char(0xe0 | (cp >> 12)); out += char(0x80 | ((cp >> 6) & 63)); out += char(0x80 | (cp & 63));
    } else {
      out += char(0xf0 | (cp >> 18)); out += char(0x80 | ((cp >> 12) & 63));
      out += char(0x80 | ((cp >> 6) & 63)); out += char(0x80 | (cp & 63));
    }
  }
  unsigned hex4() {
    if (i + 4 > t.size()) bad();
    unsigned v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = t[i++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= unsigned(c - '0');
      else if (c >= 'a' && c <= 'f') v |= unsigned(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= unsigned(c - 'A' + 10);
      else bad();
    }
    return v;
  }
  std::string string() {
    if (i >= t.size() || t[i] != '"') bad();
    ++i;
    std::string out;
    while (true) {
      if (i >= t.size()) bad();
      const char c = t[i++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) bad();
      if (c != '\\') { out += c; continue; }
      if (i >= t.size()) bad();
      const char e = t[i++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          unsigned cp = hex4();
          if (cp >= 0xd800 && cp < 0xdc00 && i + 1 < t.size() && t[i] == '\\' && t[i + 1] == 'u') {
            i += 2;
            const unsigned lo = hex4();
            if (lo < 0xdc00 || lo > 0xdfff) bad();
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          utf8(out, cp);
        } break;
        default: bad();
      }
    }
  }
  Json value(int depth) {
    if (depth > 64) bad();
    ws();
    if (i >= t.size()) bad();
    Json v;
    const char c = t[i];
    if (c == '{') {
      ++i;
      v.kind = Json::Obj;
      ws();
      if (i < t.size() && t[i] == '}') { ++i; return v; }
      while (true) {
        ws();
        std::string k = string();
        ws();
        if (i >= t.size() || t[i] != ':') bad();
        ++i;
        // a repeated key makes the whole text invalid (src/json.rs:157-166)
        for (const auto &kv : v.o)
          if (kv.first == k) bad();
        v.o.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (i < t.size() && t[i] == ',') { ++i; continue; }
        if (i < t.size() && t[i] == '}') { ++i; return v; }
        bad();
      }
    }
    if (c == '[') {
      ++i;
      v.kind = Json::Arr;
      ws();
      if (i < t.size() && t[i] == ']') { ++i; return v; }
      while (true) {
        v.a.push_back(value(depth + 1));
        ws();
        if (i < t.size() && t[i] == ',') { ++i; continue; }
        if (i < t.size() && t[i] == ']') { ++i; return v; }
        bad();
      }
    }
    if (c == '"') { v.kind = Json::Str; v.s = string(); return v; }
    if (lit("true")) { v.kind = Json::Bool; v.b = true; return v; }
    if (lit("false")) { v.kind = Json::Bool; return v; }
    if (lit("null")) return v;
    // number: -?(0|[1-9]\d*)(\.\d+)?([eE][+-]?\d+)?
    const size_t s0 = i;
    if (t[i] == '-') ++i;
    auto digits = [&] {
      const size_t k = i;
      while (i < t.size() && t[i] >= '0' && t[i] <= '9') ++i;
      return i > k;
    };
    if (i < t.size() && t[i] == '0') ++i;
    else if (!digits()) bad();
    if (i < t.size() && t[i] == '.') { ++i; if (!digits()) bad(); }
    if (i < t.size() && (t[i] == 'e' || t[i] == 'E')) {
      ++i;
      if (i < t.size() && (t[i] == '+' || t[i] == '-')) ++i;
      if (!digits()) bad();
    }
    v.kind = Json::Num;
    v.n = std::strtod(t.substr(s0, i - s0).c_str(), nullptr);
    return v;
  }
};

}  // namespace

const Json &Json::get(const std::string &key) const {
  if (kind != Obj) return kNull;
  for (const auto &kv : o)
    if (kv.first == key) return kv.second;
  return kNull;
}

const Json &Json::at(size_t idx) const { return kind == Arr && idx < a.size() ? a[idx] : kNull; }

const std::string &Json::str() const { return kind == Str ? s : kEmpty; }

Json Json::parse(const std::string &text, const char *what) {
  Reader r{text, what};
  Json v = r.value(0);
  r.ws();
  if (r.i != text.size()) r.bad();
  return v;
}

}  // namespace lg
