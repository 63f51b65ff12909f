// Seeded synthetic "laya-decoder" GGUF images for the workload shapes.
//
// The file carries general.architecture = "ggmlc" with laya.model_name = "laya-decoder",
// a name the reference's describe() rejects cleanly ("unsupported ggmlc model",
// src/models/mod.rs:48) instead of misloading, and tensor/metadata layout as written by
// GGUF v3 writers (header, key/values, tensor table, 32-byte aligned data).
//
// Values come from a counter-based SplitMix64 stream keyed by (seed, tensor index, draw
// index), so any element can be regenerated independently and the fill parallelises.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "common.h"
#include "gguf.h"

namespace lg {
namespace {

constexpr uint64_t kGolden = 0x9e3779b97f4a7c15ull;

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

struct Stream {
  uint64_t base;
  Stream(uint64_t seed, uint64_t tensor) : base(mix64(seed + 0x632be59bd9b4e019ull * (tensor + 1))) {}
  uint64_t u64(uint64_t i) const { return mix64(base + (i + 1) * kGolden); }
  double uniform(uint64_t i) const { return (double(u64(i) >> 11) + 0.5) * 0x1.0p-53; }
  // Box-Muller over draws (i, i+1)
  double normal(uint64_t i) const {
    const double a = uniform(i), b = uniform(i + 1);
    return std::sqrt(-2.0 * std::log(a)) * std::cos(6.283185307179586 * b);
  }
};

// f32 -> IEEE binary16, round to nearest even, with subnormals, Inf and NaN.
uint16_t float_to_half(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) return uint16_t(sign | 0x7c00u | (man ? 0x200u : 0u));
  int e = int(exp) - 127 + 15;
  if (e >= 31) return uint16_t(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return uint16_t(sign);
    man |= 0x800000u;
    const int shift = 14 - e;  // 24-bit significand -> subnormal half
    uint32_t h = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1))) ++h;
    return uint16_t(sign | h);
  }
  uint32_t h = (uint32_t(e) << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;  // may carry into the exponent: fine
  return uint16_t(sign | h);
}

enum class Fill { Normal, Ones, NearOne, Q8, Q4K, Q6K, Cos, Sin, LogUniform };

struct Spec {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t kind;
  Fill fill;
  double sigma;
  uint64_t offset = 0, bytes = 0;
};

struct Preset {
  const char *name;
  int L, d, hq, hkv, hd, f, V, ctx;
  double eps, theta;
  uint32_t emb, norm, q, k, v, o, gate, up, down, head;
  bool bias, fused_qkv, fused_wi, ones_norm;
  double w_sigma;  // F16 weight sigma
};

const Preset kPresets[] = {
    // CPU-runnable plumbing model: F16, 6 x d512, MHA 8 x 64, SwiGLU 1408.
    {"plumbing-f16", 6, 512, 8, 8, 64, 1408, 32000, 2048, 1e-5, 1e4, LG_F16, LG_F32, LG_F16,
     LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, false, true, true, true, 0.02},
    // Q8_0 decoder, 24 x d2048, MHA 16 x 128, FFN 5632; Q8_0 head.
    {"q8-2048", 24, 2048, 16, 16, 128, 5632, 32000, 4096, 1e-5, 1e4, LG_F16, LG_F16, LG_Q8_0,
     LG_Q8_0, LG_Q8_0, LG_Q8_0, LG_Q8_0, LG_Q8_0, LG_Q8_0, LG_Q8_0, false, true, true, false, 0.02},
    // Q4_K_M 7B Qwen2 shape: GQA 28/4 x 128, FFN 18944, QKV bias, theta 1e6.
    {"q4km-7b", 28, 3584, 28, 4, 128, 18944, 152064, 4096, 1e-6, 1e6, LG_F16, LG_F32, LG_Q4_K,
     LG_Q4_K, LG_Q6_K, LG_Q4_K, LG_Q4_K, LG_Q4_K, LG_Q6_K, LG_Q6_K, true, false, true, false, 0.02},
    // Same shape, F16 weights, long context.
    {"f16-7b", 28, 3584, 28, 4, 128, 18944, 152064, 10240, 1e-6, 1e6, LG_F16, LG_F32, LG_F16,
     LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, true, true, true, false, 0.02},
    // Small test shapes: hd 64 GQA (F16, bias), hd 128 MHA (Q8_0), hd 128 GQA K-quants.
    {"tiny-f16", 2, 256, 4, 2, 64, 512, 512, 512, 1e-5, 1e4, LG_F16, LG_F32, LG_F16, LG_F16,
     LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, true, true, true, false, 0.05},
    {"tiny-q8", 2, 256, 2, 2, 128, 512, 1024, 512, 1e-5, 1e4, LG_F16, LG_F16, LG_Q8_0, LG_Q8_0,
     LG_Q8_0, LG_Q8_0, LG_Q8_0, LG_Q8_0, LG_Q8_0, LG_Q8_0, false, true, true, false, 0.02},
    {"tiny-q4k", 2, 512, 4, 2, 128, 512, 1024, 512, 1e-6, 1e6, LG_F16, LG_F32, LG_Q4_K, LG_Q4_K,
     LG_Q6_K, LG_Q4_K, LG_Q4_K, LG_Q4_K, LG_Q6_K, LG_Q6_K, true, false, true, false, 0.02},
    {"tiny-f16-128", 2, 512, 4, 2, 128, 512, 1024, 512, 1e-5, 1e4, LG_F16, LG_F32, LG_F16, LG_F16,
     LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, true, true, true, false, 0.03},
    // tiny-f16 with a RoPE table past the decode attention's 65,536 tokens (its longest-context test)
    {"tiny-long", 2, 256, 4, 2, 64, 512, 512, 65600, 1e-5, 1e4, LG_F16, LG_F32, LG_F16, LG_F16,
     LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, LG_F16, true, true, true, false, 0.05},
    // Q4_K rows wider than the decode GEMV's register prologue: K 5120 (q, k, v, o, gate, up) and
    // 9472 (down), GQA 40/5, one layer.
    {"wide-q4k", 1, 5120, 40, 5, 128, 9472, 1024, 512, 1e-6, 1e6, LG_F16, LG_F32, LG_Q4_K, LG_Q4_K,
     LG_Q4_K, LG_Q4_K, LG_Q4_K, LG_Q4_K, LG_Q4_K, LG_Q6_K, true, false, true, false, 0.02},
};

const Preset *find_preset(const char *name) {
  for (const auto &p : kPresets)
    if (!std::strcmp(p.name, name)) return &p;
  return nullptr;
}

// ---- GGUF writer ----
struct Writer {
  std::vector<uint8_t> head;
  void bytes(const void *p, size_t n) {
    const uint8_t *b = static_cast<const uint8_t *>(p);
    head.insert(head.end(), b, b + n);
  }
  template <class T>
  void put(T v) { bytes(&v, sizeof v); }
  void str(const std::string &s) {
    put<uint64_t>(s.size());
    bytes(s.data(), s.size());
  }
  void kv_u32(const std::string &k, uint32_t v) { str(k); put<uint32_t>(4); put<uint32_t>(v); }
  void kv_u64(const std::string &k, uint64_t v) { str(k); put<uint32_t>(10); put<uint64_t>(v); }
  void kv_f32(const std::string &k, float v) { str(k); put<uint32_t>(6); put<float>(v); }
  void kv_str(const std::string &k, const std::string &v) { str(k); put<uint32_t>(8); str(v); }
  void kv_strs(const std::string &k, const std::vector<std::string> &v) {
    str(k);
    put<uint32_t>(9);
    put<uint32_t>(8);
    put<uint64_t>(v.size());
    for (const auto &e : v) str(e);
  }
};

Fill weight_fill(uint32_t kind) {
  switch (kind) {
    case LG_Q8_0: return Fill::Q8;
    case LG_Q4_K: return Fill::Q4K;
    case LG_Q6_K: return Fill::Q6K;
    default: return Fill::Normal;
  }
}

void fill_tensor(const Spec &s, uint64_t seed, uint64_t tidx, uint8_t *dst, uint64_t lo,
                 uint64_t hi, const Preset &p) {
  Stream rng(seed, tidx);
  switch (s.fill) {
    case Fill::Normal:
    case Fill::Ones:
    case Fill::NearOne:
    case Fill::LogUniform: {
      for (uint64_t e = lo; e < hi; ++e) {
        float v;
        if (s.fill == Fill::Ones) v = 1.0f;
        else if (s.fill == Fill::NearOne) v = float(0.75 + 0.5 * rng.uniform(e));
        else if (s.fill == Fill::LogUniform) v = float(std::log(1.0 + 15.0 * rng.uniform(e)));
        else v = float(s.sigma * rng.normal(2 * e));
        if (s.kind == LG_F32) std::memcpy(dst + 4 * e, &v, 4);
        else {
          uint16_t h = float_to_half(v);
          std::memcpy(dst + 2 * e, &h, 2);
        }
      }
    } break;
    case Fill::Q8: {  // [f16 d][32 x i8]: d = f16(|N(0,0.002)|), codes U{-127..127}
      for (uint64_t b = lo; b < hi; ++b) {
        uint8_t *c = dst + 34 * b;
        const uint64_t base = b * 16;
        uint16_t d = float_to_half(float(std::fabs(0.002 * rng.normal(base))));
        std::memcpy(c, &d, 2);
        for (int j = 0; j < 8; ++j) {
          uint64_t u = rng.u64(base + 2 + j);
          for (int t = 0; t < 4; ++t) {
            const uint32_t chunk = uint32_t(u >> (16 * t)) & 0xffffu;
            c[2 + 4 * j + t] = uint8_t(int8_t(int((chunk * 255u) >> 16) - 127));
          }
        }
      }
    } break;
    // Zero-centred blocks (dmin = 8 d, m = round(15 s / 16)), as a quantiser makes them from zero-mean
    // weights: the block minimum cancels the nibble mean.  Independent d/dmin draws with scales and
    // mins U{0..63} would give every matrix a mean of about 0.17 (std 0.26); through 28 layers that
    // builds a common-mode residual whose SwiGLU products (~3.6e5) leave f16's range.
    case Fill::Q4K: {
      for (uint64_t b = lo; b < hi; ++b) {
        uint8_t *c = dst + 144 * b;
        const uint64_t base = b * 32;
        const float df = float(std::fabs(0.001 * rng.normal(base)));
        const uint16_t d = float_to_half(df);
        const uint16_t dm = float_to_half(half_to_float(d) * 8.0f);
        std::memcpy(c, &d, 2);
        std::memcpy(c + 2, &dm, 2);
        uint8_t sv[8], mv[8];
        const uint64_t u = rng.u64(base + 2);
        for (int j = 0; j < 8; ++j) {
          sv[j] = uint8_t(1 + ((u >> (8 * j)) & 0xffu) % 63);
          mv[j] = uint8_t(std::min(63, int(std::lround(sv[j] * 15.0 / 16.0))));
        }
        uint8_t *sc = c + 4;
        for (int j = 0; j < 4; ++j) {
          sc[j] = uint8_t((sv[j] & 63) | ((sv[j + 4] >> 4) << 6));
          sc[j + 4] = uint8_t((mv[j] & 63) | ((mv[j + 4] >> 4) << 6));
          sc[j + 8] = uint8_t((sv[j + 4] & 15) | ((mv[j + 4] & 15) << 4));
        }
        for (int j = 0; j < 16; ++j) {
          const uint64_t r = rng.u64(base + 3 + j);
          std::memcpy(c + 16 + 8 * j, &r, 8);
        }
      }
    } break;
    case Fill::Q6K: {  // [ql 128][qh 64][16 x i8 scales U{1..127}][f16 d = |N(0,2e-5)|]
      for (uint64_t b = lo; b < hi; ++b) {
        uint8_t *c = dst + 210 * b;
        const uint64_t base = b * 32;
        for (int j = 0; j < 24; ++j) {
          const uint64_t r = rng.u64(base + j);
          std::memcpy(c + 8 * j, &r, 8);
        }
        for (int j = 0; j < 2; ++j) {
          const uint64_t r = rng.u64(base + 24 + j);
          for (int t = 0; t < 8; ++t) c[192 + 8 * j + t] = uint8_t(1 + ((r >> (8 * t)) & 0xffu) % 127);
        }
        const uint16_t d = float_to_half(float(std::fabs(2e-5 * rng.normal(base + 26))));
        std::memcpy(c + 208, &d, 2);
      }
    } break;
    case Fill::Cos:
    case Fill::Sin: {  // [ctx][hd] table, rotate-half frequencies theta^(-2 (j mod hd/2) / hd)
      const int hd = p.hd, half = hd / 2;
      for (uint64_t e = lo; e < hi; ++e) {
        const uint64_t pos = e / hd;
        const int j = int(e % hd) % half;
        const double theta = s.sigma > 0 ? s.sigma : p.theta;  // per-table base when the spec carries one
        const double ang = double(pos) * std::pow(theta, -2.0 * j / hd);
        const float v = float(s.fill == Fill::Cos ? std::cos(ang) : std::sin(ang));
        std::memcpy(dst + 4 * e, &v, 4);
      }
    } break;
  }
}

uint64_t units(const Spec &s) {
  uint64_t count = 1;
  for (auto d : s.dims) count *= d;
  switch (s.fill) {
    case Fill::Q8: return count / 32;
    case Fill::Q4K:
    case Fill::Q6K: return count / 256;
    default: return count;
  }
}

// Lays out the tensors (32-byte aligned data; `meta` must carry general.alignment = 32), writes
// header + `meta` (nmeta key/values) + tensor table, and fills the data section in parallel.
void emit_image(std::vector<Spec> &specs, const Writer &meta, int nmeta, uint64_t seed, const Preset &p,
                uint8_t **out, uint64_t *out_len) {
  const uint64_t align = 32;
  uint64_t off = 0;
  for (auto &s : specs) {
    uint64_t count = 1;
    for (auto v : s.dims) count *= v;
    uint64_t block, size;
    layout(s.kind, &block, &size);
    s.bytes = count / block * size;
    s.offset = off;
    off = (off + s.bytes + align - 1) & ~(align - 1);
  }
  Writer w;
  w.bytes("GGUF", 4);
  w.put<uint32_t>(3);
  w.put<uint64_t>(specs.size());
  w.put<uint64_t>(uint64_t(nmeta));
  w.bytes(meta.head.data(), meta.head.size());
  for (const auto &s : specs) {
    w.str(s.name);
    w.put<uint32_t>(uint32_t(s.dims.size()));
    for (auto v : s.dims) w.put<uint64_t>(v);
    w.put<uint32_t>(s.kind);
    w.put<uint64_t>(s.offset);
  }
  const uint64_t data_start = (w.head.size() + align - 1) & ~(align - 1);
  const uint64_t total = data_start + off;
  uint8_t *img = static_cast<uint8_t *>(std::malloc(total));
  if (!img) fail(LG_ERR_OOM, "cannot allocate %llu bytes for the synthetic image",
                 (unsigned long long)total);
  std::memcpy(img, w.head.data(), w.head.size());
  std::memset(img + w.head.size(), 0, data_start - w.head.size());
  for (size_t i = 0; i < specs.size(); ++i) {
    const auto &s = specs[i];
    const uint64_t end = (i + 1 < specs.size()) ? specs[i + 1].offset : off;
    std::memset(img + data_start + s.offset + s.bytes, 0, end - s.offset - s.bytes);
  }
  // parallel fill over (tensor, unit range) chunks
  struct Chunk { size_t t; uint64_t lo, hi; };
  std::vector<Chunk> chunks;
  for (size_t t = 0; t < specs.size(); ++t) {
    const uint64_t n = units(specs[t]);
    const uint64_t step = 1 << 16;
    for (uint64_t lo = 0; lo < n; lo += step) chunks.push_back({t, lo, std::min(n, lo + step)});
  }
  unsigned nth = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> pool;
  std::atomic<size_t> next{0};
  for (unsigned t = 0; t < nth; ++t)
    pool.emplace_back([&] {
      for (size_t c; (c = next.fetch_add(1)) < chunks.size();) {
        const auto &ch = chunks[c];
        fill_tensor(specs[ch.t], seed, ch.t, img + data_start + specs[ch.t].offset, ch.lo, ch.hi, p);
      }
    });
  for (auto &t : pool) t.join();
  *out = img;
  *out_len = total;
}

// ---- OpenThai-SystemOne (Qwen3.5 hybrid text tower + 256-slot head) ----
// Tensor names, shapes and kinds as written by scripts/convert-openthai.py:52-85 (F16 for
// every tensor of rank >= 2, F32 vectors); config keys as checked by
// src/models/openthai/model.rs:97-126.  Every fourth layer is full attention, the rest are
// gated DeltaNet, as in the Qwen3.5 layer_types list.
struct OtPreset {
  const char *name;
  int L, d, f, hq, hkv, nh, V, ctx, state;
  int answer;     // answer_token_id
  int opt_base;   // id of <|ts_opt_0|>; slots 0..254 follow
  int ctl_base;   // ids of <|ts_q|>, <|ts_state|>, <|ts_choice|>, <|ts_score|>, <|ts_noul|>
};

const OtPreset kOtPresets[] = {
    // The reference checkpoint's shape: 24 layers (18 DeltaNet + 6 full), d 1024, FFN 3584,
    // 8/2 heads x 256, 16 linear heads x 128, vocab 248339.
    {"openthai-0.8b", 24, 1024, 3584, 8, 2, 16, 248339, 4096, 2048, 248082, 247800, 248070},
    // Small test shape with the same head geometry (8/2 heads x 256 dims, 128-dim
    // linear heads, conv 4): 4 layers (3 DeltaNet + 1 full), d 256, 2 linear heads.
    {"openthai-tiny", 4, 256, 512, 8, 2, 2, 1024, 1024, 512, 970, 700, 960},
};

const OtPreset *find_ot_preset(const char *name) {
  for (const auto &p : kOtPresets)
    if (!std::strcmp(p.name, name)) return &p;
  return nullptr;
}

void synth_openthai(OtPreset p, uint64_t seed, int n_layers, uint8_t **out, uint64_t *out_len) {
  if (n_layers > 0) p.L = n_layers;
  const uint64_t d = p.d, f = p.f, hd = 256, lk = 128, nh = p.nh;
  const uint64_t cd = 3 * nh * lk;  // conv channels: q | k | v
  std::vector<Spec> specs;
  auto add = [&](const std::string &n, std::vector<uint64_t> dims, uint32_t kind, Fill fill, double sigma) {
    specs.push_back(Spec{n, std::move(dims), kind, fill, sigma});
  };
  std::string types;
  add("model.embed_tokens.weight", {d, uint64_t(p.V)}, LG_F16, Fill::Normal, 0.02);
  for (int l = 0; l < p.L; ++l) {
    const std::string i = "model.layers." + std::to_string(l) + ".";
    const bool full = l % 4 == 3;
    types += std::string(l ? "," : "") + (full ? "\"full_attention\"" : "\"linear_attention\"");
    add(i + "input_layernorm.weight", {d}, LG_F32, Fill::Normal, 0.1);  // zero-centred (offset 1)
    if (full) {
      add(i + "self_attn.q_proj.weight", {d, 2 * p.hq * hd}, LG_F16, Fill::Normal, 0.02);
      add(i + "self_attn.k_proj.weight", {d, p.hkv * hd}, LG_F16, Fill::Normal, 0.02);
      add(i + "self_attn.v_proj.weight", {d, p.hkv * hd}, LG_F16, Fill::Normal, 0.02);
      add(i + "self_attn.o_proj.weight", {p.hq * hd, d}, LG_F16, Fill::Normal, 0.02);
      add(i + "self_attn.q_norm.weight", {hd}, LG_F32, Fill::Normal, 0.1);
      add(i + "self_attn.k_norm.weight", {hd}, LG_F32, Fill::Normal, 0.1);
    } else {
      add(i + "linear_attn.in_proj_qkv.weight", {d, cd}, LG_F16, Fill::Normal, 0.02);
      add(i + "linear_attn.in_proj_z.weight", {d, nh * lk}, LG_F16, Fill::Normal, 0.02);
      add(i + "linear_attn.in_proj_a.weight", {d, nh}, LG_F16, Fill::Normal, 0.02);
      add(i + "linear_attn.in_proj_b.weight", {d, nh}, LG_F16, Fill::Normal, 0.02);
      add(i + "linear_attn.out_proj.weight", {nh * lk, d}, LG_F16, Fill::Normal, 0.02);
      add(i + "linear_attn.conv1d.weight", {4, 1, cd}, LG_F16, Fill::Normal, 0.3);
      add(i + "linear_attn.dt_bias", {nh}, LG_F32, Fill::Normal, 0.5);
      add(i + "linear_attn.A_log", {nh}, LG_F32, Fill::LogUniform, 0);
      add(i + "linear_attn.norm.weight", {lk}, LG_F32, Fill::NearOne, 0);
    }
    add(i + "post_attention_layernorm.weight", {d}, LG_F32, Fill::Normal, 0.1);
    add(i + "mlp.gate_proj.weight", {d, f}, LG_F16, Fill::Normal, 0.02);
    add(i + "mlp.up_proj.weight", {d, f}, LG_F16, Fill::Normal, 0.02);
    add(i + "mlp.down_proj.weight", {f, d}, LG_F16, Fill::Normal, 0.02);
  }
  add("model.norm.weight", {d}, LG_F32, Fill::Normal, 0.1);
  add("slot_head.weight", {d, 256}, LG_F16, Fill::Normal, 0.02);
  add("slot_head.bias", {256}, LG_F32, Fill::Normal, 0.1);
  add("log_temperature", {3}, LG_F32, Fill::Normal, 0.1);

  char cfg[2048];
  std::snprintf(cfg, sizeof cfg,
                "{\"model_type\":\"openthai_systemone\",\"n_slots\":256,\"abstain_slot\":255,"
                "\"answer_token_id\":%d,\"text_config\":{\"hidden_size\":%d,\"intermediate_size\":%d,"
                "\"num_hidden_layers\":%d,\"head_dim\":256,\"num_attention_heads\":%d,"
                "\"num_key_value_heads\":%d,\"linear_conv_kernel_dim\":4,\"linear_key_head_dim\":128,"
                "\"linear_value_head_dim\":128,\"linear_num_key_heads\":%d,\"linear_num_value_heads\":%d,"
                "\"vocab_size\":%d,\"rms_norm_eps\":1e-06,\"rope_parameters\":{\"rope_theta\":10000000,"
                "\"partial_rotary_factor\":0.25,\"rope_type\":\"default\"},\"layer_types\":[",
                p.answer, p.d, p.f, p.L, p.hq, p.hkv, p.nh, p.nh, p.V);
  const std::string config = std::string(cfg) + types + "]}}";
  // token strings: placeholders, then the decide control tokens at their ids
  std::vector<std::string> tokens(p.V);
  for (int i = 0; i < p.V; ++i) tokens[i] = "t" + std::to_string(i);
  tokens[198] = "\xc4\x8a";  // byte-level BPE newline
  tokens[25] = ":";
  for (int s = 0; s < 255; ++s) tokens[p.opt_base + s] = "<|ts_opt_" + std::to_string(s) + "|>";
  const char *ctl[5] = {"<|ts_q|>", "<|ts_state|>", "<|ts_choice|>", "<|ts_score|>", "<|ts_noul|>"};
  for (int j = 0; j < 5; ++j) tokens[p.ctl_base + j] = ctl[j];
  tokens[p.answer] = "<|ts_answer|>";

  Writer w;
  w.kv_str("general.architecture", "openthai_systemone");
  w.kv_str("general.name", std::string("OpenThai-SystemOne synthetic ") + p.name);
  w.kv_u32("general.alignment", 32);
  w.kv_str("openthai.config", config);
  w.kv_u32("openthai.context_length", uint32_t(p.ctx));
  w.kv_u32("openthai.state_length", uint32_t(p.state));
  w.kv_str("tokenizer.ggml.model", "gpt2");
  w.kv_strs("tokenizer.ggml.tokens", tokens);
  w.kv_u64("laya.synthetic.seed", seed);
  w.kv_str("laya.synthetic.preset", p.name);
  Preset none{};
  emit_image(specs, w, 10, seed, none, out, out_len);
}

// ---- Laya (ModernBERT encoder + 2-layer decision head) ----
// Tensor names, metadata and the compiled-graph description (ggmlc.graph_spec) as the reference
// loader reads them (src/models/laya/model.rs:60-291): linears are graph nodes of opcode 29
// (inputs weight, x[, bias]) and opcode 200 (bias add on a linear's output), layer norms nodes of
// opcode 201 named layer_norm, layer_norm_1, ... (inputs x[, weight[, bias]], attribute eps),
// attentions nodes of opcode 74 whose last input is the mask (the global layers share the first
// attention's mask).  Every third trunk layer is global (0, 3, 6, ...), the rest use the local
// window.
struct LayaPreset {
  const char *name;
  int L, d, hd, f, V, max_len, head_f, act_f;
};

const LayaPreset kLayaPresets[] = {
    // ModernBERT-base shape: 22 layers, d 768, 12 heads x 64, GeGLU 1152, vocab 50368.
    {"laya-english", 22, 768, 64, 1152, 50368, 512, 768, 256},
    // Small test shape: 4 layers (0 and 3 global), d 128, 2 heads x 64.
    {"laya-tiny", 4, 128, 64, 192, 1024, 512, 128, 64},
};

const LayaPreset *find_laya_preset(const char *name) {
  for (const auto &p : kLayaPresets)
    if (!std::strcmp(p.name, name)) return &p;
  return nullptr;
}

void synth_laya(LayaPreset p, uint64_t seed, int n_layers, uint8_t **out, uint64_t *out_len) {
  if (n_layers > 0) p.L = n_layers;
  const uint64_t d = p.d, f = p.f;
  std::vector<Spec> specs;
  auto add = [&](const std::string &n, std::vector<uint64_t> dims, uint32_t kind, Fill fill, double sigma) {
    specs.push_back(Spec{n, std::move(dims), kind, fill, sigma});
  };
  // graph description
  std::string tensors, nodes;
  int next_id = 0;
  auto tid = [&](const std::string &name) {
    const int id = next_id++;
    tensors += (tensors.empty() ? "" : ",") + std::string("\"") + std::to_string(id) + "\":{\"name\":\"" + name + "\"}";
    return id;
  };
  auto node = [&](const std::string &body) { nodes += (nodes.empty() ? "" : ",") + body; };
  int x = tid("input");
  int norm_index = 0;
  auto layer_norm = [&](bool weight, bool bias) {
    const std::string nm = norm_index == 0 ? "layer_norm" : "layer_norm_" + std::to_string(norm_index);
    std::string ins = std::to_string(x);
    if (weight) {
      add("ln." + std::to_string(norm_index) + ".weight", {d}, LG_F32, Fill::NearOne, 0);
      ins += "," + std::to_string(tid("ln." + std::to_string(norm_index) + ".weight"));
    }
    if (bias) {
      add("ln." + std::to_string(norm_index) + ".bias", {d}, LG_F32, Fill::Normal, 0.05);
      ins += "," + std::to_string(tid("ln." + std::to_string(norm_index) + ".bias"));
    }
    const int y = tid(nm + ".out");
    node("{\"opcode\":201,\"name\":\"" + nm + "\",\"inputs\":[" + ins + "],\"outputs\":[" + std::to_string(y) +
         "],\"attributes\":{\"eps\":1e-05}}");
    ++norm_index;
    x = y;
  };
  // bias_mode: 0 none, 1 as the linear's third input, 2 as a separate add node
  auto linear = [&](const std::string &key, uint64_t cols, uint64_t rows, int bias_mode, double sigma) {
    add(key + ".weight", rows == 1 ? std::vector<uint64_t>{cols} : std::vector<uint64_t>{cols, rows}, LG_F16,
        Fill::Normal, sigma);
    std::string ins = std::to_string(tid(key + ".weight")) + "," + std::to_string(x);
    if (bias_mode == 1) {
      add(key + ".bias", {rows}, LG_F32, Fill::Normal, 0.05);
      ins += "," + std::to_string(tid(key + ".bias"));
    }
    const int y = tid(key + ".out");
    node("{\"opcode\":29,\"name\":\"" + key + "\",\"inputs\":[" + ins + "],\"outputs\":[" + std::to_string(y) + "]}");
    if (bias_mode == 2) {
      add(key + ".bias_add", {rows}, LG_F32, Fill::Normal, 0.05);
      const int y2 = tid(key + ".biased");
      node("{\"opcode\":200,\"inputs\":[" + std::to_string(y) + "," + std::to_string(tid(key + ".bias_add")) +
           "],\"outputs\":[" + std::to_string(y2) + "]}");
      x = y2;
    } else {
      x = y;
    }
  };
  const int mask_full = tid("mask_full"), mask_local = tid("mask_local");
  auto attention = [&](bool full) {
    const int y = tid("attn.out");
    node("{\"opcode\":74,\"inputs\":[" + std::to_string(x) + "," + std::to_string(full ? mask_full : mask_local) +
         "],\"outputs\":[" + std::to_string(y) + "]}");
    x = y;
  };
  add("tok_emb.weight", {d, uint64_t(p.V)}, LG_F16, Fill::Normal, 0.5);
  layer_norm(true, false);  // embedding norm
  for (int l = 0; l < p.L; ++l) {
    const std::string i = std::to_string(l);
    if (l > 0) layer_norm(true, false);
    linear("qkv." + i, d, 3 * d, l == 1 ? 1 : 0, 0.03);
    attention(l % 3 == 0);
    linear("wo." + i, d, d, l == 2 ? 2 : 0, 0.03);
    layer_norm(true, false);
    linear("mlp_wi." + i, d, 2 * f, 0, 0.03);
    linear("mlp_wo." + i, f, d, 0, 0.03);
  }
  layer_norm(true, false);  // final norm
  add("type_emb.weight", {d, 3}, LG_F32, Fill::Normal, 0.1);
  for (int h = 0; h < 2; ++h) {
    const std::string i = std::to_string(h);
    layer_norm(true, true);
    linear("head_qkv." + i, d, 3 * d, 1, 0.03);
    attention(true);
    linear("head_wo." + i, d, d, 1, 0.03);
    layer_norm(true, true);
    linear("head_fc1." + i, d, uint64_t(p.head_f), 1, 0.05);
    linear("head_fc2." + i, uint64_t(p.head_f), d, 1, 0.03);
  }
  layer_norm(true, true);  // scorer norm
  linear("scorer_fc1", d, d, 1, 0.05);
  linear("scorer_fc2", d, 1, 1, 0.05);
  linear("act_fc1", d + 4, uint64_t(p.act_f), 1, 0.05);
  linear("act_fc2", uint64_t(p.act_f), 2, 1, 0.05);
  // RoPE tables [max_len][hd]: rotate-half frequencies, theta 160000 (global) and 10000 (local)
  add("cos_full", {uint64_t(p.hd), uint64_t(p.max_len)}, LG_F32, Fill::Cos, 160000.0);
  add("sin_full", {uint64_t(p.hd), uint64_t(p.max_len)}, LG_F32, Fill::Sin, 160000.0);
  add("cos_slide", {uint64_t(p.hd), uint64_t(p.max_len)}, LG_F32, Fill::Cos, 10000.0);
  add("sin_slide", {uint64_t(p.hd), uint64_t(p.max_len)}, LG_F32, Fill::Sin, 10000.0);
  const std::string graph = "{\"tensors\":{" + tensors + "},\"nodes\":[" + nodes + "]}";

  Writer w;
  w.kv_str("general.architecture", "ggmlc");
  w.kv_str("general.name", std::string("Laya synthetic ") + p.name);
  w.kv_u32("general.alignment", 32);
  w.kv_str("laya.model_name", "laya");
  w.kv_str("laya.checkpoint", std::string("laya-synthetic-") + p.name);
  w.kv_u32("laya.max_opts", 16);
  w.kv_u32("laya.max_len", uint32_t(p.max_len));
  w.kv_u32("laya.head_max_len", 192);
  w.kv_u32("laya.cls_token_id", uint32_t(p.V - 3));
  w.kv_u32("laya.sep_token_id", uint32_t(p.V - 2));
  w.kv_u32("laya.mask_token_id", uint32_t(p.V - 1));
  w.kv_str("laya.temperature", "[1.25,0.9,1.1]");
  w.kv_str("laya.temperature_by_options", "{\"choice:2\":1.05,\"choice:3-5\":1.2}");
  w.kv_str("ggmlc.graph_spec", graph);
  w.kv_u64("laya.synthetic.seed", seed);
  w.kv_str("laya.synthetic.preset", p.name);
  Preset rope{};
  rope.hd = p.hd;
  emit_image(specs, w, 16, seed, rope, out, out_len);
}

}  // namespace

// Builds the image; caller frees with free().
void synth_image(const char *preset, uint64_t seed, int n_layers, uint8_t **out, uint64_t *out_len) {
  if (const LayaPreset *lp = find_laya_preset(preset)) {
    synth_laya(*lp, seed, n_layers, out, out_len);
    return;
  }
  if (const OtPreset *op = find_ot_preset(preset)) {
    synth_openthai(*op, seed, n_layers, out, out_len);
    return;
  }
  const Preset *pp = find_preset(preset);
  if (!pp) fail(LG_ERR_INVALID, "unknown synthetic preset %s", preset);
  Preset p = *pp;
  if (n_layers > 0) p.L = n_layers;
  const uint64_t d = p.d, qw = uint64_t(p.hq) * p.hd, kvw = uint64_t(p.hkv) * p.hd, f = p.f;
  std::vector<Spec> specs;
  auto add = [&](const std::string &n, std::vector<uint64_t> dims, uint32_t kind, Fill fill,
                 double sigma) { specs.push_back(Spec{n, std::move(dims), kind, fill, sigma}); };
  const Fill norm_fill = p.ones_norm ? Fill::Ones : Fill::NearOne;
  add("tok_emb.weight", {d, uint64_t(p.V)}, p.emb, Fill::Normal, 0.02);
  for (int l = 0; l < p.L; ++l) {
    const std::string i = std::to_string(l);
    add("attn_norm." + i + ".weight", {d}, p.norm, norm_fill, 0);
    if (p.fused_qkv) {
      add("qkv." + i + ".weight", {d, qw + 2 * kvw}, p.q, weight_fill(p.q), p.w_sigma);
      if (p.bias) add("qkv." + i + ".bias", {qw + 2 * kvw}, LG_F32, Fill::Normal, 0.1);
    } else {
      add("q." + i + ".weight", {d, qw}, p.q, weight_fill(p.q), p.w_sigma);
      add("k." + i + ".weight", {d, kvw}, p.k, weight_fill(p.k), p.w_sigma);
      add("v." + i + ".weight", {d, kvw}, p.v, weight_fill(p.v), p.w_sigma);
      if (p.bias) {
        add("q." + i + ".bias", {qw}, LG_F32, Fill::Normal, 0.1);
        add("k." + i + ".bias", {kvw}, LG_F32, Fill::Normal, 0.1);
        add("v." + i + ".bias", {kvw}, LG_F32, Fill::Normal, 0.1);
      }
    }
    add("wo." + i + ".weight", {qw, d}, p.o, weight_fill(p.o), p.w_sigma);
    add("ffn_norm." + i + ".weight", {d}, p.norm, norm_fill, 0);
    if (p.fused_wi) {
      add("mlp_wi." + i + ".weight", {d, 2 * f}, p.gate, weight_fill(p.gate), p.w_sigma);
    } else {
      add("gate." + i + ".weight", {d, f}, p.gate, weight_fill(p.gate), p.w_sigma);
      add("up." + i + ".weight", {d, f}, p.up, weight_fill(p.up), p.w_sigma);
    }
    add("mlp_wo." + i + ".weight", {f, d}, p.down, weight_fill(p.down), p.w_sigma);
  }
  add("final_norm.weight", {d}, p.norm, norm_fill, 0);
  add("output.weight", {d, uint64_t(p.V)}, p.head, weight_fill(p.head), p.w_sigma);
  add("cos_full", {uint64_t(p.hd), uint64_t(p.ctx)}, LG_F32, Fill::Cos, 0);
  add("sin_full", {uint64_t(p.hd), uint64_t(p.ctx)}, LG_F32, Fill::Sin, 0);

  Writer w;
  w.kv_str("general.architecture", "ggmlc");
  w.kv_str("general.name", std::string("laya-decoder synthetic ") + p.name);
  w.kv_u32("general.alignment", 32);
  w.kv_str("laya.model_name", "laya-decoder");
  w.kv_u32("laya.mask_token_id", 0);
  w.kv_u32("laya.decoder.block_count", uint32_t(p.L));
  w.kv_u32("laya.decoder.embedding_length", uint32_t(p.d));
  w.kv_u32("laya.decoder.head_count", uint32_t(p.hq));
  w.kv_u32("laya.decoder.head_count_kv", uint32_t(p.hkv));
  w.kv_u32("laya.decoder.key_length", uint32_t(p.hd));
  w.kv_u32("laya.decoder.feed_forward_length", uint32_t(p.f));
  w.kv_u32("laya.decoder.vocab_size", uint32_t(p.V));
  w.kv_u32("laya.decoder.context_length", uint32_t(p.ctx));
  w.kv_f32("laya.decoder.layer_norm_rms_epsilon", float(p.eps));
  w.kv_f32("laya.decoder.rope_freq_base", float(p.theta));
  w.kv_u64("laya.synthetic.seed", seed);
  w.kv_str("laya.synthetic.preset", p.name);
  emit_image(specs, w, 17, seed, p, out, out_len);
}

}  // namespace lg
