// Device-side weight decoding shared by the dequant, GEMV and GEMM kernels.
// All arithmetic here is written so that it cannot be contracted into FMA: the
// dequantised f32 value must be bit-identical to src/gguf.rs:250-336.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "lg.h"

namespace lg {

// IEEE binary16 bits -> f32 with the reference's exact rules (src/gguf.rs:226-246),
// including NaN payloads (no quieting), done with integer operations.
__device__ __forceinline__ float half_bits(uint32_t x) {
  const uint32_t sign = (x & 0x8000u) << 16;
  const uint32_t e = (x >> 10) & 31u;
  const uint32_t m = x & 1023u;
  if (e == 0) {
    if (m == 0) return __uint_as_float(sign);
    const float v = __fmul_rn(float(m), 1.0f / 16777216.0f);
    return sign ? -v : v;
  }
  if (e == 31) return __uint_as_float(sign | 0x7f800000u | (m << 13));
  return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

// Q4_K 6-bit (scale, min) of sub-block j from the 12 packed bytes (src/gguf.rs:287-296).
__device__ __forceinline__ void q4k_scale_min(const uint8_t *sc, int j, uint32_t &s, uint32_t &m) {
  if (j < 4) {
    s = sc[j] & 63u;
    m = sc[j + 4] & 63u;
  } else {
    s = (sc[j + 4] & 15u) | ((uint32_t(sc[j - 4]) >> 6) << 4);
    m = (uint32_t(sc[j + 4]) >> 4) | ((uint32_t(sc[j]) >> 6) << 4);
  }
}

// Q6_K 6-bit code of element w (0..255) of a block (src/gguf.rs:314-324).
__device__ __forceinline__ uint32_t q6k_code(const uint8_t *c, int w, int &scale_index) {
  const uint8_t *ql = c, *qh = c + 128;
  const int n = w >> 7, r = w & 127, j = r >> 5, l = r & 31;
  const int lo = n * 64 + l;
  const uint32_t hi = qh[n * 32 + l];
  scale_index = n * 8 + l / 16 + j * 2;
  switch (j) {
    case 0: return (ql[lo] & 15u) | ((hi & 3u) << 4);
    case 1: return (ql[lo + 32] & 15u) | (((hi >> 2) & 3u) << 4);
    case 2: return (uint32_t(ql[lo]) >> 4) | (((hi >> 4) & 3u) << 4);
    default: return (uint32_t(ql[lo + 32]) >> 4) | (((hi >> 6) & 3u) << 4);
  }
}

// Dequantised weight of the repacked layouts (kernels.h), each product and difference rounded
// on its own as src/gguf.rs:301-303 and :326-330 form them (no contraction into FMA here, whatever
// the including file allows): Q4_K (d*sc) * q - (dmin*m) from the pair (a, b) = (d*sc, dmin*m);
// Q6_K (d*sc) * (code - 32).
__device__ __forceinline__ float kq4_weight(float a, uint32_t q, float b) {
#pragma clang fp contract(off)
  return a * float(q) - b;
}
__device__ __forceinline__ float kq6_weight(float a, int q) {
#pragma clang fp contract(off)
  return a * float(q);
}

}  // namespace lg
