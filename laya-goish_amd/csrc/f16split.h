// hi/lo f16 planes of f32 values: hi = f16(v), lo = f16(v - hi), so hi + lo carries about 22
// significant bits of v (the split-precision MFMA operands).
#pragma once
#include <hip/hip_runtime.h>

namespace lg {

// v as an opaque f32 register value.  A split of a computed value needs it: otherwise the
// compiler may contract the multiply that produced v into a mixed-precision FMA that rounds the
// exact product straight to f16 (v_fma_mix*) for one of the two conversions, while the other
// converts the f32-rounded product.  When those two roundings differ (a double-rounding tie,
// about one element in 8192) the stored hi + lo is a whole f16 ulp away from v.
__device__ __forceinline__ float f32_pin(float v) {
  asm("" : "+v"(v));
  return v;
}

__device__ __forceinline__ void split_f16(float v, _Float16 &hi, _Float16 &lo) {
  v = f32_pin(v);
  hi = _Float16(v);
  lo = _Float16(v - float(hi));
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// v - float(h[SEL]) in one v_fma_mix_f32 (v + h * -1, the f16 operand widened inside the
// instruction).  The difference of v and its own f16 rounding is exact in f32, as in split_f16.
template <int SEL>
__device__ __forceinline__ float sub_f16(float v, f16x2 h) {
  float d;
  if constexpr (SEL == 0)
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h), "v"(v));
  else
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h), "v"(v));
  return d;
}

// split_f16 of eight values, two at a time (packed conversions): the same hi and lo bits in
// two instructions a value instead of four.
__device__ __forceinline__ void split8_pk(const float *v, f16x8 &hi, f16x8 &lo) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const f32x2 w = {f32_pin(v[e]), f32_pin(v[e + 1])};
    const f16x2 h = __builtin_convertvector(w, f16x2);
    const f16x2 l = __builtin_convertvector((f32x2{sub_f16<0>(w[0], h), sub_f16<1>(w[1], h)}), f16x2);
    hi[e] = h[0];
    hi[e + 1] = h[1];
    lo[e] = l[0];
    lo[e + 1] = l[1];
  }
}

// Rotate-half RoPE of one pair (u at dim j, v at dim j + hd/2) with the table entries of both dims
// (src/tensor.rs:158-172): a = u cos_j - v sin_j, c = v cos_{j+hd/2} + u sin_{j+hd/2}, every product
// and sum rounded on its own as the reference forms them (no contraction into FMA here, whatever
// the including file allows).  Shared by every kernel that writes the KV cache, so a token's
// cached k has the same bits whichever kernel rotated it.
__device__ __forceinline__ void rope_pair(float u, float v, float c0, float s0, float c1, float s1, float &a,
                                          float &c) {
#pragma clang fp contract(off)
  a = u * c0 - v * s0;
  c = v * c1 + u * s1;
}

}  // namespace lg
