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

}  // namespace lg
