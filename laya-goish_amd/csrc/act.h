// Activations shared by the GEMM epilogues of gemm_tiles.h and gemm_wide.h, so that every tiling of a
// gated projection rounds the same way.
#pragma once
#include <hip/hip_runtime.h>

namespace lg {

// tanh-approximated GELU of src/tensor.rs:129-131
__device__ __forceinline__ float gelu_tanh(float x) {
  return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * x * (1.0f + 0.044715f * x * x)));
}

}  // namespace lg
