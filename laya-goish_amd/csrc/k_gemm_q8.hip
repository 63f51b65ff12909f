// Exact Q8_0 prefill GEMM tiles (A as hi/lo f16 planes, codes exact, block scale applied in f32
// per 32-element block).  This translation unit is compiled with MFMA results in VGPRs
// (-mllvm -amdgpu-mfma-vgpr-form, set by the Makefile): the partial sum of each block then
// feeds the scale FMAs directly instead of through AGPR reads.
#include "gemm_tiles.h"

namespace lg {

bool launch_gemm_q8_exact(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi,
                          float *C, _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias,
                          hipStream_t st) {
  // 128 x 128 x 64 tiles, one LDS stage with register prefetch: best of a sweep at the
  // 35,840-token shapes (two workgroups per CU, 244 VGPRs).
  return launch_cfg<LG_Q8_0, SPLIT, 64, 2, 2, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st);
}

}  // namespace lg
