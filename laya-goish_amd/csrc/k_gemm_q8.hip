// Exact prefill GEMMs: the 128 x 128 Q8_0 tiles (A as hi/lo f16 planes, codes exact, block scale
// applied in f32 per 32-element block) and the 256 x 256 large-batch kernels of gemm_wide.h.
// This translation unit is compiled with MFMA results in VGPRs (-mllvm -amdgpu-mfma-vgpr-form,
// set by the Makefile): the partial sum of each Q8_0 block then feeds the scale FMAs directly
// instead of through AGPR reads.
#include <algorithm>

#include "gemm_wide.h"
#include "gemm_tiles.h"

namespace lg {

bool launch_gemm_q8_exact(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi,
                          float *C, _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias,
                          hipStream_t st) {
  // 128 x 128 x 64 tiles, one LDS stage with register prefetch: best of a sweep at the
  // 35,840-token shapes (two workgroups per CU, 244 VGPRs).
  return launch_cfg<LG_Q8_0, SPLIT, 64, 2, 2, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st);
}

namespace {
int device_cus() {
  static thread_local int dev = -1, cus = 0;
  int d = 0;
  HIP_CHECK(hipGetDevice(&d));
  if (d != dev) {
    HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, d));
    dev = d;
  }
  return cus;
}
}  // namespace

bool launch_gemm_wide(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi, float *C,
                      _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, hipStream_t st) {
  using namespace wide;
  if (!A || !Alo || M <= 0 || !W.pc) return false;
  int mode;
  switch (W.kind) {
    case LG_Q8_0: mode = WQ8; if (!W.pcs) return false; break;
    case LG_F16: mode = W1; break;
    case LG_Q4_K:
    case LG_Q6_K: mode = W2; if (!W.pcl) return false; break;
    default: return false;
  }
  if (epi != Epi::F32 && epi != Epi::ADD && epi != Epi::SWIGLU) return false;
  const bool glu = epi == Epi::SWIGLU;
  const int N = W.rows, K = W.cols;
  if (K % BK != 0 || N % BN != 0) return false;  // gated: 128 gate + 128 up rows a tile
  const int NT = glu ? (N / 2) / (BN / 2) : N / BN;
  if (int64_t(N) * K * 2 >= (int64_t(1) << 32)) return false;  // 32-bit buffer offsets of the weights
  // fewer 256 x 256 tiles than CUs leaves CUs idle: the 128 x 128 tiles fill the device better
  if (int64_t((M + BM - 1) / BM) * NT < device_cus()) return false;
  if (glu ? (C16 == nullptr || ldc < N / 2) : (C == nullptr || ldc < N)) return false;

  // one kernel per (epilogue, mode); the LDS limit is raised once per kernel
  typedef void (*Fn)(const _Float16 *, const _Float16 *, int, int, const _Float16 *, const _Float16 *,
                     const float *, int, float *, _Float16 *, _Float16 *, int, const float *, int, int, int);
  static const Fn fns[3][3] = {
      {gemm_wide_kernel<int(Epi::F32), WQ8>, gemm_wide_kernel<int(Epi::F32), W1>, gemm_wide_kernel<int(Epi::F32), W2>},
      {gemm_wide_kernel<int(Epi::ADD), WQ8>, gemm_wide_kernel<int(Epi::ADD), W1>, gemm_wide_kernel<int(Epi::ADD), W2>},
      {gemm_wide_kernel<int(Epi::SWIGLU), WQ8>, gemm_wide_kernel<int(Epi::SWIGLU), W1>,
       gemm_wide_kernel<int(Epi::SWIGLU), W2>}};
  static const int lds_bytes[3] = {Geo<WQ8>::kLdsBytes, Geo<W1>::kLdsBytes, Geo<W2>::kLdsBytes};
  static bool attr[3][3] = {};
  const int ei = epi == Epi::F32 ? 0 : epi == Epi::ADD ? 1 : 2;
  const Fn fn = fns[ei][mode];
  if (!attr[ei][mode]) {
    HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  lds_bytes[mode]));
    attr[ei][mode] = true;
  }
  // activation rows per launch: the planes' buffer offsets are 32-bit
  const int64_t rows_cap = ((int64_t(1) << 31) - 1) / (int64_t(K) * 2) / BM * BM;
  LG_REQUIRE(rows_cap > 0, "gemm: K=%d too large", K);
  KernelTimer *timer = kernel_timer();
  const KernelTimer whole = timer ? *timer : KernelTimer{};
  for (int m0 = 0; m0 < M;) {
    const int Mc = int(std::min<int64_t>(M - m0, rows_cap));
    if (timer) {
      timer->start = m0 == 0 ? whole.start : nullptr;
      timer->stop = m0 + Mc >= M ? whole.stop : nullptr;
    }
    const int MT = (Mc + BM - 1) / BM;
    LG_REQUIRE(int64_t(MT) * NT < (int64_t(1) << 31), "gemm: grid too large");
    const _Float16 *Ac = A + int64_t(m0) * K, *Alc = Alo + int64_t(m0) * K;
    float *Cc = C ? C + int64_t(m0) * ldc : nullptr;
    _Float16 *C16c = C16 ? C16 + int64_t(m0) * ldc : nullptr, *C16lc = C16lo ? C16lo + int64_t(m0) * ldc : nullptr;
    launch_timed(fn, dim3(MT * NT), dim3(THREADS), lds_bytes[mode], st, Ac, Alc, Mc, K,
                 static_cast<const _Float16 *>(W.pc), static_cast<const _Float16 *>(W.pcl),
                 static_cast<const float *>(W.pcs), N, Cc, C16c, C16lc, ldc, bias, MT, NT, N / 2);
    m0 += Mc;
  }
  if (timer) *timer = whole;
  return true;
}

}  // namespace lg
