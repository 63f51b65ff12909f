// Exact Q8_0 prefill GEMM tiles (A as hi/lo f16 planes, codes exact, block scale applied in f32
// per 32-element block).  This translation unit is compiled with MFMA results in VGPRs
// (-mllvm -amdgpu-mfma-vgpr-form, set by the Makefile): the partial sum of each block then
// feeds the scale FMAs directly instead of through AGPR reads.
#include <algorithm>

#include "gemm_q8x.h"
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

bool launch_gemm_q8x(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi, float *C,
                     _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, hipStream_t st) {
  using namespace q8x;
  if (W.kind != LG_Q8_0 || !W.pc || !W.pcs || !A || !Alo || M <= 0) return false;
  if (epi != Epi::F32 && epi != Epi::ADD && epi != Epi::SWIGLU) return false;
  const bool glu = epi == Epi::SWIGLU;
  const int N = W.rows, K = W.cols;
  if (K % BK != 0 || (glu ? N % BN : N % BN) != 0) return false;  // gated: 128 gate + 128 up rows a tile
  const int NT = glu ? (N / 2) / (BN / 2) : N / BN;
  if (int64_t(N) * K * 2 >= (int64_t(1) << 32)) return false;  // 32-bit buffer offsets of the codes
  // fewer 256 x 256 tiles than CUs leaves CUs idle: the 128 x 128 tiles fill the device better
  if (int64_t((M + BM - 1) / BM) * NT < device_cus()) return false;
  if (glu ? (C16 == nullptr || ldc < N / 2) : (C == nullptr || ldc < N)) return false;

  static bool attr[4] = {false, false, false, false};
  auto set_lds_limit = [&](Epi e) {
    const void *fn = e == Epi::F32   ? reinterpret_cast<const void *>(gemm_q8x_kernel<int(Epi::F32)>)
                     : e == Epi::ADD ? reinterpret_cast<const void *>(gemm_q8x_kernel<int(Epi::ADD)>)
                                     : reinterpret_cast<const void *>(gemm_q8x_kernel<int(Epi::SWIGLU)>);
    if (!attr[int(e)]) {
      HIP_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES));
      attr[int(e)] = true;
    }
  };
  set_lds_limit(epi);
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
    const dim3 grid(MT * NT), block(THREADS);
    const _Float16 *Ac = A + int64_t(m0) * K, *Alc = Alo + int64_t(m0) * K;
    float *Cc = C ? C + int64_t(m0) * ldc : nullptr;
    _Float16 *C16c = C16 ? C16 + int64_t(m0) * ldc : nullptr, *C16lc = C16lo ? C16lo + int64_t(m0) * ldc : nullptr;
    switch (epi) {
      case Epi::F32:
        launch_timed(gemm_q8x_kernel<int(Epi::F32)>, grid, block, LDS_BYTES, st, Ac, Alc, Mc, K, W.pc, W.pcs, N,
                     Cc, C16c, C16lc, ldc, bias, MT, NT, N / 2);
        break;
      case Epi::ADD:
        launch_timed(gemm_q8x_kernel<int(Epi::ADD)>, grid, block, LDS_BYTES, st, Ac, Alc, Mc, K, W.pc, W.pcs, N,
                     Cc, C16c, C16lc, ldc, bias, MT, NT, N / 2);
        break;
      default:
        launch_timed(gemm_q8x_kernel<int(Epi::SWIGLU)>, grid, block, LDS_BYTES, st, Ac, Alc, Mc, K, W.pc, W.pcs, N,
                     Cc, C16c, C16lc, ldc, bias, MT, NT, N / 2);
        break;
    }
    m0 += Mc;
  }
  if (timer) *timer = whole;
  return true;
}

size_t q8x_copy_bytes(int rows, int cols) {
  return size_t(rows) * size_t(cols) * 2 + size_t(rows) * size_t(cols / 32) * 4;
}

void launch_q8x_prefill_copy(const DevMatrix &w, hipStream_t st) {
  LG_REQUIRE(w.kind == LG_Q8_0 && w.pc && w.pcs && w.cols % 32 == 0 && w.rows > 0, "q8x copy: bad matrix");
  const int64_t blocks = int64_t(w.rows) * (w.cols / 32);
  LG_REQUIRE((blocks + 255) / 256 < (int64_t(1) << 31), "q8x copy: matrix too large");
  hipLaunchKernelGGL(q8x::q8x_prefill_copy_kernel, dim3(unsigned((blocks + 255) / 256)), dim3(256), 0, st,
                     static_cast<const int8_t *>(w.q), static_cast<const uint16_t *>(w.s), w.rows, w.cols, w.pc,
                     w.pcs);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
