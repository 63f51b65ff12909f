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
  // Short launches (single requests): 32 x 32 tiles over two LDS stages when fewer than 128 tiles of
  // 64 x 64 cover the output, else 64 x 128 tiles when fewer than 256 of 128 x 128 would; the same
  // per-element sequence, so the same bits (a 144-token request on the 24-layer d2048 model 8.46 ->
  // 4.97 ms, 560 tokens 9.66 -> 8.29 ms, 1024 tokens 11.89 -> 10.35 ms).
  if (W.cols % 128 == 0) {
    const bool glu = epi == Epi::SWIGLU || epi == Epi::GEGLU;
    const int outN = glu ? W.rows / 2 : W.rows;
    if (int64_t((M + 63) / 64) * (outN / 64) < 128 &&
        (glu ? launch_cfg<LG_Q8_0, SPLIT, 128, 1, 2, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)
             : launch_cfg<LG_Q8_0, SPLIT, 128, 1, 1, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st)))
      return true;
    if (int64_t((M + 127) / 128) * (outN / 128) < 256 &&
        launch_cfg<LG_Q8_0, SPLIT, 128, 2, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st))
      return true;
  }
  // 128 x 128 x 64 tiles, one LDS stage with register prefetch: best of a sweep at the
  // 35,840-token shapes (two workgroups per CU, 244 VGPRs).
  return launch_cfg<LG_Q8_0, SPLIT, 64, 4, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st);
}

bool launch_gemm_q8_small_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                               const RopeKvOut &ro, hipStream_t st) {
  const bool ok = launch_cfg_rope<LG_Q8_0, SPLIT, 128, 1, 2>(A, Alo, M, W, bias, ro, st);
  if (ok) HIP_CHECK(hipGetLastError());
  return ok;
}

bool launch_gemm_q4_exact(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi,
                          float *C, _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias,
                          hipStream_t st, const _Float16 *ks) {
  // the Q8_0 geometry: 128 x 128 x 64 tiles, one LDS stage (the correction's four planes size it)
  LG_REQUIRE(ks, "gemm: an exact Q4_K launch needs its activation's chunk sums");
  // short launches: 32 x 128 tiles over two LDS stages, or 64 x 128 tiles (the Q8_0 rule with the
  // 128 x 128 tiles kept from 192 of them: at 224, a 1024-token request's o projection, they are faster)
  if (W.cols % 128 == 0) {
    const bool glu = epi == Epi::SWIGLU || epi == Epi::GEGLU;
    const int outN = glu ? W.rows / 2 : W.rows;
    if (int64_t((M + 63) / 64) * (outN / 64) < 128 &&
        launch_cfg<LG_Q4_K, SPLIT, 64, 1, 4, 2>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st, ks))
      return true;
    if (int64_t((M + 127) / 128) * (outN / 128) < 192 &&
        launch_cfg<LG_Q4_K, SPLIT, 64, 2, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st, ks))
      return true;
  }
  return launch_cfg<LG_Q4_K, SPLIT, 64, 4, 4, 1>(A, Alo, M, W, epi, C, C16, C16lo, ldc, bias, st, ks);
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

namespace {
// the wide kernel's mode for W, or -1 when it does not take an M-row launch of W with epilogue
// EPI (an Epi value or wide::kEpiRopeKv)
int wide_mode(int M, const DevMatrix &W, int EPI) {
  using namespace wide;
  if (M <= 0 || !W.pc) return -1;
  int mode;
  switch (W.kind) {
    case LG_Q8_0: mode = WQ8; if (!W.pcs) return -1; break;
    case LG_F16: mode = W1; break;
    case LG_Q4_K:  // the two-pass copy (codes, scales, correction planes), or hi/lo planes
      if (needs_ksum(W)) {
        mode = WQ4;
        if (!W.pcs || !W.pcl) return -1;
      } else {
        mode = W2;
        if (!W.pcl) return -1;
      }
      break;
    case LG_Q6_K: mode = W2; if (!W.pcl) return -1; break;
    default: return -1;
  }
  if (EPI != int(Epi::F32) && EPI != int(Epi::ADD) && EPI != int(Epi::SWIGLU) && EPI != int(Epi::GEGLU) &&
      EPI != kEpiRopeKv && EPI != kEpiLayaRope)
    return -1;
  const bool glu = EPI == int(Epi::SWIGLU) || EPI == int(Epi::GEGLU);
  const int N = W.rows, K = W.cols;
  if (K % BK != 0 || N % BN != 0) return -1;  // gated: 128 gate + 128 up rows a tile
  const int NT = glu ? (N / 2) / (BN / 2) : N / BN;
  if (int64_t(N) * K * 2 >= (int64_t(1) << 32)) return -1;  // 32-bit buffer offsets of the weights
  // fewer 256 x 256 tiles than 5/8 of the CUs leaves too many idle: the 128 x 128 tiles fill the device
  // better.  Between that and one tile per CU the 256 x 256 tiles still win (F16 at 1437 rows x 7168 gated,
  // 168 tiles: 50.3 against 60.0 us; 2048 x 6144, 192 tiles: 91.7 against 120.4; 3000 x 5120, 240 tiles:
  // 57.1 against 77.2), and below it they lose (1437 x 5120, 120 tiles: 48.1 against 41.8)
  if (int64_t((M + BM - 1) / BM) * NT * 8 < int64_t(device_cus()) * 5) return -1;
  return mode;
}

typedef void (*WideFn)(const _Float16 *, const _Float16 *, int, int, const _Float16 *, const _Float16 *,
                       const float *, int, float *, _Float16 *, _Float16 *, int, const float *, int, int, int,
                       RopeKvOut, wide::KqCorr);

// one kernel per (epilogue, mode), its LDS limit raised on the current device
template <int EPI>
WideFn wide_fn(int mode) {
  using namespace wide;
  static const WideFn fns[4] = {gemm_wide_kernel<EPI, WQ8>, gemm_wide_kernel<EPI, W1>, gemm_wide_kernel<EPI, W2>,
                                gemm_wide_kernel<EPI, WQ4>};
  static const int lds_bytes[4] = {Geo<WQ8>::kLdsBytes, Geo<W1>::kLdsBytes, Geo<W2>::kLdsBytes, Geo<WQ4>::kLdsBytes};
  grant_lds(reinterpret_cast<const void *>(fns[mode]), size_t(lds_bytes[mode]));
  return fns[mode];
}

// launches fn over the M rows in chunks whose activation planes stay within 32-bit buffer offsets
void launch_wide(WideFn fn, int mode, const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W,
                 bool glu, float *C, _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, const RopeKvOut &ro,
                 hipStream_t st, const _Float16 *ks) {
  using namespace wide;
  static const int lds_bytes[4] = {Geo<WQ8>::kLdsBytes, Geo<W1>::kLdsBytes, Geo<W2>::kLdsBytes, Geo<WQ4>::kLdsBytes};
  const int N = W.rows, K = W.cols;
  const int NT = glu ? (N / 2) / (BN / 2) : N / BN;
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
    RopeKvOut rc = ro;  // per-row tables and q planes of the rotating epilogues start at row m0
    if (rc.tok_pos) rc.tok_pos += m0;
    if (rc.tok_page) rc.tok_page += m0;
    if (rc.q16) rc.q16 += int64_t(m0) * ro.hq * 128;
    if (rc.q16lo) rc.q16lo += int64_t(m0) * ro.hq * 128;
    KqCorr kq;
    if (mode == WQ4) {
      kq.kp = W.pkp;
      kq.ks = ks + int64_t(m0) * W.pkp;
      kq.kslo = ks + (int64_t(M) + m0) * W.pkp;
      kq.bh = W.pcl;
      kq.bl = W.pcl + int64_t(N) * W.pkp;
      kq.rs = W.pcr;
    }
    launch_timed(fn, dim3(MT * NT), dim3(THREADS), lds_bytes[mode], st, Ac, Alc, Mc, K,
                 static_cast<const _Float16 *>(W.pc), static_cast<const _Float16 *>(W.pcl),
                 static_cast<const float *>(W.pcs), N, Cc, C16c, C16lc, ldc, bias, MT, NT, N / 2, rc, kq);
    m0 += Mc;
  }
  if (timer) *timer = whole;
}
}  // namespace

bool gemm_wide_takes(int M, const DevMatrix &W, Epi epi) { return wide_mode(M, W, int(epi)) >= 0; }

bool launch_gemm_wide(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi, float *C,
                      _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, hipStream_t st, const _Float16 *ks) {
  using namespace wide;
  if (!A || !Alo) return false;
  const int mode = wide_mode(M, W, int(epi));
  if (mode < 0) return false;
  LG_REQUIRE(mode != WQ4 || ks, "gemm: an exact Q4_K launch needs its activation's chunk sums");
  const bool glu = epi == Epi::SWIGLU || epi == Epi::GEGLU;
  const int N = W.rows;
  if (glu ? (C16 == nullptr || ldc < N / 2) : (C == nullptr || ldc < N)) return false;
  const WideFn fn = epi == Epi::F32      ? wide_fn<int(Epi::F32)>(mode)
                    : epi == Epi::ADD    ? wide_fn<int(Epi::ADD)>(mode)
                    : epi == Epi::SWIGLU ? wide_fn<int(Epi::SWIGLU)>(mode)
                                         : wide_fn<int(Epi::GEGLU)>(mode);
  launch_wide(fn, mode, A, Alo, M, W, glu, C, C16, C16lo, ldc, bias, RopeKvOut{}, st, ks);
  return true;
}

bool launch_gemm_wide_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                           const RopeKvOut &ro, hipStream_t st, const _Float16 *ks) {
  using namespace wide;
  if (!A || !Alo) return false;
  const int mode = wide_mode(M, W, kEpiRopeKv);
  if (mode < 0) return false;
  LG_REQUIRE(mode != WQ4 || ks, "gemm: an exact Q4_K launch needs its activation's chunk sums");
  if (ro.hd != 128 || ro.col0 % 128 != 0 || ro.col0 / 128 + W.rows / 128 > ro.hq + 2 * ro.hkv) return false;
  LG_REQUIRE(ro.cosT && ro.sinT && ro.tok_pos && ro.tok_page && ro.q16 && ro.q16lo && ro.kpool && ro.vpool,
             "gemm rope: missing output");
  LG_REQUIRE(ro.page_tokens >= 4 && ro.page_tokens % 4 == 0 && ro.page_stride > 0, "gemm rope: bad page geometry");
  LG_REQUIRE(ro.kv_planes == 1 || ro.kv_planes == 2, "gemm rope: KV pools hold 1 or 2 planes, not %d", ro.kv_planes);
  launch_wide(wide_fn<kEpiRopeKv>(mode), mode, A, Alo, M, W, false, nullptr, nullptr, nullptr, 0, bias, ro, st, ks);
  return true;
}

void launch_gemm_wide_laya_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                                const float *cosT, const float *sinT, const int32_t *tok_pos, int heads, float *C,
                                int ldc, hipStream_t st, const _Float16 *ks) {
  using namespace wide;
  LG_REQUIRE(A && Alo && C && cosT && sinT && tok_pos, "gemm laya rope: missing operand");
  const int mode = wide_mode(M, W, kEpiLayaRope);
  LG_REQUIRE(mode >= 0, "gemm laya rope: the 256 x 256 GEMM does not take %d rows of this matrix", M);
  LG_REQUIRE(mode != WQ4 || ks, "gemm: an exact Q4_K launch needs its activation's chunk sums");
  LG_REQUIRE(heads > 0 && heads % 2 == 0 && W.rows == 3 * heads * 64 && ldc >= W.rows,
             "gemm laya rope: %d rows are not q|k|v of an even number of 64-dim heads (%d)", W.rows, heads);
  RopeKvOut ro;
  ro.cosT = cosT;
  ro.sinT = sinT;
  ro.tok_pos = tok_pos;
  ro.hq = heads;
  ro.hd = 64;
  launch_wide(wide_fn<kEpiLayaRope>(mode), mode, A, Alo, M, W, false, C, nullptr, nullptr, ldc, bias, ro, st, ks);
}

}  // namespace lg
