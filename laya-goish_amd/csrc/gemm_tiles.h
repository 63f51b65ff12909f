// Prefill GEMM tiles for gfx950 (shared by the k_gemm*.hip translation units): C = A . W^T on MFMA v_mfma_f32_32x32x16_f16, f32 accumulation,
// weights dequantised into LDS, epilogue fused (bias, residual add, SwiGLU, f16 store).
//
// Numeric modes (selected by the caller):
//   FAST  : A in f16, W dequantised to f16 (RNE); one MFMA pass.
//   SPLIT : A given as two f16 planes (hi = f16(a), lo = f16(a - hi)), so A carries ~22
//           significand bits.  F16 weights are exact in f16 -> 2 passes (hi, lo).
//           Q8_0 codes are exact in f16 and the block scale is applied in f32 per 32-element
//           block (partial sums on MFMA, acc += d * partial) -> 2 passes, weights exact.
//   SPLIT3: K-quants (Q4_K, Q6_K) whose dequantised f32 weight needs 24 bits: W is split into
//           hi/lo f16 too and acc += Ah.Bh + Al.Bh + Ah.Bl -> 3 passes.
// The split modes reproduce f32 arithmetic to ~2^-22 relative per product, which the
// ill-conditioned synthetic workloads need to stay within the parity bars.
//
// Geometry: 256 threads = 4 wave64s in a 2 x 2 arrangement; each wave owns WTM x WTN MFMA
// blocks of 32 x 32, so a workgroup tile is (64 WTM) x (64 WTN) x BK.  STAGES = 2 ping-pongs
// two LDS buffers (one barrier per K step, next tile's global loads in flight during the
// MFMAs); STAGES = 1 uses one buffer with the next tile prefetched into registers.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "kernels.h"
#include "f16split.h"
#include "quant.h"

namespace lg {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum Mode { FAST = 0, SPLIT = 1, SPLIT3 = 2 };


__device__ __forceinline__ float silu(float g) { return g * (1.0f / (1.0f + __expf(-g))); }
// tanh-approximated GELU of src/tensor.rs:129-131
__device__ __forceinline__ float gelu_tanh(float x) {
  return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * x * (1.0f + 0.044715f * x * x)));
}

// f16 bits -> f32 with the hardware conversion (exact for every finite value and infinity;
// a NaN scale gives NaN outputs either way).
__device__ __forceinline__ float hw_half(uint32_t x) { return float(__builtin_bit_cast(_Float16, uint16_t(x))); }

__device__ __forceinline__ void put8(const float *v, _Float16 *hi, _Float16 *lo, bool split) {
  half8 h, l;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    _Float16 a, b;
    split_f16(v[j], a, b);
    h[j] = a;
    l[j] = b;
  }
  *reinterpret_cast<half8 *>(hi) = h;
  if (split) *reinterpret_cast<half8 *>(lo) = l;
}

// ---------------------------------------------------------------- B tile loaders
// A BNT x BK weight tile is cut into 16-byte chunks; thread t handles chunks t + 256 i.
// fetch(): global -> registers;  store(): registers -> LDS rows (stride LDK), dequantised.
// wrow(r) maps a local tile row to its weight row.
template <uint32_t KIND, int MODE, int BK, int BNT>
struct BLoad {
  // elements of the K dimension covered by one chunk
  static constexpr int kElems = KIND == LG_F16 ? 8 : (KIND == LG_Q4_K && BK == 64) ? 32 : 16;
  static constexpr int kCPR = BK / kElems;            // chunks per row
  static constexpr int kPer = BNT * kCPR / 256;        // chunks per thread
  static_assert(kPer >= 1 && BNT * kCPR % 256 == 0, "tile does not split over 256 threads");
  static constexpr bool kQ4 = KIND == LG_Q4_K;
  // register storage as ext_vectors (arrays of a struct tend to be placed in scratch)
  typedef uint32_t uvec __attribute__((ext_vector_type(4 * kPer)));
  typedef float fvec __attribute__((ext_vector_type(kPer)));
  typedef uint32_t rvec __attribute__((ext_vector_type(kPer)));
  uvec v;
  fvec sa, sb;    // scale terms of the chunk (low plane)
  fvec sa2, sb2;  // Q4_K, BK == 64: high-nibble sub-block
  rvec raw;       // Q8_0: raw f16 scale bits
  int plane = 0;  // Q4_K, BK == 32: which nibble of each byte
  // Q8_0: buffer resources of codes and scales; per-chunk byte offsets fixed at init, the K
  // position goes in the scalar offset (the host keeps rows * cols below 2^31)
  __amdgpu_buffer_rsrc_t rq, rs;
  rvec qoff, soff;

  template <class RowMap>
  __device__ __forceinline__ void init(const DevMatrix &W, RowMap wrow, int t) {
    if constexpr (KIND == LG_Q8_0) {
      rq = __builtin_amdgcn_make_buffer_rsrc(W.q, 0, W.rows * W.cols, kBufferFlags);
      rs = __builtin_amdgcn_make_buffer_rsrc(W.s, 0, W.rows * (W.cols / 32) * 2, kBufferFlags);
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int id = t + 256 * i, r = id / kCPR, c = id % kCPR;
        const int n = wrow(r);
        qoff[i] = uint32_t(n * W.cols + c * 16);
        soff[i] = uint32_t((n * (W.cols / 32) + c * 16 / 32) * 2);
      }
    }
  }
  __device__ __forceinline__ void put(int i, uint4 x) {
    v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
  }
  __device__ __forceinline__ uint4 get(int i) const { return make_uint4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]); }

  template <class RowMap>
  __device__ __forceinline__ void fetch(const DevMatrix &W, RowMap wrow, int k0, int t) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int id = t + 256 * i, r = id / kCPR, c = id % kCPR;
      const int64_t n = wrow(r);
      if constexpr (KIND == LG_F16) {
        put(i, *reinterpret_cast<const uint4 *>(static_cast<const _Float16 *>(W.q) + n * W.cols + k0 + c * 8));
      } else if constexpr (KIND == LG_Q8_0) {
        put(i, __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, qoff[i], k0, 0)));
        raw[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff[i], (k0 / 32) * 2, 0);
      } else if constexpr (KIND == LG_Q6_K) {
        const int k = k0 + c * 16;
        put(i, *reinterpret_cast<const uint4 *>(static_cast<const int8_t *>(W.q) + n * W.cols + k));
        sa[i] = static_cast<const float *>(W.s)[n * (W.cols / 16) + k / 16];
      } else {  // Q4_K
        const uint8_t *rowq = static_cast<const uint8_t *>(W.q) + n * (W.cols / 2);
        const float2 *s = static_cast<const float2 *>(W.s) + n * (W.cols / 32);
        if constexpr (BK == 64) {  // bytes [k0/2 + 16c, +16): elements 16c+j (lo) and 32+16c+j (hi)
          put(i, *reinterpret_cast<const uint4 *>(rowq + k0 / 2 + 16 * c));
          const float2 s0 = s[k0 / 32], s1 = s[k0 / 32 + 1];
          sa[i] = s0.x;
          sb[i] = s0.y;
          sa2[i] = s1.x;
          sb2[i] = s1.y;
        } else {  // one nibble plane: bytes [(k0/64)*32 + 16c, +16)
          put(i, *reinterpret_cast<const uint4 *>(rowq + (k0 / 64) * 32 + 16 * c));
          const float2 s0 = s[k0 / 32];
          sa[i] = s0.x;
          sb[i] = s0.y;
        }
      }
    }
    if constexpr (kQ4 && BK == 32) plane = (k0 % 64) >= 32;
  }

  template <int LDK>
  __device__ __forceinline__ void store(_Float16 *Bs, _Float16 *Bl, float *Ds, int t) {
    constexpr bool kSplitB = MODE == SPLIT3;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int id = t + 256 * i, r = id / kCPR, c = id % kCPR;
      const uint32_t w[4] = {v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
      if constexpr (KIND == LG_F16) {
        *reinterpret_cast<uint4 *>(Bs + r * LDK + c * 8) = get(i);
      } else if constexpr (KIND == LG_Q8_0 && MODE == SPLIT) {
        // exact codes as f16: bytes (q ^ 0x80) under a 0x64 high byte read as f16 are
        // 1024 + q + 128 exactly; one packed f16 subtraction of 1152 leaves q
        uint32_t h[8];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t u = w[d] ^ 0x80808080u;
          h[2 * d] = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
          h[2 * d + 1] = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
        }
        typedef _Float16 half2v __attribute__((ext_vector_type(2)));
        const half2v bias = {_Float16(1152.0f), _Float16(1152.0f)};
        uint32_t q[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, h[e]) - bias);
        *reinterpret_cast<uint4 *>(Bs + r * LDK + c * 16) = make_uint4(q[0], q[1], q[2], q[3]);
        *reinterpret_cast<uint4 *>(Bs + r * LDK + c * 16 + 8) = make_uint4(q[4], q[5], q[6], q[7]);
        if ((c * 16) % 32 == 0) Ds[r * (BK / 32) + c * 16 / 32] = hw_half(raw[i]);
      } else if constexpr (KIND == LG_Q8_0) {  // FAST: f16(d) * code rounds the exact product once
        static_assert(MODE == FAST, "Q8_0 tiles are FAST or SPLIT");
        half8 o0, o1;
        const _Float16 d = __builtin_bit_cast(_Float16, uint16_t(raw[i]));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          o0[j] = _Float16(int8_t(w[j / 4] >> (8 * (j % 4)))) * d;
          o1[j] = _Float16(int8_t(w[2 + j / 4] >> (8 * (j % 4)))) * d;
        }
        *reinterpret_cast<half8 *>(Bs + r * LDK + c * 16) = o0;
        *reinterpret_cast<half8 *>(Bs + r * LDK + c * 16 + 8) = o1;
      } else if constexpr (KIND == LG_Q6_K) {
        float f[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) f[j] = kq6_weight(sa[i], int8_t(w[j / 4] >> (8 * (j % 4))));
        put8(f, Bs + r * LDK + c * 16, Bl + r * LDK + c * 16, kSplitB);
        put8(f + 8, Bs + r * LDK + c * 16 + 8, Bl + r * LDK + c * 16 + 8, kSplitB);
      } else {  // Q4_K
        float lo[16], hi[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t byte = (w[j / 4] >> (8 * (j % 4))) & 0xffu;
          if constexpr (BK == 64) {
            lo[j] = kq4_weight(sa[i], byte & 15u, sb[i]);
            hi[j] = kq4_weight(sa2[i], byte >> 4, sb2[i]);
          } else {
            lo[j] = kq4_weight(sa[i], plane ? (byte >> 4) : (byte & 15u), sb[i]);
          }
        }
        put8(lo, Bs + r * LDK + c * 16, Bl + r * LDK + c * 16, kSplitB);
        put8(lo + 8, Bs + r * LDK + c * 16 + 8, Bl + r * LDK + c * 16 + 8, kSplitB);
        if constexpr (BK == 64) {
          put8(hi, Bs + r * LDK + 32 + c * 16, Bl + r * LDK + 32 + c * 16, kSplitB);
          put8(hi + 8, Bs + r * LDK + 32 + c * 16 + 8, Bl + r * LDK + 32 + c * 16 + 8, kSplitB);
        }
      }
    }
  }
};

// Tile order: the hardware hands consecutive workgroups to the 8 XCDs round-robin; give
// each XCD a contiguous range of tiles, and inside it walk groups of GM M-tiles so that the
// concurrently running tiles of one XCD share A rows and weight rows through its L2.
__device__ __forceinline__ void tile_coords(int bid, int nblk, int MT, int NT, int &mt, int &nt) {
  int t = bid;
  if ((nblk & 7) == 0) t = (bid & 7) * (nblk >> 3) + (bid >> 3);
#ifndef LG_GEMM_GROUP_M
#define LG_GEMM_GROUP_M 4
#endif
  constexpr int GM = LG_GEMM_GROUP_M;  // from a sweep of 1..32 at the 35,840-token shapes (within 3%)
  const int group = t / (GM * NT);
  const int first = group * GM;
  const int gm = min(MT - first, GM);
  const int in = t - group * GM * NT;
  mt = first + in % gm;
  nt = in / gm;
}

#define MFMA(a, b, c) __builtin_amdgcn_mfma_f32_32x32x16_f16((a), (b), (c), 0, 0, 0)

// Activation tile loader: BMW x BK halves (+ the lo plane), 16-byte chunks per thread, read with
// buffer loads: the per-thread byte offsets are fixed at init (rows >= M clamped to M - 1, never
// stored), the K position goes in the scalar offset.  The host keeps M * K * 2 below 2^31.
template <int BMW, int BK, bool SPLITA>
struct ALoad {
  static constexpr int kPer = BMW * BK / 8 / 256;
  static constexpr int kRowStep = 256 / (BK / 8);  // rows between a thread's chunks
  typedef uint32_t vec __attribute__((ext_vector_type(4 * kPer)));
  typedef uint32_t ovec __attribute__((ext_vector_type(kPer < 2 ? 2 : kPer)));
  vec v, vl;
  ovec off;
  __amdgpu_buffer_rsrc_t ra, rl;
  __device__ __forceinline__ void init(const _Float16 *A_, const _Float16 *Alo_, int m0, int M, int K, int t) {
    const int bytes = M * K * 2;
    ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(A_), 0, bytes, kBufferFlags);
    if constexpr (SPLITA) rl = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(Alo_), 0, bytes, kBufferFlags);
    const int row0 = m0 + t / (BK / 8), col = (t % (BK / 8)) * 8;
#pragma unroll
    for (int i = 0; i < kPer; ++i) off[i] = uint32_t((min(row0 + i * kRowStep, M - 1) * K + col) * 2);
  }
  __device__ __forceinline__ void fetch(int k0) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, off[i], k0 * 2, 0));
      v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
      if constexpr (SPLITA) {
        const uint4 y = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rl, off[i], k0 * 2, 0));
        vl[4 * i] = y.x; vl[4 * i + 1] = y.y; vl[4 * i + 2] = y.z; vl[4 * i + 3] = y.w;
      }
    }
  }
  template <int LDK>
  __device__ __forceinline__ void store(_Float16 *As, _Float16 *Al, int t) {
    const int r = t / (BK / 8), c = (t % (BK / 8)) * 8;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int at = (r + i * kRowStep) * LDK + c;
      *reinterpret_cast<uint4 *>(As + at) = make_uint4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
      if constexpr (SPLITA)
        *reinterpret_cast<uint4 *>(Al + at) = make_uint4(vl[4 * i], vl[4 * i + 1], vl[4 * i + 2], vl[4 * i + 3]);
    }
  }
};

// MFMAs of one staged K tile into acc (see the mode table at the top of the file).
template <uint32_t KIND, int MODE, int BK, int WTM, int WTN, int LDK>
__device__ __forceinline__ void mma_tile(f32x16 (&acc)[WTM][WTN], const _Float16 *As, const _Float16 *Al,
                                         const _Float16 *Bs, const _Float16 *Bl, const float *Ds, int wm,
                                         int wn, int lane) {
  constexpr bool kSplitA = MODE != FAST;
  constexpr bool kSplitB = MODE == SPLIT3;
  constexpr bool kScaled = MODE == SPLIT && KIND == LG_Q8_0;
  const int arow = (wm * (32 * WTM) + (lane & 31)) * LDK;
  const int brow = (wn * (32 * WTN) + (lane & 31)) * LDK;
  if constexpr (kScaled) {
    // per Q8_0 block and output block: a 4-MFMA chain into a partial p, then acc += d * p.
    // One partial is live at a time, so it stays in VGPRs and the scale FMAs of one chain
    // can issue under the MFMAs of the next.  Same operation order as the variant below.
    const f32x16 zero = {};
#pragma unroll
    for (int blk = 0; blk < BK / 32; ++blk) {
      half8 ah[2][WTM], al[2][WTM], b[2][WTN];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int kc = blk * 32 + kk * 16 + (lane >> 5) * 8;
#pragma unroll
        for (int j = 0; j < WTN; ++j) b[kk][j] = *reinterpret_cast<const half8 *>(Bs + brow + j * 32 * LDK + kc);
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
          ah[kk][i] = *reinterpret_cast<const half8 *>(As + arow + i * 32 * LDK + kc);
          al[kk][i] = *reinterpret_cast<const half8 *>(Al + arow + i * 32 * LDK + kc);
        }
      }
      float dj[WTN];
#pragma unroll
      for (int j = 0; j < WTN; ++j) dj[j] = Ds[(wn * (32 * WTN) + j * 32 + (lane & 31)) * (BK / 32) + blk];
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
          f32x16 p = MFMA(ah[0][i], b[0][j], zero);
          p = MFMA(al[0][i], b[0][j], p);
          p = MFMA(ah[1][i], b[1][j], p);
          p = MFMA(al[1][i], b[1][j], p);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += dj[j] * p[r];
        }
    }
  } else if constexpr (MODE == FAST) {
    // fragments of step kk+1 are read from LDS while the MFMAs of step kk issue
    constexpr int KS = BK / 16;
    half8 ca[WTM], cb[WTN];
    {
      const int kc = (lane >> 5) * 8;
#pragma unroll
      for (int j = 0; j < WTN; ++j) cb[j] = *reinterpret_cast<const half8 *>(Bs + brow + j * 32 * LDK + kc);
#pragma unroll
      for (int i = 0; i < WTM; ++i) ca[i] = *reinterpret_cast<const half8 *>(As + arow + i * 32 * LDK + kc);
    }
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      half8 na[WTM], nb[WTN];
      if (kk + 1 < KS) {
        const int kc = (kk + 1) * 16 + (lane >> 5) * 8;
#pragma unroll
        for (int j = 0; j < WTN; ++j) nb[j] = *reinterpret_cast<const half8 *>(Bs + brow + j * 32 * LDK + kc);
#pragma unroll
        for (int i = 0; i < WTM; ++i) na[i] = *reinterpret_cast<const half8 *>(As + arow + i * 32 * LDK + kc);
      }
#pragma unroll
      for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) acc[i][j] = MFMA(ca[i], cb[j], acc[i][j]);
      if (kk + 1 < KS) {
        // interleave: one LDS read, then a share of the MFMAs
        constexpr int R = WTM + WTN, Mf = WTM * WTN;
#pragma unroll
        for (int q = 0; q < R; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, Mf / R, 0);
        }
#pragma unroll
        for (int i = 0; i < WTM; ++i) ca[i] = na[i];
#pragma unroll
        for (int j = 0; j < WTN; ++j) cb[j] = nb[j];
      }
    }
  } else {
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int kc = kk * 16 + (lane >> 5) * 8;
      half8 b[WTN], c[kSplitB ? WTN : 1];
#pragma unroll
      for (int j = 0; j < WTN; ++j) {
        b[j] = *reinterpret_cast<const half8 *>(Bs + brow + j * 32 * LDK + kc);
        if constexpr (kSplitB) c[j] = *reinterpret_cast<const half8 *>(Bl + brow + j * 32 * LDK + kc);
      }
#pragma unroll
      for (int i = 0; i < WTM; ++i) {
        const half8 a = *reinterpret_cast<const half8 *>(As + arow + i * 32 * LDK + kc);
        half8 l;
        if constexpr (kSplitA) l = *reinterpret_cast<const half8 *>(Al + arow + i * 32 * LDK + kc);
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
          acc[i][j] = MFMA(a, b[j], acc[i][j]);
          if constexpr (kSplitA) acc[i][j] = MFMA(l, b[j], acc[i][j]);
          if constexpr (kSplitB) acc[i][j] = MFMA(a, c[j], acc[i][j]);
        }
      }
    }
  }
}

template <int MODE, int BK, int WTM, int WTN, int STAGES>
struct Cfg {
  static constexpr int kBM = 64 * WTM, kBN = 64 * WTN;
  static constexpr int kLDK = BK + 8;  // 16-byte row pad: conflict-free b128 LDS reads
  static constexpr bool kSplitA = MODE != FAST;
  static constexpr bool kSplitB = MODE == SPLIT3;
  static constexpr int kAPlane = kBM * kLDK;   // halves
  static constexpr int kBPlane = kBN * kLDK;   // halves
  static constexpr int kStageHalves = kAPlane * (kSplitA ? 2 : 1) + kBPlane * (kSplitB ? 2 : 1);
  static constexpr int kStageBytes = kStageHalves * 2 + kBN * (BK / 32) * 4;  // + block scales
  static constexpr int kLdsBytes = STAGES * kStageBytes;
};

template <uint32_t KIND, int EPI, int MODE, int BK, int WTM, int WTN, int STAGES>
__global__ __launch_bounds__(256) void gemm_kernel(const _Float16 *__restrict__ A,
                                                   const _Float16 *__restrict__ Alo, int M, int K,
                                                   DevMatrix W, float *__restrict__ C,
                                                   _Float16 *__restrict__ C16,
                                                   _Float16 *__restrict__ C16lo, int ldc,
                                                   const float *__restrict__ bias, int MT, int NT,
                                                   int ffn) {
  using CF = Cfg<MODE, BK, WTM, WTN, STAGES>;
  constexpr int BMW = CF::kBM, BNT = CF::kBN, LDK = CF::kLDK;
  constexpr bool kSplitA = CF::kSplitA, kSplitB = CF::kSplitB;
  constexpr bool kScaled = MODE == SPLIT && KIND == LG_Q8_0;
  static_assert(WTN % 2 == 0 || (EPI != int(Epi::SWIGLU) && EPI != int(Epi::GEGLU)),
                "gated epilogues pair gate and up blocks inside a wave");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int mt, nt;
  tile_coords(blockIdx.x, gridDim.x, MT, NT, mt, nt);
  const int m0 = mt * BMW;

  auto stage_ptrs = [&](int st, _Float16 *&As, _Float16 *&Al, _Float16 *&Bs, _Float16 *&Bl, float *&Ds) {
    _Float16 *base = reinterpret_cast<_Float16 *>(lds + st * CF::kStageBytes);
    As = base;
    Al = kSplitA ? base + CF::kAPlane : base;
    Bs = base + CF::kAPlane * (kSplitA ? 2 : 1);
    Bl = kSplitB ? Bs + CF::kBPlane : Bs;
    Ds = reinterpret_cast<float *>(base + CF::kStageHalves);
  };
  // local weight-tile row -> weight row
  auto wrow = [&](int r) -> int {
    if (EPI == int(Epi::SWIGLU) || EPI == int(Epi::GEGLU)) {
      // wave column r/(32 WTN); block jb = (r/32) % WTN: gate for jb < WTN/2, up otherwise
      const int wc = r / (32 * WTN), jb = (r >> 5) % WTN;
      const int up = jb >= WTN / 2, jj = jb % (WTN / 2);
      return up * ffn + nt * (BNT / 2) + wc * (16 * WTN) + jj * 32 + (r & 31);
    }
    return nt * BNT + r;
  };

  using BL = BLoad<KIND, MODE, BK, BNT>;
  using AL = ALoad<BMW, BK, kSplitA>;
  AL al;
  al.init(A, Alo, m0, M, K, t);
  BL bl;
  bl.init(W, wrow, t);
  f32x16 acc[WTM][WTN];
#pragma unroll
  for (int i = 0; i < WTM; ++i)
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = K / BK;
  al.fetch(0);
  bl.fetch(W, wrow, 0, t);
  if constexpr (STAGES == 2) {
    {
      _Float16 *As, *Al, *Bs, *Bl;
      float *Ds;
      stage_ptrs(0, As, Al, Bs, Bl, Ds);
      al.template store<LDK>(As, Al, t);
      bl.template store<LDK>(Bs, Bl, Ds, t);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) {  // in flight during the MFMAs below
        al.fetch((kt + 1) * BK);
        bl.fetch(W, wrow, (kt + 1) * BK, t);
      }
      _Float16 *As, *Al, *Bs, *Bl;
      float *Ds;
      stage_ptrs(cur, As, Al, Bs, Bl, Ds);
      mma_tile<KIND, MODE, BK, WTM, WTN, LDK>(acc, As, Al, Bs, Bl, Ds, wm, wn, lane);
      if (kt + 1 < nk) {
        stage_ptrs(cur ^ 1, As, Al, Bs, Bl, Ds);
        al.template store<LDK>(As, Al, t);
        bl.template store<LDK>(Bs, Bl, Ds, t);
      }
      __syncthreads();
    }
  } else {
    _Float16 *As, *Al, *Bs, *Bl;
    float *Ds;
    stage_ptrs(0, As, Al, Bs, Bl, Ds);
    for (int kt = 0; kt < nk; ++kt) {
      __syncthreads();
      al.template store<LDK>(As, Al, t);
      bl.template store<LDK>(Bs, Bl, Ds, t);
      __syncthreads();
      if (kt + 1 < nk) {
        al.fetch((kt + 1) * BK);
        bl.fetch(W, wrow, (kt + 1) * BK, t);
      }
      mma_tile<KIND, MODE, BK, WTM, WTN, LDK>(acc, As, Al, Bs, Bl, Ds, wm, wn, lane);
    }
  }

  // epilogue: acc[i][j] register r -> row (r/4)*8 + (lane/32)*4 + r%4, column lane%32
  const int col_in = lane & 31;
#pragma unroll
  for (int i = 0; i < WTM; ++i) {
    // the residual add reads a 32-row block's values first, all in one round trip (rows past M read
    // row M - 1 and are not stored)
    float cv[16][EPI == int(Epi::ADD) ? WTN : 1];
    if constexpr (EPI == int(Epi::ADD)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = min(m0 + wm * (32 * WTM) + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3), M - 1);
#pragma unroll
        for (int j = 0; j < WTN; ++j) cv[r][j] = C[int64_t(row) * ldc + nt * BNT + wn * (32 * WTN) + j * 32 + col_in];
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * (32 * WTM) + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (row >= M) continue;
      if (EPI == int(Epi::SWIGLU) || EPI == int(Epi::GEGLU)) {
#pragma unroll
        for (int jj = 0; jj < WTN / 2; ++jj) {
          const int col = nt * (BNT / 2) + wn * (16 * WTN) + jj * 32 + col_in;
          const float g = acc[i][jj][r];
          const float v = (EPI == int(Epi::SWIGLU) ? silu(g) : gelu_tanh(g)) * acc[i][jj + WTN / 2][r];
          _Float16 h, hl;
          split_f16(v, h, hl);
          C16[int64_t(row) * ldc + col] = h;
          if (C16lo) C16lo[int64_t(row) * ldc + col] = hl;
        }
      } else {
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
          const int col = nt * BNT + wn * (32 * WTN) + j * 32 + col_in;
          float v = acc[i][j][r];
          if (EPI == int(Epi::F32)) {
            if (bias) v += bias[col];
            C[int64_t(row) * ldc + col] = v;
          } else if constexpr (EPI == int(Epi::ADD)) {
            if (bias) v += bias[col];
            C[int64_t(row) * ldc + col] = cv[r][j] + v;
          } else {
            if (bias) v += bias[col];
            if (EPI == int(Epi::RELU16)) v = fmaxf(v, 0.0f);
            _Float16 h, hl;
            split_f16(v, h, hl);
            C16[int64_t(row) * ldc + col] = h;
            if (C16lo) C16lo[int64_t(row) * ldc + col] = hl;
          }
        }
      }
    }
  }
}

template <uint32_t KIND, int MODE, int BK, int WTM, int WTN, int STAGES>
bool launch_cfg(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi, float *C,
                _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, hipStream_t st) {
  using CF = Cfg<MODE, BK, WTM, WTN, STAGES>;
  const bool glu = epi == Epi::SWIGLU || epi == Epi::GEGLU;
  if (glu && WTN % 2) return false;  // gated epilogues need gate and up blocks in one wave
  const int outN = glu ? W.rows / 2 : W.rows;
  const int tileN = glu ? CF::kBN / 2 : CF::kBN;
  if (outN % tileN) return false;
  const int NT = outN / tileN;
  const int K = W.cols, ffn = W.rows / 2;
  if (KIND == LG_Q8_0)
    LG_REQUIRE(int64_t(W.rows) * W.cols < (1ll << 31), "gemm: Q8_0 matrix beyond 2 GiB of codes");
  // buffer offsets of A are 32-bit: launch row blocks of at most 2 GiB of activations each
  const int64_t rows_cap = ((1ll << 31) - 1) / (int64_t(K) * 2) / CF::kBM * CF::kBM;
  LG_REQUIRE(rows_cap > 0, "gemm: K=%d too large", K);
  // an installed kernel timer spans the launches of all row blocks: start on the first, stop on the last
  KernelTimer *timer = kernel_timer();
  const KernelTimer whole = timer ? *timer : KernelTimer{};
  for (int m0 = 0; m0 < M;) {
    const int Mc = int(std::min<int64_t>(M - m0, rows_cap));
    if (timer) {
      timer->start = m0 == 0 ? whole.start : nullptr;
      timer->stop = m0 + Mc >= M ? whole.stop : nullptr;
    }
    const int MT = (Mc + CF::kBM - 1) / CF::kBM;
    LG_REQUIRE(int64_t(MT) * NT < (1ll << 31), "gemm: grid too large");
    const dim3 grid(MT * NT), block(256);
    const _Float16 *Ac = A + int64_t(m0) * K, *Alc = Alo ? Alo + int64_t(m0) * K : nullptr;
    float *Cc = C ? C + int64_t(m0) * ldc : nullptr;
    _Float16 *C16c = C16 ? C16 + int64_t(m0) * ldc : nullptr, *C16lc = C16lo ? C16lo + int64_t(m0) * ldc : nullptr;
#define LAUNCH(E)                                                                                              \
  do {                                                                                                         \
    auto fn = gemm_kernel<KIND, E, MODE, BK, WTM, WTN, STAGES>;                                                \
    static bool attr = false;                                                                                  \
    if (!attr) {                                                                                               \
      HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(fn),                                        \
                                    hipFuncAttributeMaxDynamicSharedMemorySize, CF::kLdsBytes));                \
      attr = true;                                                                                             \
    }                                                                                                          \
    launch_timed(fn, grid, block, CF::kLdsBytes, st, Ac, Alc, Mc, K, W, Cc, C16c, C16lc, ldc, bias, MT, NT,    \
                 ffn);                                                                                         \
  } while (0)
    switch (epi) {
      case Epi::F32: LAUNCH(0); break;
      case Epi::ADD: LAUNCH(1); break;
      case Epi::F16: LAUNCH(2); break;
      case Epi::SWIGLU:
        if constexpr (WTN % 2 == 0) LAUNCH(3);
        break;
      case Epi::GEGLU:
        if constexpr (WTN % 2 == 0) LAUNCH(4);
        break;
      case Epi::RELU16: LAUNCH(5); break;
    }
    m0 += Mc;
  }
  if (timer) *timer = whole;
#undef LAUNCH
  return true;
}

}  // namespace

// Exact Q8_0 tiles, built in their own translation unit (k_gemm_q8.hip) with MFMA results in
// VGPRs, where the per-block scale FMAs read the partial sums without AGPR copies.
bool launch_gemm_q8_exact(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi,
                          float *C, _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias,
                          hipStream_t st);

// Exact GEMM on 256 x 256 tiles over the weight's prefill copy (gemm_wide.h: Q8_0, F16, Q4_K,
// Q6_K), for launches with at least as many tiles as the device has CUs.  Same per-element
// operation order as the exact 128 x 128 tiles, so the two give the same bits.  Returns false
// (nothing launched) when the matrix has no prefill copy or the shape or epilogue is not one it
// takes.
bool launch_gemm_wide(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi, float *C,
                      _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, hipStream_t st);

}  // namespace lg
