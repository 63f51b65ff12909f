// Prefill GEMM tiles for gfx950 (shared by the k_gemm*.hip translation units): C = A . W^T on MFMA
// v_mfma_f32_16x16x32_f16 (each instruction one 32-deep K chunk), f32 accumulation, weights
// dequantised into LDS, epilogue fused (bias, residual add, SwiGLU, f16 store).
//
// Numeric modes (selected by the caller):
//   FAST  : A in f16, W dequantised to f16 (RNE); one MFMA pass.
//   SPLIT : A given as two f16 planes (hi = f16(a), lo = f16(a - hi)), so A carries ~22
//           significand bits.  F16 weights are exact in f16 -> 2 passes (hi, lo).
//           Q8_0 codes are exact in f16 and the block scale is applied in f32 per 32-element
//           block (partial sums on MFMA, acc += d * partial) -> 2 passes, weights exact.
//           Q4_K with the two-pass prefill copy (DevMatrix::pcr): w = A q - B per 32-element
//           sub-block, codes q exact in f16 and A applied per sub-block as the Q8_0 scale (2 passes),
//           after a correction GEMM of depth K/32 over the activation's chunk sums and -B (3 passes):
//           x.w = sum_c A_c (x_c . q_c) - sum_c B_c (sum x_c).
//   SPLIT3: K-quants (Q4_K, Q6_K) whose dequantised f32 weight needs 24 bits: W is split into
//           hi/lo f16 too and acc += Ah.Bh + Al.Bh + Ah.Bl -> 3 passes.
// The split modes reproduce f32 arithmetic to ~2^-22 relative per product, which the
// ill-conditioned synthetic workloads need to stay within the parity bars.
//
// Geometry: 256 threads = 4 wave64s in a 2 x 2 arrangement; each wave owns a (16 HM) x (16 HN)
// tile, HM x HN MFMA blocks of 16 x 16, so a workgroup tile is (32 HM) x (32 HN) x BK.  STAGES = 2 ping-pongs
// two LDS buffers (one barrier per K step, next tile's global loads in flight during the
// MFMAs); STAGES = 1 uses one buffer with the next tile prefetched into registers.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>

#include "act.h"
#include "common.h"
#include "kernels.h"
#include "f16split.h"
#include "quant.h"

namespace lg {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum Mode { FAST = 0, SPLIT = 1, SPLIT3 = 2 };


__device__ __forceinline__ float silu(float g) { return g * (1.0f / (1.0f + __expf(-g))); }

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
      } else if constexpr (KIND == LG_Q4_K && MODE == SPLIT) {
        // two-pass form: the codes as f16 (exact, 0..15; bytes under a 0x64 high byte read as f16 are
        // 1024 + q, one packed subtraction leaves q) and the sub-block scales A = d*sc; the low nibbles
        // are elements 16c + j of the 64-deep step, the high nibbles 32 + 16c + j
        static_assert(BK == 64, "two-pass Q4_K tiles take 64-deep K steps");
        typedef _Float16 half2v __attribute__((ext_vector_type(2)));
        const half2v bias = {_Float16(1024.0f), _Float16(1024.0f)};
        uint32_t lo8[8], hi8[8];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t ul = w[d] & 0x0f0f0f0fu, uh = (w[d] >> 4) & 0x0f0f0f0fu;
          lo8[2 * d] = __builtin_amdgcn_perm(0x64646464u, ul, 0x04010400u);
          lo8[2 * d + 1] = __builtin_amdgcn_perm(0x64646464u, ul, 0x04030402u);
          hi8[2 * d] = __builtin_amdgcn_perm(0x64646464u, uh, 0x04010400u);
          hi8[2 * d + 1] = __builtin_amdgcn_perm(0x64646464u, uh, 0x04030402u);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          lo8[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, lo8[e]) - bias);
          hi8[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, hi8[e]) - bias);
        }
        *reinterpret_cast<uint4 *>(Bs + r * LDK + c * 16) = make_uint4(lo8[0], lo8[1], lo8[2], lo8[3]);
        *reinterpret_cast<uint4 *>(Bs + r * LDK + c * 16 + 8) = make_uint4(lo8[4], lo8[5], lo8[6], lo8[7]);
        *reinterpret_cast<uint4 *>(Bs + r * LDK + 32 + c * 16) = make_uint4(hi8[0], hi8[1], hi8[2], hi8[3]);
        *reinterpret_cast<uint4 *>(Bs + r * LDK + 32 + c * 16 + 8) = make_uint4(hi8[4], hi8[5], hi8[6], hi8[7]);
        if (c == 0) {
          Ds[r * 2] = sa[i];
          Ds[r * 2 + 1] = sa2[i];
        }
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

#define MFMA(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

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

// MFMAs of one staged K tile into acc (see the mode table at the top of the file).  Operand
// layout of v_mfma_f32_16x16x32_f16: lane l holds row (l % 16) of a 16-row A block and column
// (l % 16) of a 16-column B block, k = 8 (l / 16) .. + 8 of the 32-deep chunk; the result block
// holds rows 4 (l / 16) .. + 4 of column l % 16.  Per output element and 32-deep chunk the
// operation sequence is (acc as f32):
//   FAST  : acc += A.W
//   SPLIT : F16 weights: acc += A_hi.W, acc += A_lo.W;  Q8_0 / Q4_K codes: p = A_hi.W, p += A_lo.W,
//           acc += d * p (d the chunk's Q8_0 block scale or Q4_K sub-block scale d*sc, f32 FMA);
//           a two-pass Q4_K launch first runs its correction (SPLIT3 order over the chunk sums and
//           the -B 2^e planes) and multiplies acc by 2^-e per column
//   SPLIT3: acc += A_hi.W_hi, acc += A_lo.W_hi, acc += A_hi.W_lo
// gemm_wide.h keeps the same sequences, so both tilings give the same bits.
template <uint32_t KIND, int MODE, int BK, int HM, int HN, int LDK>
__device__ __forceinline__ void mma_tile(f32x4 (&acc)[HM][HN], const _Float16 *As, const _Float16 *Al,
                                         const _Float16 *Bs, const _Float16 *Bl, const float *Ds, int wm,
                                         int wn, int lane) {
  constexpr bool kSplitA = MODE != FAST;
  constexpr bool kSplitB = MODE == SPLIT3;
  constexpr bool kScaled = MODE == SPLIT && (KIND == LG_Q8_0 || KIND == LG_Q4_K);
  constexpr int MI = HM, NJ = HN;
  const int arow = (wm * (16 * HM) + (lane & 15)) * LDK;
  const int brow = (wn * (16 * HN) + (lane & 15)) * LDK;
  const int kl = (lane >> 4) * 8;
  const f32x4 zero = {};
#pragma unroll
  for (int blk = 0; blk < BK / 32; ++blk) {
    const int kc = blk * 32 + kl;
    half8 ah[MI], al[kSplitA ? MI : 1], b[NJ], c[kSplitB ? NJ : 1];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      b[j] = *reinterpret_cast<const half8 *>(Bs + brow + j * 16 * LDK + kc);
      if constexpr (kSplitB) c[j] = *reinterpret_cast<const half8 *>(Bl + brow + j * 16 * LDK + kc);
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      ah[i] = *reinterpret_cast<const half8 *>(As + arow + i * 16 * LDK + kc);
      if constexpr (kSplitA) al[i] = *reinterpret_cast<const half8 *>(Al + arow + i * 16 * LDK + kc);
    }
    if constexpr (kScaled) {
      float dj[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) dj[j] = Ds[(wn * (16 * HN) + j * 16 + (lane & 15)) * (BK / 32) + blk];
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          f32x4 p = MFMA(ah[i], b[j], zero);
          p = MFMA(al[i], b[j], p);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] += dj[j] * p[r];
        }
    } else {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          acc[i][j] = MFMA(ah[i], b[j], acc[i][j]);
          if constexpr (kSplitA) acc[i][j] = MFMA(al[i], b[j], acc[i][j]);
          if constexpr (kSplitB) acc[i][j] = MFMA(ah[i], c[j], acc[i][j]);
        }
    }
  }
}

template <int MODE, int BK, int HM, int HN, int STAGES>
struct Cfg {
  static constexpr int kBM = 32 * HM, kBN = 32 * HN;
  static constexpr int kLDK = BK + 8;  // 16-byte row pad: conflict-free b128 LDS reads
  static constexpr bool kSplitA = MODE != FAST;
  static constexpr bool kSplitB = MODE == SPLIT3;
  static constexpr int kAPlane = kBM * kLDK;   // halves
  static constexpr int kBPlane = kBN * kLDK;   // halves
  static constexpr int kStageHalves = kAPlane * (kSplitA ? 2 : 1) + kBPlane * (kSplitB ? 2 : 1);
  static constexpr int kStageBytes = kStageHalves * 2 + kBN * (BK / 32) * 4;  // + block scales
  static constexpr int kLdsBytes = STAGES * kStageBytes;
};

// LDS of one launch: a two-pass Q4_K launch's correction stages four planes (SPLIT3) in the same space.
template <uint32_t KIND, int MODE, int BK, int HM, int HN, int STAGES>
constexpr int lds_bytes() {
  constexpr int main = Cfg<MODE, BK, HM, HN, STAGES>::kLdsBytes;
  constexpr int corr = Cfg<SPLIT3, BK, HM, HN, 1>::kStageBytes;
  return KIND == LG_Q4_K && MODE == SPLIT && corr > main ? corr : main;
}

// Epilogue of a q|k|v projection that rotates and stores q, k and v itself (RopeKvOut), as the RoPE
// kernel would from the f32 rows: tiles of 64 weight rows (HN == 2), each wave's two 16-row blocks a
// rotate-half pair of 16 dims each (d and d + hd/2 of one head), so the pair sits in one lane.
constexpr int kTileEpiRope = 16;

// ks / kslo: the chunk-sum planes of a two-pass Q4_K launch ([M][W.pkp] each), unused otherwise.
// ro: the q|k|v outputs of EPI == kTileEpiRope (row r of the launch is ro's row ro_row0 + r).
template <uint32_t KIND, int EPI, int MODE, int BK, int HM, int HN, int STAGES>
__global__ __launch_bounds__(256) void gemm_kernel(const _Float16 *__restrict__ A,
                                                   const _Float16 *__restrict__ Alo, int M, int K,
                                                   DevMatrix W, float *__restrict__ C,
                                                   _Float16 *__restrict__ C16,
                                                   _Float16 *__restrict__ C16lo, int ldc,
                                                   const float *__restrict__ bias, int MT, int NT,
                                                   int ffn, const _Float16 *__restrict__ ks,
                                                   const _Float16 *__restrict__ kslo, RopeKvOut ro, int ro_row0) {
  using CF = Cfg<MODE, BK, HM, HN, STAGES>;
  constexpr int BMW = CF::kBM, BNT = CF::kBN, LDK = CF::kLDK;
  constexpr bool kSplitA = CF::kSplitA, kSplitB = CF::kSplitB;
  constexpr bool kScaled = MODE == SPLIT && (KIND == LG_Q8_0 || KIND == LG_Q4_K);
  static_assert(HN % 2 == 0 || (EPI != int(Epi::SWIGLU) && EPI != int(Epi::GEGLU)),
                "gated epilogues pair gate and up blocks inside a wave");
  static_assert(EPI != kTileEpiRope || HN == 2, "the rotating epilogue takes 64-row tiles");
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
      // wave column r/(16 HN); 16-row block jb = (r/16) % HN: gate for jb < HN/2, up otherwise
      const int wc = r / (16 * HN), jb = (r >> 4) % HN;
      const int up = jb >= HN / 2, jj = jb % (HN / 2);
      return up * ffn + nt * (BNT / 2) + wc * (8 * HN) + jj * 16 + (r & 15);
    }
    if (EPI == kTileEpiRope) {
      // tile nt: pair offsets 32 (nt % (hd/64)) .. + 32 of head nt / (hd/64) of this part; wave column
      // r/32 takes 16 of them, block (r/16) % 2 the first or the second dim of each pair
      const int hpt = ro.hd / 64, p = (nt % hpt) * 32 + (r / 32) * 16 + (r & 15);
      return (nt / hpt) * ro.hd + p + ((r >> 4) & 1) * (ro.hd / 2);
    }
    return nt * BNT + r;
  };

  using BL = BLoad<KIND, MODE, BK, BNT>;
  using AL = ALoad<BMW, BK, kSplitA>;
  AL al;
  al.init(A, Alo, m0, M, K, t);
  BL bl;
  bl.init(W, wrow, t);
  constexpr int MI = HM, NJ = HN;
  f32x4 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;

  if constexpr (KIND == LG_Q4_K && MODE == SPLIT) {
    // correction of the two-pass form: acc = (sum_c ks[m][c] (-B[n][c] 2^e_n)) 2^-e_n, a GEMM of depth
    // W.pkp over the chunk sums and the correction planes (f16 hi/lo each, SPLIT3 order), staged
    // four planes at a time through one LDS buffer with the next step prefetched into registers
    using CC = Cfg<SPLIT3, BK, HM, HN, 1>;
    const int kp = W.pkp;
    DevMatrix Ch = W;  // the correction planes read as F16 matrices [rows][kp]
    Ch.kind = LG_F16;
    Ch.cols = kp;
    Ch.q = W.pcl;
    DevMatrix Cl = Ch;
    Cl.q = W.pcl + int64_t(W.rows) * kp;
    ALoad<BMW, BK, true> ka;
    ka.init(ks, kslo, m0, M, kp, t);
    BLoad<LG_F16, SPLIT3, BK, BNT> ch, cl;
    _Float16 *Cs = reinterpret_cast<_Float16 *>(lds);
    _Float16 *Csl = Cs + CC::kAPlane, *Cb = Cs + 2 * CC::kAPlane, *Cbl = Cb + CC::kBPlane;
    const int nkc = kp / BK;
    ka.fetch(0);
    ch.fetch(Ch, wrow, 0, t);
    cl.fetch(Cl, wrow, 0, t);
    for (int kt = 0; kt < nkc; ++kt) {
      if (kt) __syncthreads();
      ka.template store<LDK>(Cs, Csl, t);
      ch.template store<LDK>(Cb, Cb, nullptr, t);
      cl.template store<LDK>(Cbl, Cbl, nullptr, t);
      __syncthreads();
      if (kt + 1 < nkc) {
        ka.fetch((kt + 1) * BK);
        ch.fetch(Ch, wrow, (kt + 1) * BK, t);
        cl.fetch(Cl, wrow, (kt + 1) * BK, t);
      }
      mma_tile<LG_F16, SPLIT3, BK, HM, HN, LDK>(acc, Cs, Csl, Cb, Cbl, nullptr, wm, wn, lane);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float rs = W.pcr[wrow(wn * (16 * HN) + j * 16 + (lane & 15))];
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] *= rs;
    }
    __syncthreads();  // the main loop's stores reuse the LDS
  }

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
      mma_tile<KIND, MODE, BK, HM, HN, LDK>(acc, As, Al, Bs, Bl, Ds, wm, wn, lane);
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
      mma_tile<KIND, MODE, BK, HM, HN, LDK>(acc, As, Al, Bs, Bl, Ds, wm, wn, lane);
    }
  }

  if constexpr (EPI == kTileEpiRope) {
    // each lane holds dims d = p and d + hd/2 (blocks 0 and 1) of four rows; the values are the f32
    // acc (+ bias) an F32 epilogue would store, rotated by rope_pair and split by split_f16 as the RoPE
    // kernel does: q to scaled hi/lo planes [M][hq hd], k to its K page row, v to its V page column
    const int hd = ro.hd, half = hd / 2, hpt = hd / 64;
    const int p = (nt % hpt) * 32 + wn * 16 + (lane & 15);
    const int pcol = (nt / hpt) * hd + p;  // output column of dim p within this part
    const int head = (ro.col0 + pcol) / hd;
    const int part = head < ro.hq ? 0 : head < ro.hq + ro.hkv ? 1 : 2;  // q, k, v
    const int PT = ro.page_tokens, plane = PT * hd, kvp = ro.kv_planes;
    const float b0 = bias ? bias[pcol] : 0.0f, b1 = bias ? bias[pcol + half] : 0.0f;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * (16 * HM) + i * 16 + (lane >> 4) * 4 + r;
        if (row >= M) continue;
        const int grow = ro_row0 + row;
        const int pos = ro.tok_pos[grow];
        const int64_t page = ro.tok_page[grow];
        float v0 = acc[i][0][r], v1 = acc[i][1][r];
        if (bias) {
          v0 += b0;
          v1 += b1;
        }
        _Float16 h, l;
        if (part < 2) {
          const int64_t tb = int64_t(pos) * hd + p;
          float a, c;
          rope_pair(v0, v1, ro.cosT[tb], ro.sinT[tb], ro.cosT[tb + half], ro.sinT[tb + half], a, c);
          if (part == 0) {
            _Float16 *dh = ro.q16 + int64_t(grow) * (ro.hq * hd) + head * hd + p;
            _Float16 *dl = ro.q16lo + int64_t(grow) * (ro.hq * hd) + head * hd + p;
            split_f16(a * ro.qscale, h, l);
            dh[0] = h;
            dl[0] = l;
            split_f16(c * ro.qscale, h, l);
            dh[half] = h;
            dl[half] = l;
          } else {
            const int64_t blk = page * ro.page_stride + int64_t(head - ro.hq) * plane;
            _Float16 *dh = ro.kpool + kvp * blk + (pos % PT) * hd + p;
            split_f16(a, h, l);
            dh[0] = h;
            if (kvp == 2) dh[plane] = l;
            split_f16(c, h, l);
            dh[half] = h;
            if (kvp == 2) dh[plane + half] = l;
          }
        } else {
          const int64_t blk = page * ro.page_stride + int64_t(head - ro.hq - ro.hkv) * plane;
          _Float16 *dh = ro.vpool + kvp * blk + int64_t(p) * PT + (pos % PT);
          split_f16(v0, h, l);
          dh[0] = h;
          if (kvp == 2) dh[plane] = l;
          split_f16(v1, h, l);
          dh[int64_t(half) * PT] = h;
          if (kvp == 2) dh[plane + int64_t(half) * PT] = l;
        }
      }
    }
    return;
  }

  // epilogue: acc[i][j] register r -> row 16 i + 4 (lane / 16) + r, column 16 j + lane % 16 of the
  // wave tile
  const int col_in = lane & 15;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    // the residual add reads a 16-row block's values first, all in one round trip (rows past M read
    // row M - 1 and are not stored)
    float cv[4][EPI == int(Epi::ADD) ? NJ : 1];
    if constexpr (EPI == int(Epi::ADD)) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = min(m0 + wm * (16 * HM) + i * 16 + (lane >> 4) * 4 + r, M - 1);
#pragma unroll
        for (int j = 0; j < NJ; ++j) cv[r][j] = C[int64_t(row) * ldc + nt * BNT + wn * (16 * HN) + j * 16 + col_in];
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + wm * (16 * HM) + i * 16 + (lane >> 4) * 4 + r;
      if (row >= M) continue;
      if (EPI == int(Epi::SWIGLU) || EPI == int(Epi::GEGLU)) {
        // gate block j pairs with up block j + NJ / 2 (the same output columns)
#pragma unroll
        for (int j = 0; j < NJ / 2; ++j) {
          const int col = nt * (BNT / 2) + wn * (8 * HN) + j * 16 + col_in;
          const float g = acc[i][j][r];
          const float v = (EPI == int(Epi::SWIGLU) ? silu(g) : gelu_tanh(g)) * acc[i][j + NJ / 2][r];
          _Float16 h, hl;
          split_f16(v, h, hl);
          C16[int64_t(row) * ldc + col] = h;
          if (C16lo) C16lo[int64_t(row) * ldc + col] = hl;
        }
      } else {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int col = nt * BNT + wn * (16 * HN) + j * 16 + col_in;
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

template <uint32_t KIND, int MODE, int BK, int HM, int HN, int STAGES>
bool launch_cfg(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi, float *C,
                _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, hipStream_t st,
                const _Float16 *ks = nullptr) {
  using CF = Cfg<MODE, BK, HM, HN, STAGES>;
  const bool glu = epi == Epi::SWIGLU || epi == Epi::GEGLU;
  if (glu && HN % 2) return false;  // gated epilogues need gate and up blocks in one wave
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
    const _Float16 *ksc = ks ? ks + int64_t(m0) * W.pkp : nullptr;
    const _Float16 *kslc = ks ? ks + (int64_t(M) + m0) * W.pkp : nullptr;
    constexpr int lds = lds_bytes<KIND, MODE, BK, HM, HN, STAGES>();
#define LAUNCH(E)                                                                                              \
  do {                                                                                                         \
    auto fn = gemm_kernel<KIND, E, MODE, BK, HM, HN, STAGES>;                                                  \
    grant_lds(reinterpret_cast<const void *>(fn), lds);                                                        \
    launch_timed(fn, grid, block, lds, st, Ac, Alc, Mc, K, W, Cc, C16c, C16lc, ldc, bias, MT, NT, ffn, ksc,     \
                 kslc, RopeKvOut{}, 0);                                                                        \
  } while (0)
    switch (epi) {
      case Epi::F32: LAUNCH(0); break;
      case Epi::ADD: LAUNCH(1); break;
      case Epi::F16: LAUNCH(2); break;
      case Epi::SWIGLU:
        if constexpr (HN % 2 == 0) LAUNCH(3);
        break;
      case Epi::GEGLU:
        if constexpr (HN % 2 == 0) LAUNCH(4);
        break;
      case Epi::RELU16: LAUNCH(5); break;
    }
    m0 += Mc;
  }
  if (timer) *timer = whole;
#undef LAUNCH
  return true;
}

// The q|k|v projection (or a column range of it, ro.col0 a multiple of hd) on tiles of BM x 64 weight
// rows with the rotating epilogue; false (nothing launched) when the shape does not fit.
template <uint32_t KIND, int MODE, int BK, int HM, int STAGES>
bool launch_cfg_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                     const RopeKvOut &ro, hipStream_t st, const _Float16 *ks = nullptr) {
  using CF = Cfg<MODE, BK, HM, 2, STAGES>;
  if ((ro.hd != 64 && ro.hd != 128) || W.rows % ro.hd || ro.col0 % ro.hd || !Alo || !ro.q16lo) return false;
  const int K = W.cols, NT = W.rows / 64;
  const int64_t rows_cap = ((1ll << 31) - 1) / (int64_t(K) * 2) / CF::kBM * CF::kBM;
  if (int64_t(M) > rows_cap) return false;
  const int MT = (M + CF::kBM - 1) / CF::kBM;
  const dim3 grid(MT * NT), block(256);
  constexpr int lds = lds_bytes<KIND, MODE, BK, HM, 2, STAGES>();
  auto fn = gemm_kernel<KIND, kTileEpiRope, MODE, BK, HM, 2, STAGES>;
  grant_lds(reinterpret_cast<const void *>(fn), lds);
  const _Float16 *kslc = ks ? ks + int64_t(M) * W.pkp : nullptr;
  launch_timed(fn, grid, block, lds, st, A, Alo, M, K, W, static_cast<float *>(nullptr), static_cast<_Float16 *>(nullptr),
               static_cast<_Float16 *>(nullptr), 0, bias, MT, NT, W.rows / 2, ks, kslc, ro, 0);
  return true;
}

}  // namespace

// Exact Q8_0 tiles, built in their own translation unit (k_gemm_q8.hip) with MFMA results in
// VGPRs, where the per-block scale FMAs read the partial sums without AGPR copies.
bool launch_gemm_q8_exact(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi,
                          float *C, _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias,
                          hipStream_t st);
// launch_gemm_small_rope for Q8_0 weights (the exact Q8_0 tiles' translation unit).
bool launch_gemm_q8_small_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                               const RopeKvOut &ro, hipStream_t st);
// Exact two-pass Q4_K tiles (the same translation unit): codes, sub-block scales and the correction
// over the activation's chunk sums ks.
bool launch_gemm_q4_exact(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi,
                          float *C, _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias,
                          hipStream_t st, const _Float16 *ks);

// Exact GEMM on 256 x 256 tiles over the weight's prefill copy (gemm_wide.h: Q8_0, F16, Q4_K,
// Q6_K), for launches with at least as many tiles as the device has CUs.  Same per-element
// operation order as the exact 128 x 128 tiles, so the two give the same bits.  Returns false
// (nothing launched) when the matrix has no prefill copy or the shape or epilogue is not one it
// takes.
bool launch_gemm_wide(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, Epi epi, float *C,
                      _Float16 *C16, _Float16 *C16lo, int ldc, const float *bias, hipStream_t st,
                      const _Float16 *ks = nullptr);

}  // namespace lg
