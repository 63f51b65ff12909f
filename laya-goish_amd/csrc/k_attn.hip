// Causal GQA attention over the paged KV cache (gfx950).
//
// Reference semantics (src/models/openthai/model.rs:276-294, generalised to hq/hkv heads):
// for query i of head h, kv head kh = h / (hq/hkv), s_j = dot(q_i, k_j) / sqrt(hd) for
// j <= pos_i, p = softmax(s), out = sum_j p_j v_j.
//
// KV page layout (one layer, one page of P = 64 tokens), element type f16 or f32:
//   K: [hkv][P][hd] (row per token)     V: [hkv][hd][P] (column per token)
//
// Prefill: one wave per (32-query tile, query head).  S^T = K . Q^T on MFMA 32x32x16 f16, so
// each lane owns one query column and the online softmax reduces over its own registers plus
// one lane swap; O^T = V^T . P^T then consumes P straight from registers.  With an f32 cache
// and hi/lo query planes every product is split (hi.hi + lo.hi + hi.lo: three MFMAs), which
// keeps scores and outputs f32-faithful.
//
// Decode (one new token): one workgroup per (kv head, page): coalesced reads of the page's K
// rows and V columns, RoPE of the group's query heads (and, on the last page, of the new key,
// which it also writes into the cache), f32 scores for every query head of the group, partial
// (max, sum, out) per page; a second launch combines the pages of each query head.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "f16split.h"
#include "wave.h"

namespace lg {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int P = 64;  // tokens per page
constexpr float kLog2e = 1.4426950408889634f;

#define MFMA(a, b, c) __builtin_amdgcn_mfma_f32_32x32x16_f16((a), (b), (c), 0, 0, 0)

__device__ __forceinline__ void split8(const float *v, half8 &hi, half8 &lo) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    _Float16 h, l;
    split_f16(v[j], h, l);
    hi[j] = h;
    lo[j] = l;
  }
}

// SPLIT == false: f16 cache, f16 q.  SPLIT == true: f32 cache, q as hi/lo planes.
template <int HD, bool SPLIT>
__global__ __launch_bounds__(64) void attn_prefill_kernel(
    const _Float16 *__restrict__ q16, const _Float16 *__restrict__ q16lo, int hq, KvGeom g,
    const void *__restrict__ kpool, const void *__restrict__ vpool, const int32_t *__restrict__ pages,
    int max_pages, const int32_t *__restrict__ tile_seq, const int32_t *__restrict__ tile_row0,
    const int32_t *__restrict__ tile_pos0, const int32_t *__restrict__ tile_n,
    _Float16 *__restrict__ out16, _Float16 *__restrict__ out16lo) {
  using KV = typename std::conditional<SPLIT, float, _Float16>::type;
  constexpr int KT = HD / 16;  // k-steps of the QK^T product
  constexpr int DB = HD / 32;  // 32-wide d blocks of the output
  // Workgroups are dealt to the 8 XCDs round-robin (i -> XCD i % 8).  Map them so each XCD
  // takes one contiguous range of (head, tile) pairs, tiles fastest: all query tiles of one
  // (sequence, head) then run on one XCD and read that sequence's K/V through one L2.
  const int total = gridDim.x, ntiles = total / hq;
  const int xcd = blockIdx.x % 8, per = total / 8, rem = total % 8;
  const int logical = xcd * per + min(xcd, rem) + blockIdx.x / 8;
  const int tile = logical % ntiles, h = logical / ntiles;
  const int lane = threadIdx.x, qi = lane & 31, hl = lane >> 5;
  const int seq = tile_seq[tile], row0 = tile_row0[tile], pos0 = tile_pos0[tile], n = tile_n[tile];
  const int kh = h / (hq / g.hkv);
  const int qw = hq * HD;
  const int qpos = pos0 + qi;
  const bool live = qi < n;

  // Q^T operand: lane holds q[qi][16t + 8*hl .. +8]
  half8 qr[KT], ql[SPLIT ? KT : 1];
  {
    const int64_t off = int64_t(row0 + min(qi, n - 1)) * qw + h * HD + hl * 8;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      qr[t] = *reinterpret_cast<const half8 *>(q16 + off + 16 * t);
      if (SPLIT) ql[t] = *reinterpret_cast<const half8 *>(q16lo + off + 16 * t);
    }
  }
  f32x16 acc[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  const float scale = kLog2e / sqrtf(float(HD));
  const int last = pos0 + n - 1;
  const int32_t *ptab = pages + int64_t(seq) * max_pages;
  const KV *kbase = static_cast<const KV *>(kpool);
  const KV *vbase = static_cast<const KV *>(vpool);

  for (int kt = 0; kt <= last / P; ++kt) {
    const int64_t page = ptab[kt];
    const KV *Kp = kbase + page * g.page_stride + int64_t(kh) * P * HD;
    const KV *Vp = vbase + page * g.page_stride + int64_t(kh) * HD * P;
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
      const KV *kr = Kp + (kb * 32 + qi) * HD + hl * 8;
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        if constexpr (SPLIT) {
          float kv[8];
          const float4 a = *reinterpret_cast<const float4 *>(kr + 16 * t);
          const float4 b = *reinterpret_cast<const float4 *>(kr + 16 * t + 4);
          kv[0] = a.x; kv[1] = a.y; kv[2] = a.z; kv[3] = a.w;
          kv[4] = b.x; kv[5] = b.y; kv[6] = b.z; kv[7] = b.w;
          half8 kh8, kl8;
          split8(kv, kh8, kl8);
          s[kb] = MFMA(kh8, qr[t], s[kb]);
          s[kb] = MFMA(kl8, qr[t], s[kb]);
          s[kb] = MFMA(kh8, ql[t], s[kb]);
        } else {
          s[kb] = MFMA(*reinterpret_cast<const half8 *>(kr + 16 * t), qr[t], s[kb]);
        }
      }
    }
    // s[kb][r] <-> key kt*P + kb*32 + (r/4)*8 + hl*4 + r%4, query qi
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt * P + kb * 32 + (r >> 2) * 8 + hl * 4 + (r & 3);
        const float v = (key <= qpos && live) ? s[kb][r] * scale : -INFINITY;
        s[kb][r] = v;
        mt = fmaxf(mt, v);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mn = fmaxf(m, mt);
    const float alpha = mn == -INFINITY ? 1.0f : exp2f(m - mn);
    float rs = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = mn == -INFINITY ? 0.0f : exp2f(s[kb][r] - mn);
        s[kb][r] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 32);
    l = l * alpha + rs;
    m = mn;
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[b][r] *= alpha;
    // O^T += V^T . P^T over four 16-key chunks
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = s[c >> 1][(c & 1) * 8 + e];
      half8 ph, pl;
      if constexpr (SPLIT) split8(pv, ph, pl);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) ph[e] = _Float16(pv[e]);
#pragma unroll
      for (int b = 0; b < DB; ++b) {
        const KV *vr = Vp + (b * 32 + qi) * P + 16 * c + hl * 4;
        if constexpr (SPLIT) {
          const float4 lo4 = *reinterpret_cast<const float4 *>(vr);
          const float4 hi4 = *reinterpret_cast<const float4 *>(vr + 8);
          const float vv[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
          half8 vh, vl;
          split8(vv, vh, vl);
          acc[b] = MFMA(vh, ph, acc[b]);
          acc[b] = MFMA(vl, ph, acc[b]);
          acc[b] = MFMA(vh, pl, acc[b]);
        } else {
          const half4 lo = *reinterpret_cast<const half4 *>(vr);
          const half4 hi = *reinterpret_cast<const half4 *>(vr + 8);
          const half8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          acc[b] = MFMA(va, ph, acc[b]);
        }
      }
    }
  }
  if (!live) return;
  const float inv = 1.0f / l;
  const int64_t obase = int64_t(row0 + qi) * qw + h * HD;
  // acc[b][r] <-> d = b*32 + (r/4)*8 + hl*4 + r%4
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      half4 o, olo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        _Float16 oh, ol;
        split_f16(acc[b][r4 * 4 + j] * inv, oh, ol);
        o[j] = oh;
        olo[j] = ol;
      }
      const int64_t at = obase + b * 32 + r4 * 8 + hl * 4;
      *reinterpret_cast<half4 *>(out16 + at) = o;
      if (SPLIT) *reinterpret_cast<half4 *>(out16lo + at) = olo;
    }
}

// Position of key k (0..63) inside a V row in LDS: bits 2 and 3 swapped, so the eight keys one
// lane feeds to the O^T product (16c + 4hl + {0..3}, 16c + 8 + 4hl + {0..3}) sit in one
// 16-byte run at 16c + 8hl.
__device__ __forceinline__ int vperm(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

// Prefill, grouped: one workgroup of four waves per (group of <= 4 consecutive query tiles of
// one sequence, query head).  Each K/V page of the group passes through LDS once, already
// in MFMA operand form (hi/lo f16 planes with an f32 cache), and serves all four tiles; the
// next page is fetched into registers while the current one is consumed.  Wave w computes
// tile w with the arithmetic of attn_prefill_kernel, term for term, so both kernels give
// bit-identical outputs.
template <int HD, bool SPLIT>
__global__ __launch_bounds__(256, 1) void attn_prefill_grp_kernel(
    const _Float16 *__restrict__ q16, const _Float16 *__restrict__ q16lo, int hq, KvGeom g,
    const void *__restrict__ kpool, const void *__restrict__ vpool, const int32_t *__restrict__ pages,
    int max_pages, const int32_t *__restrict__ grp_first, const int32_t *__restrict__ grp_count,
    const int32_t *__restrict__ tile_seq, const int32_t *__restrict__ tile_row0,
    const int32_t *__restrict__ tile_pos0, const int32_t *__restrict__ tile_n,
    _Float16 *__restrict__ out16, _Float16 *__restrict__ out16lo) {
  using KV = typename std::conditional<SPLIT, float, _Float16>::type;
  constexpr int KT = HD / 16, DB = HD / 32;
  constexpr int NPL = SPLIT ? 2 : 1;      // f16 planes per operand
  constexpr int KS = HD + 8, VS = P + 8;  // padded LDS row strides (halves): conflict-free reads
  constexpr int EPL = SPLIT ? 4 : 8;      // KV values per 16-byte load
  constexpr int NLD = P * HD / (256 * EPL);
  static_assert(NLD * 256 * EPL == P * HD, "page must split evenly over 256 threads");
  __shared__ __align__(16) _Float16 kls[NPL][P * KS];
  __shared__ __align__(16) _Float16 vls[NPL][HD * VS];

  // Same XCD-contiguous mapping as attn_prefill_kernel, over (head, group) pairs.
  const int total = gridDim.x, ngroups = total / hq;
  const int xcd = blockIdx.x % 8, per = total / 8, rem = total % 8;
  const int logical = xcd * per + min(xcd, rem) + blockIdx.x / 8;
  const int grp = logical % ngroups, h = logical / ngroups;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, qi = lane & 31, hl = lane >> 5;
  const int t0 = grp_first[grp], cnt = grp_count[grp];
  const bool active = wave < cnt;
  const int tile = t0 + min(wave, cnt - 1);
  const int seq = tile_seq[tile], row0 = tile_row0[tile], pos0 = tile_pos0[tile], n = tile_n[tile];
  const int glast = tile_pos0[t0 + cnt - 1] + tile_n[t0 + cnt - 1] - 1;
  const int kh = h / (hq / g.hkv);
  const int qw = hq * HD;
  const int qpos = pos0 + qi;
  const bool live = qi < n;

  half8 qr[KT], ql[SPLIT ? KT : 1];
  {
    const int64_t off = int64_t(row0 + min(qi, n - 1)) * qw + h * HD + hl * 8;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      qr[t] = *reinterpret_cast<const half8 *>(q16 + off + 16 * t);
      if (SPLIT) ql[t] = *reinterpret_cast<const half8 *>(q16lo + off + 16 * t);
    }
  }
  f32x16 acc[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  const float scale = kLog2e / sqrtf(float(HD));
  const int npages = glast / P + 1;
  const int mypages = active ? (pos0 + n - 1) / P + 1 : 0;
  const int32_t *ptab = pages + int64_t(seq) * max_pages;
  const KV *kbase = static_cast<const KV *>(kpool) + int64_t(kh) * P * HD;
  const KV *vbase = static_cast<const KV *>(vpool) + int64_t(kh) * HD * P;

  uint4 kreg[NLD], vreg[NLD];
  // page-table entry of the page after the one in flight: loaded one iteration ahead, so the
  // K/V prefetch never waits on a page-table round trip
  int32_t next_page = ptab[min(1, npages - 1)];
  {
    const int64_t page = ptab[0];
    const uint4 *ks = reinterpret_cast<const uint4 *>(kbase + page * g.page_stride);
    const uint4 *vs = reinterpret_cast<const uint4 *>(vbase + page * g.page_stride);
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      kreg[j] = ks[tid + 256 * j];
      vreg[j] = vs[tid + 256 * j];
    }
  }

  for (int kt = 0; kt < npages; ++kt) {
    __syncthreads();  // every wave is done reading the previous page
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int e0 = (tid + 256 * j) * EPL;  // first value of this load within the page
      const int kro = (e0 / HD) * KS + e0 % HD;
      const int vd = e0 / P, vk = e0 % P;
      if constexpr (SPLIT) {
        const float4 kf = __builtin_bit_cast(float4, kreg[j]);
        const float4 vf = __builtin_bit_cast(float4, vreg[j]);
        const float kv[4] = {kf.x, kf.y, kf.z, kf.w}, vv[4] = {vf.x, vf.y, vf.z, vf.w};
        half4 khi, klo, vhi, vlo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 a, b, c, d;
          split_f16(kv[e], a, b);
          split_f16(vv[e], c, d);
          khi[e] = a;
          klo[e] = b;
          vhi[e] = c;
          vlo[e] = d;
        }
        *reinterpret_cast<half4 *>(&kls[0][kro]) = khi;
        *reinterpret_cast<half4 *>(&kls[1][kro]) = klo;
        const int vo = vd * VS + vperm(vk);
        *reinterpret_cast<half4 *>(&vls[0][vo]) = vhi;
        *reinterpret_cast<half4 *>(&vls[1][vo]) = vlo;
      } else {
        *reinterpret_cast<uint4 *>(&kls[0][kro]) = kreg[j];
        const half8 v8 = __builtin_bit_cast(half8, vreg[j]);
        const half4 va = {v8[0], v8[1], v8[2], v8[3]}, vb = {v8[4], v8[5], v8[6], v8[7]};
        *reinterpret_cast<half4 *>(&vls[0][vd * VS + vperm(vk)]) = va;
        *reinterpret_cast<half4 *>(&vls[0][vd * VS + vperm(vk + 4)]) = vb;
      }
    }
    __syncthreads();
    if (kt + 1 < npages) {
      const int64_t page = next_page;
      next_page = ptab[min(kt + 2, npages - 1)];
      const uint4 *ks = reinterpret_cast<const uint4 *>(kbase + page * g.page_stride);
      const uint4 *vs = reinterpret_cast<const uint4 *>(vbase + page * g.page_stride);
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
        kreg[j] = ks[tid + 256 * j];
        vreg[j] = vs[tid + 256 * j];
      }
    }
    if (kt >= mypages) continue;

    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
      const int ro = (kb * 32 + qi) * KS + hl * 8;
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const half8 kh8 = *reinterpret_cast<const half8 *>(&kls[0][ro + 16 * t]);
        if constexpr (SPLIT) {
          const half8 kl8 = *reinterpret_cast<const half8 *>(&kls[1][ro + 16 * t]);
          s[kb] = MFMA(kh8, qr[t], s[kb]);
          s[kb] = MFMA(kl8, qr[t], s[kb]);
          s[kb] = MFMA(kh8, ql[t], s[kb]);
        } else {
          s[kb] = MFMA(kh8, qr[t], s[kb]);
        }
      }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt * P + kb * 32 + (r >> 2) * 8 + hl * 4 + (r & 3);
        const float v = (key <= qpos && live) ? s[kb][r] * scale : -INFINITY;
        s[kb][r] = v;
        mt = fmaxf(mt, v);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mn = fmaxf(m, mt);
    const float alpha = mn == -INFINITY ? 1.0f : exp2f(m - mn);
    float rs = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = mn == -INFINITY ? 0.0f : exp2f(s[kb][r] - mn);
        s[kb][r] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 32);
    l = l * alpha + rs;
    m = mn;
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[b][r] *= alpha;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = s[c >> 1][(c & 1) * 8 + e];
      half8 ph, pl;
      if constexpr (SPLIT) split8(pv, ph, pl);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) ph[e] = _Float16(pv[e]);
#pragma unroll
      for (int b = 0; b < DB; ++b) {
        const int vo = (b * 32 + qi) * VS + 16 * c + hl * 8;
        const half8 vh = *reinterpret_cast<const half8 *>(&vls[0][vo]);
        if constexpr (SPLIT) {
          const half8 vl = *reinterpret_cast<const half8 *>(&vls[1][vo]);
          acc[b] = MFMA(vh, ph, acc[b]);
          acc[b] = MFMA(vl, ph, acc[b]);
          acc[b] = MFMA(vh, pl, acc[b]);
        } else {
          acc[b] = MFMA(vh, ph, acc[b]);
        }
      }
    }
  }
  if (!active || !live) return;
  const float inv = 1.0f / l;
  const int64_t obase = int64_t(row0 + qi) * qw + h * HD;
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      half4 o, olo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        _Float16 oh, ol;
        split_f16(acc[b][r4 * 4 + j] * inv, oh, ol);
        o[j] = oh;
        olo[j] = ol;
      }
      const int64_t at = obase + b * 32 + r4 * 8 + hl * 4;
      *reinterpret_cast<half4 *>(out16 + at) = o;
      if (SPLIT) *reinterpret_cast<half4 *>(out16lo + at) = olo;
    }
}

// ---------------------------------------------------------------- decode
// part layout: [nseq][hq][max_pages][2 + HD] = (max, sum, out[HD]) of one page.
// One 256-thread workgroup per (page, kv head).  Every thread issues its query/RoPE loads, then
// all of its K and V loads: K rows and V columns of the page are read as consecutive 16-byte
// words (thread t takes word t + 256 i), so each load instruction covers one contiguous
// kilobyte per wave.  A thread thus holds E consecutive dims of NL keys (K) and E consecutive
// keys of NL dims (V).  Meanwhile the group's query heads are rotated into LDS and, on the page
// that holds the new token, its k (rotated) and v are written into the cache and substituted
// for the stale slot in the registers just loaded.  Scores are reduced over the lanes of a key
// with DPP moves, the page softmax runs on one wave per head, then P.V reduces over the lanes
// of a dim.
template <int HD, int GRP, typename KV>
__device__ __forceinline__ void attn_decode_page(const float *__restrict__ qkv, int hq, const KvGeom &g,
                                                 const float *__restrict__ cosT,
                                                 const float *__restrict__ sinT, int pos,
                                                 KV *__restrict__ kpool, KV *__restrict__ vpool,
                                                 const int32_t *__restrict__ pages, float *pbase,
                                                 int64_t hstride);
template <int HD, int GRP, typename KV>
__global__ __launch_bounds__(256) void attn_decode_kernel(const float *__restrict__ qkv, int hq, KvGeom g,
                                                          const float *__restrict__ cosT,
                                                          const float *__restrict__ sinT, int pos,
                                                          KV *__restrict__ kpool, KV *__restrict__ vpool,
                                                          const int32_t *__restrict__ pages, int max_pages,
                                                          float *__restrict__ part) {
  static_assert(HD == 64 || HD == 128, "decode attention is written for head_dim 64 and 128");
  const int pi = blockIdx.x, kh = blockIdx.y;
  float *pbase = part + (int64_t(kh * GRP) * max_pages + pi) * (2 + HD);
  const int64_t hstride = int64_t(max_pages) * (2 + HD);
  attn_decode_page<HD, GRP, KV>(qkv, hq, g, cosT, sinT, pos, kpool, vpool, pages, pbase, hstride);
}

// Combine the per-page partials (max, sum, out[HD]) of one query head: pb points at its page 0,
// np pages.  A separate launch: handing the partials over to a last-arriving page workgroup
// would need an agent-scope release (an L2 write-back on this part) in every page workgroup,
// which measured slower than the launch.  Thread (d, half) owns output dim d over the pages half, half + 2, ...; each batch
// of 2*CB pages is loaded in one round trip together with the page maxima and sums (indices
// clamped, surplus pages weighted 0).  All 256 threads of the workgroup take part.
template <int HD>
__device__ __forceinline__ void combine_head(const float *__restrict__ pb, int np, float *__restrict__ outh) {
  constexpr int NPART = 256 / HD;  // threads per output dim: 2 (head_dim 128) or 4 (64)
  static_assert(NPART * HD == 256, "256 threads over the output dims");
  constexpr int CB = 64 / NPART;   // pages per thread per batch
  const int t = threadIdx.x;
  __shared__ float wm[1024], wl[1024];
  __shared__ float red[4], sacc[NPART][HD], sl[NPART];
  const int d = t & (HD - 1), part = t / HD;
  // page maxima and sums (np <= 1024: four per thread), then the first batch of outputs
  float m4[4], l4[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = min(t + 256 * u, np - 1);
    m4[u] = pb[int64_t(i) * (2 + HD)];
    l4[u] = pb[int64_t(i) * (2 + HD) + 1];
  }
  float ov[CB];
#pragma unroll
  for (int u = 0; u < CB; ++u) ov[u] = pb[int64_t(min(part + NPART * u, np - 1)) * (2 + HD) + 2 + d];
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (t + 256 * u < np) M = fmaxf(M, m4[u]);
  M = wave_max_dpp(M);
  if ((t & 63) == 0) red[t >> 6] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = t + 256 * u;
    if (i < np) {
      wm[i] = m4[u] == -INFINITY ? 0.0f : __expf(m4[u] - M);
      wl[i] = l4[u];
    }
  }
  __syncthreads();
  float acc = 0.0f, L = 0.0f;
  for (int b0 = 0; b0 < np; b0 += NPART * CB) {
    if (b0 > 0) {
#pragma unroll
      for (int u = 0; u < CB; ++u) ov[u] = pb[int64_t(min(b0 + part + NPART * u, np - 1)) * (2 + HD) + 2 + d];
    }
#pragma unroll
    for (int u = 0; u < CB; ++u) {
      const int i = b0 + part + NPART * u;
      if (i < np) {
        acc += ov[u] * wm[i];
        L += wl[i] * wm[i];
      }
    }
  }
  sacc[part][d] = acc;
  if (d == 0) sl[part] = L;
  __syncthreads();
  if (t < HD) {
    float a = 0.0f, l = 0.0f;
#pragma unroll
    for (int q = 0; q < NPART; ++q) {
      a += sacc[q][t];
      l += sl[q];
    }
    outh[t] = a / l;
  }
  __syncthreads();  // the shared arrays are reused by the caller's next head
}

// Combine as its own launch: one workgroup per (query head, sequence).
template <int HD>
__global__ __launch_bounds__(256) void attn_decode_combine(const float *__restrict__ part, int hq,
                                                           int max_pages,
                                                           const int32_t *__restrict__ ctx_len, int ctx_all,
                                                           float *__restrict__ out) {
  const int h = blockIdx.x, s = blockIdx.y;
  const int np = ((ctx_len ? ctx_len[s] : ctx_all) + P - 1) / P;
  combine_head<HD>(part + ((int64_t(s) * hq + h) * max_pages) * (2 + HD), np, out + (int64_t(s) * hq + h) * HD);
}

// One page of one kv head: scores, page softmax and P.V for each query head.
template <int HD, int GRP, typename KV>
__device__ __forceinline__ void attn_decode_page(const float *__restrict__ qkv, int hq, const KvGeom &g,
                                                 const float *__restrict__ cosT,
                                                 const float *__restrict__ sinT, int pos,
                                                 KV *__restrict__ kpool, KV *__restrict__ vpool,
                                                 const int32_t *__restrict__ pages, float *pbase,
                                                 int64_t hstride) {
  constexpr int E = 16 / sizeof(KV);          // elements per 16-byte word: 4 (f32) or 8 (f16)
  constexpr int NL = P * HD / E / 256;        // words per thread of K (and of V)
  constexpr int LPK = HD / E;                 // lanes per key row of K
  constexpr int LPD = P / E;                  // lanes per dim column of V
  constexpr int HALF = HD / 2;
  constexpr int NQP = (GRP * HALF + 255) / 256;  // rotation pairs per thread
  static_assert(LPK == 8 || LPK == 16 || LPK == 32, "key rows span 8, 16 or 32 lanes");
  static_assert(LPD == 8 || LPD == 16, "dim columns span 8 or 16 lanes");
  const int pi = blockIdx.x, kh = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int len = pos + 1;
  const int64_t page = pages[pi];
  KV *Kp = kpool + page * g.page_stride + int64_t(kh) * P * HD;
  KV *Vp = vpool + page * g.page_stride + int64_t(kh) * HD * P;
  const float *cs = cosT + int64_t(pos) * HD, *sn = sinT + int64_t(pos) * HD;
  // query rotation inputs and the new token's k/v first (small); every load is unconditional
  // (clamped index) so that none is sunk behind the page loads
  float qu[NQP], qv[NQP], c0[NQP], c1[NQP], s0[NQP], s1[NQP];
#pragma unroll
  for (int e = 0; e < NQP; ++e) {
    const int idx = min(t + 256 * e, GRP * HALF - 1);
    const int gq = idx / HALF, j = idx % HALF;
    const float *qr = qkv + (kh * GRP + gq) * HD;
    qu[e] = qr[j];
    qv[e] = qr[j + HALF];
    c0[e] = cs[j];
    c1[e] = cs[j + HALF];
    s0[e] = sn[j];
    s1[e] = sn[j + HALF];
  }
  const int jn = t & (HALF - 1);  // new key: thread t < HALF rotates pair (jn, jn + HALF)
  const float *kr0 = qkv + (hq + kh) * HD;
  const float nku = kr0[jn], nkv = kr0[jn + HALF];
  const float nc0 = cs[jn], nc1 = cs[jn + HALF], ns0 = sn[jn], ns1 = sn[jn + HALF];
  const float nvv = qkv[(hq + g.hkv + kh) * HD + min(max(t - HALF, 0), HD - 1)];
  __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the page's: they return first
  uint4 kr[NL], vr[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) kr[i] = reinterpret_cast<const uint4 *>(Kp)[t + 256 * i];
#pragma unroll
  for (int i = 0; i < NL; ++i) vr[i] = reinterpret_cast<const uint4 *>(Vp)[t + 256 * i];
  // RoPE (src/models/openthai/model.rs:276-294 applies it to q and k before the dot products)
  __shared__ float qs[GRP * HD + HD];  // tail: landing row for idle threads
  __shared__ float nka[256], nkb[256], nvs[256];  // new k (pairs j, j + HD/2) and v staged per thread
  __shared__ float sc[GRP][P];
#pragma unroll
  for (int e = 0; e < NQP; ++e) {
    const int idx = t + 256 * e;
    const int gq = idx / HALF, j = idx % HALF;
    const int row = idx < GRP * HALF ? gq : GRP;
    qs[row * HD + j] = qu[e] * c0[e] - qv[e] * s0[e];
    qs[row * HD + j + HALF] = qv[e] * c1[e] + qu[e] * s1[e];
  }
  const bool cur = pi == pos / P;  // this page holds the new token (uniform per workgroup)
  const int slot = pos % P;
  {  // the new token's rotated k and its v, computed and staged in LDS by every thread (idle
     // threads write junk to their own slots), so their loads stay ahead of the page's; only
     // the page that holds the slot stores them into the cache
    const KV a = KV(nku * nc0 - nkv * ns0), b = KV(nkv * nc1 + nku * ns1), v = KV(nvv);
    nka[t] = float(a);
    nkb[t] = float(b);
    nvs[t] = float(v);
    if (cur) {
      if (t < HALF) {
        Kp[slot * HD + t] = a;
        Kp[slot * HD + t + HALF] = b;
      } else if (t < HALF + HD) {
        Vp[(t - HALF) * P + slot] = v;
      }
    }
  }
  __syncthreads();
  const int kd0 = (t * E) % HD;   // K: first dim of this thread's words (same for every i)
  const int vk0 = (t * E) % P;    // V: first key of this thread's words (same for every i)
  if (cur) {  // the registers hold the slot as it was before this step: use the new values
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      KV *k8 = reinterpret_cast<KV *>(&kr[i]);
      if ((t + 256 * i) * E / HD == slot)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int dd = kd0 + e;
          k8[e] = KV(dd < HALF ? nka[dd] : nkb[dd - HALF]);
        }
      KV *v8 = reinterpret_cast<KV *>(&vr[i]);
      const int dim = (t + 256 * i) * E / P;
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (vk0 + e == slot) v8[e] = KV(nvs[HALF + dim]);
    }
  }
  const float inv_sqrt = 1.0f / sqrtf(float(HD));
#pragma unroll
  for (int gq = 0; gq < GRP; ++gq) {
    float q[E];
#pragma unroll
    for (int e = 0; e < E; ++e) q[e] = qs[gq * HD + kd0 + e];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const KV *k8 = reinterpret_cast<const KV *>(&kr[i]);
      float d = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) d = fmaf(q[e], float(k8[e]), d);
      const int key = (t + 256 * i) * E / HD;
      if constexpr (LPK == 32) {
        d = half_sum_odd_rows(d);  // lanes 16-31 / 48-63 hold the key's sum
        if ((lane & 31) == 16) sc[gq][key] = pi * P + key < len ? d * inv_sqrt : -INFINITY;
      } else if constexpr (LPK == 16) {
        d = row_sum(d);
        if ((lane & 15) == 0) sc[gq][key] = pi * P + key < len ? d * inv_sqrt : -INFINITY;
      } else {
        d = group8_sum(d);
        if ((lane & 7) == 0) sc[gq][key] = pi * P + key < len ? d * inv_sqrt : -INFINITY;
      }
    }
  }
  __syncthreads();
  // page softmax per query head: wave w handles heads w, w + 4, ...
  for (int gq = wave; gq < GRP; gq += 4) {
    const float v = sc[gq][lane];
    const float mx = wave_max_dpp(v);
    const float p = v == -INFINITY ? 0.0f : __expf(v - mx);
    const float sum = wave_sum_dpp(p);
    sc[gq][lane] = p;
    if (lane == 0) {
      pbase[gq * hstride] = mx;
      pbase[gq * hstride + 1] = sum;
    }
  }
  __syncthreads();
#pragma unroll
  for (int gq = 0; gq < GRP; ++gq) {
    float p[E];
#pragma unroll
    for (int e = 0; e < E; ++e) p[e] = sc[gq][vk0 + e];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const KV *v8 = reinterpret_cast<const KV *>(&vr[i]);
      float a = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) a = fmaf(p[e], float(v8[e]), a);
      a = LPD == 16 ? row_sum(a) : group8_sum(a);
      if ((lane & (LPD - 1)) == 0) pbase[gq * hstride + 2 + (t + 256 * i) * E / P] = a;
    }
  }
}

}  // namespace

void launch_attn_prefill(const _Float16 *q16, const _Float16 *q16_lo, int T, int hq,
                         const KvGeom &g, const void *kpool, const void *vpool,
                         const int32_t *pages, int max_pages, const int32_t *tile_seq,
                         const int32_t *tile_row0, const int32_t *tile_pos0,
                         const int32_t *tile_n, int ntiles, const int32_t *grp_first,
                         const int32_t *grp_count, int ngroups, _Float16 *out16,
                         _Float16 *out16_lo, hipStream_t st) {
  LG_REQUIRE(g.page_tokens == P, "attention: page size must be %d", P);
  LG_REQUIRE(hq % g.hkv == 0, "attention: hq %% hkv != 0");
  LG_REQUIRE(ntiles > 0 && T > 0, "attention: empty batch");
  const bool split = q16_lo != nullptr;
  LG_REQUIRE(split == (g.kv32 != 0), "attention: split queries need the f32 cache and vice versa");
  LG_REQUIRE(!split || out16_lo, "attention: split path needs the lo output plane");
  LG_REQUIRE(int64_t(ntiles) * hq < (1ll << 31), "attention: too many tiles");
  if (grp_first && g.hd == 128) {
    LG_REQUIRE(ngroups > 0 && ngroups <= ntiles, "attention: bad tile groups");
    const dim3 grid(ngroups * hq), block(256);
    if (split)
      hipLaunchKernelGGL((attn_prefill_grp_kernel<128, true>), grid, block, 0, st, q16, q16_lo, hq, g,
                         kpool, vpool, pages, max_pages, grp_first, grp_count, tile_seq, tile_row0,
                         tile_pos0, tile_n, out16, out16_lo);
    else
      hipLaunchKernelGGL((attn_prefill_grp_kernel<128, false>), grid, block, 0, st, q16, q16_lo, hq, g,
                         kpool, vpool, pages, max_pages, grp_first, grp_count, tile_seq, tile_row0,
                         tile_pos0, tile_n, out16, out16_lo);
    HIP_CHECK(hipGetLastError());
    return;
  }
  const dim3 grid(ntiles * hq), block(64);
#define LAUNCH(HDV, S)                                                                              \
  hipLaunchKernelGGL((attn_prefill_kernel<HDV, S>), grid, block, 0, st, q16, q16_lo, hq, g, kpool, vpool, \
                     pages, max_pages, tile_seq, tile_row0, tile_pos0, tile_n, out16, out16_lo)
  if (g.hd == 64) {
    if (split) LAUNCH(64, true); else LAUNCH(64, false);
  } else if (g.hd == 128) {
    if (split) LAUNCH(128, true); else LAUNCH(128, false);
  } else {
    fail(LG_ERR_UNSUPPORTED, "attention: head_dim %d not supported (64, 128)", g.hd);
  }
#undef LAUNCH
  HIP_CHECK(hipGetLastError());
}

int64_t attn_decode_scratch_floats(int nseq, int hq, int hd, int max_ctx) {
  const int64_t pages = (max_ctx + P - 1) / P;
  return int64_t(nseq) * hq * pages * (2 + hd);
}

void launch_attn_decode(const float *qkv, int hq, const KvGeom &g, const float *cosT, const float *sinT,
                        int pos, void *kpool, void *vpool, const int32_t *pages, int max_pages,
                        float *part, float *out, hipStream_t st) {
  LG_REQUIRE(g.page_tokens == P, "attention: page size must be %d", P);
  LG_REQUIRE(g.hd == 128 || g.hd == 64, "decode attention: head_dim %d not supported (64, 128)", g.hd);
  LG_REQUIRE(pos >= 0, "decode attention: negative position");
  const int np = pos / P + 1;
  LG_REQUIRE(np <= max_pages, "decode attention: context exceeds the page table");
  LG_REQUIRE(np <= 1024, "decode attention: context of %d pages exceeds the combine stage", np);
  const int grp = hq / g.hkv;
  const dim3 grid(np, g.hkv), block(256);
#define CASE(HDV, G)                                                                                     \
  case G:                                                                                                \
    if (g.kv32)                                                                                          \
      hipLaunchKernelGGL((attn_decode_kernel<HDV, G, float>), grid, block, 0, st, qkv, hq, g, cosT, sinT, \
                         pos, static_cast<float *>(kpool), static_cast<float *>(vpool), pages, max_pages, \
                         part);                                                                          \
    else                                                                                                 \
      hipLaunchKernelGGL((attn_decode_kernel<HDV, G, _Float16>), grid, block, 0, st, qkv, hq, g, cosT,    \
                         sinT, pos, static_cast<_Float16 *>(kpool), static_cast<_Float16 *>(vpool), pages, \
                         max_pages, part);                                                               \
    break;
  if (g.hd == 128) {
    switch (grp) {
      CASE(128, 1) CASE(128, 2) CASE(128, 4) CASE(128, 7) CASE(128, 8)
      default: fail(LG_ERR_UNSUPPORTED, "decode attention: group size %d not supported", grp);
    }
  } else {
    switch (grp) {
      CASE(64, 1) CASE(64, 2) CASE(64, 4) CASE(64, 7) CASE(64, 8)
      default: fail(LG_ERR_UNSUPPORTED, "decode attention: group size %d not supported", grp);
    }
  }
#undef CASE
  HIP_CHECK(hipGetLastError());
  if (g.hd == 128)
    hipLaunchKernelGGL((attn_decode_combine<128>), dim3(hq, 1), dim3(256), 0, st, part, hq, max_pages,
                       static_cast<const int32_t *>(nullptr), pos + 1, out);
  else
    hipLaunchKernelGGL((attn_decode_combine<64>), dim3(hq, 1), dim3(256), 0, st, part, hq, max_pages,
                       static_cast<const int32_t *>(nullptr), pos + 1, out);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
