// Causal GQA attention over the paged KV cache (gfx950).
//
// Reference semantics (src/models/openthai/model.rs:276-294, generalised to hq/hkv heads):
// for query i of head h, kv head kh = h / (hq/hkv), s_j = dot(q_i, k_j) / sqrt(hd) for
// j <= pos_i, p = softmax(s), out = sum_j p_j v_j.
//
// KV page layout (one layer, one page of P = 64 tokens), per kv head:
//   K: [P][hd] (row per token)     V: [hd][P] (column per token)
// in f16 (FAST, KV16) or as two f16 planes (EXACT: the hi plane hi = f16(v), then the lo plane
// lo = f16(v - hi), each of that layout; hi + lo holds v to about 22 significant bits).
//
// Prefill: one workgroup per (group of query tiles, kv head, block of the kv head's query
// heads), MFMA 16x16x32 f16.  Queries and probabilities as hi/lo planes over a split cache make
// every product hi.hi + lo.hi + hi.lo (three MFMAs), which keeps scores and outputs f32-faithful;
// over an f16 cache, hi.c + lo.c (two MFMAs): exact in the query and probability, the cache value
// as stored.
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
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int P = 64;  // tokens per page

#define MFMA(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

// Prefill.  Work item: (tile group, kv head kh, head block hb).  A tile group is <= T
// consecutive 32-query tiles of one sequence, a head block GB consecutive query heads of kh's
// group of G = hq / hkv.  Wave w computes head kh * G + hb * GB + w % GB on tile w / GB of the
// group, so all W = GB * T waves read the same K/V pages: each page passes through LDS once per
// workgroup.  Pages are copied global -> LDS by LDS-DMA loads (16 bytes a lane, no registers),
// double-buffered: page kt + 1 is in flight while page kt is consumed, one barrier per page.
//
// S^T = K . Q^T on MFMA 16x16x32 f16 (one instruction per 32-deep chunk of the head dim), keys as
// rows and queries as columns, in 16 x 16 blocks: a wave's 32 queries are two query blocks qb, a
// page's 64 keys four key blocks (ck, h) of two 32-key chunks ck.  Lane l feeds row r = l % 16 of a
// key block, and row r of block (ck, h) is key ck * 32 + 8 (r / 4) + 4 h + r % 4: the result leaves
// lane l (query l % 16 of its block) with keys ck * 32 + 8 g + 4 h + 0..3, g = l / 16, so its scores
// of (ck, 0) and (ck, 1) together are the eight keys ck * 32 + 8 g + 0..7 that its P^T operand of
// O^T = V^T . P^T takes against one 16-byte run of a V row.  A query's 64 scores of a page sit in the
// four lanes l % 16 + 16 g; the online softmax reduces over them with two lane swaps.  Each wave
// runs eight independent score chains and sixteen output chains, so no MFMA waits on the one
// before it.
// LDS: K rows unpadded, the 16-byte chunk x of key row R at slot x ^ kswz(R), so the sixteen rows
// an operand read takes fall in distinct 16-byte bank groups; V rows (one dim, 64 keys) carry one
// pad slot for the same reason.
// NQ: planes of the queries and of P (2: hi/lo, 1: f16); NKV: planes of the cache (2: hi/lo,
// 1: f16).  (2, 2): three MFMAs a product (hi.hi + lo.hi + hi.lo); (2, 1): two (hi.c + lo.c);
// (1, 1): one.
template <int HD>
__device__ __forceinline__ int kswz(int row) {
  return HD == 128 ? ((row & 3) | (((row >> 3) & 3) << 2)) : ((row & 3) | (((row >> 3) & 1) << 2));
}

template <int HD, int NPL>
struct PrefillStage {
  static constexpr int KC = HD / 8;                // 16-byte chunks per K row (no pad)
  static constexpr int VC = P / 8, VRS = VC + 1;   // chunks and slots per V row (one dim, 64 keys)
  static constexpr int KPL = P * KC, VPL = HD * VRS;  // slots per plane
  static_assert(KPL % 64 == 0 && VPL % 64 == 0, "planes fill whole 64-slot blocks");
  static constexpr int KSLOTS = NPL * KPL, SLOTS = NPL * (KPL + VPL);
  static constexpr int BLOCKS = SLOTS / 64;  // one LDS-DMA instruction of one wave per block
  static constexpr int BYTES = SLOTS * 16;
};

__device__ __forceinline__ half8 lds_half8(const unsigned char *base, int slot) {
  return *reinterpret_cast<const half8 *>(base + slot * 16);
}

// STG: LDS stages of K/V pages.  2: page kt + 1 is in flight while page kt is consumed (one workgroup of
// up to 8 waves per CU: 128 KiB of LDS at head_dim 128).  1: each page is loaded, then consumed, and
// two workgroups of 4 waves share a CU, one computing while the other waits for its page (the short
// sequences, where a workgroup's start and its few pages' waits dominate).
template <int HD, int NQ, int NKV, int W, int GB, int STG>
__global__ __launch_bounds__(64 * W, STG == 1 ? 2 : 1) void attn_prefill_kernel(
    const _Float16 *__restrict__ q16, const _Float16 *__restrict__ q16lo, int hq, KvGeom g,
    const _Float16 *__restrict__ kpool, const _Float16 *__restrict__ vpool, const int32_t *__restrict__ pages,
    int max_pages, const int32_t *__restrict__ grp_first, const int32_t *__restrict__ grp_count,
    const int32_t *__restrict__ tile_seq, const int32_t *__restrict__ tile_row0,
    const int32_t *__restrict__ tile_pos0, const int32_t *__restrict__ tile_n,
    _Float16 *__restrict__ out16, _Float16 *__restrict__ out16lo) {
  static_assert(NKV <= NQ, "an f16 query over a split cache is not a mode");
  using S = PrefillStage<HD, NKV>;
  constexpr int NC = HD / 32, DB = HD / 16;  // 32-deep chunks of the head dim, 16-dim output blocks
  constexpr int NI = (S::BLOCKS + W - 1) / W;  // LDS-DMA instructions per wave per page
  static_assert(STG == 1 || STG == 2, "one or two LDS stages");
  __shared__ __align__(16) unsigned char lds[STG * S::BYTES];

  // XCD-contiguous mapping: workgroups are dealt to the 8 XCDs round-robin (i -> XCD i % 8);
  // each XCD takes one contiguous range of (head block, tile group) pairs, groups fastest, so
  // the pages of one sequence and kv head are read through one L2.
  const int G = hq / g.hkv, nhb = G / GB;
  const int total = gridDim.x, ngroups = total / (g.hkv * nhb);
  const int xcd = blockIdx.x % 8, per = total / 8, rem = total % 8;
  const int logical = xcd * per + min(xcd, rem) + blockIdx.x / 8;
  const int grp = logical % ngroups, hsel = logical / ngroups;
  const int kh = hsel / nhb, hb = hsel % nhb;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, qg = lane >> 4;
  const int t0 = grp_first[grp], cnt = grp_count[grp];
  const bool active = wave / GB < cnt;
  const int tile = t0 + min(wave / GB, cnt - 1);
  const int h = kh * G + hb * GB + wave % GB;
  const int row0 = tile_row0[tile], pos0 = tile_pos0[tile], n = tile_n[tile];
  const int seq = tile_seq[t0];  // every tile of a group belongs to one sequence
  const int glast = tile_pos0[t0 + cnt - 1] + tile_n[t0 + cnt - 1] - 1;
  const int qw = hq * HD;

  // this lane's byte offset inside the kv head's K (or V) block for each of its DMA slots; pad
  // slots get an offset past the block, which the buffer load turns into zeros without a read
  constexpr uint32_t kHeadBytes = uint32_t(NKV) * P * HD * 2;
  uint32_t off[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int b = i * W + wave, slot = b * 64 + lane;
    uint32_t o = kHeadBytes;
    if (b < S::BLOCKS) {
      if (slot < S::KSLOTS) {
        const int p = slot / S::KPL, r = slot % S::KPL, row = r / S::KC, x = (r % S::KC) ^ kswz<HD>(row);
        o = uint32_t(((p * P + row) * HD + x * 8) * 2);
      } else {
        const int s2 = slot - S::KSLOTS, p = s2 / S::VPL, r = s2 % S::VPL, d = r / S::VRS, x = r % S::VRS;
        if (x < S::VC) o = uint32_t(((p * HD + d) * P + x * 8) * 2);
      }
    }
    off[i] = o;
  }
  const int32_t *ptab = pages + int64_t(seq) * max_pages;
  const int64_t page_halves = int64_t(NKV) * g.page_stride;  // halves per page of one layer
  const int64_t head_halves = int64_t(NKV) * P * HD;         // halves per kv head of one page
  auto issue = [&](int32_t page, int st) {
    const int64_t base = int64_t(page) * page_halves + kh * head_halves;
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(kpool + base), 0, kHeadBytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(vpool + base), 0, kHeadBytes, kBufferFlags);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int b = i * W + wave;
      if (b >= S::BLOCKS) break;
#if defined(__HIP_DEVICE_COMPILE__)
      // device pass only: with a run-time voffset this builtin keeps the host pass from
      // emitting the kernel's launch stub (the host never runs kernel bodies)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(b * 64 < S::KSLOTS ? rk : rv,
                                               (__attribute__((address_space(3))) void *)(lds + st * S::BYTES + b * 1024),
                                               16, off[i], 0, 0, 0);
#endif
    }
  };

  // queries qb * 16 + lr of the tile (rows past n repeat row n - 1 and are never stored), the eight
  // dims 32 c + 8 g .. + 8 of each 32-deep chunk c
  half8 qr[2][NC], ql[2][NQ == 2 ? NC : 1];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int64_t qo = int64_t(row0 + min(qb * 16 + lr, n - 1)) * qw + h * HD + qg * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qr[qb][c] = *reinterpret_cast<const half8 *>(q16 + qo + 32 * c);
      if constexpr (NQ == 2) ql[qb][c] = *reinterpret_cast<const half8 *>(q16lo + qo + 32 * c);
    }
  }
  f32x4 acc[2][DB];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[qb][b][r] = 0.0f;
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
  const int npages = glast / P + 1;
  const int mypages = active ? (pos0 + n - 1) / P + 1 : 0;
  // this lane's K operand rows: key ck * 32 + 8 (lr / 4) + 4 h + lr % 4 of block (ck, h); their
  // chunk swizzle depends on lr only
  const int kr0 = 8 * (lr >> 2) + (lr & 3), ksw = kswz<HD>(kr0);

  issue(ptab[0], 0);
  // page-table entry of the page after the one in flight, read one iteration ahead so that no
  // DMA issue waits on a page-table round trip
  int32_t next_page = ptab[min(1, npages - 1)];
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int kt = 0; kt < npages; ++kt) {
    const int st = STG == 2 ? kt & 1 : 0;
    if (STG == 2 && kt + 1 < npages) {
      const int32_t page = next_page;
      next_page = ptab[min(kt + 2, npages - 1)];
      issue(page, st ^ 1);
    }
    if (kt < mypages) {
      const unsigned char *stage = lds + st * S::BYTES;
      const unsigned char *kl_ = stage + S::KPL * 16 * (NKV - 1);  // K lo plane (= hi when NKV 1)
      const unsigned char *vh_ = stage + S::KSLOTS * 16, *vl_ = vh_ + S::VPL * 16 * (NKV - 1);
      f32x4 s[2][2][2];  // [qb][ck][h]
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int ck = 0; ck < 2; ++ck)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int r = 0; r < 4; ++r) s[qb][ck][hh][r] = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int ck = 0; ck < 2; ++ck)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int slot = (ck * 32 + kr0 + 4 * hh) * S::KC + ((4 * c + qg) ^ ksw);
            const half8 kh8 = lds_half8(stage, slot);
            if constexpr (NQ == 2 && NKV == 2) {
              const half8 kl8 = lds_half8(kl_, slot);
#pragma unroll
              for (int qb = 0; qb < 2; ++qb) {
                s[qb][ck][hh] = MFMA(kh8, qr[qb][c], s[qb][ck][hh]);
                s[qb][ck][hh] = MFMA(kl8, qr[qb][c], s[qb][ck][hh]);
                s[qb][ck][hh] = MFMA(kh8, ql[qb][c], s[qb][ck][hh]);
              }
            } else if constexpr (NQ == 2) {
#pragma unroll
              for (int qb = 0; qb < 2; ++qb) {
                s[qb][ck][hh] = MFMA(kh8, qr[qb][c], s[qb][ck][hh]);
                s[qb][ck][hh] = MFMA(kh8, ql[qb][c], s[qb][ck][hh]);
              }
            } else {
#pragma unroll
              for (int qb = 0; qb < 2; ++qb) s[qb][ck][hh] = MFMA(kh8, qr[qb][c], s[qb][ck][hh]);
            }
          }
      // s[qb][ck][h][e] <-> key kt * P + ck * 32 + 8 qg + 4 h + e, query qb * 16 + lr.  The queries
      // come pre-multiplied by log2(e) / sqrt(hd), so s is the base-2 logit.  Only a page that
      // reaches past the tile's first query needs the causal mask.
      if (kt * P + P - 1 > pos0) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const int lim = pos0 + qb * 16 + lr - kt * P - 8 * qg;  // mask offsets ck * 32 + 4 h + e above
#pragma unroll
          for (int ck = 0; ck < 2; ++ck)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (ck * 32 + 4 * hh + e > lim) s[qb][ck][hh][e] = -INFINITY;
        }
      }
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        float mt = -INFINITY;
#pragma unroll
        for (int ck = 0; ck < 2; ++ck)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int e = 0; e < 4; ++e) mt = fmaxf(mt, s[qb][ck][hh][e]);
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        // A lane's exponent base m moves only when one of its query's scores exceeds it by more
        // than 8, so p = 2^(s - m) <= 256; l and acc carry the same base, so out = acc / l is
        // unchanged.  The rescale is skipped unless some lane of the wave moves; the others
        // multiply by exactly 1, so a query's arithmetic never depends on the other queries of its
        // wave.  Key 0 is visible to every query, so m is finite from the first page on and
        // 2^(-inf - m) = 0 drops masked keys.
        const bool grow = mt > m[qb] + 8.0f;
        if (__any(grow)) {
          const float mn = grow ? mt : m[qb];
          const float alpha = __builtin_amdgcn_exp2f(m[qb] - mn);
          l[qb] *= alpha;
#pragma unroll
          for (int b = 0; b < DB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[qb][b][r] *= alpha;
          m[qb] = mn;
        }
        float rs = 0.0f;
#pragma unroll
        for (int ck = 0; ck < 2; ++ck)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float p = __builtin_amdgcn_exp2f(s[qb][ck][hh][e] - m[qb]);
              s[qb][ck][hh][e] = p;
              rs += p;
            }
        rs += __shfl_xor(rs, 16);
        rs += __shfl_xor(rs, 32);
        l[qb] += rs;
      }
      // O^T += V^T . P^T over the two 32-key chunks: lane l's P^T operand is keys ck * 32 + 8 qg + 0..7
      // of its query, against dims 16 b + lr of V at the same keys
#pragma unroll
      for (int ck = 0; ck < 2; ++ck) {
        half8 ph[2], pl[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          float pv[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pv[e] = s[qb][ck][0][e];
            pv[4 + e] = s[qb][ck][1][e];
          }
          if constexpr (NQ == 2) split8_pk(pv, ph[qb], pl[qb]);
          else
#pragma unroll
            for (int e = 0; e < 8; ++e) ph[qb][e] = _Float16(pv[e]);
        }
#pragma unroll
        for (int b = 0; b < DB; ++b) {
          const int vo = (b * 16 + lr) * S::VRS + 4 * ck + qg;
          const half8 vh = lds_half8(vh_, vo);
          if constexpr (NQ == 2 && NKV == 2) {
            const half8 vl = lds_half8(vl_, vo);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
              acc[qb][b] = MFMA(vh, ph[qb], acc[qb][b]);
              acc[qb][b] = MFMA(vl, ph[qb], acc[qb][b]);
              acc[qb][b] = MFMA(vh, pl[qb], acc[qb][b]);
            }
          } else if constexpr (NQ == 2) {
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
              acc[qb][b] = MFMA(vh, ph[qb], acc[qb][b]);
              acc[qb][b] = MFMA(vh, pl[qb], acc[qb][b]);
            }
          } else {
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) acc[qb][b] = MFMA(vh, ph[qb], acc[qb][b]);
          }
        }
      }
    }
    if (STG == 1 && kt + 1 < npages) {  // every wave is done with the stage: load page kt + 1 into it
      __syncthreads();
      const int32_t page = next_page;
      next_page = ptab[min(kt + 2, npages - 1)];
      issue(page, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of page kt + 1 has landed
    __syncthreads();
  }
  if (!active) return;
  // acc[qb][b][r] <-> dim 16 b + 4 qg + r of query qb * 16 + lr
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    if (qb * 16 + lr >= n) continue;
    const float inv = 1.0f / l[qb];
    const int64_t obase = int64_t(row0 + qb * 16 + lr) * qw + h * HD + 4 * qg;
#pragma unroll
    for (int b = 0; b < DB; ++b) {
      half4 o, olo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        _Float16 oh, ol;
        split_f16(acc[qb][b][j] * inv, oh, ol);
        o[j] = oh;
        olo[j] = ol;
      }
      const int64_t at = obase + b * 16;
      *reinterpret_cast<half4 *>(out16 + at) = o;
      if constexpr (NQ == 2) *reinterpret_cast<half4 *>(out16lo + at) = olo;
    }
  }
}

// ---------------------------------------------------------------- decode
// part layout: [hq][max_pages][2 + HD] = (max, sum, out[HD]) of one page.
// One 256-thread workgroup per (page, kv head).  Every thread issues its query/RoPE loads, then
// all of its K and V loads: K rows and V columns of the page are read as consecutive 16-byte
// words (thread t takes word t + 256 i), so each load instruction covers one contiguous
// kilobyte per wave.  A thread thus holds E consecutive dims of NL keys (K) and E consecutive
// keys of NL dims (V).  Meanwhile the group's query heads are rotated into LDS and, on the page
// that holds the new token, its k (rotated) and v are substituted for the stale slot in the
// registers just loaded.  Scores are reduced over the lanes of a key with DPP moves, the page
// softmax runs on one wave per head, then P.V reduces over the lanes of a dim.  The new token's
// k and v are stored into the cache by an extra workgroup per kv head (grid column np), which
// reads no page and so finishes long before the page workgroups: a store in the page's own
// workgroup would hold it, one of the launch's last to finish, until the write is acknowledged.
// Pool value formats: float, _Float16, or SplitKV: per (page, kv head) block an f16 hi plane and
// then an f16 lo plane (hi = f16(v), lo = f16(v - hi)), each laid out as the f16 pool is.
struct SplitKV {};
template <typename KV>
struct KvFmt {
  using elem = KV;
  static constexpr int NPL = 1;
};
template <>
struct KvFmt<SplitKV> {
  using elem = _Float16;
  static constexpr int NPL = 2;
};

// The new token's rotated k and its v (f16, or hi/lo planes) into slot pos % P of its page, for
// kv head kh; threads 0 .. HD-1 take part (k pair (t, t + HD/2) for t < HD/2, v dim t).  The same
// rope_pair and split as the page workgroup that substitutes the slot in its registers, so the
// cache holds the values that step's scores used.
template <int HD, typename KV>
__device__ __forceinline__ void store_new_kv(const float *__restrict__ qkv, int hq, const KvGeom &g,
                                             const float *__restrict__ cosT, const float *__restrict__ sinT,
                                             int pos, typename KvFmt<KV>::elem *__restrict__ kpool,
                                             typename KvFmt<KV>::elem *__restrict__ vpool,
                                             const int32_t *__restrict__ pages, int kh) {
  using T = typename KvFmt<KV>::elem;
  constexpr int NPL = KvFmt<KV>::NPL, HALF = HD / 2, PLANE = P * HD;
  const int t = threadIdx.x;
  if (t >= HD) return;
  const int64_t page = pages[pos / P];
  const int slot = pos % P;
  T *Kp = kpool + page * (NPL * g.page_stride) + int64_t(kh) * NPL * P * HD;
  T *Vp = vpool + page * (NPL * g.page_stride) + int64_t(kh) * NPL * HD * P;
  const float *cs = cosT + int64_t(pos) * HD, *sn = sinT + int64_t(pos) * HD;
  const int j = t & (HALF - 1);
  const float *kr0 = qkv + (hq + kh) * HD;
  const float ku = kr0[j], kv = kr0[j + HALF], c0 = cs[j], c1 = cs[j + HALF], s0 = sn[j], s1 = sn[j + HALF];
  const float nv = qkv[(hq + g.hkv + kh) * HD + t];
  float a, b;
  rope_pair(ku, kv, c0, s0, c1, s1, a, b);
  if constexpr (NPL == 2) {
    _Float16 vh, vl;
    split_f16(nv, vh, vl);
    Vp[t * P + slot] = vh;
    Vp[PLANE + t * P + slot] = vl;
    if (t < HALF) {
      _Float16 ah, al, bh, bl;
      split_f16(a, ah, al);
      split_f16(b, bh, bl);
      Kp[slot * HD + t] = ah;
      Kp[PLANE + slot * HD + t] = al;
      Kp[slot * HD + t + HALF] = bh;
      Kp[PLANE + slot * HD + t + HALF] = bl;
    }
  } else {
    Vp[t * P + slot] = T(nv);
    if (t < HALF) {
      Kp[slot * HD + t] = T(a);
      Kp[slot * HD + t + HALF] = T(b);
    }
  }
}

template <int HD, int GRP, typename KV>
__device__ __forceinline__ void attn_decode_page(const float *__restrict__ qkv, int hq, const KvGeom &g,
                                                 const float *__restrict__ cosT,
                                                 const float *__restrict__ sinT, int pos,
                                                 typename KvFmt<KV>::elem *__restrict__ kpool,
                                                 typename KvFmt<KV>::elem *__restrict__ vpool,
                                                 const int32_t *__restrict__ pages, float *pbase,
                                                 int64_t hstride, int kh, int qh0);
// Grid (np + 1, hkv * split): workgroup row y serves query heads y * GRP .. y * GRP + GRP - 1 of kv head
// y / split (split = query heads per kv head / GRP: a kv head's group of query heads dealt over `split`
// workgroups when the grid would otherwise be too small to fill the part).
template <int HD, int GRP, typename KV>
__global__ __launch_bounds__(256) void attn_decode_kernel(const float *__restrict__ qkv, int hq, KvGeom g,
                                                          const float *__restrict__ cosT,
                                                          const float *__restrict__ sinT, int pos,
                                                          typename KvFmt<KV>::elem *__restrict__ kpool,
                                                          typename KvFmt<KV>::elem *__restrict__ vpool,
                                                          const int32_t *__restrict__ pages, int max_pages,
                                                          float *__restrict__ part, int split) {
  static_assert(HD == 64 || HD == 128, "decode attention is written for head_dim 64 and 128");
  const int pi = blockIdx.x, kh = blockIdx.y / split, qh0 = blockIdx.y * GRP;
  if (pi == pos / P + 1) {  // the extra column: store the new token's k and v, read no page
    if (blockIdx.y % split == 0) store_new_kv<HD, KV>(qkv, hq, g, cosT, sinT, pos, kpool, vpool, pages, kh);
    return;
  }
  float *pbase = part + (int64_t(qh0) * max_pages + pi) * (2 + HD);
  const int64_t hstride = int64_t(max_pages) * (2 + HD);
  attn_decode_page<HD, GRP, KV>(qkv, hq, g, cosT, sinT, pos, kpool, vpool, pages, pbase, hstride, kh, qh0);
}

// Combine launch: one 256-thread workgroup per query head h: out = sum_i w_i out_i / sum_i w_i sum_i
// over the page partials (max_i, sum_i, out_i) of h, with w_i = exp(max_i - M) and M the largest
// page maximum.  Thread (d, part) owns output dim d over the pages part, part + NPART, ...
// (NPART = 256 / HD; one part per wave), so its page index is wave-uniform.  Every wave finds M
// and the total sum_i w_i sum_i itself from lane-distributed maxima and sums (lane j: pages j,
// j + 64, ...), and takes the weight of a page from the lane that computed it, so the only
// barrier is the final sum over the parts.  The maxima and the first batch of 64 pages are loaded
// before the first is waited for.  A separate launch: handing the partials over to a
// last-arriving page workgroup would need an agent-scope release (an L2 write-back on this part)
// in every page workgroup, which measured slower than the launch.
template <int HD>
__global__ __launch_bounds__(256) void attn_decode_combine(const float *__restrict__ part, int max_pages, int np,
                                                           float *__restrict__ out) {
  constexpr int NPART = 256 / HD;  // threads per output dim: 2 (head_dim 128) or 4 (64)
  static_assert(NPART * HD == 256, "256 threads over the output dims");
  constexpr int CB = 64 / NPART;   // pages per thread per batch of 64
  constexpr int ROW = 2 + HD;
  const int h = blockIdx.x, t = threadIdx.x, lane = t & 63, d = t & (HD - 1);
  const int pw = __builtin_amdgcn_readfirstlane(t / HD);  // this wave's part
  const float *pb = part + int64_t(h) * max_pages * ROW;
  float mx[16];  // page maxima, np <= 1024
#pragma unroll
  for (int c = 0; c < 16; ++c)
    if (c * 64 < np) mx[c] = pb[int64_t(min(c * 64 + lane, np - 1)) * ROW];
  float mb, lb, ov[CB];
  auto load_batch = [&](int b0) {
    const int i = min(b0 + lane, np - 1);
    mb = pb[int64_t(i) * ROW];
    lb = pb[int64_t(i) * ROW + 1];
#pragma unroll
    for (int u = 0; u < CB; ++u) ov[u] = pb[int64_t(min(b0 + pw + NPART * u, np - 1)) * ROW + 2 + d];
  };
  load_batch(0);
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < 16; ++c)
    if (c * 64 < np) M = fmaxf(M, mx[c]);
  M = wave_max_dpp(M);
  float acc = 0.0f, lsum = 0.0f;
  for (int b0 = 0; b0 < np; b0 += 64) {
    if (b0 > 0) load_batch(b0);
    // weight of page b0 + lane (0 past the last page)
    const float w = b0 + lane < np && mb != -INFINITY ? __expf(mb - M) : 0.0f;
    lsum = fmaf(lb, w, lsum);
#pragma unroll
    for (int u = 0; u < CB; ++u) {
      const int k = pw + NPART * u;  // wave-uniform page of the batch
      if (b0 + k < np) acc = fmaf(ov[u], lane_value(w, k), acc);
    }
  }
  const float L = wave_sum_dpp(lsum);
  __shared__ float sacc[NPART][HD];
  sacc[pw][d] = acc;
  __syncthreads();
  if (t < HD) {
    float a = 0.0f;
#pragma unroll
    for (int q = 0; q < NPART; ++q) a += sacc[q][t];
    out[int64_t(h) * HD + t] = a / L;
  }
}

// One page of one kv head: scores, page softmax and P.V for each query head.
template <int HD, int GRP, typename KV>
__device__ __forceinline__ void attn_decode_page(const float *__restrict__ qkv, int hq, const KvGeom &g,
                                                 const float *__restrict__ cosT,
                                                 const float *__restrict__ sinT, int pos,
                                                 typename KvFmt<KV>::elem *__restrict__ kpool,
                                                 typename KvFmt<KV>::elem *__restrict__ vpool,
                                                 const int32_t *__restrict__ pages, float *pbase,
                                                 int64_t hstride, int kh, int qh0) {
  using T = typename KvFmt<KV>::elem;
  constexpr int NPL = KvFmt<KV>::NPL;
  constexpr int E = 16 / sizeof(T);           // values per 16-byte word: 4 (f32) or 8 (f16 planes)
  constexpr int NL = P * HD / E / 256;        // words per thread of K (and of V), per plane
  constexpr int LPK = HD / E;                 // lanes per key row of K
  constexpr int LPD = P / E;                  // lanes per dim column of V
  constexpr int HALF = HD / 2;
  constexpr int NQP = (GRP * HALF + 255) / 256;  // rotation pairs per thread
  static_assert(LPK == 8 || LPK == 16 || LPK == 32, "key rows span 8, 16 or 32 lanes");
  static_assert(LPD == 8 || LPD == 16, "dim columns span 8 or 16 lanes");
  const int pi = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int len = pos + 1;
  const int64_t page = pages[pi];
  // hi plane (the only one unless split); the lo plane follows one plane (P * HD values) later
  T *Kp = kpool + page * (NPL * g.page_stride) + int64_t(kh) * NPL * P * HD;
  T *Vp = vpool + page * (NPL * g.page_stride) + int64_t(kh) * NPL * HD * P;
  constexpr int PLANE = P * HD;
  const float *cs = cosT + int64_t(pos) * HD, *sn = sinT + int64_t(pos) * HD;
  // query rotation inputs and the new token's k/v first (small); every load is unconditional
  // (clamped index) so that none is sunk behind the page loads
  float qu[NQP], qv[NQP], c0[NQP], c1[NQP], s0[NQP], s1[NQP];
#pragma unroll
  for (int e = 0; e < NQP; ++e) {
    const int idx = min(t + 256 * e, GRP * HALF - 1);
    const int gq = idx / HALF, j = idx % HALF;
    const float *qr = qkv + (qh0 + gq) * HD;
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
  uint4 kr[NL], vr[NL], krl[NPL == 2 ? NL : 1], vrl[NPL == 2 ? NL : 1];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    kr[i] = reinterpret_cast<const uint4 *>(Kp)[t + 256 * i];
    if constexpr (NPL == 2) krl[i] = reinterpret_cast<const uint4 *>(Kp + PLANE)[t + 256 * i];
  }
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    vr[i] = reinterpret_cast<const uint4 *>(Vp)[t + 256 * i];
    if constexpr (NPL == 2) vrl[i] = reinterpret_cast<const uint4 *>(Vp + PLANE)[t + 256 * i];
  }
  // RoPE (src/models/openthai/model.rs:276-294 applies it to q and k before the dot products)
  __shared__ float qs[GRP * HD + HD];  // tail: landing row for idle threads
  __shared__ float nka[256], nkb[256], nvs[256];  // new k (pairs j, j + HD/2) and v staged per thread
  __shared__ float sc[GRP][P];
#pragma unroll
  for (int e = 0; e < NQP; ++e) {
    const int idx = t + 256 * e;
    const int gq = idx / HALF, j = idx % HALF;
    const int row = idx < GRP * HALF ? gq : GRP;
    float ra, rc;
    rope_pair(qu[e], qv[e], c0[e], s0[e], c1[e], s1[e], ra, rc);
    qs[row * HD + j] = ra;
    qs[row * HD + j + HALF] = rc;
  }
  const bool cur = pi == pos / P;  // this page holds the new token (uniform per workgroup)
  const int slot = pos % P;
  {  // the new token's rotated k and its v as the cache holds them (store_new_kv, in the extra
     // workgroup column, stores the same values), staged in LDS by every thread (idle threads
     // write junk to their own slots) so that their loads stay ahead of the page's
    float a, b;
    rope_pair(nku, nkv, nc0, ns0, nc1, ns1, a, b);
    if constexpr (NPL == 2) {
      _Float16 ah, al, bh, bl, vh, vl;
      split_f16(a, ah, al);
      split_f16(b, bh, bl);
      split_f16(nvv, vh, vl);
      nka[t] = float(ah) + float(al);
      nkb[t] = float(bh) + float(bl);
      nvs[t] = float(vh) + float(vl);
    } else {
      nka[t] = float(T(a));
      nkb[t] = float(T(b));
      nvs[t] = float(T(nvv));
    }
  }
  __syncthreads();
  const int kd0 = (t * E) % HD;   // K: first dim of this thread's words (same for every i)
  const int vk0 = (t * E) % P;    // V: first key of this thread's words (same for every i)
  // element e of word w (+ its lo plane word wl when split), as the value the cache holds
  auto put = [&](uint4 &w, uint4 &wl, int e, float v) {
    if constexpr (NPL == 2) {
      _Float16 hi, lo;
      split_f16(v, hi, lo);  // v = hi + lo exactly: this gives back the stored planes
      reinterpret_cast<_Float16 *>(&w)[e] = hi;
      reinterpret_cast<_Float16 *>(&wl)[e] = lo;
    } else {
      reinterpret_cast<T *>(&w)[e] = T(v);
    }
  };
  auto get = [&](const uint4 &w, const uint4 &wl, int e) -> float {
    if constexpr (NPL == 2)
      return float(reinterpret_cast<const _Float16 *>(&w)[e]) + float(reinterpret_cast<const _Float16 *>(&wl)[e]);
    else
      return float(reinterpret_cast<const T *>(&w)[e]);
  };
  if (cur) {  // the registers hold the slot as it was before this step: use the new values
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if ((t + 256 * i) * E / HD == slot)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int dd = kd0 + e;
          put(kr[i], krl[NPL == 2 ? i : 0], e, dd < HALF ? nka[dd] : nkb[dd - HALF]);
        }
      const int dim = (t + 256 * i) * E / P;
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (vk0 + e == slot) put(vr[i], vrl[NPL == 2 ? i : 0], e, nvs[HALF + dim]);
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
      float d = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) d = fmaf(q[e], get(kr[i], krl[NPL == 2 ? i : 0], e), d);
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
      float a = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) a = fmaf(p[e], get(vr[i], vrl[NPL == 2 ? i : 0], e), a);
      a = LPD == 16 ? row_sum(a) : group8_sum(a);
      if ((lane & (LPD - 1)) == 0) pbase[gq * hstride + 2 + (t + 256 * i) * E / P] = a;
    }
  }
}

}  // namespace

namespace {
// (GB, T): query heads per workgroup and tiles per group for a GQA group of G heads.  Eight
// waves (two per SIMD) where G allows; G = 7 takes seven.
struct PrefillShape {
  int gb, t;
};
PrefillShape prefill_shape(int G) {
  switch (G) {
    case 2: return {2, 4};
    case 4: return {4, 2};
    case 7: return {7, 1};
    case 8: return {8, 1};
    default: return {1, 8};
  }
}
// Sequences up to this long take the single-stage form for one query head per kv head (MHA): groups of
// 4 tiles, 4 waves, two workgroups per CU.
constexpr int kShortSeq = 1024;
}  // namespace

int attn_prefill_group_tiles(int hq, int hkv, int max_len) {
  return hq == hkv && max_len <= kShortSeq ? 4 : prefill_shape(hq / hkv).t;
}

void launch_attn_prefill(const _Float16 *q16, const _Float16 *q16_lo, int T, int hq,
                         const KvGeom &g, const void *kpool, const void *vpool,
                         const int32_t *pages, int max_pages, const int32_t *tile_seq,
                         const int32_t *tile_row0, const int32_t *tile_pos0,
                         const int32_t *tile_n, int ntiles, const int32_t *grp_first,
                         const int32_t *grp_count, int ngroups, int group_tiles, _Float16 *out16,
                         _Float16 *out16_lo, hipStream_t st) {
  LG_REQUIRE(g.page_tokens == P, "attention: page size must be %d", P);
  LG_REQUIRE(g.hkv > 0 && hq % g.hkv == 0, "attention: hq %% hkv != 0");
  LG_REQUIRE(ntiles > 0 && T > 0, "attention: empty batch");
  const bool split = q16_lo != nullptr;
  LG_REQUIRE(split || !g.split, "attention: the split cache needs split queries");
  LG_REQUIRE(!split || out16_lo, "attention: split path needs the lo output plane");
  LG_REQUIRE(grp_first && grp_count && ngroups > 0 && ngroups <= ntiles, "attention: bad tile groups");
  const int G = hq / g.hkv;
  const bool single = G == 1 && group_tiles == 4;  // attn_prefill_group_tiles' short-sequence form
  const PrefillShape sh = single ? PrefillShape{1, 4} : prefill_shape(G);
  LG_REQUIRE(group_tiles == sh.t, "attention: groups of %d tiles, kernel shape of %d", group_tiles, sh.t);
  const int64_t nwg = int64_t(ngroups) * g.hkv * (G / sh.gb);
  LG_REQUIRE(nwg < (1ll << 31), "attention: too many tiles");
  const dim3 grid{static_cast<uint32_t>(nwg)}, block{static_cast<uint32_t>(64 * sh.gb * sh.t)};
  const _Float16 *kp = static_cast<const _Float16 *>(kpool), *vp = static_cast<const _Float16 *>(vpool);
#define LAUNCH(HDV, NQV, NKVV, WV, GBV, STGV)                                                             \
  hipLaunchKernelGGL((attn_prefill_kernel<HDV, NQV, NKVV, WV, GBV, STGV>), grid, block, 0, st, q16, q16_lo, hq, g, kp, vp, \
                     pages, max_pages, grp_first, grp_count, tile_seq, tile_row0, tile_pos0, tile_n, out16,    \
                     out16_lo)
#define SHAPES(HDV, NQV, NKVV)                                                 \
  if (single) {                                                                \
    LAUNCH(HDV, NQV, NKVV, 4, 1, 1);                                           \
  } else {                                                                     \
    switch (sh.gb) {                                                           \
      case 2: LAUNCH(HDV, NQV, NKVV, 8, 2, 2); break;                          \
      case 4: LAUNCH(HDV, NQV, NKVV, 8, 4, 2); break;                          \
      case 7: LAUNCH(HDV, NQV, NKVV, 7, 7, 2); break;                          \
      case 8: LAUNCH(HDV, NQV, NKVV, 8, 8, 2); break;                          \
      default: LAUNCH(HDV, NQV, NKVV, 8, 1, 2); break;                         \
    }                                                                          \
  }
  if (g.hd == 128) {
    if (g.split) { SHAPES(128, 2, 2) } else if (split) { SHAPES(128, 2, 1) } else { SHAPES(128, 1, 1) }
  } else if (g.hd == 64) {
    if (g.split) { SHAPES(64, 2, 2) } else if (split) { SHAPES(64, 2, 1) } else { SHAPES(64, 1, 1) }
  } else {
    fail(LG_ERR_UNSUPPORTED, "attention: head_dim %d not supported (64, 128)", g.hd);
  }
#undef SHAPES
#undef LAUNCH
  HIP_CHECK(hipGetLastError());
}

int64_t attn_decode_scratch_floats(int hq, int hd, int max_pages) { return int64_t(hq) * max_pages * (2 + hd); }

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
  // a grid of few (page, kv head) workgroups (short contexts, few kv heads: 68 at 1024 tokens of the 7B
  // shape) cannot keep the part busy: then each workgroup serves one query head, `grp` per page and kv
  // head (their page reads meet in the caches); every query head's arithmetic is the same either way
  // (group sizes without their own instance always take this form)
  const bool inst = grp == 1 || grp == 2 || grp == 4 || grp == 7 || grp == 8;
  const bool by_head = grp > 1 && (!inst || int64_t(np + 1) * g.hkv < 512);
  const int gsel = by_head ? 1 : grp, split = by_head ? grp : 1;
  const dim3 grid(np + 1, g.hkv * split), block(256);  // column np stores the new token
#define CASE(HDV, G)                                                                                     \
  case G:                                                                                                \
    if (g.split)                                                                                         \
      hipLaunchKernelGGL((attn_decode_kernel<HDV, G, SplitKV>), grid, block, 0, st, qkv, hq, g, cosT, sinT, \
                         pos, static_cast<_Float16 *>(kpool), static_cast<_Float16 *>(vpool), pages,    \
                         max_pages, part, split);                                                        \
    else                                                                                                 \
      hipLaunchKernelGGL((attn_decode_kernel<HDV, G, _Float16>), grid, block, 0, st, qkv, hq, g, cosT,    \
                         sinT, pos, static_cast<_Float16 *>(kpool), static_cast<_Float16 *>(vpool), pages, \
                         max_pages, part, split);                                                        \
    break;
  if (g.hd == 128) {
    switch (gsel) {
      CASE(128, 1) CASE(128, 2) CASE(128, 4) CASE(128, 7) CASE(128, 8)
      default: fail(LG_ERR_UNSUPPORTED, "decode attention: group size %d not supported", grp);
    }
  } else {
    switch (gsel) {
      CASE(64, 1) CASE(64, 2) CASE(64, 4) CASE(64, 7) CASE(64, 8)
      default: fail(LG_ERR_UNSUPPORTED, "decode attention: group size %d not supported", grp);
    }
  }
#undef CASE
  HIP_CHECK(hipGetLastError());
  if (g.hd == 128)
    hipLaunchKernelGGL((attn_decode_combine<128>), dim3(hq), dim3(256), 0, st, part, max_pages, np, out);
  else
    hipLaunchKernelGGL((attn_decode_combine<64>), dim3(hq), dim3(256), 0, st, part, max_pages, np, out);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
