// Causal GQA attention over the paged F16 KV cache (gfx950).
//
// Reference semantics (src/models/openthai/model.rs:276-294, generalised to hq/hkv heads):
// for query i of head h, kv head kh = h / (hq/hkv), s_j = dot(q_i, k_j) / sqrt(hd) for
// j <= pos_i, p = softmax(s), out = sum_j p_j v_j.
//
// KV page layout (one layer, one page of P = 64 tokens):
//   K: [hkv][P][hd] (row per token)     V: [hkv][hd][P] (column per token)
//
// Prefill: one wave per (32-query tile, query head).  S^T = K . Q^T on MFMA 32x32x16 f16, so
// each lane owns one query column and the online softmax reduces over its own registers plus
// one lane swap; O^T = V^T . P^T then consumes P straight from registers.
//
// Decode: one wave per (sequence, kv head, page): coalesced 16 KB reads of the page's K rows
// and V columns, f32 scores for every query head of the group, partial (max, sum, out) per
// page; a second kernel combines the pages.
#include <hip/hip_runtime.h>

#include "common.h"
#include "kernels.h"

namespace lg {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int P = 64;  // tokens per page
constexpr float kLog2e = 1.4426950408889634f;

template <int HD>
__global__ __launch_bounds__(64) void attn_prefill_kernel(
    const _Float16 *__restrict__ q16, int hq, KvGeom g, const _Float16 *__restrict__ kpool,
    const _Float16 *__restrict__ vpool, const int32_t *__restrict__ pages, int max_pages,
    const int32_t *__restrict__ tile_seq, const int32_t *__restrict__ tile_row0,
    const int32_t *__restrict__ tile_pos0, const int32_t *__restrict__ tile_n,
    _Float16 *__restrict__ out16) {
  constexpr int KT = HD / 16;  // k-steps of the QK^T product
  constexpr int DB = HD / 32;  // 32-wide d blocks of the output
  const int tile = blockIdx.x, h = blockIdx.y;
  const int lane = threadIdx.x, qi = lane & 31, hl = lane >> 5;
  const int seq = tile_seq[tile], row0 = tile_row0[tile], pos0 = tile_pos0[tile], n = tile_n[tile];
  const int kh = h / (hq / g.hkv);
  const int qw = hq * HD;
  const int qpos = pos0 + qi;
  const bool live = qi < n;

  // Q^T operand: lane holds q[qi][16t + 8*hl .. +8]
  half8 qr[KT];
  {
    const _Float16 *qp = q16 + int64_t(row0 + min(qi, n - 1)) * qw + h * HD + hl * 8;
#pragma unroll
    for (int t = 0; t < KT; ++t) qr[t] = *reinterpret_cast<const half8 *>(qp + 16 * t);
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

  for (int kt = 0; kt <= last / P; ++kt) {
    const int64_t page = ptab[kt];
    const _Float16 *Kp = kpool + page * g.page_stride + int64_t(kh) * P * HD;
    const _Float16 *Vp = vpool + page * g.page_stride + int64_t(kh) * HD * P;
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
      const _Float16 *kr = Kp + (kb * 32 + qi) * HD + hl * 8;
#pragma unroll
      for (int t = 0; t < KT; ++t)
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(kr + 16 * t),
                                                       qr[t], s[kb], 0, 0, 0);
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
      half8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = _Float16(s[c >> 1][(c & 1) * 8 + e]);
#pragma unroll
      for (int b = 0; b < DB; ++b) {
        const _Float16 *vr = Vp + (b * 32 + qi) * P + 16 * c + hl * 4;
        const half4 lo = *reinterpret_cast<const half4 *>(vr);
        const half4 hi = *reinterpret_cast<const half4 *>(vr + 8);
        const half8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, acc[b], 0, 0, 0);
      }
    }
  }
  if (!live) return;
  const float inv = 1.0f / l;
  _Float16 *op = out16 + int64_t(row0 + qi) * qw + h * HD;
  // acc[b][r] <-> d = b*32 + (r/4)*8 + hl*4 + r%4
#pragma unroll
  for (int b = 0; b < DB; ++b)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      half4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = _Float16(acc[b][r4 * 4 + j] * inv);
      *reinterpret_cast<half4 *>(op + b * 32 + r4 * 8 + hl * 4) = o;
    }
}

// ---------------------------------------------------------------- decode
// part layout: [nseq][hq][max_pages][2 + HD] = (max, sum, out[HD]) of one page.
template <int HD, int GRP>
__global__ __launch_bounds__(64) void attn_decode_kernel(const float *__restrict__ q32, int hq, KvGeom g,
                                                         const _Float16 *__restrict__ kpool,
                                                         const _Float16 *__restrict__ vpool,
                                                         const int32_t *__restrict__ pages,
                                                         int max_pages,
                                                         const int32_t *__restrict__ ctx_len,
                                                         float *__restrict__ part) {
  static_assert(HD == 128, "decode attention is written for head_dim 128");
  const int pi = blockIdx.x, kh = blockIdx.y, s = blockIdx.z;
  const int lane = threadIdx.x;
  const int len = ctx_len[s];
  float *pbase = part + ((int64_t(s) * hq + kh * GRP) * max_pages + pi) * (2 + HD);
  const int64_t hstride = int64_t(max_pages) * (2 + HD);
  if (pi * P >= len) {
    if (lane == 0)
      for (int gq = 0; gq < GRP; ++gq) {
        pbase[gq * hstride] = -INFINITY;
        pbase[gq * hstride + 1] = 0.0f;
      }
    return;
  }
  const int64_t page = pages[int64_t(s) * max_pages + pi];
  const uint4 *Kp = reinterpret_cast<const uint4 *>(kpool + page * g.page_stride + int64_t(kh) * P * HD);
  const uint4 *Vp = reinterpret_cast<const uint4 *>(vpool + page * g.page_stride + int64_t(kh) * HD * P);
  uint4 kv[16], vv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) kv[i] = Kp[i * 64 + lane];  // key lane/16 + 4i, dims (lane%16)*8
#pragma unroll
  for (int i = 0; i < 16; ++i) vv[i] = Vp[i * 64 + lane];  // d lane/8 + 8i, keys (lane%8)*8
  __shared__ float sc[GRP][P];
  const float inv_sqrt = 1.0f / sqrtf(float(HD));
#pragma unroll
  for (int gq = 0; gq < GRP; ++gq) {
    const float *q = q32 + int64_t(s) * hq * HD + (kh * GRP + gq) * HD + (lane & 15) * 8;
    float qv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) qv[j] = q[j];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const _Float16 *kh8 = reinterpret_cast<const _Float16 *>(&kv[i]);
      float d = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) d += qv[j] * float(kh8[j]);
      d += __shfl_xor(d, 1);
      d += __shfl_xor(d, 2);
      d += __shfl_xor(d, 4);
      d += __shfl_xor(d, 8);
      const int key = (lane >> 4) + 4 * i;
      if ((lane & 15) == 0) sc[gq][key] = (pi * P + key < len) ? d * inv_sqrt : -INFINITY;
    }
  }
  __syncthreads();
#pragma unroll
  for (int gq = 0; gq < GRP; ++gq) {
    const float v = sc[gq][lane];
    float mx = v;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    const float p = v == -INFINITY ? 0.0f : __expf(v - mx);
    float sum = p;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    __syncthreads();
    sc[gq][lane] = p;
    __syncthreads();
    float o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const _Float16 *v8 = reinterpret_cast<const _Float16 *>(&vv[i]);
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) a += sc[gq][(lane & 7) * 8 + j] * float(v8[j]);
      a += __shfl_xor(a, 1);
      a += __shfl_xor(a, 2);
      a += __shfl_xor(a, 4);
      o[i] = a;
    }
    float *pp = pbase + gq * hstride;
    if (lane == 0) {
      pp[0] = mx;
      pp[1] = sum;
    }
    if ((lane & 7) == 0)
#pragma unroll
      for (int i = 0; i < 16; ++i) pp[2 + (lane >> 3) + 8 * i] = o[i];
  }
}

__global__ __launch_bounds__(128) void attn_decode_combine(const float *__restrict__ part, int hq, int hd,
                                                           int max_pages,
                                                           const int32_t *__restrict__ ctx_len,
                                                           float *__restrict__ out) {
  const int h = blockIdx.x, s = blockIdx.y;
  const int np = (ctx_len[s] + P - 1) / P;
  const float *pb = part + (int64_t(s) * hq + h) * max_pages * (2 + hd);
  float M = -INFINITY;
  for (int i = 0; i < np; ++i) M = fmaxf(M, pb[int64_t(i) * (2 + hd)]);
  float L = 0.0f, acc = 0.0f;
  const int d = threadIdx.x;
  for (int i = 0; i < np; ++i) {
    const float *p = pb + int64_t(i) * (2 + hd);
    if (p[0] == -INFINITY) continue;
    const float w = __expf(p[0] - M);
    L += p[1] * w;
    if (d < hd) acc += p[2 + d] * w;
  }
  if (d < hd) out[(int64_t(s) * hq + h) * hd + d] = acc / L;
}

}  // namespace

void launch_attn_prefill(const _Float16 *q16, int T, int hq, const KvGeom &g,
                         const _Float16 *kpool, const _Float16 *vpool, const int32_t *pages,
                         int max_pages, const int32_t *tile_seq, const int32_t *tile_row0,
                         const int32_t *tile_pos0, const int32_t *tile_n, int ntiles,
                         _Float16 *out16, hipStream_t st) {
  LG_REQUIRE(g.page_tokens == P, "attention: page size must be %d", P);
  LG_REQUIRE(hq % g.hkv == 0, "attention: hq %% hkv != 0");
  LG_REQUIRE(ntiles > 0 && T > 0, "attention: empty batch");
  const dim3 grid(ntiles, hq), block(64);
  switch (g.hd) {
    case 64:
      hipLaunchKernelGGL(attn_prefill_kernel<64>, grid, block, 0, st, q16, hq, g, kpool, vpool, pages,
                         max_pages, tile_seq, tile_row0, tile_pos0, tile_n, out16);
      break;
    case 128:
      hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, block, 0, st, q16, hq, g, kpool, vpool, pages,
                         max_pages, tile_seq, tile_row0, tile_pos0, tile_n, out16);
      break;
    default: fail(LG_ERR_UNSUPPORTED, "attention: head_dim %d not supported (64, 128)", g.hd);
  }
  HIP_CHECK(hipGetLastError());
}

int64_t attn_decode_scratch_floats(int nseq, int hq, int hd, int max_ctx) {
  const int64_t pages = (max_ctx + P - 1) / P;
  return int64_t(nseq) * hq * pages * (2 + hd);
}

void launch_attn_decode(const float *q32, int nseq, int hq, const KvGeom &g,
                        const _Float16 *kpool, const _Float16 *vpool, const int32_t *pages,
                        int max_pages, const int32_t *ctx_len, int max_ctx, float *part,
                        float *out, hipStream_t st) {
  LG_REQUIRE(g.page_tokens == P, "attention: page size must be %d", P);
  LG_REQUIRE(g.hd == 128, "decode attention: head_dim %d not supported (128)", g.hd);
  LG_REQUIRE(nseq > 0 && max_ctx > 0, "decode attention: empty");
  const int np = (max_ctx + P - 1) / P;
  LG_REQUIRE(np <= max_pages, "decode attention: context exceeds the page table");
  const int grp = hq / g.hkv;
  const dim3 grid(np, g.hkv, nseq), block(64);
  switch (grp) {
#define CASE(G)                                                                                   \
  case G:                                                                                         \
    hipLaunchKernelGGL((attn_decode_kernel<128, G>), grid, block, 0, st, q32, hq, g, kpool, vpool, \
                       pages, max_pages, ctx_len, part);                                         \
    break;
    CASE(1) CASE(2) CASE(4) CASE(7) CASE(8)
#undef CASE
    default: fail(LG_ERR_UNSUPPORTED, "decode attention: group size %d not supported", grp);
  }
  hipLaunchKernelGGL(attn_decode_combine, dim3(hq, nseq), dim3(128), 0, st, part, hq, g.hd, max_pages,
                     ctx_len, out);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
