// Dequantisation and repacking kernels.
//
// Bit-exactness: fp contraction is off for this file and every product/difference uses
// the _rn intrinsics, so each operation rounds once, in the reference's order.
#pragma clang fp contract(off)
#include <hip/hip_runtime.h>

#include "common.h"
#include "f16split.h"
#include "kernels.h"
#include "quant.h"

namespace lg {

int64_t DevMatrix::bytes() const {
  const int64_t n = int64_t(rows) * cols;
  switch (kind) {
    case LG_F32: return n * 4;
    case LG_F16: return n * 2;
    case LG_Q8_0: return n + n / 32 * 2;
    case LG_Q4_K: return n / 2 + n / 32 * 8;
    case LG_Q6_K: return n + n / 16 * 4;
    default: return 0;
  }
}

int64_t DevMatrix::gguf_bytes() const {
  const int64_t n = int64_t(rows) * cols;
  switch (kind) {
    case LG_F32: return n * 4;
    case LG_F16: return n * 2;
    case LG_Q8_0: return n / 32 * 34;
    case LG_Q4_K: return n / 256 * 144;
    case LG_Q6_K: return n / 256 * 210;
    default: return 0;
  }
}

namespace {

__device__ __forceinline__ float h2(const uint8_t *b) { return half_bits(uint32_t(b[0]) | (uint32_t(b[1]) << 8)); }

// One thread per output element, straight from GGUF blocks (src/gguf.rs:250-336).
__global__ void dequant_gguf(uint32_t kind, const uint8_t *__restrict__ src, uint64_t nelem,
                             float *__restrict__ dst) {
  const uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= nelem) return;
  float v = 0.0f;
  switch (kind) {
    case LG_F32: v = __uint_as_float(uint32_t(src[4 * e]) | (uint32_t(src[4 * e + 1]) << 8) |
                                     (uint32_t(src[4 * e + 2]) << 16) | (uint32_t(src[4 * e + 3]) << 24));
      break;
    case LG_F16: v = h2(src + 2 * e); break;
    case LG_Q8_0: {
      const uint8_t *c = src + 34 * (e / 32);
      v = __fmul_rn(h2(c), float(int8_t(c[2 + e % 32])));
    } break;
    case LG_Q4_0: {
      const uint8_t *c = src + 18 * (e / 32);
      const int j = int(e % 32);
      const uint32_t q = j < 16 ? (c[2 + j] & 15u) : (uint32_t(c[2 + j - 16]) >> 4);
      v = __fmul_rn(h2(c), __fsub_rn(float(q), 8.0f));
    } break;
    case LG_Q4_K: {
      const uint8_t *c = src + 144 * (e / 256);
      const int w = int(e % 256), g = w / 64, t = (w % 64) / 32, j = w % 32;
      uint32_t s, m;
      q4k_scale_min(c + 4, g * 2 + t, s, m);
      const uint32_t q = c[16 + g * 32 + j];
      const uint32_t nib = t ? (q >> 4) : (q & 15u);
      v = __fsub_rn(__fmul_rn(__fmul_rn(h2(c), float(s)), float(nib)), __fmul_rn(h2(c + 2), float(m)));
    } break;
    case LG_Q6_K: {
      const uint8_t *c = src + 210 * (e / 256);
      int si;
      const uint32_t q = q6k_code(c, int(e % 256), si);
      v = __fmul_rn(__fmul_rn(h2(c + 208), float(int8_t(c[192 + si]))), __fsub_rn(float(q), 32.0f));
    } break;
  }
  dst[e] = v;
}

// ---- repack: one thread per GGUF block ----
__global__ void repack_q8(const uint8_t *__restrict__ src, uint64_t nblocks, int8_t *__restrict__ q,
                          uint16_t *__restrict__ s) {
  const uint64_t b = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t *c = src + 34 * b;
  s[b] = uint16_t(c[0] | (c[1] << 8));
  for (int j = 0; j < 32; ++j) q[32 * b + j] = int8_t(c[2 + j]);
}

__global__ void repack_q4k(const uint8_t *__restrict__ src, uint64_t nblocks, uint8_t *__restrict__ q,
                           float2 *__restrict__ s) {
  const uint64_t b = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t *c = src + 144 * b;
  const float d = h2(c), dm = h2(c + 2);
  for (int j = 0; j < 8; ++j) {
    uint32_t sc, m;
    q4k_scale_min(c + 4, j, sc, m);
    s[8 * b + j] = make_float2(__fmul_rn(d, float(sc)), __fmul_rn(dm, float(m)));
  }
  for (int j = 0; j < 128; ++j) q[128 * b + j] = c[16 + j];
}

__global__ void repack_q6k(const uint8_t *__restrict__ src, uint64_t nblocks, int8_t *__restrict__ q,
                           float *__restrict__ s) {
  const uint64_t b = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t *c = src + 210 * b;
  const float d = h2(c + 208);
  for (int j = 0; j < 16; ++j) s[16 * b + j] = __fmul_rn(d, float(int8_t(c[192 + j])));
  for (int w = 0; w < 256; ++w) {
    int si;
    q[256 * b + w] = int8_t(int(q6k_code(c, w, si)) - 32);
  }
}

// f32 weight from the repacked layout -- the arithmetic the GEMV kernels use.
// Q4_K / Q6_K weight (n, k) of the repacked layout.
__device__ __forceinline__ float kquant_weight(const DevMatrix &W, uint64_t n, uint64_t k) {
  const uint64_t cols = uint64_t(W.cols);
  if (W.kind == LG_Q4_K) {
    const uint8_t byte = static_cast<const uint8_t *>(W.q)[n * (cols / 2) + (k / 64) * 32 + (k % 32)];
    const uint32_t nib = (k % 64) >= 32 ? (byte >> 4) : (byte & 15u);
    const float2 ab = static_cast<const float2 *>(W.s)[n * (cols / 32) + k / 32];
    return kq4_weight(ab.x, nib, ab.y);
  }
  return kq6_weight(static_cast<const float *>(W.s)[n * (cols / 16) + k / 16],
                    static_cast<const int8_t *>(W.q)[n * cols + k]);
}

__global__ void dequant_repacked(DevMatrix W, float *__restrict__ dst) {
  const uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t cols = uint64_t(W.cols);
  if (e >= uint64_t(W.rows) * cols) return;
  const uint64_t n = e / cols, k = e % cols;
  float v = 0.0f;
  switch (W.kind) {
    case LG_F32: v = static_cast<const float *>(W.q)[e]; break;
    case LG_F16: v = half_bits(static_cast<const uint16_t *>(W.q)[e]); break;
    case LG_Q8_0:
      v = __fmul_rn(half_bits(static_cast<const uint16_t *>(W.s)[n * (cols / 32) + k / 32]),
                    float(static_cast<const int8_t *>(W.q)[e]));
      break;
    case LG_Q4_K:
    case LG_Q6_K: v = kquant_weight(W, n, k); break;
  }
  dst[e] = v;
}

// Prefill copy of a K-quant matrix: the weight split into f16 hi / lo planes, one element each.
__global__ void split_planes_kernel(DevMatrix W, _Float16 *__restrict__ hi, _Float16 *__restrict__ lo) {
  const uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t cols = uint64_t(W.cols);
  if (e >= uint64_t(W.rows) * cols) return;
  _Float16 h, l;
  split_f16(kquant_weight(W, e / cols, e % cols), h, l);
  hi[e] = h;
  lo[e] = l;
}

// Prefill copy of a Q8_0 matrix: codes [rows][cols] int8 -> f16, scales [rows][cols/32] f16 -> f32
// transposed to [cols/32][rows].  One 32-element block per thread.
__global__ void q8_prefill_copy_kernel(const int8_t *__restrict__ q, const uint16_t *__restrict__ s, int rows,
                                       int cols, _Float16 *__restrict__ codes, float *__restrict__ scales) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int nb = cols / 32;
  if (i >= int64_t(rows) * nb) return;
  const int n = int(i / nb), kb = int(i % nb);
  const int8_t *src = q + int64_t(n) * cols + kb * 32;
  _Float16 *dst = codes + int64_t(n) * cols + kb * 32;
#pragma unroll
  for (int e = 0; e < 32; ++e) dst[e] = _Float16(float(src[e]));
  scales[int64_t(kb) * rows + n] = half_bits(s[i]);
}

// Prefill copy of a Q4_K matrix in the two-pass form (DevMatrix::pc, pcs, pcl, pcr), one wave per
// row: codes as f16, the sub-block scales A = d*sc transposed, and the correction planes of -B =
// -(dmin*m) scaled by the row's power of two 2^e (its largest |B| into [2^13, 2^14), so the f16 lo
// plane stays out of the subnormals) with 2^-e kept per row.  Scaling by 2^e is exact.
__global__ __launch_bounds__(256) void q4k_prefill_copy_kernel(const uint8_t *__restrict__ q, const float2 *__restrict__ s,
                                                               int rows, int cols, int kp, _Float16 *__restrict__ codes,
                                                               float *__restrict__ ascale, _Float16 *__restrict__ bh,
                                                               _Float16 *__restrict__ bl, float *__restrict__ rs) {
  const int row = int(blockIdx.x) * 4 + int(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int nb = cols / 32;
  const float2 *sr = s + int64_t(row) * nb;
  float mx = 0.0f;
  for (int c = lane; c < nb; c += 64) mx = fmaxf(mx, fabsf(sr[c].y));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  int e = 0;  // a zero or non-finite maximum leaves the row unscaled
  if (mx > 0.0f && mx <= 3.4e38f) {
    int ex;
    (void)frexpf(mx, &ex);  // mx = f 2^ex, f in [0.5, 1)
    e = 14 - ex;
  }
  const float up = ldexpf(1.0f, e);
  if (lane == 0) rs[row] = ldexpf(1.0f, -e);
  for (int c = lane; c < kp; c += 64) {
    _Float16 h = _Float16(0.0f), l = _Float16(0.0f);
    if (c < nb) {
      split_f16(-(sr[c].y * up), h, l);
      ascale[int64_t(c) * rows + row] = sr[c].x;
    }
    bh[int64_t(row) * kp + c] = h;
    bl[int64_t(row) * kp + c] = l;
  }
  // byte j of each 64-element group holds element j (low nibble) and j + 32 (high nibble)
  const uint8_t *qr = q + int64_t(row) * (cols / 2);
  for (int k = lane; k < cols; k += 64) {
    const uint32_t byte = qr[(k / 64) * 32 + (k % 32)];
    codes[int64_t(row) * cols + k] = _Float16(float((k % 64) >= 32 ? (byte >> 4) : (byte & 15u)));
  }
}

// Chunk sums of hi/lo activation planes (launch_chunk_sums): one 32-element chunk per thread.
__global__ __launch_bounds__(256) void chunk_sums_kernel(const _Float16 *__restrict__ A, const _Float16 *__restrict__ Alo,
                                                         int M, int K, int kp, _Float16 *__restrict__ ks) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= int64_t(M) * kp) return;
  const int m = int(i / kp), c = int(i % kp);
  float sum = 0.0f;
  if (c < K / 32) {
    const uint4 *h = reinterpret_cast<const uint4 *>(A + int64_t(m) * K + c * 32);
    const uint4 *l = reinterpret_cast<const uint4 *>(Alo + int64_t(m) * K + c * 32);
    uint4 hv[4], lv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      hv[u] = h[u];
      lv[u] = l[u];
    }
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const h8 a = __builtin_bit_cast(h8, hv[u]), b = __builtin_bit_cast(h8, lv[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += f32_pin(float(a[e]) + float(b[e]));  // hi + lo is exact in f32
    }
  }
  _Float16 hh, ll;
  split_f16(sum, hh, ll);
  ks[i] = hh;
  ks[int64_t(M) * kp + i] = ll;
}

inline unsigned grid_for(uint64_t n, unsigned block) { return unsigned((n + block - 1) / block); }

}  // namespace

void launch_dequant(uint32_t kind, const uint8_t *src, uint64_t nblocks, float *dst, hipStream_t st) {
  uint64_t block, size;
  switch (kind) {
    case LG_F32: block = 1; size = 4; break;
    case LG_F16: block = 1; size = 2; break;
    case LG_Q4_0: block = 32; size = 18; break;
    case LG_Q8_0: block = 32; size = 34; break;
    case LG_Q4_K: block = 256; size = 144; break;
    case LG_Q6_K: block = 256; size = 210; break;
    default: fail(LG_ERR_UNSUPPORTED, "unsupported GGML tensor type %u", kind);
  }
  (void)size;
  const uint64_t n = nblocks * block;
  if (n == 0) return;
  LG_REQUIRE(n / 256 < (1ull << 31), "dequant: tensor too large for one launch");
  hipLaunchKernelGGL(dequant_gguf, dim3(grid_for(n, 256)), dim3(256), 0, st, kind, src, n, dst);
  HIP_CHECK(hipGetLastError());
}

void launch_repack(uint32_t kind, const uint8_t *src, int rows, int cols, DevMatrix &w, hipStream_t st) {
  LG_REQUIRE(w.q != nullptr && rows > 0 && cols > 0, "repack: empty matrix");
  const uint64_t n = uint64_t(rows) * uint64_t(cols);
  switch (kind) {
    case LG_F32:
      HIP_CHECK(hipMemcpyAsync(w.q, src, n * 4, hipMemcpyDeviceToDevice, st));
      return;
    case LG_F16:
      HIP_CHECK(hipMemcpyAsync(w.q, src, n * 2, hipMemcpyDeviceToDevice, st));
      return;
    case LG_Q8_0:
      LG_REQUIRE(cols % 32 == 0 && w.s, "repack: Q8_0 rows must be whole blocks");
      hipLaunchKernelGGL(repack_q8, dim3(grid_for(n / 32, 256)), dim3(256), 0, st, src, n / 32,
                         static_cast<int8_t *>(w.q), static_cast<uint16_t *>(w.s));
      break;
    case LG_Q4_K:
      LG_REQUIRE(cols % 256 == 0 && w.s, "repack: Q4_K rows must be whole blocks");
      hipLaunchKernelGGL(repack_q4k, dim3(grid_for(n / 256, 128)), dim3(128), 0, st, src, n / 256,
                         static_cast<uint8_t *>(w.q), static_cast<float2 *>(w.s));
      break;
    case LG_Q6_K:
      LG_REQUIRE(cols % 256 == 0 && w.s, "repack: Q6_K rows must be whole blocks");
      hipLaunchKernelGGL(repack_q6k, dim3(grid_for(n / 256, 128)), dim3(128), 0, st, src, n / 256,
                         static_cast<int8_t *>(w.q), static_cast<float *>(w.s));
      break;
    default:
      fail(LG_ERR_UNSUPPORTED, "no device layout for GGML tensor type %u", kind);
  }
  HIP_CHECK(hipGetLastError());
}

size_t prefill_copy_bytes(uint32_t kind, int rows, int cols) {
  const size_t n = size_t(rows) * size_t(cols);
  switch (kind) {
    case LG_Q8_0: return n * 2 + size_t(rows) * size_t(cols / 32) * 4;
    case LG_Q4_K:
      return n * 2 + size_t(rows) * size_t(cols / 32) * 4 + size_t(rows) * size_t(ksum_cols(cols)) * 4 + size_t(rows) * 4;
    case LG_Q6_K: return n * 4;
  }
  return 0;
}

void launch_chunk_sums(const _Float16 *A, const _Float16 *Alo, int M, int K, int kp, _Float16 *ks, hipStream_t st) {
  LG_REQUIRE(A && Alo && ks && M > 0 && K % 32 == 0 && kp >= K / 32, "chunk sums: bad arguments");
  const int64_t n = int64_t(M) * kp;
  LG_REQUIRE((n + 255) / 256 < (int64_t(1) << 31), "chunk sums: too many rows");
  hipLaunchKernelGGL(chunk_sums_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, A, Alo, M, K, kp, ks);
  HIP_CHECK(hipGetLastError());
}

void launch_prefill_copy(const DevMatrix &w, hipStream_t st) {
  const int64_t n = int64_t(w.rows) * w.cols;
  LG_REQUIRE(w.rows > 0 && w.cols > 0 && w.pc, "prefill copy: bad matrix");
  if (w.kind == LG_Q8_0) {
    LG_REQUIRE(w.pcs && w.cols % 32 == 0, "prefill copy: Q8_0 needs scales and whole blocks");
    const int64_t blocks = n / 32;
    LG_REQUIRE((blocks + 255) / 256 < (int64_t(1) << 31), "prefill copy: matrix too large");
    hipLaunchKernelGGL(q8_prefill_copy_kernel, dim3(unsigned((blocks + 255) / 256)), dim3(256), 0, st,
                       static_cast<const int8_t *>(w.q), static_cast<const uint16_t *>(w.s), w.rows, w.cols, w.pc,
                       w.pcs);
  } else if (w.kind == LG_Q4_K) {
    LG_REQUIRE(w.pcs && w.pcl && w.pcr && w.cols % 256 == 0 && w.pkp == ksum_cols(w.cols),
               "prefill copy: Q4_K needs codes, scales, correction planes and whole super-blocks");
    hipLaunchKernelGGL(q4k_prefill_copy_kernel, dim3(unsigned((w.rows + 3) / 4)), dim3(256), 0, st,
                       static_cast<const uint8_t *>(w.q), static_cast<const float2 *>(w.s), w.rows, w.cols, w.pkp, w.pc,
                       w.pcs, w.pcl, w.pcl + int64_t(w.rows) * w.pkp, w.pcr);
  } else if (w.kind == LG_Q6_K) {
    LG_REQUIRE(w.pcl && w.cols % 256 == 0, "prefill copy: K-quant needs both planes and whole super-blocks");
    LG_REQUIRE((n + 255) / 256 < (int64_t(1) << 31), "prefill copy: matrix too large");
    hipLaunchKernelGGL(split_planes_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, w, w.pc, w.pcl);
  } else {
    fail(LG_ERR_UNSUPPORTED, "prefill copy: GGML type %u has none", w.kind);
  }
  HIP_CHECK(hipGetLastError());
}

void launch_dequant_repacked(const DevMatrix &w, float *dst, hipStream_t st) {
  const uint64_t n = uint64_t(w.rows) * uint64_t(w.cols);
  LG_REQUIRE(n / 256 < (1ull << 31), "dequant: matrix too large for one launch");
  hipLaunchKernelGGL(dequant_repacked, dim3(grid_for(n, 256)), dim3(256), 0, st, w, dst);
  HIP_CHECK(hipGetLastError());
}

}  // namespace lg
