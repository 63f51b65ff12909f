// Exact Q8_0 prefill GEMM for large batches (gfx950): C = A . W^T with A given as f16 hi/lo
// planes and W as Q8_0 (codes exact in f16, one f32 scale per 32-element block).
//
// Per 32 x 32 output block and Q8_0 block the partial sum is one chain of four MFMAs
// (v_mfma_f32_32x32x16_f16: hi and lo planes of A against the codes, two 16-deep k halves),
// then acc += d * partial in f32 -- the operation order of the 128 x 128 tiles in
// gemm_tiles.h, so both give the same bits.
//
// Operands come from the weight's prefill copy (DevMatrix::pc, pcs): codes as f16 [N][K]
// and scales as f32 [K/32][N], written once at upload, so every operand byte reaches LDS by
// LDS-DMA (buffer_load ... lds, 16 bytes a lane) with no register staging and no conversion.
//
// Geometry: 512 threads = 8 wave64s (2 per SIMD), workgroup tile 256 x 256, K steps of 32
// (one Q8_0 block), three LDS stages (147 KiB): stage k + 2 is in flight while stage k is
// consumed, one barrier per step.  Wave w owns rows 64 (w / 2) .. + 64 and columns
// 128 (w % 2) .. + 128 of the tile (2 x 4 MFMA blocks).
//
// LDS rows are 64 bytes (four 16-byte chunks); logical chunk c of row r sits in slot
// c ^ ((r >> 2) & 3), so the 16 lanes of each quarter of an operand read fall in 16 distinct
// 16-byte bank groups.  The DMA side writes whole 1 KiB blocks: lane L of a block fetches the
// global chunk that belongs in its slot.
#pragma once
#include <hip/hip_runtime.h>

#include "common.h"
#include "f16split.h"
#include "kernels.h"

namespace lg {
namespace q8x {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 32, STAGES = 3, WAVES = 8, THREADS = 64 * WAVES;
constexpr int ROWB = BK * 2;                        // bytes per LDS row of one plane
constexpr int PLANE = BM * ROWB;                    // 16 KiB
constexpr int A_HI = 0, A_LO = PLANE, B_OFF = 2 * PLANE, S_OFF = 3 * PLANE;
constexpr int STAGE_BYTES = S_OFF + BN * 4;         // + f32 scales of the step
constexpr int LDS_BYTES = STAGES * STAGE_BYTES;     // 150,528
constexpr int MIN_PER_WAVE = 3 * PLANE / 1024 / WAVES;  // DMA instructions per wave and stage (wave 0: + 1)
static_assert(BM == BN, "A and B planes share one slot layout");

__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }

#define Q8X_MFMA(a, b, c) __builtin_amdgcn_mfma_f32_32x32x16_f16((a), (b), (c), 0, 0, 0)

__device__ __forceinline__ float silu_f(float g) { return g * (1.0f / (1.0f + __expf(-g))); }

// EPI: Epi values (F32, ADD, F16 planes, SWIGLU).  For SWIGLU the workgroup's 256 weight rows
// are 128 gate rows and the 128 matching up rows: wave column wn holds gate rows in its blocks
// 0, 1 and the up rows of the same output columns in blocks 2, 3.
template <int EPI>
__global__ __launch_bounds__(THREADS, 1) void gemm_q8x_kernel(
    const _Float16 *__restrict__ A, const _Float16 *__restrict__ Alo, int M, int K,
    const _Float16 *__restrict__ Wc, const float *__restrict__ Ws, int N, float *__restrict__ C,
    _Float16 *__restrict__ C16, _Float16 *__restrict__ C16lo, int ldc, const float *__restrict__ bias,
    int MT, int NT, int ffn) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr bool kGlu = EPI == int(Epi::SWIGLU);
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: scalar DMA setup
  const int wm = wave >> 1, wn = wave & 1;

  // tile order: consecutive workgroups go to the 8 XCDs round-robin; each XCD takes a
  // contiguous range of tiles, walked in groups of 4 M-tiles so that the concurrently
  // resident tiles of one XCD share A rows and weight rows through its L2
  int mt, nt;
  {
    const int nblk = gridDim.x;
    int id = blockIdx.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);
    constexpr int GM = 4;
    const int group = id / (GM * NT), first = group * GM;
    const int gm = min(MT - first, GM), in = id - group * GM * NT;
    mt = first + in % gm;
    nt = in / gm;
  }
  const int m0 = mt * BM;

  // weight row of local B row r
  auto wrow = [&](int r) -> int {
    if constexpr (kGlu) {
      const int wc = r >> 7, jb = (r >> 5) & 3, up = jb >> 1, jj = jb & 1;
      return up * ffn + nt * (BN / 2) + wc * 64 + jj * 32 + (r & 31);
    } else {
      return nt * BN + r;
    }
  };

  // DMA: a stage is 48 operand blocks of 1 KiB (16 per plane: A hi, A lo, codes) plus one of
  // scales.  Wave w issues operand blocks w + 8 i, i = 0..5 -- i = 0, 1 in the A hi plane,
  // 2, 3 in the A lo plane, 4, 5 in the codes -- and wave 0 also the scale block.
  static_assert(PLANE / 1024 == 2 * WAVES, "two blocks of each plane per wave");
  const uint32_t abytes = uint32_t(M) * uint32_t(K) * 2u;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(A), 0, abytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(Alo), 0, abytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(Wc), 0, uint32_t(N) * uint32_t(K) * 2u, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(Ws), 0, uint32_t(N) * uint32_t(K / 32) * 4u, kBufferFlags);
  uint32_t aoff[2], boff[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int slot = (wave + WAVES * h) * 64 + lane;  // 16-byte slot inside a plane
    const int row = slot >> 2, c = (slot & 3) ^ swz(row);
    aoff[h] = uint32_t(m0 + row) * uint32_t(K) * 2u + uint32_t(c) * 16u;  // rows >= M: past the buffer -> zeros
    boff[h] = uint32_t(wrow(row)) * uint32_t(K) * 2u + uint32_t(c) * 16u;
  }
  const uint32_t soff = uint32_t(wrow(4 * lane)) * 4u;  // four consecutive weight rows' scales
  const int nk = K / BK;
  auto issue = [&](int kt, int st) {
#if defined(__HIP_DEVICE_COMPILE__)
    // device pass only: with a run-time voffset this builtin keeps the host pass from
    // emitting the kernel's launch stub (the host never runs kernel bodies)
    typedef __attribute__((address_space(3))) void *lds_ptr;
    uint8_t *base = lds + st * STAGE_BYTES;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int blk = (wave + WAVES * h) * 1024;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr)(base + A_HI + blk), 16, aoff[h], kt * BK * 2, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, (lds_ptr)(base + A_LO + blk), 16, aoff[h], kt * BK * 2, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr)(base + B_OFF + blk), 16, boff[h], kt * BK * 2, 0, 0);
    }
    if (wave == 0) __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(base + S_OFF), 16, soff, kt * N * 4, 0, 0);
#endif
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // operand read offsets: row (lane & 31) of each 32-row block, chunk 2 kk + (lane >> 5)
  const int lr = lane & 31, sw = swz(lr);
  const int ac0 = (wm * 64 + lr) * ROWB, bc0 = (wn * 128 + lr) * ROWB;
  const int ch0 = ((0 + (lane >> 5)) ^ sw) * 16, ch1 = ((2 + (lane >> 5)) ^ sw) * 16;
  const f32x16 zero = {};

  issue(0, 0);
  if (nk > 1) issue(1, 1);
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(MIN_PER_WAVE) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // every wave has its part of stage kt in LDS and is done reading stage kt - 1; a bare
    // barrier (no fence), so the DMA of stage kt + 1 stays in flight across it
    asm volatile("s_barrier" ::: "memory");
    if (kt + 2 < nk) issue(kt + 2, (kt + 2) % STAGES);
    const uint8_t *st = lds + (kt % STAGES) * STAGE_BYTES;
    float d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = *reinterpret_cast<const float *>(st + S_OFF + (wn * 128 + j * 32 + lr) * 4);
    half8 ah[2][2], al[2][2], b[2][4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int ch = kk ? ch1 : ch0;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ah[kk][i] = *reinterpret_cast<const half8 *>(st + A_HI + ac0 + i * 32 * ROWB + ch);
        al[kk][i] = *reinterpret_cast<const half8 *>(st + A_LO + ac0 + i * 32 * ROWB + ch);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) b[kk][j] = *reinterpret_cast<const half8 *>(st + B_OFF + bc0 + j * 32 * ROWB + ch);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x16 p = Q8X_MFMA(ah[0][i], b[0][j], zero);
        p = Q8X_MFMA(al[0][i], b[0][j], p);
        p = Q8X_MFMA(ah[1][i], b[1][j], p);
        p = Q8X_MFMA(al[1][i], b[1][j], p);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] += d[j] * p[r];
      }
  }

  // epilogue: acc[i][j] register r -> row (r/4)*8 + (lane/32)*4 + r%4, column lane%32
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (row >= M) continue;
      if constexpr (kGlu) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int col = nt * (BN / 2) + wn * 64 + jj * 32 + lr;
          const float v = silu_f(acc[i][jj][r]) * acc[i][jj + 2][r];
          _Float16 h, hl;
          split_f16(v, h, hl);
          C16[int64_t(row) * ldc + col] = h;
          if (C16lo) C16lo[int64_t(row) * ldc + col] = hl;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int col = nt * BN + wn * 128 + j * 32 + lr;
          float v = acc[i][j][r];
          if (bias) v += bias[col];
          if constexpr (EPI == int(Epi::F32)) {
            C[int64_t(row) * ldc + col] = v;
          } else if constexpr (EPI == int(Epi::ADD)) {
            C[int64_t(row) * ldc + col] += v;
          } else {
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
#undef Q8X_MFMA

// Prefill copy of a repacked Q8_0 matrix: codes [rows][cols] int8 -> f16, scales
// [rows][cols/32] f16 -> f32 transposed to [cols/32][rows].
__global__ void q8x_prefill_copy_kernel(const int8_t *__restrict__ q, const uint16_t *__restrict__ s, int rows,
                                        int cols, _Float16 *__restrict__ codes, float *__restrict__ scales) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;  // one 32-element block each
  const int nb = cols / 32;
  if (i >= int64_t(rows) * nb) return;
  const int n = int(i / nb), kb = int(i % nb);
  const int8_t *src = q + int64_t(n) * cols + kb * 32;
  _Float16 *dst = codes + int64_t(n) * cols + kb * 32;
#pragma unroll
  for (int e = 0; e < 32; ++e) dst[e] = _Float16(float(src[e]));
  scales[int64_t(kb) * rows + n] = float(__builtin_bit_cast(_Float16, s[i]));
}

}  // namespace q8x
}  // namespace lg
