// Exact prefill GEMM for large batches (gfx950): C = A . W^T with A given as f16 hi/lo planes
// and W read from its prefill copy (DevMatrix::pc, pcl, pcs), written once at upload so that
// every operand byte reaches LDS by LDS-DMA (buffer_load ... lds, 16 bytes a lane) with no
// register staging and no conversion.  Three weight forms (MODE):
//   WQ8: Q8_0 -- codes as f16 (exact) [N][K] and block scales as f32 [K/32][N].  Per 16 x 16
//        output block and Q8_0 block the partial sum is a chain of two MFMAs (A hi, then A lo,
//        against the codes), then acc += d * partial in f32.
//   W1 : F16 weights [N][K] (the weights themselves, no copy): per 32-deep k chunk
//        acc += A_hi . W, then acc += A_lo . W.
//   W2 : Q6_K (and Q4_K without the two-pass copy) -- the dequantised f32 weight split into f16 hi
//        and lo planes [N][K]: per 32-deep k chunk acc += A_hi . W_hi, A_lo . W_hi, A_hi . W_lo.
//   WQ4: Q4_K in the two-pass form w = A q - B (A = d*sc, B = dmin*m per 32-element sub-block):
//        first the correction acc = (sum_c ks[m][c] (-B[n][c] 2^e_n)) 2^-e_n over the activation's
//        chunk sums (KqCorr; W2's order and stage layout, depth K/32 rounded up to 128), then WQ8's
//        loop over the codes (exact in f16) with A as the per-chunk scale.
// Each mode keeps the per-element operation order of the 128 x 128 tiles in gemm_tiles.h, so
// both give the same bits (all on v_mfma_f32_16x16x32_f16 with f32 accumulation: one
// instruction per 32-deep chunk).
//
// Geometry: 512 threads = 8 wave64s (2 per SIMD), workgroup tile 256 x 256, K steps of 32.
// WQ8 and W1 keep three LDS stages, W2 two (its stage holds four planes).  Wave w owns rows
// 64 (w / 2) .. + 64 and columns 128 (w % 2) .. + 128 of the tile (4 x 8 MFMA blocks of
// 16 x 16).  The two wave groups of a workgroup (waves 0-3 and 4-7) run half a step apart
// (ping-pong, below), one barrier per half step.
//
// LDS rows are 64 bytes (four 16-byte chunks); logical chunk c of row r sits in slot
// c ^ ((r >> 2) & 3), so the 16 lanes of each quarter of an operand read (16 rows, one chunk)
// fall in 16 distinct 16-byte bank groups.  The DMA side writes whole 1 KiB blocks: lane L of a
// block fetches the global chunk that belongs in its slot.
#pragma once
#include <hip/hip_runtime.h>

#include "act.h"
#include "common.h"
#include "f16split.h"
#include "kernels.h"

namespace lg {
namespace wide {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum Mode { WQ8 = 0, W1 = 1, W2 = 2, WQ4 = 3 };
// epilogue of the fused q|k|v projection (RoPE, q planes, KV cache stores; RopeKvOut)
constexpr int kEpiRopeKv = 16;
// epilogue of the encoder's q|k|v projection: f32 rows as Epi::F32 stores them, q and k rotated
// (head_dim 64; RopeKvOut's cosT, sinT, tok_pos and hq)
constexpr int kEpiLayaRope = 17;

constexpr int BM = 256, BN = 256, BK = 32, WAVES = 8, THREADS = 64 * WAVES;
constexpr int ROWB = BK * 2;      // bytes per LDS row of one plane
constexpr int PLANE = BM * ROWB;  // 16 KiB
static_assert(BM == BN, "A and B planes share one slot layout");
static_assert(PLANE / 1024 == 2 * WAVES, "two 1 KiB blocks of each plane per wave");

// Q4_K correction operands of one two-pass launch (WQ4): the activation's chunk sums and the weight's
// -B 2^e planes, f16 hi and lo [rows][kp] each, and 2^-e per weight row (DevMatrix::pcl, pcr).
struct KqCorr {
  const _Float16 *ks = nullptr, *kslo = nullptr;
  const _Float16 *bh = nullptr, *bl = nullptr;
  const float *rs = nullptr;
  int kp = 0;
};

template <int MODE>
struct Geo {
  static constexpr int kBPlanes = MODE == W2 ? 2 : 1;
  static constexpr bool kScales = MODE == WQ8 || MODE == WQ4;
  static constexpr int kAHi = 0, kALo = PLANE, kBHi = 2 * PLANE, kBLo = 3 * PLANE;
  static constexpr int kScl = (2 + kBPlanes) * PLANE;
  static constexpr int kStageBytes = kScl + (kScales ? BN * 4 : 0);
  static constexpr int kStages = MODE == W2 ? 2 : 3;
  static constexpr int kLdsBytes = kStages * kStageBytes;  // WQ8, WQ4 150,528; W1 147,456; W2 131,072
};

__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }

#define WIDE_MFMA(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

__device__ __forceinline__ float silu_f(float g) { return g * (1.0f / (1.0f + __expf(-g))); }

// EPI: Epi values (F32, ADD, SWIGLU, GEGLU), kEpiRopeKv or kEpiLayaRope.  For SWIGLU and GEGLU the workgroup's 256 weight
// rows are 128 gate rows and the 128 matching up rows: wave column wn holds gate rows in its column blocks
// 0-3 and the up rows of the same output columns in blocks 4-7.
template <int EPI, int MODE>
__global__ __launch_bounds__(THREADS, 1) void gemm_wide_kernel(
    const _Float16 *__restrict__ A, const _Float16 *__restrict__ Alo, int M, int K,
    const _Float16 *__restrict__ Wh, const _Float16 *__restrict__ Wl, const float *__restrict__ Ws, int N,
    float *__restrict__ C, _Float16 *__restrict__ C16, _Float16 *__restrict__ C16lo, int ldc,
    const float *__restrict__ bias, int MT, int NT, int ffn, RopeKvOut ro, KqCorr kq) {
  using G = Geo<MODE>;
  constexpr bool kScaled = G::kScales;  // WQ8, WQ4: per-chunk scale FMAs over code partial sums
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr bool kGlu = EPI == int(Epi::SWIGLU) || EPI == int(Epi::GEGLU);
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
#ifndef LG_WIDE_GROUP_M
#define LG_WIDE_GROUP_M 4
#endif
    constexpr int GM = LG_WIDE_GROUP_M;
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

  // DMA.  Rows past M sit past the end of the A buffers: the buffer unit answers them with zeros.
  const uint32_t abytes = uint32_t(M) * uint32_t(K) * 2u, wbytes = uint32_t(N) * uint32_t(K) * 2u;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(A), 0, abytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(Alo), 0, abytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(Wh), 0, wbytes, kBufferFlags);
  __amdgpu_buffer_rsrc_t rc = rb, rs = rb;
  if constexpr (MODE == W2) rc = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(Wl), 0, wbytes, kBufferFlags);
  if constexpr (kScaled)
    rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(Ws), 0, uint32_t(N) * uint32_t(K / 32) * 4u, kBufferFlags);
  // WQ8 and W1: every wave moves the blocks wave and wave + 8 of each plane (A hi, A lo, W hi);
  // wave 0 also moves the scale block.  W2: the four waves of group 1 move everything, wave
  // 4 + b the blocks b, b + 4, b + 8, b + 12 of each of the four planes.  Block b + q holds the
  // rows of block b shifted by 16 q, which for A and for every weight row map (wrow) is a
  // wave-uniform byte offset: the buffer instruction's scalar offset.
  constexpr int BSTEP = MODE == W2 ? 4 : 8;  // block stride of a wave's blocks
  const int grp = wave >> 2, wb = MODE == W2 ? (wave & 3) : wave;
  uint32_t aoff, boff;
  {
    const int slot = wb * 64 + lane;  // 16-byte slot inside a plane (block wb)
    const int row = slot >> 2, c = (slot & 3) ^ swz(row);
    aoff = uint32_t(m0 + row) * uint32_t(K) * 2u + uint32_t(c) * 16u;
    boff = uint32_t(wrow(row)) * uint32_t(K) * 2u + uint32_t(c) * 16u;
  }
  const uint32_t soff = uint32_t(wrow(4 * lane)) * 4u;  // four consecutive weight rows' scales
  const int nk = K / BK;
#if defined(__HIP_DEVICE_COMPILE__)
  typedef __attribute__((address_space(3))) void *lds_ptr;
#endif
  // one DMA instruction of step kt into stage st: plane pl (0 A hi, 1 A lo, 2 W hi, 3 W lo) of
  // block wb + BSTEP h
  auto dma = [&](int kt, int st, int pl, int h) {
#if defined(__HIP_DEVICE_COMPILE__)
    // device pass only: with a run-time voffset this builtin keeps the host pass from
    // emitting the kernel's launch stub (the host never runs kernel bodies)
    uint8_t *base = lds + st * G::kStageBytes;
    const int blk = (wb + BSTEP * h) * 1024, dr = 16 * BSTEP * h;  // block, row shift
    const uint32_t ka = uint32_t(kt * BK * 2) + uint32_t(dr) * uint32_t(K) * 2u;
    const uint32_t kb = uint32_t(kt * BK * 2) + uint32_t(wrow(dr) - wrow(0)) * uint32_t(K) * 2u;
    if (pl == 0) __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr)(base + G::kAHi + blk), 16, aoff, ka, 0, 0);
    if (pl == 1) __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, (lds_ptr)(base + G::kALo + blk), 16, aoff, ka, 0, 0);
    if (pl == 2) __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr)(base + G::kBHi + blk), 16, boff, kb, 0, 0);
    if (pl == 3) __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (lds_ptr)(base + G::kBLo + blk), 16, boff, kb, 0, 0);
#endif
  };
  auto dma_scale = [&](int kt, int st) {
#if defined(__HIP_DEVICE_COMPILE__)
    if constexpr (kScaled)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(lds + st * G::kStageBytes + G::kScl), 16, soff,
                                               kt * N * 4, 0, 0);
#endif
  };
  constexpr int NPL = 2 + G::kBPlanes;  // planes per stage
  constexpr int NBW = 16 / BSTEP;          // blocks per plane of a moving wave
  // this wave's part of step kt: NBW * NPL instructions (wave 0: + the scale block)
  auto issue = [&](int kt, int st) {
#pragma unroll
    for (int h = 0; h < NBW; ++h)
#pragma unroll
      for (int pl = 0; pl < NPL; ++pl) dma(kt, st, pl, h);
    if (wave == 0) dma_scale(kt, st);
  };

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;

  // operand reads: lane l takes row (l % 16) of each 16-row block and chunk l / 16 of its 64-byte
  // row; every block starts at a multiple of 16 rows, so the slot swizzle depends on the lane only
  const int lr = lane & 15;
  const int ach = ((lane >> 4) ^ swz(lr)) * 16;
  const int ac0 = (wm * 64 + lr) * ROWB + ach, bc0 = (wn * 128 + lr) * ROWB + ach;
  const f32x4 zero = {};
  // one step's operands, read from LDS stage k % S by read_step and consumed by compute_step
  struct Frag {
    half8 ah[4], al[4], b[8], c[8];
    float d[8];
  };
  auto read_step = [&](int k, Frag &f) {
    const uint8_t *st = lds + (k % G::kStages) * G::kStageBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f.ah[i] = *reinterpret_cast<const half8 *>(st + G::kAHi + ac0 + i * 16 * ROWB);
      f.al[i] = *reinterpret_cast<const half8 *>(st + G::kALo + ac0 + i * 16 * ROWB);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f.b[j] = *reinterpret_cast<const half8 *>(st + G::kBHi + bc0 + j * 16 * ROWB);
      if constexpr (MODE == W2) f.c[j] = *reinterpret_cast<const half8 *>(st + G::kBLo + bc0 + j * 16 * ROWB);
    }
    if constexpr (kScaled) {
#pragma unroll
      for (int j = 0; j < 8; ++j) f.d[j] = *reinterpret_cast<const float *>(st + G::kScl + (wn * 128 + j * 16 + lr) * 4);
    }
    // the reads have returned: the barrier after this phase frees the stage for the DMA
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };
  // dkt >= 0: the six A/W DMA instructions of this wave's part of step dkt (into stage dst) issue
  // one per column block j = 1 .. 6, between the MFMAs
  auto compute_step = [&](const Frag &f, int dkt, int dst) {
    if constexpr (kScaled) {
      // software pipeline over the wave's eight column blocks j: the eight MFMAs of column j (the
      // hi then lo chains of its four row blocks, interleaved) issue between the sixteen scale
      // FMAs of column j - 1 (two sets of four partial sums)
      f32x4 p[2][4];
#pragma unroll
      for (int j = 0; j <= 8; ++j) {
        if (j < 8) {
#pragma unroll
          for (int i = 0; i < 4; ++i) p[j & 1][i] = WIDE_MFMA(f.ah[i], f.b[j], zero);
#pragma unroll
          for (int i = 0; i < 4; ++i) p[j & 1][i] = WIDE_MFMA(f.al[i], f.b[j], p[j & 1][i]);
        }
        if (j > 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j - 1][r] += f.d[j - 1] * p[(j - 1) & 1][i][r];
        }
        const bool dm = dkt >= 0 && j >= 1 && j <= 6;
        if (dm) dma(dkt, dst, (j - 1) % 3, (j - 1) / 3);
        if (j == 0) {
          __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // column 0's MFMAs
        } else if (j < 8) {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA of column j
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two FMAs of column j - 1
            if (dm && q == 3) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one DMA
          }
        } else {
          __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);  // column 7's FMAs
        }
      }
    } else if constexpr (MODE == W1) {
      // per element: A_hi.W, then A_lo.W; column by column, the four row blocks' chains interleaved
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = WIDE_MFMA(f.ah[i], f.b[j], acc[i][j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = WIDE_MFMA(f.al[i], f.b[j], acc[i][j]);
        const bool dm = dkt >= 0 && j >= 1 && j <= 6;
        if (dm) {
          dma(dkt, dst, (j - 1) % 3, (j - 1) / 3);
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        }
      }
    } else {
      // per element: A_hi.W_hi, A_lo.W_hi, A_hi.W_lo; column by column, the four row blocks'
      // chains interleaved; dkt >= 0 (group 1): its sixteen DMA instructions, two per column
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = WIDE_MFMA(f.ah[i], f.b[j], acc[i][j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = WIDE_MFMA(f.al[i], f.b[j], acc[i][j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = WIDE_MFMA(f.ah[i], f.c[j], acc[i][j]);
        if (dkt >= 0) {
          dma(dkt, dst, (2 * j) % 4, (2 * j) / 4);
          dma(dkt, dst, (2 * j + 1) % 4, (2 * j + 1) / 4);
          __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
      }
    }
  };
  // a bare barrier (no fence): the DMA in flight stays in flight across it; no instruction is
  // scheduled across it, so a phase's MFMAs and FMAs stay in that phase
  auto barrier = [] {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Ping-pong (WQ8, W1): the two wave groups (waves 0-3 and 4-7, one of each per SIMD) alternate
  // between reading a step's operands from LDS into registers (read_step) and computing on them
  // (compute_step), half a step apart: in phase 2k group 0 reads step k while group 1 computes
  // step k - 1, in phase 2k + 1 group 0 computes step k while group 1 reads it, one barrier after
  // each phase.  So every SIMD always has one wave issuing MFMAs while the other waits on LDS, and
  // the reading wave runs at the higher issue priority, so its LDS reads overlap the MFMAs.
  // DMA, interleaved with the MFMAs of the compute phases so that no phase waits on the buffer
  // unit: group 0 moves its part of step k + 2 while computing step k (phase 2k + 1), group 1 its
  // part of step k + 3 while computing step k (phase 2k + 2); wave 0 moves the scales of step
  // k + 2 when it starts reading step k (phase 2k).  Each of those stages last held a step both
  // groups have finished reading (k - 1 and k), and a read phase ends when its LDS reads have
  // returned, so the barrier after it also frees the stage.  Every wave ends each phase waiting
  // for all but its last six DMA instructions: that completes group 0's part of step k + 1 by the
  // end of phase 2k + 1 and group 1's by the end of phase 2k + 1 (its read of step k), before
  // group 0 reads step k + 1 in phase 2k + 2.  Steps past the last are fetched too (the buffer
  // unit answers reads past the end with zeros and nothing reads those stages), so every wait has
  // the same count and no branch separates the MFMAs from the DMA.  Both groups run the same loop
  // and pass 2 nk + 2 barriers.
  if constexpr (MODE == WQ4) {
    // The correction of the two-pass Q4_K form, before the main loop: acc = (sum_c ks[m][c]
    // (-B[n][c] 2^e_n)) 2^-e_n over kq.kp sub-block columns, in W2's per-element order and stage
    // layout (four planes, two stages).  Every wave moves blocks wave and wave + 8 of each plane, one
    // step ahead of the reads.
    using GC = Geo<W2>;
    static_assert(GC::kStages * GC::kStageBytes <= G::kLdsBytes, "the correction's stages fit the LDS");
    const int kp = kq.kp;
    const uint32_t ksb = uint32_t(M) * uint32_t(kp) * 2u, kbb = uint32_t(N) * uint32_t(kp) * 2u;
    const __amdgpu_buffer_rsrc_t r0 = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(kq.ks), 0, ksb, kBufferFlags);
    const __amdgpu_buffer_rsrc_t r1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(kq.kslo), 0, ksb, kBufferFlags);
    const __amdgpu_buffer_rsrc_t r2 = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(kq.bh), 0, kbb, kBufferFlags);
    const __amdgpu_buffer_rsrc_t r3 = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(kq.bl), 0, kbb, kBufferFlags);
    uint32_t kao, kbo;
    {
      const int slot = wave * 64 + lane, row = slot >> 2, c = (slot & 3) ^ swz(row);
      kao = uint32_t(m0 + row) * uint32_t(kp) * 2u + uint32_t(c) * 16u;
      kbo = uint32_t(wrow(row)) * uint32_t(kp) * 2u + uint32_t(c) * 16u;
    }
    auto cdma = [&](int kt, int st) {
#if defined(__HIP_DEVICE_COMPILE__)
      uint8_t *base = lds + st * GC::kStageBytes;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int blk = (wave + 8 * h) * 1024, dr = 128 * h;  // block, row shift
        const uint32_t ka = uint32_t(kt * BK * 2) + uint32_t(dr) * uint32_t(kp) * 2u;
        const uint32_t kb = uint32_t(kt * BK * 2) + uint32_t(wrow(dr) - wrow(0)) * uint32_t(kp) * 2u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r0, (lds_ptr)(base + GC::kAHi + blk), 16, kao, ka, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r1, (lds_ptr)(base + GC::kALo + blk), 16, kao, ka, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r2, (lds_ptr)(base + GC::kBHi + blk), 16, kbo, kb, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r3, (lds_ptr)(base + GC::kBLo + blk), 16, kbo, kb, 0, 0);
      }
#endif
    };
    const int nkc = kp / BK;
    cdma(0, 0);
    for (int kt = 0; kt < nkc; ++kt) {
      if (kt + 1 < nkc) {  // step kt + 1 into the other stage, which every wave finished reading
        cdma(kt + 1, (kt + 1) & 1);
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      barrier();
      const uint8_t *st = lds + (kt & 1) * GC::kStageBytes;
      half8 ah[4], al[4], b[8], c[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ah[i] = *reinterpret_cast<const half8 *>(st + GC::kAHi + ac0 + i * 16 * ROWB);
        al[i] = *reinterpret_cast<const half8 *>(st + GC::kALo + ac0 + i * 16 * ROWB);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        b[j] = *reinterpret_cast<const half8 *>(st + GC::kBHi + bc0 + j * 16 * ROWB);
        c[j] = *reinterpret_cast<const half8 *>(st + GC::kBLo + bc0 + j * 16 * ROWB);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = WIDE_MFMA(ah[i], b[j], acc[i][j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = WIDE_MFMA(al[i], b[j], acc[i][j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = WIDE_MFMA(ah[i], c[j], acc[i][j]);
      }
      barrier();  // the stage is free for step kt + 2
    }
    float rsc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) rsc[j] = kq.rs[wrow(wn * 128 + j * 16 + lr)];
    // the scale loads land before the main loop's DMA, whose waits count only its own instructions
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] *= rsc[j];
  }

  constexpr int S = G::kStages;
  if constexpr (MODE != W2) {
    static_assert(S == 3 && NPL == 3, "ping-pong: three stages of three planes");
    // prologue: both groups' parts of steps 0 and 1, group 1's part of step 2
    issue(0, 0);
    issue(1, 1);
    if (grp == 1) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) dma(2, 2, pl, h);
      asm volatile("s_waitcnt vmcnt(12)" ::: "memory");  // step 0
    } else if (kScaled && wave == 0) {
      asm volatile("s_waitcnt vmcnt(7)" ::: "memory");  // step 0 and its scales
    } else {
      asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    }
    barrier();
    if (grp == 1) barrier();  // group 1 runs half a step behind
    for (int k = 0; k < nk; ++k) {
      Frag f;
      __builtin_amdgcn_s_setprio(2);
      if (wave == 0) dma_scale(k + 2, (k + 2) % S);
      read_step(k, f);
      asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
      barrier();
      __builtin_amdgcn_s_setprio(0);
      compute_step(f, k + 2 + grp, (k + 2 + grp) % S);
      asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
      barrier();
    }
    if (grp == 0) barrier();
  } else {
    // W2, two stages of four planes: the same ping-pong, group 1 moving every block.  In phase
    // 2k + 2 it moves step k + 2 (into the stage step k held, which both groups finished reading
    // by phase 2k + 1) between the MFMAs of its compute phase of step k; it waits for that step at
    // the end of its read phase of step k + 1 (phase 2k + 3), before group 0 reads it in 2k + 4.
    if (grp == 1) {
      issue(0, 0);
      issue(1, 1);
      asm volatile("s_waitcnt vmcnt(16)" ::: "memory");  // step 0
    }
    barrier();
    if (grp == 1) barrier();
    for (int k = 0; k < nk; ++k) {
      Frag f;
      __builtin_amdgcn_s_setprio(2);
      read_step(k, f);
      if (grp == 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // step k + 1
      barrier();
      __builtin_amdgcn_s_setprio(0);
      compute_step(f, grp == 1 ? k + 2 : -1, k % S);  // one call: two would spill
      barrier();
    }
    if (grp == 0) barrier();
  }

  // epilogue: acc[i][j] register r -> row 16 i + 4 (lane / 16) + r, column 16 j + lane % 16 of the
  // wave tile
  if constexpr (kGlu) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (row >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int col = nt * (BN / 2) + wn * 64 + j * 16 + lr;
          const float g = acc[i][j][r];
          const float v = (EPI == int(Epi::SWIGLU) ? silu_f(g) : gelu_tanh(g)) * acc[i][j + 4][r];
          _Float16 h, hl;
          split_f16(v, h, hl);
          C16[int64_t(row) * ldc + col] = h;
          if (C16lo) C16lo[int64_t(row) * ldc + col] = hl;
        }
      }
    }
  } else if constexpr (EPI == kEpiRopeKv) {
    // the wave's 128 columns are one head: q (rotated, scaled, hi/lo planes [M][hq * 128]), k
    // (rotated, K page rows) or v (V page columns); each value is the f32 acc (+ bias) the F32
    // epilogue would store, rotated by rope_pair and split by split_f16 as the RoPE kernel does
    const int head = (ro.col0 + nt * BN + wn * 128) >> 7;
    const int part = head < ro.hq ? 0 : head < ro.hq + ro.hkv ? 1 : 2;  // q, k, v
    const int PT = ro.page_tokens, plane = PT * 128;
    const int kvp = ro.kv_planes;  // pool planes: 2 (hi, lo) or 1 (f16, the hi value)
    float bv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) bv[j] = bias ? bias[nt * BN + wn * 128 + j * 16 + lr] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rb = m0 + wm * 64 + i * 16 + (lane >> 4) * 4;  // this lane's four rows rb .. rb + 3
      int pos[4], page[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = min(rb + r, M - 1);
        pos[r] = ro.tok_pos[row];
        page[r] = ro.tok_page[row];
      }
      float v[8][4];
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[j][r] = acc[i][j][r];
          if (bias) v[j][r] += bv[j];
        }
      if (part < 2) {
        // rotate-half pairs (d, d + 64): column blocks j and j + 4 of the same lane
        float cs[4][4][4];  // [r][j][cos d, sin d, cos d + 64, sin d + 64]
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t tb = int64_t(pos[r]) * 128 + j * 16 + lr;
            cs[r][j][0] = ro.cosT[tb];
            cs[r][j][1] = ro.sinT[tb];
            cs[r][j][2] = ro.cosT[tb + 64];
            cs[r][j][3] = ro.sinT[tb + 64];
          }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb + r;
          if (row >= M) continue;
          _Float16 *dh, *dl;
          if (part == 0) {
            dh = ro.q16 + int64_t(row) * (ro.hq * 128) + head * 128;
            dl = ro.q16lo + int64_t(row) * (ro.hq * 128) + head * 128;
          } else {
            const int64_t blk = int64_t(page[r]) * ro.page_stride + int64_t(head - ro.hq) * plane;
            dh = ro.kpool + kvp * blk + (pos[r] % PT) * 128;
            dl = dh + plane;
          }
          const bool lo = part == 0 || kvp == 2;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float a, c;
            rope_pair(v[j][r], v[j + 4][r], cs[r][j][0], cs[r][j][1], cs[r][j][2], cs[r][j][3], a, c);
            if (part == 0) {
              a *= ro.qscale;
              c *= ro.qscale;
            }
            _Float16 h, l;
            split_f16(a, h, l);
            dh[j * 16 + lr] = h;
            if (lo) dl[j * 16 + lr] = l;
            split_f16(c, h, l);
            dh[j * 16 + lr + 64] = h;
            if (lo) dl[j * 16 + lr + 64] = l;
          }
        }
      } else {
        // V page columns [128][PT]: the four rows are four consecutive slots of a column when they
        // are consecutive positions of one page starting at a multiple of 4 (one 8-byte store a
        // plane), else one slot at a time
        bool quad = rb + 3 < M && (pos[0] & 3) == 0;
#pragma unroll
        for (int r = 1; r < 4; ++r) quad = quad && pos[r] == pos[0] + r && page[r] == page[0];
        typedef _Float16 half4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int d = j * 16 + lr;
          half4 h4, l4;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            _Float16 h, l;
            split_f16(v[j][r], h, l);
            h4[r] = h;
            l4[r] = l;
          }
          if (quad) {
            const int64_t blk = int64_t(page[0]) * ro.page_stride + int64_t(head - ro.hq - ro.hkv) * plane;
            _Float16 *dh = ro.vpool + kvp * blk + int64_t(d) * PT + (pos[0] % PT);
            *reinterpret_cast<half4 *>(dh) = h4;
            if (kvp == 2) *reinterpret_cast<half4 *>(dh + plane) = l4;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (rb + r >= M) continue;
              const int64_t blk = int64_t(page[r]) * ro.page_stride + int64_t(head - ro.hq - ro.hkv) * plane;
              _Float16 *dh = ro.vpool + kvp * blk + int64_t(d) * PT + (pos[r] % PT);
              dh[0] = h4[r];
              if (kvp == 2) dh[plane] = l4[r];
            }
          }
        }
      }
    }
  } else if constexpr (EPI == kEpiLayaRope) {
    // the wave's 128 columns are two 64-dim heads of q, k or v (the q width hq * 64 is a multiple of
    // 128); q and k pairs (d, d + 32) are column blocks j and j + 2 of the same lane, rotated by
    // rope_pair from the row's position as the encoder's RoPE kernel rotates the F32 epilogue's values
    const int cw = nt * BN + wn * 128;
    const bool rot = cw < 2 * ro.hq * 64;
    float bv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) bv[j] = bias ? bias[cw + j * 16 + lr] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (row >= M) continue;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          v[j] = acc[i][j][r];
          if (bias) v[j] += bv[j];
        }
        if (rot) {
          const int64_t tb = int64_t(ro.tok_pos[row]) * 64;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (j & 2) continue;  // blocks 0, 1, 4, 5 hold dims d < 32 of their head
            const int64_t e = tb + (j & 1) * 16 + lr;
            float a, c;
            rope_pair(v[j], v[j + 2], ro.cosT[e], ro.sinT[e], ro.cosT[e + 32], ro.sinT[e + 32], a, c);
            v[j] = a;
            v[j + 2] = c;
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) C[int64_t(row) * ldc + cw + j * 16 + lr] = v[j];
      }
    }
  } else {
    float bv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) bv[j] = bias ? bias[nt * BN + wn * 128 + j * 16 + lr] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // the residual add reads a 16-row block's 32 values per lane in one round trip (rows past M
      // read row M - 1 and are not stored), then adds and stores
      float cv[4][8];
      if constexpr (EPI == int(Epi::ADD)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = min(m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r, M - 1);
#pragma unroll
          for (int j = 0; j < 8; ++j) cv[r][j] = C[int64_t(row) * ldc + nt * BN + wn * 128 + j * 16 + lr];
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (row >= M) continue;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int col = nt * BN + wn * 128 + j * 16 + lr;
          float v = acc[i][j][r];
          if (bias) v += bv[j];
          if constexpr (EPI == int(Epi::F32)) C[int64_t(row) * ldc + col] = v;
          else C[int64_t(row) * ldc + col] = cv[r][j] + v;
        }
      }
    }
  }
}
#undef WIDE_MFMA

}  // namespace wide
}  // namespace lg
