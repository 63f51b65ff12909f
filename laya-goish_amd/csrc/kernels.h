// Host-side launchers of the gfx950 kernels.  Every launcher checks the shapes its kernel
// and grid assume before launching, and throws lg::Error(LG_ERR_INVALID/UNSUPPORTED)
// instead of launching anything out of bounds.
#pragma once
#include <hip/hip_runtime.h>

#include <hip/hip_ext.h>

#include <cmath>
#include <cstdint>

#include "lg.h"

namespace lg {

// Kernel timing: while a KernelTimer is installed on the calling thread, the GEMV and GEMM
// launchers start their (single) kernel with hipExtLaunchKernelGGL, which records `start` and
// `stop` when that kernel itself starts and ends, so the interval excludes dispatch gaps.
struct KernelTimer {
  hipEvent_t start = nullptr, stop = nullptr;
};
KernelTimer *&kernel_timer();

// hipLaunchKernelGGL, or its timed form when a KernelTimer is installed.
template <typename F, typename... Args>
inline void launch_timed(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
  if (KernelTimer *t = kernel_timer())
    hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(lds), st, t->start, t->stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
}

// Raise `kernel`'s dynamic LDS limit on the current device to `lds` bytes (no-op up to 64 KiB); done
// once per (device, kernel, size), thread-safe.
void grant_lds(const void *kernel, size_t lds);

// Repacked device layout of one weight matrix W[rows][cols] (y = x . W^T).
//   F32 : q = float[rows][cols]
//   F16 : q = half[rows][cols]
//   Q8_0: q = int8[rows][cols] (codes), s = half[rows][cols/32] (block scale d)
//   Q4_K: q = uint8[rows][cols/2]; each 64-element group is 32 bytes whose byte j holds
//         element j (low nibble) and j+32 (high nibble), as inside a GGUF Q4_K block;
//         s = float2[rows][cols/32] = (d*sc, dmin*m) per 32-element sub-block
//   Q6_K: q = int8[rows][cols] holding (code - 32); s = float[rows][cols/16] = d*sc
// Dequantised weight (bit-identical to src/gguf.rs:264-332):
//   Q8_0: half(d) * q     Q4_K: (d*sc)*q - (dmin*m)     Q6_K: (d*sc)*(q-32)
struct DevMatrix {
  uint32_t kind = 0;
  int rows = 0, cols = 0;
  void *q = nullptr;
  void *s = nullptr;
  // Prefill copy (exact-mode decoder matrices, set once at upload; null otherwise), the operand
  // form the large-batch GEMM (gemm_wide.h) moves to LDS by DMA with no conversion on the way:
  //   Q8_0 : pc = codes as f16 [rows][cols], pcs = block scales as f32 [cols/32][rows]
  //   F16  : pc = q (the weights themselves; no copy)
  //   Q4_K : the two-pass form of w = A q - B (A = d*sc, B = dmin*m per 32-element sub-block):
  //          pc = codes q as f16 [rows][cols], pcs = A as f32 [cols/32][rows] (the Q8_0 form), and
  //          the correction sum_c B[n][c] * ksum[m][c] as a GEMM of depth pkp = ksum_cols(cols):
  //          pcl = -B[n][c] * 2^e_n split into f16 hi [rows][pkp] then lo [rows][pkp] (zero past
  //          cols/32), pcr = 2^-e_n [rows], e_n putting the row's largest |B| in [2^13, 2^14)
  //   Q6_K : pc / pcl = f16 hi / lo planes [rows][cols] of the dequantised f32 weight
  _Float16 *pc = nullptr;
  _Float16 *pcl = nullptr;
  float *pcs = nullptr;
  float *pcr = nullptr;
  int pkp = 0;
  int64_t bytes() const;  // HBM bytes of q + s
  int64_t gguf_bytes() const;  // bytes of the same matrix in GGUF blocks
};

enum class Epi : int {
  F32 = 0,     // C[m][n]  = acc (+ bias[n])
  ADD = 1,     // C[m][n] += acc (+ bias[n]) (residual stream update)
  F16 = 2,     // C16[m][n] = half(acc (+ bias[n]))
  SWIGLU = 3,  // C16[m][j] = half(silu(acc_gate) * acc_up), W rows [0,f) gate, [f,2f) up
  GEGLU = 4,   // as SWIGLU with the tanh GELU of src/tensor.rs:129-131 (prefill GEMM only)
  RELU16 = 5,  // C16[m][n] = half(max(acc + bias[n], 0)) (prefill GEMM only)
};

// Standalone dequant of raw GGUF blocks (device pointers), bit-exact with gguf::decode.
void launch_dequant(uint32_t kind, const uint8_t *src, uint64_t nblocks, float *dst,
                    hipStream_t st);

// Repack raw GGUF blocks (device) of a [rows][cols] matrix into the DevMatrix layout.
void launch_repack(uint32_t kind, const uint8_t *src, int rows, int cols, DevMatrix &w,
                   hipStream_t st);

// Prefill copy (DevMatrix::pc, pcl, pcs) of a repacked Q8_0 / Q4_K / Q6_K matrix: device bytes
// it needs (0 for kinds that need none), and the conversion from w.q / w.s into the buffers
// w.pc, w.pcl, w.pcs already point at.  The K-quant planes split the weight exactly as the
// exact-mode GEMM tiles do (gemm_tiles.h), so both GEMMs see the same operand bits.
size_t prefill_copy_bytes(uint32_t kind, int rows, int cols);
void launch_prefill_copy(const DevMatrix &w, hipStream_t st);

// Depth of the Q4_K correction GEMM: one column per 32-element sub-block, rounded up to 128.
inline int ksum_cols(int cols) { return (cols / 32 + 127) / 128 * 128; }
// Chunk sums of an activation given as f16 hi/lo planes [M][K]: ks[m][c] = sum over the 32 elements
// k of chunk c of (hi + lo), left to right in f32, split into f16 hi [M][kp] then lo [M][kp] planes
// (zero for c >= K/32).  The Q4_K correction GEMM's activation operand.
void launch_chunk_sums(const _Float16 *A, const _Float16 *Alo, int M, int K, int kp, _Float16 *ks, hipStream_t st);

// Prefill GEMM: out = A[M][K] (half, row-major, lda = K) . W^T with epilogue `epi`.
// A_lo == nullptr: one f16 pass.  A_lo != nullptr: A = A + A_lo (hi/lo f16 planes) and the
// weights are applied exactly (split-precision MFMA, f32-faithful).  f16 outputs (Epi::F16,
// Epi::SWIGLU) are written as hi/lo planes when C16_lo != nullptr.
// For Epi::SWIGLU the output has W.rows/2 columns.
// ks: the chunk sums of A (launch_chunk_sums, hi plane then lo plane of M x W.pkp), required by an
// exact Q4_K launch whose matrix has the two-pass prefill copy (W.pcr), ignored otherwise.
void launch_gemm(const _Float16 *A, const _Float16 *A_lo, int M, const DevMatrix &W, Epi epi, float *C,
                 _Float16 *C16, _Float16 *C16_lo, int ldc, const float *bias, hipStream_t st,
                 const _Float16 *ks = nullptr);
// True when an exact launch of W needs the chunk sums of its activation (Q4_K, two-pass copy).
inline bool needs_ksum(const DevMatrix &W) { return W.kind == LG_Q4_K && W.pcr != nullptr; }

// Generic f32 GEMM for shapes the tiled kernel does not take (any M, N, K), F32/F16/Q weights.
void launch_gemm_generic(const float *X, int M, const DevMatrix &W, const float *bias, float *Y,
                         hipStream_t st);

// Decode GEMV over f32 x[K] (M = 1): y[n] = x . W[n] with epilogue (F32/ADD/SWIGLU-f32).
// For Epi::SWIGLU, y has W.rows/2 entries (f32).  `x` may be fused with an RMSNorm:
// when norm_w != nullptr the kernel computes h = x * rsqrt(mean(x^2)+eps) * norm_w first.
void launch_gemv(const float *x, const DevMatrix &W, Epi epi, float *y, const float *bias,
                 const float *norm_w, float eps, hipStream_t st);

// Row RMSNorm: y = x * (1/sqrt(dot(x,x)/d + eps)) * w   (src/models/openthai/model.rs:84-94)
// written as f16 (y) or as hi/lo f16 planes (y, y_lo) when y_lo != nullptr.
void launch_rmsnorm_f16(const float *x, int rows, int d, const float *w, float eps, _Float16 *y,
                        _Float16 *y_lo, hipStream_t st);
void launch_rmsnorm_f32(const float *x, int rows, int d, const float *w, float eps, float *y,
                        hipStream_t st);

// Launch-floor probe: `launches` dependent launches of a plain read kernel, each over its own zero-filled
// slice of `bytes` (~2 GiB of slices in all: HBM reads), on a stream of its own (current device); returns
// the average microseconds per launch.
double probe_read_chain(size_t bytes, int launches);

// Embedding rows (F16 or F32 table [vocab][d]) -> f32 x[T][d].
void launch_embed(const void *table, uint32_t kind, const int32_t *ids, int T, int d, int vocab,
                  float *x, hipStream_t st);

// KV page geometry shared by the attention and rope kernels.
struct KvGeom {
  int page_tokens = 64;  // tokens per page
  int hkv = 0, hd = 0;
  int split = 0;             // value format of the pools: 0 = f16, 1 = f16 hi plane + f16 lo plane
  int64_t layer_stride = 0;  // values between layers of the K (or V) pool
  int64_t page_stride = 0;   // values per page of one layer: hkv * page_tokens * hd
};
// Pool layout of one layer: [page][kv head][plane][...] where a plane is K rows [page_tokens][hd]
// or V columns [hd][page_tokens] of f16; a split pool has two planes per (page, kv head), hi
// then lo (hi = f16(v), lo = f16(v - hi)), an f16 pool one.

// The factor launch_rope_kv_tiles (and the fused q|k|v epilogue) folds into q: log2(e) / sqrt(hd),
// so that the attention kernels work on base-2 logits.
inline float attn_q_scale(int hd) { return 1.4426950408889634f / std::sqrt(float(hd)); }

// Outputs of the q|k|v projection's fused epilogue (launch_gemm_wide_rope): the f32 result
// (+ bias) is rotated and stored exactly as launch_rope_kv_tiles stores it from the f32 rows.
// head_dim 128; the launch's output columns are heads col0 / 128 .. of the q|k|v layout (q heads,
// then k heads, then v heads).
struct RopeKvOut {
  const float *cosT = nullptr, *sinT = nullptr;          // [ctx][128]
  const int32_t *tok_pos = nullptr, *tok_page = nullptr;  // per activation row: position, its page
  _Float16 *q16 = nullptr, *q16lo = nullptr;              // [M][hq * 128] hi / lo planes
  _Float16 *kpool = nullptr, *vpool = nullptr;            // the layer's pools
  int64_t page_stride = 0;                                // as KvGeom::page_stride
  int hq = 0, hkv = 0, hd = 128, page_tokens = 64, col0 = 0;  // hd: must be 128
  float qscale = 1.0f;                                    // attn_q_scale(128)
  int kv_planes = 2;                                      // 2: hi/lo pool planes; 1: f16 pools
};

// The 256 x 256 exact GEMM (gemm_wide.h) of a q|k|v projection, or a column range of it, with the
// RoPE and KV cache stores of launch_rope_kv_tiles as its epilogue: q to f16 hi/lo planes
// (scaled), k and v into the pools (hi/lo planes, or f16 when ro.kv_planes is 1) at each row's
// position and page.  Returns false (nothing
// launched) when the wide kernel does not take the launch (gemm_wide_takes) or the layout is not
// one the epilogue covers (head_dim 128, col0 a multiple of 128).
bool launch_gemm_wide_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                           const RopeKvOut &ro, hipStream_t st, const _Float16 *ks = nullptr);
// Whether the 256 x 256 exact GEMM takes an M-row launch of W with epilogue epi (shape, prefill
// copy and tile count; pointers are checked at launch).
bool gemm_wide_takes(int M, const DevMatrix &W, Epi epi);
// The encoder's q|k|v projection (W rows: q, k, v of `heads` 64-dim heads, an even count) on the
// 256 x 256 exact GEMM, its epilogue storing the f32 rows [M][ldc] with q and k rotated: the same bits
// as the F32 GEMM followed by launch_laya_rope.  Only for launches gemm_wide_takes(M, W, Epi::F32)
// accepts; anything else fails.  cosT, sinT: [ctx][64]; tok_pos: per row.
void launch_gemm_wide_laya_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                                const float *cosT, const float *sinT, const int32_t *tok_pos, int heads, float *C,
                                int ldc, hipStream_t st, const _Float16 *ks = nullptr);
// Short launches (fewer than 128 tiles of 64 x 64) of an F16 or Q8_0 q|k|v projection in the exact
// split mode: the 32-row tile GEMM with the same rotating epilogue as launch_gemm_wide_rope (head_dim
// 64 or 128, ro.col0 a multiple of it), the same bits as the F32 GEMM followed by the RoPE kernel.
// gemm_small_rope_takes tells whether launch_gemm_small_rope launches (it returns false otherwise).
bool gemm_small_rope_takes(int M, const DevMatrix &W, int hd);
bool launch_gemm_small_rope(const _Float16 *A, const _Float16 *Alo, int M, const DevMatrix &W, const float *bias,
                            const RopeKvOut &ro, hipStream_t st);

// RoPE on q and k of q|k|v rows ((hq+2hkv)*hd f32) with tables cos/sin[ctx][hd], q written
// out, k and v written into the K page rows [hkv][page_tokens][hd] and V page columns
// [hkv][hd][page_tokens] of the layer pools (value format per g.split).
// This form: a prefill batch, one workgroup per attention tile (<= 32 consecutive tokens
// of one sequence, rows row0.., positions pos0..); q goes to f16 planes, multiplied by
// log2(e) / sqrt(hd) (the scaled base-2 logit form launch_attn_prefill expects).  head_dim <= 128.
void launch_rope_kv_tiles(const float *qkv, int hq, const KvGeom &g, const float *cosT,
                          const float *sinT, const int32_t *pages, int max_pages,
                          const int32_t *tile_seq, const int32_t *tile_row0, const int32_t *tile_pos0,
                          const int32_t *tile_n, int ntiles, _Float16 *q16, _Float16 *q16_lo,
                          void *kpool, void *vpool, hipStream_t st);

// Causal prefill attention over the paged cache, queries as launch_rope_kv_tiles leaves them
// (pre-scaled by log2(e) / sqrt(hd)).  Work items: tiles of 32 query rows of one
// sequence (tile_seq, tile_row0 = first batch row, tile_pos0 = its position, tile_n rows).
// q16_lo != nullptr selects the split-precision path, over the split cache (g.split) or an f16
// one; the output is then written as hi/lo planes (out16, out16_lo).  f16 queries need the f16
// cache.  Tiles go in groups (grp_first[i],
// grp_count[i] for i < ngroups) of at most group_tiles = attn_prefill_group_tiles(hq, hkv, max_len)
// consecutive tiles of one sequence (max_len: the longest sequence of the batch, its own tokens
// included); each group's workgroups share every K/V page through LDS.  head_dim 64 or 128.
// A query's output does not depend on which group or batch its tile is in.
int attn_prefill_group_tiles(int hq, int hkv, int max_len);
void launch_attn_prefill(const _Float16 *q16, const _Float16 *q16_lo, int T, int hq,
                         const KvGeom &g, const void *kpool, const void *vpool,
                         const int32_t *pages, int max_pages, const int32_t *tile_seq,
                         const int32_t *tile_row0, const int32_t *tile_pos0,
                         const int32_t *tile_n, int ntiles, const int32_t *grp_first,
                         const int32_t *grp_count, int ngroups, int group_tiles, _Float16 *out16,
                         _Float16 *out16_lo, hipStream_t st);

// Decode attention for one new token at position pos of one sequence: q|k|v row `qkv` (before
// RoPE); RoPE of q and k (tables cos/sin[ctx][hd]) and the k/v write into the cache slot are
// fused in.  Split over the pages 0..pos/64 into `part` (attn_decode_scratch_floats(hq, hd,
// max_pages) floats, max_pages = the length of the page table), then combined per query head by
// a second launch into out[hq * hd].
void launch_attn_decode(const float *qkv, int hq, const KvGeom &g, const float *cosT, const float *sinT,
                        int pos, void *kpool, void *vpool, const int32_t *pages, int max_pages,
                        float *part, float *out, hipStream_t st);
int64_t attn_decode_scratch_floats(int hq, int hd, int max_pages);

// Gather rows, final RMSNorm and the option head: logits[r][j] = h_r . W[ids[j]] (+ bias[ids[j]]).
void launch_head_rows(const float *x, const int32_t *rows, int R, int d, const float *norm_w,
                      float eps, const DevMatrix &W, const float *bias, const int32_t *vocab_ids, int nv,
                      float *logits, hipStream_t st);

// Option scoring over logits[R][k]: probabilities and log-softmax at temperature t.
void launch_option_scores(const float *logits, int R, int k, float temperature, float *probs,
                          float *logprobs, hipStream_t st);

// Full-vocabulary argmax of logits[V] (first maximum wins) -> out[0], or -1 when the maximum is not
// finite (inf or no comparable value).  One launch of one workgroup; part_v / part_i (64 entries each,
// reserved by the decode workspaces) are not used by it.
void launch_argmax(const float *logits, int V, int32_t *out, float *part_v, int32_t *part_i,
                   hipStream_t st);
// launch_argmax, then the chosen token's embedding row (table[V][d], F16 or F32, the vocabulary of the
// logits) into x[d] by the same workgroup: the next decode step's input without its own launch.
void launch_argmax_embed(const float *logits, int V, int32_t *out, const void *table, uint32_t kind, int d, float *x,
                         hipStream_t st);

// f32 -> f16 (round to nearest even), n elements; with y_lo, also the residual plane
// y_lo = f16(x - y).
void launch_cvt_f16(const float *x, int64_t n, _Float16 *y, _Float16 *y_lo, hipStream_t st);

// f32 weights from the repacked layout of W, row-major [rows][cols] (bit-exact dequant).
void launch_dequant_repacked(const DevMatrix &w, float *dst, hipStream_t st);

// ---- OpenThai-SystemOne mixers (k_openthai.hip), src/models/openthai/model.rs:244-362 ----
// Gated DeltaNet, per token: causal conv (kernel 4) + silu over the q|k|v columns of the
// projection row [q|k|v (3*nh*128) | z (nh*128) | a (nh) | b (nh) | pad] (ldp floats), then
// qk[T][nh][query 128 | key 128] (L2-normalised; query also / sqrt(128)), vbuf[T][nh*128],
// gb[T][nh][log-decay, beta].  tok_pos = index of each row in its sequence.
void launch_ot_delta_prep(const float *proj, int ldp, int T, const int32_t *tok_pos, const float *conv,
                          const float *alog, const float *dt, int nh, float *qk, float *vbuf, float *gb,
                          hipStream_t st);
// The recurrent scan over each sequence (rows seq_row0[s] .. + seq_n[s] of T, the longest max_n tokens):
// out[nh][8][T][16] (head, block of 16 value columns, row), in chunks of 32 tokens (two launches: the
// chunks' local terms in parallel, then the state carried from chunk to chunk).  chunk_ws holds
// ot_delta_chunk_floats(T, nseq, nh) floats.
size_t ot_delta_chunk_floats(int T, int nseq, int nh);
void launch_ot_delta_scan(const float *qk, const float *vbuf, const float *gb, const int32_t *seq_row0,
                          const int32_t *seq_n, int nseq, int T, int max_n, int nh, float *chunk_ws, float *out,
                          hipStream_t st);
// rms(out head, norm_w) * silu(z) with z at column zcol of the projection row -> f16 planes; out in the
// scan's layout.
void launch_ot_delta_out(const float *o, int T, int nh, const float *norm_w, const float *proj, int ldp, int zcol,
                         _Float16 *y, _Float16 *ylo, hipStream_t st);
// Full attention: per-head q/k rms (weights 1 + w) + partial RoPE (tables [pos][32]) from the
// projection row [(q 256 | gate 256) x hq | k 256 x hkv | v 256 x hkv] into Qb[T][hq][256],
// Kb[T][hkv][256]; then causal GQA over 32-token tiles (tile_*: first row, position, count)
// with the output * sigmoid(gate) -> f16 planes [T][hq*256].
void launch_ot_attn_prep(const float *proj, int ldp, int T, int hq, int hkv, const int32_t *tok_pos,
                         const float *qn1, const float *kn1, const float *cosT, const float *sinT, float *Qb,
                         float *Kb, hipStream_t st);
void launch_ot_attn(const float *Qb, const float *Kb, const float *proj, int ldp, int hq, int hkv,
                    const int32_t *tile_row0, const int32_t *tile_pos0, const int32_t *tile_n, int ntiles,
                    _Float16 *y, _Float16 *ylo, hipStream_t st);
// The same attention on f32 MFMA, split over keys: work items (first row, position, rows <= 16,
// key range [klo, khi) of <= 256 keys) write partials (ot_attn_part_floats(nitems, hq) floats),
// then each 16-row tile (cb_*: first row, rows, first item, items) is merged into the planes.
// Needs (hq / hkv) % 4 == 0.
int64_t ot_attn_part_floats(int nitems, int hq);
void launch_ot_attn_mfma(const float *Qb, const float *Kb, const float *proj, int ldp, int hq, int hkv,
                         const int32_t *it_row0, const int32_t *it_pos0, const int32_t *it_nq, const int32_t *it_klo,
                         const int32_t *it_khi, int nitems, const int32_t *cb_row0, const int32_t *cb_nq,
                         const int32_t *cb_first, const int32_t *cb_n, int ncomb, float *part, _Float16 *y,
                         _Float16 *ylo, hipStream_t st);

// ---- Laya encoder (k_laya.hip), src/models/laya/model.rs:301-416, src/tensor.rs:103-192 ----
// LayerNorm of rows (rows[r] of x when rows != nullptr), w/b optional, + add[sel[seq[r]]] when
// add != nullptr, into f16 planes (y16, y16lo) or f32 (y32).  d % 4 == 0, d <= 4096.
void launch_layer_norm(const float *x, const int32_t *rows, int nrows, int d, const float *w, const float *b, float eps,
                       const float *add, const int32_t *seq, const int32_t *sel, _Float16 *y16, _Float16 *y16lo,
                       float *y32, hipStream_t st);
// Bidirectional attention over q|k|v rows [T][3d] (head dim 64), keys |i - j| <= window
// (window < 0: all), RoPE from tables [pos][64] when cosT != nullptr; 32-token tiles (tile_*),
// tile_seq -> sequence, seq_n -> its length.  Output f16 planes [T][d].
// RoPE in place on the q and k parts of q|k|v rows [T][3d]: pairs (j, j + 32) of each head,
// tables [pos][hd], row positions tok_pos[T].
void launch_laya_rope(float *qkv, int T, int d, int hd, const float *cosT, const float *sinT, const int32_t *tok_pos,
                      hipStream_t st);
// Bidirectional attention over rotated q|k|v rows of fresh sequences in tiles of <= 32 rows;
// window < 0: all keys of the sequence.  Output f16 planes [T][d].
void launch_laya_attn(const float *qkv, int d, int hd, int window, const int32_t *tile_row0, const int32_t *tile_pos0,
                      const int32_t *tile_n, const int32_t *tile_seq, const int32_t *seq_n, int ntiles, _Float16 *y,
                      _Float16 *ylo, hipStream_t st);
void launch_gelu_inplace(float *x, int64_t n, hipStream_t st);
// pooled[s] = [h[seq_row0[s]] (d), top1, top1 - top2, entropy, max(k,2)/255] over the option
// logits logits[lg_first[s] .. + lg_count[s]] (model.rs:392-403).
void launch_laya_act_features(const float *h, int d, const int32_t *seq_row0, const int32_t *lg_first,
                              const int32_t *lg_count, const float *logits, int nseq, float *pooled, hipStream_t st);

// Device int32 fill / copy helpers (small, capture-safe).
void launch_fill_i32(int32_t *p, int n, int32_t v, hipStream_t st);

}  // namespace lg
