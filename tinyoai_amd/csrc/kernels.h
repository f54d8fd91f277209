// Launch interfaces of the gfx950 kernels. Host code (the model handles and
// the C ABI) calls only these; each returns hipSuccess or the launch error.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>

#include "formats.h"

// Kernel timing for the stage profiler. While `start` is set, the decode
// kernels launch through hipExtLaunchKernelGGL with `start` and `stop`,
// which the dispatch records when the kernel begins and ends (events
// recorded around a launch also count the launch gap), and set `used`.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
  bool used = false;
};
LaunchTiming &launch_timing();  // the calling thread's

#define TINYOAI_TIMED_LAUNCH(KERNEL, GRID, BLOCK, LDS, STREAM, ...)                                        \
  do {                                                                                                       \
    LaunchTiming &lt_ = launch_timing();                                                                     \
    if (lt_.start) {                                                                                         \
      hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, LDS, STREAM, lt_.start, lt_.stop, 0, __VA_ARGS__);         \
      lt_.used = true;                                                                                       \
    } else {                                                                                                 \
      hipLaunchKernelGGL(KERNEL, GRID, BLOCK, LDS, STREAM, __VA_ARGS__);                                     \
    }                                                                                                        \
  } while (0)

// Per-layer weights of a StableLM block (stablelm.go:113-117), fused:
//   win  rows [q | k | v | gate/up], cols = hidden. Inside each q and k head
//        the rotary pair (j, j + rot/2) sits on adjacent rows 2j, 2j + 1,
//        followed by the non-rotary dims in order; gate row i and up row i
//        sit on rows 2i and 2i + 1 of the MLP section. Every consumer reads
//        row pairs (2u, 2u + 1).
//   wout rows = hidden, cols [o (hidden) | down (intermediate)]: the o and
//        down rows of one output feature, back to back.
struct LayerDev {
  MatDesc win, wout;
  const float *ln_w, *ln_b;
  // A layer whose attention and MLP matrices differ in storage format (as
  // in GGUF K-quant mixes) keeps them as sections of their own: then win
  // holds only [q | k | v] and win2 the gate/up pairs; wout holds only o
  // and wout2 down. rows == 0 when the layer is fused.
  MatDesc win2, wout2;
};

// Shapes and constants of a decoder layer, with the choices that tell
// StableLM (stablelm.go) and the legacy Llama (model.go) apart.
struct StableDims {
  int d, hd, rot, heads, kv_heads, inter, vocab;
  double eps;
  float att_scale;  // float32(sqrt(hd)), attentionScale (stablelm.go:431), model.go:433
  int norm;          // 0: LayerNorm (stablelm.go:288-305); 1: RMSNorm (model.go:591-600)
  int rope_adjacent; // rotary pairs: 0 (j, j + rot/2) (stablelm.go:309-326); 1 (2j, 2j+1) (model.go:611-618)
  int silu;          // 0: (g / (1 + e)) * u (stablelm.go:371-373); 1: (g * (1 / (1 + e))) * u (model.go:463-470)
  int win_q, win_kv; // rows of the q section and of each of the k, v sections of win
};

// KV cache of one layer: [kv_heads][cap][hd], fp32 or fp16 bits.
struct KVDev {
  void *k, *v;
  int cap;
  int half;  // 1 = fp16 storage (floatHalf rounding), 0 = fp32
};

// Where the rows of an uploaded tensor land in a fused matrix.
enum : int { ROWMAP_IDENTITY = 0, ROWMAP_HEADS = 1, ROWMAP_INTERLEAVE = 2 };
struct RowMap {
  int kind;
  int64_t offset;   // first destination row
  int hd, rot;      // ROWMAP_HEADS
  int phase;        // ROWMAP_INTERLEAVE: 0 -> rows 2i, 1 -> rows 2i + 1
};

// ---- decode (one token) ----
// Matvec launches take their grid and block size (256 or 512 threads) from
// the caller; blocks stream their share of the rows.
//
// LayerNorm(x) -> win rows with RoPE, KV append and SiLU-gate fused into
// the epilogue. pos (and token) are read from device memory; `rope` is the
// token's row of the rotary table (rot floats: cos, sin per pair), so no
// load waits for pos before the weights stream. With `emb` (a host-side
// descriptor, copied), x is first set to the embedding row of *token
// (layer 0).
hipError_t launch_decode_in(const LayerDev &w, const StableDims &s, const KVDev &kv, float *x, const MatDesc *emb,
                            const int *token, const float *rope, const int *pos, float *q_out, float *m_out,
                            int grid, int threads, hipStream_t st);
// decode_in and the layer's split-K decode attention (launch_attention's
// arguments: steps, splits, partials, counters, out) in one launch: extra
// blocks wait until every streaming wave has stored its q/k/v rows, then
// run the attention while the gate/up rows stream. fuse_ctr holds the
// layer's 1 + 16 counter lines and then one go-flag line per head (32
// words each, zero before the first launch), epoch the device int of
// launches completed on them, err the word a timed-out wait sets. Supported: Q8_0 and BF16 win
// matrices whose rows fit one column slice, head widths 64, 80 and 128,
// 256-thread blocks, steps 1 or 2.
constexpr int kFuseGroups = 16;  // group counters of the fused launch's arrival tree
bool decode_in_att_supported(const LayerDev &w, const StableDims &s, int threads, int steps);
hipError_t launch_decode_in_att(const LayerDev &w, const StableDims &s, const KVDev &kv, float *x, const MatDesc *emb,
                                const int *token, const float *rope, const int *pos, float *q_out, float *m_out,
                                int grid, int steps, int splits, float *partials, unsigned *counters, float *att_out,
                                unsigned *fuse_ctr, const int *epoch, unsigned *err, hipStream_t st);
// x = (x + o * a) + down * m (stablelm.go:365-377), one wout row per wave:
// a row holds ka values of o then, from the next chunk boundary, km values
// of down (km = 0: x = x + o * a).
hipError_t launch_decode_out(const MatDesc &wout, int ka, int km, const float *a, const float *m, float *x,
                             int grid, int threads, hipStream_t st);
// Split-K flash decode with in-kernel combine for nq queries at positions
// pos0 + j (j < nq): q [nq][heads*hd] -> out [nq][heads*hd]. A block covers
// 64 * steps positions; `splits` blocks per (query, head) must cover
// max_pos + 1 positions (<= 0: derived from max_pos). partials holds
// nq * heads * partial_region(splits, hd) floats; counters (nq * heads)
// start at 0 and are left at 0.
hipError_t launch_attention(const StableDims &s, const KVDev &kv, const float *q, const int *pos0, int nq,
                            int max_pos, float *partials, unsigned *counters, float *out, hipStream_t st,
                            int steps = 0, int splits = 0);
// Branch attention: query j sits at position rows[2j] and its own K/V at
// slot rows[2j + 1] of the branch cache sfx; positions below `prefix` come
// from kv (the shared prefix), position t >= prefix from slot rows[2j + 1]
// - rows[2j] + t of sfx (the branch's suffix, stored contiguously). Every
// query's position is at most max_pos. partials holds nq * heads *
// partial_region(max_splits, hd) floats. Head widths 8, 64, 80 and 128.
// With a prefix, at most 128 queries and a matrix-core head width, the
// prefix is attended once for all queries (launch_shared_prefix_attention)
// and the suffix splits continue from its records. max_splits must be at
// least branch_attention_records(s, prefix, max_pos, nq).
hipError_t launch_branch_attention(const StableDims &s, const KVDev &kv, const KVDev &sfx, int prefix,
                                   const float *q, const int *rows, int nq, int max_pos, float *partials,
                                   unsigned *counters, float *out, int max_splits, hipStream_t st);
int branch_attention_records(const StableDims &s, int prefix, int max_pos, int nq);
// The launch shape launch_branch_attention takes at these arguments (its
// grid and positions per block), as one integer.
int branch_attention_shape(const StableDims &s, int prefix, int max_pos, int nq);
// The shared-prefix pass on the matrix cores: nq <= 128 queries q
// [nq][heads*hd], every one past `prefix`, against cache positions
// [0, prefix) of kv, in blocks of 256 positions; block x writes the record
// {m, l, o[hd]} (natural-log max, unnormalised sums) of (query j, head h)
// at partials + (j * heads + h) * region + x * (hd + 2).
int shared_prefix_splits(int prefix);
hipError_t launch_shared_prefix_attention(const StableDims &s, const KVDev &kv, int prefix, const float *q, int nq,
                                          float *partials, int64_t region, hipStream_t st);
// Causal attention of n prefill queries on the matrix cores (head widths
// 64, 80, 96, 128): q [n][heads*hd] at positions pos0 + j -> out.
bool flash_prefill_supported(int hd);
// out (fp32, may be null) and / or the bf16 operand planes oh, ol of the
// matrix-core GEMM (null: none). With sfx, the queries are one branch's
// rows: cache positions t >= prefix come from slot sfx_slot0 + (t - prefix)
// of the branch cache sfx, positions below prefix from kv. The planes' query
// rows lie ld_o values apart (0: heads * hd). With segs (and sfx), nseg
// runs of branch rows in one launch: segs[3k..3k+2] = (first row, rows,
// slot of its first position) on the device, n = the longest run, q, pos0
// (row pairs) and out indexed by row.
// Without sfx, when the query tiles leave CUs idle and the last query's
// position (last_pos, known to the host) reaches 256, each tile's keys are
// split over several blocks whose records (in `work`, at most work_floats)
// a second kernel combines in order (null work: no splits).
hipError_t launch_flash_prefill(const StableDims &s, const KVDev &kv, const float *q, const int *pos0, int n,
                                float *out, hipStream_t st, uint16_t *oh = nullptr, uint16_t *ol = nullptr,
                                const KVDev *sfx = nullptr, int prefix = 0, int sfx_slot0 = 0, int64_t ld_o = 0,
                                const int *segs = nullptr, int nseg = 0, float *work = nullptr,
                                int64_t work_floats = 0, int last_pos = 0);
int attention_steps(int max_pos, int heads);
// The decode step's attention shape at position pos: attention_steps up to
// about 1800 positions (fused into the decode_in launch), then wider
// separate blocks (4 steps; 16 beyond about 5000 positions for head widths
// up to 80).
int decode_attention_steps(int pos, int heads, int hd);
// Floats per (query, head) in the partials buffer: max_splits records of
// hd + 2, rounded to 256 bytes.
__host__ __device__ inline int64_t partial_region(int max_splits, int hd) {
  return ((int64_t)max_splits * (hd + 2) + 63) / 64 * 64;
}

// The operand planes of the matrix-core GEMM for one value: bf16 hi (round
// to nearest even) and lo = bf16(v - hi), as launch_split_bf16 forms them.
// The empty asm keeps v one fp32 value for both conversions.
__device__ __forceinline__ void store_bf16_split(uint16_t *hi, uint16_t *lo, int64_t i, float v) {
  asm volatile("" : "+v"(v));
  const __bf16 h = (__bf16)v;
  hi[i] = __builtin_bit_cast(uint16_t, h);
  lo[i] = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)h));
}
int attention_splits(int max_pos, int steps);
// out[rows] = W * norm(x) (skipped when ln_w is null; norm as StableDims),
// for the logits head and single-matrix products.
hipError_t launch_ln_matvec(const MatDesc &w, const float *ln_w, const float *ln_b, double eps, int norm,
                            const float *x, float *out, int grid, int threads, hipStream_t st);
// x[n][cols] = rows ids[j] of an embedding matrix, bit-exact dequantized.
hipError_t launch_embed(const MatDesc &emb, const int *ids, int n, float *x, hipStream_t st);


// ---- prefill (n tokens) ----
// out (fp32, may be null) and / or bf16 operand planes oh, ol (null: none)
// with rows ldo values apart (0: d).
hipError_t launch_layer_norm_rows(const float *x, const float *w, const float *b, double eps, int n, int d,
                                  float *out, hipStream_t st, uint16_t *oh = nullptr, uint16_t *ol = nullptr,
                                  int ldo = 0);
// out[n][rows] = x[n][cols] * W^T on the vector units (any format/shape).
hipError_t launch_gemm(const MatDesc &w, const float *x, int n, float *out, hipStream_t st);
// The matrix-core product: y[M][N] (row stride ldy) = X * W^T with X given
// as bf16 planes [M][K] (xl null: one plane). Q8_0 and BF16 weights with
// K % 32 == 0. With ksplit > 1 the K range is cut in ksplit parts whose
// products go to y + s * M * ldy (s < ksplit), for the caller to sum;
// gemm_splits: the split count that fills the device for this shape (at
// most max_splits).
bool gemm_mfma_supported(const MatDesc &w);
int gemm_planes(const MatDesc &w, bool bf16_path = false);
int gemm_splits(const MatDesc &w, int M, int max_splits);
hipError_t launch_gemm_mfma(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int M, float *y, int ldy,
                            hipStream_t st, int ksplit = 1);
// Few-row products with a 5/6-bit matrix (Q4_K, Q5_K, Q6_K, Q5_1) on the
// matrix cores: y[M][N] (row stride ldy) = X * W^T, X fp32 [M][ldx]
// (16-byte aligned, ldx % 4 == 0), converted first into `stage` (16-byte
// aligned device memory of kq_rows_stage_bytes(K, M) bytes); more than 32
// rows run as slices of 32 on the grid's second dimension. With
// ks > 1 the K range is cut in ks parts whose products go to
// y + s * split_stride (0: M * ldy; a larger stride lets row slices of one
// product share the caller's split layout), for the caller to sum;
// kq_rows_splits: the split count that fills the device for this matrix
// (at most max_splits). With staged, `stage` already holds this X (a
// previous call's, same M and K).
bool kq_rows_supported(const MatDesc &w, int M);
size_t kq_rows_stage_bytes(int K, int M);
int kq_rows_splits(const MatDesc &w, int max_splits);
hipError_t launch_kq_rows(const MatDesc &w, const float *x, int ldx, int M, float *y, int ldy, int ks, void *stage,
                          hipStream_t st, bool staged = false, int64_t split_stride = 0);
// Two few-row products of the same M rows (each from its own staged X, as
// launch_kq_rows(..., staged) reads it) in one launch, each block running
// its own product's format, with the results of two launch_kq_rows calls
// with the same split counts. Formats: Q4_K and Q6_K, in either order.
struct KqProduct {
  MatDesc w;
  const void *stage;     // staged X of this product
  float *y;
  int ldy, ks;
  int64_t split_stride;  // 0: M * ldy
};
bool kq_rows_pair_supported(int fmt1, int fmt2);
// Stages two inputs of the same M <= 32 rows (K1, K2 % 32 == 0, rows ldx
// apart, 16-byte aligned) for launch_kq_rows(..., staged) in one launch,
// as two unstaged launch_kq_rows calls would (no LayerNorm).
hipError_t launch_kq_stage_pair(const float *x1, int ldx1, int K1, void *stage1, const float *x2, int ldx2, int K2,
                                void *stage2, int M, hipStream_t st);
hipError_t launch_kq_rows_pair(const KqProduct &a, const KqProduct &b, int M, hipStream_t st);
// Stages M <= 32 rows of x (K % 256 == 0) for launch_kq_rows(..., staged)
// with the LayerNorm (weights lw, bias lb, eps) applied on the way.
hipError_t launch_kq_stage_norm(const float *x, int ldx, int M, int K, const float *lw, const float *lb, double eps,
                                void *stage, hipStream_t st);
// The fused in-projection epilogue of a matrix-core win product for M
// tokens at positions *pos0 + j: RoPE'd q [M][heads*hd], K/V into the
// cache, and the SiLU-gate outputs as bf16 planes mh, ml [M][inter] (and
// fp32 m [M][inter] when m is not null), as launch_in_epilogue forms them
// from y.
struct InEpilogue {
  StableDims s;
  KVDev kv;
  const float *rope;
  const int *pos0;
  float *q;
  float *m;
  uint16_t *mh, *ml;
  int ldm;  // values between rows of mh / ml (0: inter)
};
hipError_t launch_gemm_in_epilogue(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int M,
                                   const InEpilogue &e, hipStream_t st);
// Wide-tile matrix-core products (one wave per SIMD, both operands loaded
// straight into LDS): y = X * W^T for BF16 weights with K % 32 == 0 (X as
// bf16 planes xh and xl, or xh alone for one plane), or Q8_0 weights that
// wide_q8_ok accepts (two planes, mf 1), with rows lda values apart. A launch carries one or two products of M rows each (their
// blocks side by side, the first product's first); product i cuts its K
// range in ksplit parts whose results go to y + s * split_stride. Block
// tiles are (128 * mf) x (32 * nf): gemm_wide_shape names the instances
// built.
struct WideGemm {
  MatDesc w;
  const uint16_t *xh, *xl;
  int lda;
  float *y;
  int ldy;
  int ksplit;
  int64_t split_stride;
};
bool gemm_wide_shape(int fmt, int mf, int nf);
// A Q8_0 matrix (or column view) the wide tiles take: K a multiple of 32,
// each row's fp16 block scales starting on a dword (the kernel loads them
// two blocks at a time) and its quants on 16 bytes.
inline bool wide_q8_ok(const MatDesc &w) {
  return w.fmt == FMT_Q8_0 && w.cols % 32 == 0 && w.vstride % 16 == 0 && w.mstride % 4 == 0 &&
         (reinterpret_cast<uintptr_t>(w.meta) & 3) == 0 && (reinterpret_cast<uintptr_t>(w.vals) & 15) == 0;
}
hipError_t launch_gemm_wide(const WideGemm *p, int nprod, int M, int mf, int nf, hipStream_t st);
// The in-projection (win) product with its epilogue fused (no output
// matrix), on wide tiles.
hipError_t launch_gemm_wide_in_epilogue(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int lda, int M,
                                        const InEpilogue &e, int mf, int nf, hipStream_t st);
// x fp32 [rows][k] (row stride ldx) -> bf16 hi [rows][k] and lo = x - hi.
hipError_t launch_split_bf16(const float *x, int ldx, int k, int64_t rows, uint16_t *hi, uint16_t *lo,
                             hipStream_t st);
// Epilogue of the fused in-projection for n tokens: y [n][win rows] ->
// RoPE'd q [n][heads*hd], K/V into the cache at positions pos0 + j, and
// m [n][inter] = SiLU-gate(gate, up) (m may be null), and / or m as bf16
// operand planes mh, ml (null: none; rows ldm values apart, 0: inter).
// With rows, token j sits at position rows[2j] and its K/V go to cache
// slot rows[2j + 1] (branch rows). y may hold ys partial products n * ldy
// floats apart, summed in order.
hipError_t launch_in_epilogue(const StableDims &s, const KVDev &kv, const float *y, int ldy, const float *rope,
                              const int *pos0, int n, float *q, float *m, hipStream_t st, uint16_t *mh = nullptr,
                              uint16_t *ml = nullptr, const int *rows = nullptr, int ys = 1, int ldm = 0);
// Two such epilogues of the same n branch rows (rows as above) in one
// launch, each with its own dims (sa: q/k/v, sb: gate/up), products y
// (ys partials n * ldy floats apart) and fp32 m, with the results of two
// launch_in_epilogue calls.
hipError_t launch_in_epilogue_pair(const StableDims &sa, const float *ya, int ldya, int ysa, const StableDims &sb,
                                   const float *yb, int ldyb, int ysb, const KVDev &kv, const float *rope,
                                   const int *rows, int n, float *q, float *m, hipStream_t st);
// x = (x + p) + d elementwise (stablelm.go:375-377).
// x = (x + sum_s p[s]) + sum_s d[s] over sp and sd partial products n
// floats apart (K-split GEMM outputs), summed in order.
hipError_t launch_residual(float *x, const float *p, int sp, const float *d, int sd, int64_t n, hipStream_t st);
// launch_residual over n rows of d values, then the LayerNorm of the new
// rows (launch_layer_norm_rows' arithmetic, weights w, bias b) into out
// and / or the bf16 planes oh, ol, in one pass over x: the same bits as
// the two launches.
hipError_t launch_residual_norm_rows(float *x, const float *p, int sp, const float *dd, int sd, int n, int d,
                                     const float *w, const float *b, double eps, float *out, uint16_t *oh,
                                     uint16_t *ol, hipStream_t st);
// out[i] = sum over s < sp of p[s * n + i], in order of s.
hipError_t launch_sum_splits(float *out, const float *p, int sp, int64_t n, hipStream_t st);
hipError_t launch_copy_row(const float *src, float *dst, int n, hipStream_t st);
// n 32-bit words from src to dst (both 16-byte aligned; either may be
// host-mapped memory), with 16-byte accesses.
hipError_t launch_copy_words(const void *src, void *dst, int n, hipStream_t st);

// Log probabilities of `rows` rows of logits (row stride ld floats, vocab
// entries each), normalised over the whole row in float64: chosen[r] for
// targets[r], and the count largest entries of each row as top_ids[r][k] /
// top_lp[r][k], descending with ties to the lower id (summarizeLogits,
// logprobs.go:60-95). 1 <= count <= vocab. `scratch` (16-byte aligned
// device memory of logprob_scratch_bytes(count) bytes) starts with the
// error word, which the caller zeroes first: a row holding NaN leaves its
// row + 1 there (the largest such) and no results for that row.
size_t logprob_scratch_bytes(int count);
hipError_t launch_logprobs(const float *logits, int64_t ld, int rows, int vocab, const int *targets, int count,
                           double *chosen, int *top_ids, double *top_lp, void *scratch, hipStream_t st);

// ---- the stories260K-shaped Llama, every token of a call in one launch ----
constexpr int kTinyDim = 64, kTinyHidden = 172, kTinyMaxLayers = 8, kTinyMaxSeq = 512, kTinyMaxVocab = 512,
              kTinyMaxTokens = 256;
// Packed fp32 weights, per layer: [wq | wk | wv] (128 x 64), wo (64 x 64),
// w1/w3 interleaved (344 x 64), w2 (64 x 172), rows unpadded; the buffer
// ends with kTinyPad spare bytes (reads of a row's last chunks may run past
// a matrix, never past the buffer). The K/V cache is one buffer too: per
// layer K [kv_heads][cap][8], then V the same, then kTinyPad bytes.
constexpr int64_t kTinyQkvOff = 0, kTinyWoOff = 128 * 64 * 4, kTinyW13Off = kTinyWoOff + 64 * 64 * 4,
                  kTinyW2Off = kTinyW13Off + 344 * 64 * 4, kTinyLayerBytes = kTinyW2Off + 64 * 172 * 4,
                  kTinyPad = 1024;
struct TinyLlamaArgs {
  const uint8_t *w;                  // packed weights, layers * kTinyLayerBytes + kTinyPad bytes
  const uint8_t *emb;                // [vocab][dim] fp32, also the classifier
  float *kv;                         // the K/V buffer
  const float *rms_att, *rms_ffn, *rms_final;  // [layers][dim], [layers][dim], [dim]
  const float *rope;                 // [cap][8]: (cos, sin) of pairs 0..3
  float att_scale;                   // float32(sqrt(8))
  int layers, vocab, cap, prefix, n;
  int all, last;                     // rows written: every token's (all) or the last token's (last)
  float *out;                        // [n or 1][vocab]
  unsigned *done;                    // set to `seq` (system scope) after the rows, when non-null
  unsigned seq;
  int tokens[kTinyMaxTokens];
};
bool tiny_llama_supported(int dim, int hidden, int heads, int kv_heads, int layers, int vocab, int seq);
hipError_t launch_tiny_llama(const TinyLlamaArgs &a, hipStream_t st);

// ---- weights ----
// Places raw GGUF-encoded bytes (already in device memory) of a
// [rows][cols] tensor into `dst` under `map`, starting at column col0.
hipError_t launch_repack(int fmt, const uint8_t *raw, int64_t rows, int64_t cols, const MatDesc &dst,
                         const RowMap &map, int64_t col0, hipStream_t st);
// Copies `rows` rows of row_bytes from src (contiguous) into dst (stride
// dst_stride) at byte col0b of the mapped row: placement of one plane.
hipError_t launch_place_bytes(const uint8_t *src, int64_t rows, int64_t row_bytes, uint8_t *dst, int64_t dst_stride,
                              int64_t col0b, const RowMap &map, hipStream_t st);
hipError_t launch_read_values(const MatDesc &m, int64_t offset, int64_t n, float *out, hipStream_t st);

int device_cu_count();
