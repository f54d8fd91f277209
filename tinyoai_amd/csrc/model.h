// Host-side model state behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "kernels.h"
#include "tinyoai_hip.h"

namespace tinyoai {

extern thread_local std::string g_error;
int fail(int code, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);

// One weight matrix in HBM, in the plane layout of formats.h.
struct DevMatrix {
  MatDesc desc{};
  void *mem = nullptr;
  size_t bytes = 0;
  DevMatrix() = default;
  DevMatrix(const DevMatrix &) = delete;
  DevMatrix &operator=(const DevMatrix &) = delete;
  DevMatrix(DevMatrix &&o) noexcept : desc(o.desc), mem(o.mem), bytes(o.bytes) { o.mem = nullptr; }
  ~DevMatrix();
  // Zeroed planes for a [rows][cols] matrix of format dtype.
  int create(int32_t dtype, int64_t rows, int64_t cols, hipStream_t st);
  // Places a GGUF-encoded [rows][cols] tensor of the same format at column
  // col0 (a value index) under a row map; waits for the copy to finish.
  int place(int32_t dtype, int64_t rows, int64_t cols, const void *data, uint64_t nbytes, const RowMap &map,
            int64_t col0, hipStream_t st);
  // create + place of a whole matrix.
  int upload(int32_t dtype, int64_t rows, int64_t cols, const void *data, uint64_t nbytes, hipStream_t st);
};

// A column range [col0, col0 + cols) of a matrix as a matrix of its own
// (col0 on a 16-byte chunk boundary, and on a block boundary for Q8_0).
MatDesc column_view(const MatDesc &m, int64_t col0, int64_t cols);

// Stage timings with hipEvents on the model's stream, the device-side
// counterpart of stableProfile (stablelm.go:227-250). Off by default; when
// on, every kernel launch is bracketed by two events, resolved after the
// forward synchronizes.
enum Stage : int {
  ST_EMBED, ST_DECODE_IN, ST_ATTENTION, ST_DECODE_OUT, ST_LM_HEAD, ST_PREFILL_NORM, ST_PREFILL_GEMM,
  ST_PREFILL_EPILOGUE, ST_PREFILL_ATTENTION, ST_PREFILL_ELEMENTWISE, ST_COUNT
};

struct Profiler {
  bool on = false;
  std::vector<hipEvent_t> pool;
  // (stage, start event, stop event): the events recorded around the
  // launch, or those its dispatch recorded (LaunchTiming)
  struct Mark {
    int stage;
    size_t a, b;
  };
  std::vector<Mark> marks;
  size_t used = 0;
  double ms[ST_COUNT] = {};
  int64_t count[ST_COUNT] = {};
  ~Profiler();
  hipEvent_t next();
  void begin(int stage, hipStream_t st);
  void end(hipStream_t st);
  void resolve();
  void clear();
};

// A StableLM resident on one GPU with its KV cache (stableState,
// stablelm.go:216-225, kept in HBM).
struct StableModel {
  tinyoai_stablelm_config cfg{};
  StableDims dims{};
  hipStream_t stream = nullptr;
  DevMatrix embed, head;
  std::vector<DevMatrix> mats;  // win, wout, win2, wout2 of each layer
  bool mixed_layers = false;    // some layer keeps its MLP (or down) matrices as sections of their own
  std::vector<LayerDev> layers;
  const float *norm_w = nullptr, *norm_b = nullptr;
  float *rope = nullptr;
  std::vector<float> rope_host;  // [pos][rot]: a decode token's row travels with its parameters

  // KV: one [kv_heads][cap][hd] K and V buffer per layer.
  std::vector<KVDev> kv;
  int cap = 0, offset = 0, reserve = 0, kv_half = 0;
  // Open branch sessions borrowing the resident prefix: while any is open
  // the model refuses every call that would change its KV (forward, reset,
  // set_kv_bits, limit_cache) and close, as the reference's session holds
  // the model gate (branches.go:16-22).
  int open_branches = 0;
  int busy_with_branches() const;

  // decode workspaces
  float *x = nullptr, *qbuf = nullptr, *mbuf = nullptr, *abuf = nullptr, *logits_dev = nullptr;
  int *params = nullptr;
  float *partials = nullptr;
  unsigned *counters = nullptr;
  int max_splits = 0;
  static constexpr int kPrefillSplits = 8;  // K-split partial products P and D can hold
  static constexpr int kRowStreamMax = 32;  // non-matrix-core products of at most this many rows run per row
  // prefill workspaces, `chunk` tokens each: residual X, LayerNorm H, win
  // products Y, RoPE'd queries Q, SiLU-gate M, attention A, o and down
  // products P and D, bf16 planes XH/XL of the current GEMM operand
  int chunk = 0, win_rows = 0;
  // Device parameter block (ints): [0, 16) scalars, [16, 16 + chunk) token
  // ids or the decode token's rotary row, then 2 * chunk ints of per-row
  // (position, KV slot) pairs.
  int *rows_dev() const { return params + 16 + std::max(chunk, dims.rot); }
  float *X = nullptr, *H = nullptr, *Y = nullptr, *Q = nullptr, *M = nullptr, *A = nullptr, *P = nullptr,
        *D = nullptr;
  uint16_t *XH = nullptr, *XL = nullptr;
  uint16_t *MH = nullptr, *ML = nullptr;  // the SiLU-gate outputs as bf16 planes (down projection operand)
  void *h_pinned = nullptr;
  hipEvent_t params_copied = nullptr;  // last H2D copy out of h_pinned's parameter slot
  // Host-mapped pinned memory of the decode graph: logits and the error
  // word (io_words_logits() words), then the step's parameter block (16 +
  // rot words). The graph's first kernel copies the parameters in and its
  // last the logits out, so a decode step needs no copy-engine transfer.
  void *h_io = nullptr, *d_io = nullptr;
  bool logits_mapped = false;  // the last decode step left its logits in h_io
  int io_words_logits() const { return (cfg.vocab_size + 1 + 63) / 64 * 64; }
  bool tracing = false;
  float *trace_dev = nullptr, *trace_att = nullptr, *trace_gate = nullptr;  // [L][d], [L][heads*hd], [L][inter]
  int grid_in = 0, grid_out = 0, grid_head = 0;
  int threads_in = 256, threads_out = 256, threads_head = 256;
  int att_steps = 0;  // decode attention positions per block / 64; 0 = chosen by position
  // Decode: each layer's attention runs inside its decode_in launch where
  // the shapes allow (set_launch stage 4 turns it off); one counter line
  // per layer, and the launches completed on them (parameter int 2).
  bool fuse_attention = true;
  unsigned *fuse_ctr = nullptr;  // per layer: fuse_lines() lines of 32 words (counters, then a go flag per head)
  int fuse_epoch = 0;
  int fuse_lines() const { return 1 + kFuseGroups + dims.heads; }
  size_t fuse_bytes() const { return (size_t)cfg.num_hidden_layers * fuse_lines() * 128; }

  unsigned *perr = nullptr;  // the word after the logits: an in-kernel wait timed out

  std::vector<void *> buffers;
  Profiler prof;
  // Decode graphs by attention launch shape (valid for the current KV).
  std::map<int64_t, hipGraphExec_t> graphs;
  bool use_graphs = true;
  int launch_gen = 0;  // changed by every set_launch call (part of the branch step graphs' keys)

  ~StableModel();
  int init(const tinyoai_stablelm_config &c, const tinyoai_tensor *tensors, int n);
  int alloc(void **p, size_t bytes);
  void free_kv();
  int ensure_kv(int needed);
  int upload_params(const int *head_vals, int nh, const int32_t *ids, int n, const float *row = nullptr,
                    int nrow = 0, const int *rows = nullptr);
  int enqueue_decode(int steps, int splits, bool want_logits);
  void drop_graphs();
  int decode_step(int token, int pos, bool want_logits);
  int check_wait_error(int rc);
  bool decode_fused(int steps) const;
  void reset_fused();
  // y = x * W^T; with `splits`, the product may come as *splits K-split
  // partials n * ldy floats apart (y holds max_splits of them). With
  // rowstream (branch steps), a product of at most 32 rows with a 5/6-bit
  // matrix runs on the matrix cores as one few-row product, and of at most
  // kRowStreamMax rows in another format without a matrix-core path as one
  // row-streaming matvec per row; otherwise every chunk size takes the
  // same arithmetic.
  // staged (few-row 5/6-bit products): in, the workspace already holds
  // this x from the previous product of the same shape; out, it does now.
  int project(const MatDesc &w, const float *x, int ldx, int n, float *y, int ldy, int *splits = nullptr,
              bool rowstream = false, int max_splits = kPrefillSplits, bool *staged = nullptr);
  // y = X * W^T with X already in bf16 planes xh, xl (matrix-core formats).
  // BF16-weight prefill products take bf16 activations (one plane) when
  // set: the bf16 path's accuracy (2e-2 of the logit range), about 1.3x
  // the matrix-core rate; off by default, which keeps greedy streams equal
  // to the fp32 engine's where logits nearly tie.
  bool bf16_acts = false;
  const uint16_t *lo_plane(const MatDesc &w) const { return gemm_planes(w, bf16_acts) == 2 ? XL : nullptr; }
  int project_planes(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int n, float *y, int ldy,
                     int *splits = nullptr);
  // BF16-weight prefill products on the wide-tile kernel (set_launch
  // stage 7, on by default), else on the 128 x 256 tiles; wide_layer: the
  // layer's whole prefill takes the wide-tile path.
  bool use_wide = true;
  bool wide_layer(int l) const;
  // The wide-tile in-projection forms its epilogue as a kernel of its own
  // from the product's output (the default), or in the product's own
  // launch (set_launch stage 8 on: one wave per SIMD then runs the float64
  // exp chains and scattered stores while the matrix cores idle; the 8K
  // BF16 prefill takes 129 ms against 117.5).
  bool wide_epi = false;
  // Q8_0 prefill products on wide tiles (the Q8_0 ring kernel) or on the
  // 128 x 256 tiles (launch stage 10).
  bool q8_wide = true;
  bool kq_pair = true;     // a branch step's paired launches (products, stagings, epilogues)
  bool flash_ksplit = true;  // prefill attention split over keys where its query tiles leave CUs idle (stage 9)
  int prefill_chunk(const int32_t *ids, int n, int start, bool want_logits);
  // Scoring of a forward_logprobs call: while set, prefill_chunk also
  // computes every row's logits and their log probabilities (device
  // buffers, rows from score_row on).
  struct Scoring {
    const int *targets = nullptr;
    int count = 0, row = 0;
    double *chosen = nullptr, *top_lp = nullptr;
    int *top_ids = nullptr;
    void *scratch = nullptr;  // launch_logprobs scratch (the NaN error word first)
  } scoring;
  void *score_mem = nullptr;
  size_t score_bytes = 0;
  int score_rows(int n);
  int forward_logprobs(int prefix, const int32_t *tokens, const int32_t *targets, int n, int count, float *logits,
                       double *chosen, int32_t *top_ids, double *top_lp);
  int forward(int prefix, const int32_t *tokens, int n, bool want_logits, float *logits);
  // Rows of open branches: token ids[i] extends branch br[i]; each
  // branch's rows are consecutive and continue its suffix. Writes each
  // touched branch's newest-row logits to logits[branch][vocab].
  int branch_rows(struct Branches &b, const int32_t *ids, const int32_t *br, int n, float *logits);
};

// Independent suffixes of a resident prefix (nativeBranches,
// mlx_branches.go:14-20): the prefix KV [0, prefix) of the model is read,
// never written; branch j owns the suffix positions prefix + [0, len[j]),
// held in per-layer caches laid out [kv_heads][count * scap][hd], so that
// branch j's suffix entry s is slot j * scap + s. The caches grow (to a
// power of two, at most max_len) when a branch needs more positions, as
// appendBranchKV allocates only the suffix length used
// (mlx_branches.go:50-69).
struct Branches {
  StableModel *m = nullptr;
  int prefix = 0, count = 0, max_len = 0;
  std::vector<int> len;
  int scap = 0;
  std::vector<KVDev> kv;
  float *partials = nullptr;     // split-K attention partials
  size_t partial_floats = 0;
  unsigned *counters = nullptr;  // their arrival counters (zero between launches)
  size_t counter_words = 0;
  float *last = nullptr;         // [count][hidden]: each branch's newest residual row
  int *segs = nullptr;           // [chunk][3]: the runs of an append's chunk (first row, rows, first slot)
  std::vector<int> segs_host;    // their host copy (kept until the call has synchronised)
  float *logits_host = nullptr;  // [count][vocab] pinned: a step's logits on their way to the caller
  size_t logits_bytes = 0;
  std::map<int64_t, hipGraphExec_t> graphs;  // lockstep steps by attention shape
  ~Branches();
  void free_kv();
  void drop_graphs();
  // Suffix capacity for `need` positions per branch (existing entries kept).
  int grow(int need);
  // Attention scratch for nq queries with up to `splits` splits.
  int ensure_partials(int nq, int splits);
};

// The legacy Llama of llama2.c checkpoints (Model.transformer,
// model.go:379-481) on the decode kernels, fp32 weights and KV, one token
// per step (the reference evaluates a suffix token by token as well).
struct LlamaModel {
  tinyoai_llama_config cfg{};
  StableDims att{}, mlp{};  // attention half (RMSNorm + q/k/v) and MLP half (RMSNorm + w1/w3)
  hipStream_t stream = nullptr;
  DevMatrix embed;          // token embeddings, also the classifier (model.go:476-479)
  std::vector<DevMatrix> mats;  // per layer: win (q|k|v), wo, w1/w3 interleaved, w2
  std::vector<LayerDev> att_layers, mlp_layers;
  float *rms_final = nullptr, *rope = nullptr;
  std::vector<float> rope_host;  // [pos][hs]
  std::vector<KVDev> kv;    // [kv_heads][seq_len][head] per layer
  int offset = 0;
  float *x = nullptr, *qbuf = nullptr, *abuf = nullptr, *hbuf = nullptr, *partials = nullptr;
  float *head_out = nullptr;    // [vocab]: the head's output of the last step
  float *logits_dev = nullptr;  // [rows][vocab]: the rows a forward returns
  int logits_rows = 0;
  unsigned *counters = nullptr;
  int *params = nullptr;
  int max_splits = 0;
  void *h_pinned = nullptr;
  hipEvent_t params_copied = nullptr;
  int grid_in = 1, grid_mlp = 1, grid_out = 1, grid_head = 1;
  std::map<int64_t, hipGraphExec_t> graphs;
  std::vector<void *> buffers;
  // One launch per call (launch_tiny_llama) where the shape allows: the
  // logits rows land in pinned host memory (out_host, out_rows rows).
  bool tiny_ok = false, tiny = false;
  uint8_t *tiny_w = nullptr;  // packed weights (layout in kernels.h)
  void *kv_base = nullptr;    // every layer's K and V (kv[l] points into it)
  float *out_host = nullptr, *out_dev = nullptr;
  int out_rows = 0;
  unsigned *done_host = nullptr, *done_dev = nullptr;  // completion word (mapped, coherent)
  unsigned done_seq = 0;

  ~LlamaModel();
  int init(const tinyoai_llama_config &c, const float *weights, uint64_t n_floats);
  int alloc(void **p, size_t bytes);
  int ensure_logits(int rows);
  int enqueue_step(int steps, int splits, float *logits);
  int step(int token, int pos, float *logits);
  int forward(int prefix, const int32_t *tokens, int n, bool all_logits, float *logits);
  int forward_tiny(int prefix, const int32_t *tokens, int n, bool all_logits, float *logits);
};

}  // namespace tinyoai

// One opaque handle type for both model families.
struct tinyoai_model {
  std::unique_ptr<tinyoai::StableModel> stable;
  std::unique_ptr<tinyoai::LlamaModel> llama;
};
