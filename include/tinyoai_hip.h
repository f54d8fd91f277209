/*
 * tinyoai_hip.h -- C ABI of the MI355X (gfx950) forward-pass backend.
 *
 * The entry points are what tinyoai's GPU forwarder contract binds
 * (mlx.go:45-51, mlx_llama.go:27-35, mlx_kv.go:78-91, mlx_native.go:231-244),
 * plus the weightTensor operations the kernel-level benchmarks and tests use
 * (safetensors.go:268-280, matmul.go:12-95). Plain pointers and sizes only.
 *
 * Conventions
 *  - Every call returns 0 on success or a negative TINYOAI_E* code; the
 *    message is then available from tinyoai_last_error() on the same thread.
 *  - Host buffers stay owned by the caller; the library copies what it keeps.
 *  - A handle is used by one thread at a time (the caller holds the model
 *    gate, stablelm.go:478-484 / mlx.go:291-296). Different handles are
 *    independent and run on their own HIP streams.
 *  - Cancellation stays with the caller, checked between calls; an admitted
 *    forward always completes (mlx_native.go:491-494).
 */
#ifndef TINYOAI_HIP_H
#define TINYOAI_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TINYOAI_OK 0
#define TINYOAI_EINVAL (-1)   /* invalid argument or unsupported configuration */
#define TINYOAI_EDEVICE (-2)  /* HIP runtime or kernel launch failure */
#define TINYOAI_ENOMEM (-3)   /* device or host allocation failure */

/* GGUF tensor type codes (gguf.go:183-214). Q4_K (12) is accepted although
 * the reference rejects it (gguf.go:203-204). */
#define TINYOAI_F32 0
#define TINYOAI_F16 1
#define TINYOAI_Q5_1 7
#define TINYOAI_Q8_0 8
#define TINYOAI_Q4_K 12
#define TINYOAI_Q5_K 13
#define TINYOAI_Q6_K 14
#define TINYOAI_BF16 30

typedef struct tinyoai_model tinyoai_model;
typedef struct tinyoai_weight tinyoai_weight;
typedef struct tinyoai_branches tinyoai_branches;

/* One tensor in its on-disk encoding, row-major [rows, cols] (vectors:
 * rows = 1), named as in the Hugging Face checkpoint
 * (stablelm.go:180-191); weightTensor, safetensors.go:193-197. */
typedef struct {
  const char *name;
  int32_t dtype;
  int64_t rows, cols;
  const void *data;
  uint64_t nbytes;
} tinyoai_tensor;

/* StableLMConfig after validate() (stablelm.go:18-111). */
typedef struct {
  int32_t vocab_size, hidden_size, intermediate_size, num_hidden_layers;
  int32_t num_attention_heads, num_key_value_heads, max_position_embeddings;
  int32_t bos_token_id, eos_token_id;
  double layer_norm_eps, rope_theta, partial_rotary_factor;
} tinyoai_stablelm_config;

/* llama2.c Config header (model.go:29-37). */
typedef struct {
  int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
} tinyoai_llama_config;

/* The calling thread's message for its last failed call. */
const char *tinyoai_last_error(void);

/* ---------------- StableLM forwarder (mlxForwarder, mlx.go:45-51) ---------------- */

/* Uploads every tensor named by loadStableWeights (stablelm.go:178-191) to
 * HBM and prepares fp32 KV storage (StableLMOptions{KVCache: "f32"}).
 * Layer matrices are regrouped per layer into an input-side matrix (q, k,
 * v, gate, up) and an output-side matrix (o, down). q, k and v must share
 * one storage format and gate and up one format; the attention and MLP
 * sections may differ (as GGUF K-quant mixes store them), and then each is
 * kept as a matrix of its own. Other combinations return TINYOAI_EINVAL. */
int tinyoai_stablelm_load(const tinyoai_stablelm_config *config, const tinyoai_tensor *tensors,
                          int32_t n_tensors, tinyoai_model **out);

/* Forward (mlx.go:47-48; nativeMLX.Forward, mlx_native.go:292-297):
 * replaces the resident suffix after `prefix` (0 <= prefix <= offset) with
 * `tokens`, writes their KV, and when want_logits is nonzero writes the last
 * position's fp32 logits [vocab_size] to the caller's `logits`. On success
 * the resident offset becomes prefix + n. On failure the KV is reset
 * (mlx_native.go:487-490) and the offset is 0. */
int tinyoai_stablelm_forward(tinyoai_model *m, int32_t prefix, const int32_t *tokens, int32_t n,
                             int32_t want_logits, float *logits);

/* ForwardWithLogprobs (mlx.go:53-57; mlx_native.go:300-311): the forward
 * of `tokens` after `prefix` (semantics and failure behaviour of
 * tinyoai_stablelm_forward, always with logits) that also scores position i
 * against targets[i]: chosen[i] = log p(targets[i]) and the `count` most
 * likely ids top_ids[i][count] with their log probabilities
 * top_logprobs[i][count], descending, ties to the lower id, normalised over
 * the whole vocabulary in float64 (summarizeLogits, logprobs.go:60-95).
 * `logits` receives the last position's row. 1 <= count <= vocab; every
 * target in [0, vocab). -0 and +0 rank as equal (ties to the lower id). A
 * row holding NaN is refused (TINYOAI_EINVAL, naming the position): the
 * reference's float64 max would make every value NaN. */
int tinyoai_stablelm_forward_logprobs(tinyoai_model *m, int32_t prefix, const int32_t *tokens,
                                      const int32_t *targets, int32_t n, int32_t count, float *logits,
                                      double *chosen, int32_t *top_ids, double *top_logprobs);

/* summarizeLogits (logprobs.go:60-95) on the device for `rows` caller rows
 * of logits [rows][vocab]: chosen[r] = log p(targets[r]) and the `count`
 * best ids and log probabilities per row (1 <= count <= vocab), as
 * forward_logprobs scores them; a row holding NaN is refused. */
int tinyoai_summarize_logits(const float *logits, int32_t rows, int32_t vocab, const int32_t *targets, int32_t count,
                             double *chosen, int32_t *top_ids, double *top_logprobs);

/* SetKVBits (mlx_kv.go:78-91): 16 = fp16 KV rounded with floatHalf
 * (kv_cache.go:27-65), 32 = fp32 KV (the CPU engine's StableLMOptions{KVCache:
 * "f32"}). The MLX forwarder's 8 (affine 8-bit KV in groups of 64,
 * mlx_kv.go:46-73) is rejected with TINYOAI_EINVAL. A change discards the
 * resident prefix and sets *cleared = 1. */
int tinyoai_stablelm_set_kv_bits(tinyoai_model *m, int32_t bits, int32_t *cleared);

/* LimitCache (mlx_native.go:231-244): reserves `limit` KV positions; a
 * larger retained cache is discarded and *cleared = 1. */
int tinyoai_stablelm_limit_cache(tinyoai_model *m, int32_t limit, int32_t *cleared);

/* Discards KV, keeping weights resident (nativeMLX.reset, mlx_native.go:216-224). */
int tinyoai_stablelm_reset(tinyoai_model *m);

/* Resident prefix length (nativeMLX.offset), or a negative code. */
int tinyoai_stablelm_offset(const tinyoai_model *m);

/* Releases weights, KV and the stream (mlx_native.go:247-259); refused
 * (TINYOAI_EINVAL, nothing released) while branches are open. */
int tinyoai_stablelm_close(tinyoai_model *m);

/* NewBranches (mlx_branches.go:25-33; mlxBrancher, branches.go:55-59): opens
 * `count` independent suffixes that borrow the resident prefix [0, prefix)
 * (0 <= prefix <= offset) read-only. Branch j holds the suffix positions
 * prefix + [0, length(j)); the suffix KV grows with use (in powers of two,
 * at most max_len positions per branch; 0 = up to the context), in the
 * model's KV format at opening. Head widths 8, 64, 80 and 128; count * vocab <=
 * the prefill chunk's product buffer. While branches are open the model
 * refuses forward, reset, set_kv_bits, limit_cache and close with
 * TINYOAI_EINVAL (the reference's session holds the model gate,
 * branches.go:16-22). */
int tinyoai_stablelm_branches_open(tinyoai_model *m, int32_t prefix, int32_t count, int32_t max_len,
                                   tinyoai_branches **out);
/* nativeBranches.Forward (mlx_branches.go:120-182): one token per branch,
 * branch j at position prefix + length(j); writes `count` rows of fp32
 * logits [count][vocab]. Attention combines the shared prefix with the
 * branch's own suffix under one softmax (branchAttention,
 * mlx_branches.go:98-114). TINYOAI_EINVAL for a wrong count, an invalid id,
 * or a suffix past max_len or the context; a native failure closes the
 * branches' storage (later calls fail), as Forward closes them on error. */
int tinyoai_stablelm_branches_forward(tinyoai_branches *b, const int32_t *tokens, int32_t count, float *logits);
/* Private suffixes of different lengths (no counterpart in the reference,
 * whose branches all advance one token per step): appends lengths[j] >= 1
 * tokens to branch j, the tokens given branch after branch (sum of lengths
 * ids), evaluated causally within each branch against the shared prefix;
 * writes each branch's last-row logits [count][vocab]. Errors as forward. */
int tinyoai_stablelm_branches_append(tinyoai_branches *b, const int32_t *tokens, const int32_t *lengths,
                                     int32_t count, float *logits);
/* Suffix tokens branch `branch` holds, or a negative code. */
int tinyoai_stablelm_branches_length(const tinyoai_branches *b, int32_t branch);
/* nativeBranches.Close (mlx_branches.go:36-47): frees the suffix KV; the
 * shared prefix stays. NULL is accepted. */
int tinyoai_stablelm_branches_close(tinyoai_branches *b);

/* KV snapshots (SaveCache / LoadCache, cache_file.go:49-186): the host keeps
 * the TNYKV001 container (magic, JSON header with the model identity and
 * tokens, SHA-256 trailer); these move its payload, cachePayload's byte
 * order (cache_file.go:188-216): for each layer, each kv head, K then V,
 * positions [0, n) of head_dim values, little-endian fp32 or fp16 bits as
 * the model's KV format (`half` must match it; "KV cache precision does
 * not match model options" otherwise). nbytes = layers * kv_heads * 2 * n *
 * head_dim * (half ? 2 : 4). save reads positions [0, n) of the resident
 * prefix (n <= offset); load replaces the resident cache with the payload
 * and sets the offset to n (on a copy failure the KV is reset). */
int tinyoai_stablelm_kv_save(tinyoai_model *m, int32_t n, int32_t half, void *payload, uint64_t nbytes);
int tinyoai_stablelm_kv_load(tinyoai_model *m, int32_t n, int32_t half, const void *payload, uint64_t nbytes);

/* Debug hooks for parity checks: copy KV head `kv_head` of `layer` for
 * positions [0, n) as fp32 [n][head_dim] (stableState keys/values,
 * kv_cache.go:91-96); record the residual stream after every layer for the
 * final token of each forward (the stage boundaries of stableProfile,
 * stablelm.go:339-384) and read it back as [layers][hidden]. */
int tinyoai_stablelm_read_kv(tinyoai_model *m, int32_t layer, int32_t kv_head, int32_t n, float *keys,
                             float *values);
int tinyoai_stablelm_trace(tinyoai_model *m, int32_t enable);
int tinyoai_stablelm_trace_read(tinyoai_model *m, float *residual);
/* The same trace's attention outputs [layers][heads * head_dim] (attendHeads,
 * stablelm.go:391-431) and SiLU-gate outputs [layers][intermediate]
 * (stablelm.go:371-373) of the final token. */
int tinyoai_stablelm_trace_read_stages(tinyoai_model *m, float *attention, float *gate);

/* Stage timings (stableProfile, stablelm.go:227-250): when enabled, each
 * kernel is bracketed by hipEvents on the handle's stream and its duration
 * is added to its stage: 0 embedding, 1 decode_in (layer_norm +
 * projections + rotary + kv_write + SiLU-gate), 2 attention, 3 decode_out
 * (output_projection + down + residual), 4 lm_head, 5 prefill layer_norm,
 * 6 prefill projections, 7 prefill rotary + kv_write + SiLU-gate, 8 prefill
 * attention, 9 prefill residual. Enabling clears the totals.
 * profile_read fills ms[] and counts[] (n_stages >= 10) and returns the
 * number of stages. */
int tinyoai_stablelm_profile(tinyoai_model *m, int32_t enable);
/* Launch shape of a decode matrix kernel: stage 0 decode_in, 1 decode_out,
 * 2 lm_head; `grid` blocks (> 0) of `threads` threads (256 or 512). Takes
 * effect from the next forward (cached graphs are dropped); a shape the
 * kernel cannot run makes that forward fail. The shape changes speed; the
 * per-row arithmetic stays the same (only the float64 sums of the
 * normalisation moments are grouped by wave). Stage 3 sets the decode
 * attention shape instead: `grid` = positions per block / 64 (1, 2 or 4 on
 * 4-wave blocks, 8 or 16 on 16-wave blocks; 0 = chosen from the position)
 * and `threads` is ignored. Stage 4: grid nonzero (the default) runs each
 * layer's decode attention on extra blocks of the decode_in launch, zero
 * as a launch of its own (same arithmetic). Stage 5: grid nonzero makes
 * the prefill products of BF16 matrices take bf16 activations (the bf16
 * path: within 2e-2 of the logit range, faster on the matrix cores; greedy
 * ids may then differ from the fp32 engine's where logits nearly tie),
 * zero (the default) keeps two bf16 planes per activation (16 significant
 * bits). Stage 7: grid nonzero (the default) runs the BF16-weight prefill
 * products on wide matrix-core tiles (the o and down products together
 * as K splits of one launch), zero on 128 x 256 tiles (fp32 accumulation
 * either way; the sums' order differs). Stage 8: grid nonzero forms the wide-tile in-projection's
 * epilogue in the product's own launch, zero (the default) as a kernel of
 * its own (same arithmetic). Stage 9: grid nonzero (the default) splits a
 * prefill call's attention over key ranges when its query tiles would
 * leave CUs idle (calls of fewer than about 900 tokens whose last position
 * reaches 256), the ranges' partial results combined in a fixed order; zero
 * keeps one block per query tile (the sums' order differs). Stage 10:
 * grid nonzero (the default) runs the Q8_0-weight prefill of fused layers
 * on wide tiles (the o and down products together as K splits of one
 * launch; chunks over 1024 rows also their in-projection), zero on
 * 128 x 256 tiles throughout (the quants exact either way; the sums' order
 * differs). Stage 11: grid nonzero (the default) pairs a branch step's
 * launches: the two few-row K-quant in-products (Q4_K / Q6_K q/k/v and
 * gate/up) as one launch, their two epilogues as one, and the o and down
 * products (their inputs staged together after the attention) as one;
 * zero runs each as a launch of its own (identical results). Returns 0 or
 * TINYOAI_EINVAL. */
int tinyoai_stablelm_set_launch(tinyoai_model *m, int32_t stage, int32_t grid, int32_t threads);
int tinyoai_stablelm_profile_read(tinyoai_model *m, double *ms, int64_t *counts, int32_t n_stages);

/* ---------------- legacy Llama forwarder (llamaMLXForwarder, mlx_llama.go:27-35) ---------------- */

/* `weights` is the float32 payload after the 7-int32 header, in
 * readWeights order (model.go:129-166). */
int tinyoai_llama_load(const tinyoai_llama_config *config, const float *weights, uint64_t n_floats,
                       tinyoai_model **out);
/* Forward (mlx_llama.go:30-31): evaluates `tokens` after `prefix`; writes
 * all n rows of logits ([n][vocab]) when all_logits is nonzero, else only
 * the last row. */
int tinyoai_llama_forward(tinyoai_model *m, int32_t prefix, const int32_t *tokens, int32_t n,
                          int32_t all_logits, float *logits);
int tinyoai_llama_reset(tinyoai_model *m);  /* Reset (mlx_llama.go:32-33) */
int tinyoai_llama_close(tinyoai_model *m);  /* Close (mlx_llama.go:34) */
/* Launch choice (no counterpart in the reference: a tuning and test
 * switch, like tinyoai_stablelm_set_launch). Stage 0: value nonzero (the
 * default where the model fits: dim 64, 8 query / 4 kv heads, MLP 172, at
 * most 8 layers, 512 positions and a 512-token vocabulary, the stories260K
 * shape) runs every token of a forward call in one launch of one
 * workgroup; zero runs five kernels per layer and token. The sums' order
 * differs between the two. Returns 0, or TINYOAI_EINVAL for another stage,
 * or for value nonzero on a model of another shape. */
int tinyoai_llama_set_launch(tinyoai_model *m, int32_t stage, int32_t value);

/* ---------------- single weight matrices (weightTensor, safetensors.go:193-280) ---------------- */

int tinyoai_weight_upload(int32_t dtype, int64_t rows, int64_t cols, const void *data, uint64_t nbytes,
                          tinyoai_weight **out);
/* readValues (matmul.go:12-50): n values from flat element `offset`, bit-exact. */
int tinyoai_weight_read_values(tinyoai_weight *w, int64_t offset, int64_t n, float *out);
/* mulScratch (n == 1, safetensors.go:275-280) or mulBatch (n > 1,
 * matmul.go:55-95): out[n][rows] = x[n][cols] * W^T, host buffers. */
int tinyoai_weight_mul(tinyoai_weight *w, const float *x, int32_t n, float *out);
/* The same product on device-resident buffers, enqueued on `stream`
 * (a hipStream_t; NULL = the weight's own stream) without synchronizing. */
int tinyoai_weight_mul_device(tinyoai_weight *w, const float *x_dev, int32_t n, float *out_dev, void *stream);
/* tinyoai_weight_mul_device without any allocation, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc); it has no counterpart in the reference.
 * The activations' operand planes (16 MiB) and the product's K-split
 * partials (32 MiB) live in a library array of 48 MiB on each GPU the
 * library runs on (held until the process ends), so n * cols
 * may be at most 4,194,304 (TINYOAI_EINVAL beyond) and the current device
 * must be the weight's. Calls share that array and each overwrites what
 * the previous one left there, so the library orders them: `stream` NULL
 * runs the call on one library stream per GPU (not the weight's own
 * stream), and a caller's stream first waits for the previous call on
 * that GPU, on whatever stream it ran. Under HIP stream capture no such
 * wait is recorded: captured calls that overlap on one GPU race for the
 * array. */
int tinyoai_weight_mul_device_noalloc(tinyoai_weight *w, const float *x_dev, int32_t n, float *out_dev, void *stream);
int tinyoai_weight_free(tinyoai_weight *w);

#ifdef __cplusplus
}
#endif
#endif
