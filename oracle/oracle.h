/*
 * oracle.h -- CPU restatement of tinyoai's Go scalar (float64-accumulating)
 * inference engine, used ONLY as a test checker and as the CPU baseline that
 * bench.py reports beside the GPU numbers. Product code never links this.
 *
 * Reference files restated (wbrown/tinyoai):
 *   dot.go:14-89, dot_scalar.go:9-37, matmul.go:12-95, matmul_scalar.go:7-27,
 *   quant_k.go:8-86, safetensors.go:230-264, kv_cache.go:27-109,
 *   stablelm.go:288-431, prefill.go:33-115, model.go:407-481,552-630.
 *
 * Numerics: built with -ffp-contract=off so every float32 operation rounds
 * separately, matching Go on amd64 (which never fuses x*y+z).
 */
#ifndef TINYOAI_ORACLE_H
#define TINYOAI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type codes (gguf.go:183-214); Q4_K=12 is a restatement of the
 * public GGML layout, absent from the reference. */
enum {
  OR_F32 = 0, OR_F16 = 1, OR_Q5_1 = 7, OR_Q8_0 = 8,
  OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_BF16 = 30
};

/* A row-major [rows, cols] tensor in its on-disk encoding (safetensors.go:193-197). */
typedef struct {
  int32_t dtype;
  int64_t rows, cols;
  const uint8_t *data;
} or_weight;

void or_set_threads(int n);
int or_get_threads(void);

float or_half_float(uint16_t h);
uint16_t or_float_half(float v);
int64_t or_weight_bytes(int32_t dtype, int64_t rows, int64_t cols);
void or_decode_kblock(int32_t dtype, const uint8_t *block, float *out);
void or_read_values(const or_weight *w, int64_t offset, int64_t n, float *out);
float or_at(const or_weight *w, int64_t i);

void or_mul_rows(const or_weight *w, const float *x, float *out, int64_t start, int64_t end);
void or_mul(const or_weight *w, const float *x, float *out);
void or_mul_batch(const or_weight *w, const float *x, int n, float *out);

void or_layer_norm(float *out, const float *x, int n, const or_weight *weight,
                   const or_weight *bias, double eps);
void or_stable_rotate(float *x, int len, int head, int rotary, int pos, double theta);
void or_softmax(float *x, int n);
int or_argmax(const float *v, int n);
float or_attention_dot(const float *q, const float *k, int n);

/* ---- StableLM engine (stablelm.go, prefill.go, kv_cache.go) ---- */
typedef struct {
  int32_t vocab_size, hidden_size, intermediate_size, num_hidden_layers;
  int32_t num_attention_heads, num_key_value_heads, max_position_embeddings;
  int32_t bos_token_id, eos_token_id;
  double layer_norm_eps, rope_theta, partial_rotary_factor;
} or_stablelm_config;

typedef struct or_stablelm or_stablelm;

/* tensors: [embed, head, norm.weight, norm.bias] then per layer
 * [ln.weight, ln.bias, q, k, v, o, gate, up, down]. Data is borrowed. */
or_stablelm *or_stablelm_create(const or_stablelm_config *c, const or_weight *tensors,
                                int n_tensors, int half_kv, int capacity);
void or_stablelm_destroy(or_stablelm *m);
int or_stablelm_forward(or_stablelm *m, int token, int pos, int want_logits, float *logits);
int or_stablelm_prefill(or_stablelm *m, const int32_t *ids, int n, int start, float *logits);
/* Copies layer l's K and V for kv head h, positions [0, n), expanded to fp32. */
int or_stablelm_read_kv(or_stablelm *m, int l, int h, int n, float *keys, float *values);
/* Residual stream after each layer of the last forward's final token:
 * [layers][hidden]; enabled by or_stablelm_trace(m, 1). */
void or_stablelm_trace(or_stablelm *m, int enable);
const float *or_stablelm_trace_data(or_stablelm *m);

/* ---- legacy Llama engine (model.go) ---- */
typedef struct {
  int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
} or_llama_config;

typedef struct or_llama or_llama;
/* weights: the llama2.c float32 payload following the 7-int32 header
 * (model.go:129-166), borrowed. */
or_llama *or_llama_create(const or_llama_config *c, const float *weights, size_t n_floats);
void or_llama_destroy(or_llama *m);
int or_llama_transformer(or_llama *m, int token, int pos, float *logits);

#ifdef __cplusplus
}
#endif
#endif
