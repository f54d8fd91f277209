/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of wbrown/tinyoai's Go scalar engine ("scalar-float64",
 * dot_scalar.go:19), which dot.go:10-13 names as the numerical oracle of the
 * reference. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load it, always as the checker or the timed CPU baseline, never as the
 * product path.
 *
 * Every function cites the reference file:line it follows. Parity pins:
 *   halfFloat/floatHalf   exhaustive round trip + all midpoints (kv_cache_test.go:12-44)
 *   Q5_K/Q6_K/Q5_1 decode reference golden vectors testdata/gguf q5_k/q6_k/q5_1 .bin files (quant_k_test.go:14-33)
 *   Q4_K decode           embedding into Q5_K with an all-zero high-bit plane,
 *                         whose decoder the golden vectors pin
 *   Q8_0/BF16/F32 decode  closed forms (matmul.go:12-50)
 *   matvec / mulBatch     float64 brute force (prefill_test.go:183-212)
 *   RoPE                  closed form + rope.json (stablelm_test.go:168-205)
 *   StableLM forward      expected.json logits + greedy ids (stablelm_test.go:50-82)
 *   batched prefill       sequential forward within 3e-5 (prefill_test.go:217-277)
 *   Llama transformer     the reference holds no Llama logits or tokens: pinned by
 *                         a float64 statement of the same model on stories260K at
 *                         positions 0-8 (rotations other than the identity, 8
 *                         query heads on 4 kv heads, up to 9 softmax terms),
 *                         which detects planted mistakes (swapped cos/sin, a
 *                         wrong kv head, a dropped key), and closed-form steps.
 *
 * Build: -O2 -ffp-contract=off -fopenmp (see oracle/Makefile). With contraction
 * off, every float32 operation rounds separately, like Go on amd64.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int or_get_threads(void) { return g_threads; }

static inline float f32_from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }
static inline uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t le32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* halfFloat, safetensors.go:250-264. */
float or_half_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 31, frac = h & 1023;
  if (exp == 0) {
    float v = (float)ldexp((double)frac, -24);
    return sign ? -v : v;
  }
  if (exp == 31) return f32_from_bits(sign | 0x7f800000u | frac << 13);
  return f32_from_bits(sign | (exp + 112) << 23 | frac << 13);
}

/* floatHalf, kv_cache.go:27-51: round to nearest even incl. subnormals. */
uint16_t or_float_half(float value) {
  uint32_t bits = f32_bits(value);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
  uint32_t magnitude = bits & 0x7fffffffu;
  if (magnitude >= 0x7f800000u) {
    if (magnitude > 0x7f800000u) return sign | 0x7e00;
    return sign | 0x7c00;
  }
  int exponent = (int)(magnitude >> 23) - 127 + 15;
  if (exponent >= 31) return sign | 0x7c00;
  if (exponent <= 0) {
    if (exponent < -10) return sign;
    uint32_t mantissa = (magnitude & 0x7fffffu) | 0x800000u;
    unsigned shift = (unsigned)(14 - exponent);
    uint32_t rounded = (mantissa + ((1u << (shift - 1)) - 1) + ((mantissa >> shift) & 1)) >> shift;
    return sign | (uint16_t)rounded;
  }
  magnitude += 0xfff + ((magnitude >> 13) & 1);
  return sign | (uint16_t)((magnitude >> 13) - 0x1c000);
}

/* kBlockBytes / quantBlockWidth, quant_k.go:8-24 (+ Q4_K: 144 B / 256). */
static int kblock_bytes(int32_t dtype) {
  switch (dtype) {
    case OR_Q5_1: return 24;
    case OR_Q6_K: return 210;
    case OR_Q4_K: return 144;
    default: return 176; /* Q5_K */
  }
}
static int kblock_width(int32_t dtype) { return dtype == OR_Q5_1 ? 32 : 256; }

int64_t or_weight_bytes(int32_t dtype, int64_t rows, int64_t cols) {
  int64_t n = rows * cols;
  switch (dtype) {
    case OR_F32: return n * 4;
    case OR_F16: case OR_BF16: return n * 2;
    case OR_Q8_0: return n / 32 * 34;
    case OR_Q5_1: return n / 32 * 24;
    case OR_Q4_K: return n / 256 * 144;
    case OR_Q5_K: return n / 256 * 176;
    case OR_Q6_K: return n / 256 * 210;
  }
  return -1;
}

/* Shared 6-bit scale/min unpacking of Q5_K and Q4_K (quant_k.go:69-77). */
static void kquant_scale_min(const uint8_t *scales, int group, uint8_t *scale, uint8_t *minimum) {
  if (group < 4) {
    *scale = scales[group] & 63;
    *minimum = scales[group + 4] & 63;
  } else {
    *scale = (uint8_t)((scales[group + 4] & 15) | ((scales[group - 4] >> 6) << 4));
    *minimum = (uint8_t)((scales[group + 4] >> 4) | ((scales[group] >> 6) << 4));
  }
}

/* decodeKBlock, quant_k.go:31-86; Q4_K follows the Q5_K arithmetic with no
 * high-bit plane (GGML block_q4_K: d, dmin, scales[12], qs[128]). */
void or_decode_kblock(int32_t dtype, const uint8_t *block, float *out) {
  if (dtype == OR_Q5_1) { /* quant_k.go:35-45 */
    float d = or_half_float(le16(block)), minimum = or_half_float(le16(block + 2));
    uint32_t high = le32(block + 4);
    for (int i = 0; i < 32; i++) {
      uint8_t low = (block[8 + i % 16] >> (unsigned)(i / 16 * 4)) & 15;
      uint8_t q = (uint8_t)(low | ((high >> (unsigned)i) & 1) << 4);
      float t = d * (float)q;
      out[i] = t + minimum;
    }
    return;
  }
  if (dtype == OR_Q6_K) { /* quant_k.go:47-61 */
    float d = or_half_float(le16(block + 208));
    for (int group = 0; group < 16; group++) {
      float scale = d * (float)(int8_t)block[192 + group];
      for (int j = 0; j < 16; j++) {
        int i = group * 16 + j;
        uint8_t low = (block[(i / 128) * 64 + i % 64] >> (unsigned)((i % 128) / 64 * 4)) & 15;
        uint8_t high = (block[128 + (i / 128) * 32 + i % 32] >> (unsigned)((i % 128) / 32 * 2)) & 3;
        out[i] = scale * (float)((int)(low | high << 4) - 32);
      }
    }
    return;
  }
  /* Q5_K, quant_k.go:63-85; Q4_K shares it with high == 0. */
  float d = or_half_float(le16(block)), dmin = or_half_float(le16(block + 2));
  const uint8_t *scales = block + 4;
  int q4 = dtype == OR_Q4_K;
  for (int group = 0; group < 8; group++) {
    uint8_t scale, minimum;
    kquant_scale_min(scales, group, &scale, &minimum);
    float ds = d * (float)scale, dm = dmin * (float)minimum;
    for (int j = 0; j < 32; j++) {
      uint8_t low, high;
      if (q4) {
        low = (block[16 + (group / 2) * 32 + j] >> (unsigned)(group % 2 * 4)) & 15;
        high = 0;
      } else {
        low = (block[48 + (group / 2) * 32 + j] >> (unsigned)(group % 2 * 4)) & 15;
        high = (block[16 + j] >> (unsigned)group) & 1;
      }
      float t = ds * (float)(low | high << 4);
      out[group * 32 + j] = t - dm;
    }
  }
}

/* readValues, matmul.go:12-50. */
void or_read_values(const or_weight *w, int64_t offset, int64_t n, float *out) {
  switch (w->dtype) {
    case OR_BF16:
      for (int64_t i = 0; i < n; i++) out[i] = f32_from_bits((uint32_t)le16(w->data + (offset + i) * 2) << 16);
      return;
    case OR_F32:
      for (int64_t i = 0; i < n; i++) out[i] = f32_from_bits(le32(w->data + (offset + i) * 4));
      return;
    case OR_Q8_0:
      for (int64_t i = 0; i < n;) {
        int64_t index = offset + i;
        const uint8_t *block = w->data + index / 32 * 34;
        float scale = or_half_float(le16(block));
        int64_t m = 32 - index % 32;
        if (m > n - i) m = n - i;
        for (int64_t j = 0; j < m; j++) out[i + j] = scale * (float)(int8_t)block[2 + index % 32 + j];
        i += m;
      }
      return;
    case OR_Q5_K: case OR_Q6_K: case OR_Q5_1: case OR_Q4_K: {
      int size = kblock_bytes(w->dtype), width = kblock_width(w->dtype);
      float decoded[256];
      for (int64_t i = 0; i < n;) {
        int64_t index = offset + i;
        or_decode_kblock(w->dtype, w->data + index / width * size, decoded);
        int64_t m = width - index % width;
        if (m > n - i) m = n - i;
        memcpy(out + i, decoded + index % width, (size_t)m * 4);
        i += m;
      }
      return;
    }
    default: /* F16 through at(), safetensors.go:236-237 */
      for (int64_t i = 0; i < n; i++) out[i] = or_half_float(le16(w->data + (offset + i) * 2));
  }
}

/* at, safetensors.go:230-246. */
float or_at(const or_weight *w, int64_t i) {
  float v;
  or_read_values(w, i, 1, &v);
  return v;
}

/* mulRowsScalar, dot.go:14-70: float64 accumulation, float32 result. */
void or_mul_rows(const or_weight *w, const float *x, float *out, int64_t start, int64_t end) {
  int64_t cols = w->cols;
  for (int64_t i = start; i < end; i++) {
    double sum = 0;
    switch (w->dtype) {
      case OR_Q5_K: case OR_Q6_K: case OR_Q5_1: case OR_Q4_K: { /* dot.go:22-30 */
        float decoded[256];
        for (int64_t j = 0; j < cols; j += 256) {
          int64_t n = cols - j < 256 ? cols - j : 256;
          or_read_values(w, i * cols + j, n, decoded);
          for (int64_t k = 0; k < n; k++) sum += (double)x[j + k] * (double)decoded[k];
        }
        break;
      }
      case OR_Q8_0: { /* dot.go:31-40 */
        const uint8_t *row = w->data + i * cols / 32 * 34;
        for (int64_t j = 0; j < cols; j += 32) {
          const uint8_t *block = row + j / 32 * 34;
          double dot = 0;
          for (int k = 0; k < 32; k++) dot += (double)x[j + k] * (double)(int8_t)block[2 + k];
          sum += dot * (double)or_half_float(le16(block));
        }
        break;
      }
      case OR_BF16: { /* dot.go:41-57 */
        const uint8_t *row = w->data + i * cols * 2;
        double a = 0, b = 0, c = 0, d = 0;
        int64_t j = 0;
        for (; j + 3 < cols; j += 4) {
          a += (double)x[j] * (double)f32_from_bits((uint32_t)le16(row + j * 2) << 16);
          b += (double)x[j + 1] * (double)f32_from_bits((uint32_t)le16(row + j * 2 + 2) << 16);
          c += (double)x[j + 2] * (double)f32_from_bits((uint32_t)le16(row + j * 2 + 4) << 16);
          d += (double)x[j + 3] * (double)f32_from_bits((uint32_t)le16(row + j * 2 + 6) << 16);
        }
        sum = (a + b) + (c + d);
        for (; j < cols; j++) sum += (double)x[j] * (double)f32_from_bits((uint32_t)le16(row + j * 2) << 16);
        break;
      }
      case OR_F32: { /* dot.go:58-62 */
        const uint8_t *row = w->data + i * cols * 4;
        for (int64_t j = 0; j < cols; j++) sum += (double)x[j] * (double)f32_from_bits(le32(row + j * 4));
        break;
      }
      default: /* dot.go:63-66 */
        for (int64_t j = 0; j < cols; j++) sum += (double)x[j] * (double)or_at(w, i * cols + j);
    }
    out[i] = (float)sum;
  }
}

/* mul / mulScratch with parallelRows, safetensors.go:268-280, dot.go:76-89.
 * Row ownership does not change results, so OpenMP static partitioning
 * stands in for the goroutine partition. */
void or_mul(const or_weight *w, const float *x, float *out) {
  int64_t rows = w->rows;
  int workers = g_threads < rows ? g_threads : (int)rows;
  if (rows * w->cols < (1 << 20) || workers <= 1) {
    or_mul_rows(w, x, out, 0, rows);
    return;
  }
#pragma omp parallel for num_threads(workers) schedule(static, 1)
  for (int worker = 0; worker < workers; worker++)
    or_mul_rows(w, x, out, rows * worker / workers, rows * (worker + 1) / workers);
}

/* batchDot4, matmul_scalar.go:12-27 (scalar build, batchWidth 4). */
static void batch_dot4(double *dst, const float *x, const float *w, int stride, int64_t k) {
  for (int token = 0; token < stride; token++) {
    float a = 0, b = 0, c = 0, d = 0;
    for (int64_t j = 0; j < k; j++) {
      float v = x[j * stride + token];
      a += v * w[j];
      b += v * w[k + j];
      c += v * w[2 * k + j];
      d += v * w[3 * k + j];
    }
    dst[token] += (double)a;
    dst[stride + token] += (double)b;
    dst[2 * stride + token] += (double)c;
    dst[3 * stride + token] += (double)d;
  }
}

/* mulBatch, matmul.go:55-95: token-major out[n][rows] = x[n][cols] * W^T. */
void or_mul_batch(const or_weight *w, const float *x, int n, float *out) {
  if (n == 1) {
    or_mul(w, x, out);
    return;
  }
  int64_t rows = w->rows, cols = w->cols;
  int stride = (n + 3) / 4 * 4;
  float *packed = (float *)calloc((size_t)(cols * stride), sizeof(float));
  for (int token = 0; token < n; token++)
    for (int64_t col = 0; col < cols; col++) packed[col * stride + token] = x[token * cols + col];
  int64_t groups = (rows + 3) / 4;
  int workers = g_threads < groups ? g_threads : (int)groups;
  if (rows * cols * n < (1 << 20)) workers = 1;
#pragma omp parallel num_threads(workers)
  {
    float tile[4 * 512];
    double *totals = (double *)malloc(sizeof(double) * 4 * (size_t)stride);
#pragma omp for schedule(static)
    for (int64_t group = 0; group < groups; group++) {
      int64_t row = group * 4;
      int nr = rows - row < 4 ? (int)(rows - row) : 4;
      memset(totals, 0, sizeof(double) * 4 * (size_t)stride);
      for (int64_t col = 0; col < cols; col += 512) {
        int64_t nk = cols - col < 512 ? cols - col : 512;
        if (nr != 4) memset(tile, 0, sizeof(tile));
        for (int r = 0; r < nr; r++) or_read_values(w, (row + r) * cols + col, nk, tile + r * nk);
        batch_dot4(totals, packed + col * stride, tile, stride, nk);
      }
      for (int r = 0; r < nr; r++)
        for (int token = 0; token < n; token++)
          out[(int64_t)token * rows + row + r] = (float)totals[r * stride + token];
    }
    free(totals);
  }
  free(packed);
}

/* layerNorm, stablelm.go:288-305: float64 moments, float32 affine. */
void or_layer_norm(float *out, const float *x, int n, const or_weight *weight,
                   const or_weight *bias, double eps) {
  double mean = 0, variance = 0;
  for (int i = 0; i < n; i++) mean += (double)x[i];
  mean /= (double)n;
  for (int i = 0; i < n; i++) {
    double d = (double)x[i] - mean;
    variance += d * d;
  }
  float inv = (float)(1 / sqrt(variance / (double)n + eps));
  float fm = (float)mean;
  for (int i = 0; i < n; i++) {
    float t = x[i] - fm;
    t = t * inv;
    t = t * or_at(weight, i);
    out[i] = t + or_at(bias, i);
  }
}

/* stableRotate, stablelm.go:309-326: split-half RoPE of the rotary prefix. */
void or_stable_rotate(float *x, int len, int head, int rotary, int pos, double theta) {
  for (int i = 0; i < rotary / 2; i++) {
    float expo = (float)(2 * i) / (float)rotary;
    float power = (float)pow((double)(float)theta, (double)expo);
    float inv_freq = 1.0f / power;
    float angle = (float)pos * inv_freq;
    float sn = (float)sin((double)angle), cs = (float)cos((double)angle);
    for (int h = 0; h < len; h += head) {
      float a = x[h + i], b = x[h + i + rotary / 2];
      float ac = a * cs, bs = b * sn, bc = b * cs, as = a * sn;
      x[h + i] = ac - bs;
      x[h + i + rotary / 2] = bc + as;
    }
  }
}

/* softmax, model.go:552-570. */
void or_softmax(float *x, int n) {
  if (n == 0) return;
  float max_val = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > max_val) max_val = x[i];
  float sum = 0;
  for (int i = 0; i < n; i++) {
    float d = x[i] - max_val;
    x[i] = (float)exp((double)d);
    sum += x[i];
  }
  for (int i = 0; i < n; i++) x[i] /= sum;
}

/* argmax, model.go:622-630: strict > keeps the earliest index. */
int or_argmax(const float *v, int n) {
  int best = 0;
  float best_v = v[0];
  for (int i = 1; i < n; i++)
    if (v[i] > best_v) { best = i; best_v = v[i]; }
  return best;
}

/* attentionDot, dot_scalar.go:23-29: sequential float32. */
float or_attention_dot(const float *q, const float *k, int n) {
  float score = 0;
  for (int i = 0; i < n; i++) score += q[i] * k[i];
  return score;
}

/* ===================== StableLM engine ===================== */

struct or_stablelm {
  or_stablelm_config c;
  or_weight *t; /* 4 + 9*layers */
  int half_kv, capacity;
  float **keys, **values;       /* fp32 KV [layer][kvh][cap][hd] */
  uint16_t **keys16, **values16; /* fp16 KV */
  float *x, *norm, *att_out, *proj, *gate, *up, *q, *k, *v, *att;
  float *trace;
  int trace_on;
};

static const or_weight *layer_t(const or_stablelm *m, int l, int j) { return &m->t[4 + 9 * l + j]; }

or_stablelm *or_stablelm_create(const or_stablelm_config *c, const or_weight *tensors,
                                int n_tensors, int half_kv, int capacity) {
  if (n_tensors != 4 + 9 * c->num_hidden_layers) return NULL;
  or_stablelm *m = (or_stablelm *)calloc(1, sizeof(*m));
  m->c = *c;
  m->t = (or_weight *)malloc(sizeof(or_weight) * (size_t)n_tensors);
  memcpy(m->t, tensors, sizeof(or_weight) * (size_t)n_tensors);
  m->half_kv = half_kv;
  m->capacity = capacity;
  int d = c->hidden_size, h = c->intermediate_size, L = c->num_hidden_layers;
  int kv = d / c->num_attention_heads * c->num_key_value_heads;
  m->x = calloc((size_t)d, 4); m->norm = calloc((size_t)d, 4); m->att_out = calloc((size_t)d, 4);
  m->proj = calloc((size_t)d, 4); m->gate = calloc((size_t)h, 4); m->up = calloc((size_t)h, 4);
  m->q = calloc((size_t)d, 4); m->k = calloc((size_t)kv, 4); m->v = calloc((size_t)kv, 4);
  m->att = calloc((size_t)capacity * (size_t)c->num_attention_heads, 4);
  m->trace = calloc((size_t)L * (size_t)d, 4);
  size_t kvn = (size_t)capacity * (size_t)kv;
  if (half_kv) {
    m->keys16 = calloc((size_t)L, sizeof(uint16_t *)); m->values16 = calloc((size_t)L, sizeof(uint16_t *));
    for (int l = 0; l < L; l++) { m->keys16[l] = calloc(kvn, 2); m->values16[l] = calloc(kvn, 2); }
  } else {
    m->keys = calloc((size_t)L, sizeof(float *)); m->values = calloc((size_t)L, sizeof(float *));
    for (int l = 0; l < L; l++) { m->keys[l] = calloc(kvn, 4); m->values[l] = calloc(kvn, 4); }
  }
  return m;
}

void or_stablelm_destroy(or_stablelm *m) {
  if (!m) return;
  for (int l = 0; l < m->c.num_hidden_layers; l++) {
    if (m->half_kv) { free(m->keys16[l]); free(m->values16[l]); }
    else { free(m->keys[l]); free(m->values[l]); }
  }
  free(m->keys); free(m->values); free(m->keys16); free(m->values16);
  free(m->x); free(m->norm); free(m->att_out); free(m->proj); free(m->gate); free(m->up);
  free(m->q); free(m->k); free(m->v); free(m->att); free(m->trace); free(m->t);
  free(m);
}

void or_stablelm_trace(or_stablelm *m, int enable) { m->trace_on = enable; }
const float *or_stablelm_trace_data(or_stablelm *m) { return m->trace; }

/* storeKV, kv_cache.go:55-65. */
static void store_kv(or_stablelm *m, int l, int64_t offset, const float *key, const float *value, int n) {
  if (!m->half_kv) {
    memcpy(m->keys[l] + offset, key, (size_t)n * 4);
    memcpy(m->values[l] + offset, value, (size_t)n * 4);
    return;
  }
  for (int i = 0; i < n; i++) {
    m->keys16[l][offset + i] = or_float_half(key[i]);
    m->values16[l][offset + i] = or_float_half(value[i]);
  }
}

/* KV element read; fp16 storage expands with halfFloat exactly as
 * prepareKV does (kv_cache.go:71-86). */
static inline float kv_key(const or_stablelm *m, int l, int64_t i) {
  return m->half_kv ? or_half_float(m->keys16[l][i]) : m->keys[l][i];
}
static inline float kv_value(const or_stablelm *m, int l, int64_t i) {
  return m->half_kv ? or_half_float(m->values16[l][i]) : m->values[l][i];
}

int or_stablelm_read_kv(or_stablelm *m, int l, int h, int n, float *keys, float *values) {
  int head = m->c.hidden_size / m->c.num_attention_heads;
  int64_t base = (int64_t)h * m->capacity * head;
  for (int64_t i = 0; i < (int64_t)n * head; i++) {
    keys[i] = kv_key(m, l, base + i);
    values[i] = kv_value(m, l, base + i);
  }
  return 0;
}

/* attendHeads, stablelm.go:401-427, for query heads [start,end) at pos,
 * reading q from qv and writing out; att is per-head score scratch. */
static void attend_heads(const or_stablelm *m, int l, int pos, const float *qv, float *out,
                         float *att, int start, int end) {
  const or_stablelm_config *c = &m->c;
  int head = c->hidden_size / c->num_attention_heads;
  int group = c->num_attention_heads / c->num_key_value_heads;
  int cap = m->capacity;
  float scale = (float)sqrt((double)head); /* attentionScale, stablelm.go:431 */
  float kbuf[512];
  for (int h = start; h < end; h++) {
    float *a = att + (int64_t)h * cap;
    const float *q = qv + h * head;
    int64_t offset = (int64_t)(h / group) * cap * head;
    for (int t = 0; t <= pos; t++) {
      for (int i = 0; i < head; i++) kbuf[i] = kv_key(m, l, offset + (int64_t)t * head + i);
      float score = or_attention_dot(q, kbuf, head);
      a[t] = score / scale;
    }
    or_softmax(a, pos + 1);
    float *o = out + h * head;
    memset(o, 0, (size_t)head * 4);
    for (int t = 0; t <= pos; t++) { /* attentionAdd, dot_scalar.go:33-37 */
      float score = a[t];
      for (int i = 0; i < head; i++) o[i] += score * kv_value(m, l, offset + (int64_t)t * head + i);
    }
  }
}

static void attend(const or_stablelm *m, int l, int pos, const float *qv, float *out, float *att) {
  int heads = m->c.num_attention_heads;
  int workers = g_threads < heads ? g_threads : heads;
#pragma omp parallel for num_threads(workers) schedule(static, 1)
  for (int w = 0; w < workers; w++)
    attend_heads(m, l, pos, qv, out, att, heads * w / workers, heads * (w + 1) / workers);
}

/* SiLU-gate, stablelm.go:371-373. */
static void silu_gate(float *gate, const float *up, int n) {
  for (int i = 0; i < n; i++) {
    float v = gate[i];
    float e = (float)exp(-(double)v);
    float den = 1 + e;
    float s = v / den;
    gate[i] = s * up[i];
  }
}

/* forward, stablelm.go:332-387: one token at absolute position pos. */
int or_stablelm_forward(or_stablelm *m, int token, int pos, int want_logits, float *logits) {
  const or_stablelm_config *c = &m->c;
  int d = c->hidden_size, head = d / c->num_attention_heads;
  int rotary = (int)((double)head * c->partial_rotary_factor);
  int cap = m->capacity;
  if (pos < 0 || pos >= cap || token < 0 || token >= c->vocab_size) return -1;
  or_read_values(&m->t[0], (int64_t)token * d, d, m->x);
  for (int l = 0; l < c->num_hidden_layers; l++) {
    or_layer_norm(m->norm, m->x, d, layer_t(m, l, 0), layer_t(m, l, 1), c->layer_norm_eps);
    or_mul(layer_t(m, l, 2), m->norm, m->q);
    or_mul(layer_t(m, l, 3), m->norm, m->k);
    or_mul(layer_t(m, l, 4), m->norm, m->v);
    or_stable_rotate(m->q, d, head, rotary, pos, c->rope_theta);
    or_stable_rotate(m->k, head * c->num_key_value_heads, head, rotary, pos, c->rope_theta);
    for (int h = 0; h < c->num_key_value_heads; h++) {
      int64_t offset = ((int64_t)h * cap + pos) * head;
      store_kv(m, l, offset, m->k + h * head, m->v + h * head, head);
    }
    attend(m, l, pos, m->q, m->att_out, m->att);
    or_mul(layer_t(m, l, 5), m->att_out, m->proj);
    or_mul(layer_t(m, l, 6), m->norm, m->gate);
    or_mul(layer_t(m, l, 7), m->norm, m->up);
    silu_gate(m->gate, m->up, c->intermediate_size);
    or_mul(layer_t(m, l, 8), m->gate, m->att_out);
    for (int i = 0; i < d; i++) {
      float t = m->x[i] + m->proj[i];
      m->x[i] = t + m->att_out[i];
    }
    if (m->trace_on) memcpy(m->trace + (int64_t)l * d, m->x, (size_t)d * 4);
  }
  if (want_logits) {
    or_layer_norm(m->norm, m->x, d, &m->t[2], &m->t[3], c->layer_norm_eps);
    or_mul(&m->t[1], m->norm, logits);
  }
  return 0;
}

/* prefill, prefill.go:33-115: chunks of prefillBatch=128 (matmul.go:8); a
 * one-token chunk goes through forward; logits from the last row only. */
int or_stablelm_prefill(or_stablelm *m, const int32_t *ids, int count, int start, float *logits) {
  const or_stablelm_config *c = &m->c;
  int d = c->hidden_size, hsz = c->intermediate_size, head = d / c->num_attention_heads;
  int kvh = c->num_key_value_heads, kv = head * kvh;
  int rotary = (int)((double)head * c->partial_rotary_factor);
  int cap = m->capacity;
  if (count == 0) return 0;
  if (start < 0 || start + count > cap) return -1;
  for (int i = 0; i < count; i++)
    if (ids[i] < 0 || ids[i] >= c->vocab_size) return -1;
  const int B = 128;
  float *x = malloc((size_t)B * d * 4), *norm = malloc((size_t)B * d * 4), *att_out = malloc((size_t)B * d * 4);
  float *proj = malloc((size_t)B * d * 4), *gate = malloc((size_t)B * hsz * 4), *up = malloc((size_t)B * hsz * 4);
  float *q = malloc((size_t)B * d * 4), *k = malloc((size_t)B * kv * 4), *v = malloc((size_t)B * kv * 4);
  int rc = 0;
  for (int offset = 0; offset < count; offset += B) {
    int n = count - offset < B ? count - offset : B;
    if (n == 1) {
      rc = or_stablelm_forward(m, ids[offset], start + offset, offset + n == count, logits);
      if (rc) break;
      continue;
    }
    for (int j = 0; j < n; j++) or_read_values(&m->t[0], (int64_t)ids[offset + j] * d, d, x + (int64_t)j * d);
    for (int l = 0; l < c->num_hidden_layers; l++) {
      for (int j = 0; j < n; j++)
        or_layer_norm(norm + (int64_t)j * d, x + (int64_t)j * d, d, layer_t(m, l, 0), layer_t(m, l, 1), c->layer_norm_eps);
      or_mul_batch(layer_t(m, l, 2), norm, n, q);
      or_mul_batch(layer_t(m, l, 3), norm, n, k);
      or_mul_batch(layer_t(m, l, 4), norm, n, v);
      for (int j = 0; j < n; j++) {
        or_stable_rotate(q + (int64_t)j * d, d, head, rotary, start + offset + j, c->rope_theta);
        or_stable_rotate(k + (int64_t)j * kv, kv, head, rotary, start + offset + j, c->rope_theta);
      }
      for (int j = 0; j < n; j++)
        for (int kh = 0; kh < kvh; kh++) {
          int64_t at = ((int64_t)kh * cap + start + offset + j) * head;
          store_kv(m, l, at, k + (int64_t)j * kv + kh * head, v + (int64_t)j * kv + kh * head, head);
        }
      /* attendBatch in the scalar build (attentionBatchWidth 1,
       * attention_scalar.go:7) evaluates every query with attendHeads. */
      {
        int heads = c->num_attention_heads;
        int tasks = n * heads;
        int workers = g_threads < tasks ? g_threads : tasks;
#pragma omp parallel num_threads(workers)
        {
          float *att = malloc((size_t)cap * heads * 4);
#pragma omp for schedule(static)
          for (int task = 0; task < tasks; task++) {
            int h = task / n, j = task % n;
            attend_heads(m, l, start + offset + j, q + (int64_t)j * d, att_out + (int64_t)j * d, att, h, h + 1);
          }
          free(att);
        }
      }
      or_mul_batch(layer_t(m, l, 5), att_out, n, proj);
      or_mul_batch(layer_t(m, l, 6), norm, n, gate);
      or_mul_batch(layer_t(m, l, 7), norm, n, up);
      silu_gate(gate, up, n * hsz);
      or_mul_batch(layer_t(m, l, 8), gate, n, att_out);
      for (int64_t i = 0; i < (int64_t)n * d; i++) {
        float t = x[i] + proj[i];
        x[i] = t + att_out[i];
      }
      if (m->trace_on) memcpy(m->trace + (int64_t)l * d, x + (int64_t)(n - 1) * d, (size_t)d * 4);
    }
    if (offset + n == count) {
      memcpy(m->x, x + (int64_t)(n - 1) * d, (size_t)d * 4);
      or_layer_norm(m->norm, m->x, d, &m->t[2], &m->t[3], c->layer_norm_eps);
      or_mul(&m->t[1], m->norm, logits);
    }
  }
  free(x); free(norm); free(att_out); free(proj); free(gate); free(up); free(q); free(k); free(v);
  return rc;
}

/* ===================== legacy Llama engine ===================== */

struct or_llama {
  or_llama_config c;
  const float *emb, *rms_att, *wq, *wk, *wv, *wo, *rms_ffn, *w1, *w2, *w3, *rms_final, *fcr, *fci;
  float *x, *xb, *xb2, *hb, *hb2, *q, *k, *v, *att, *key_cache, *value_cache;
};

/* readWeights order, model.go:129-166. */
or_llama *or_llama_create(const or_llama_config *c, const float *w, size_t n_floats) {
  int64_t dim = c->dim, hidden = c->hidden_dim, L = c->n_layers, vocab = c->vocab_size, seq = c->seq_len;
  int64_t hs = dim / c->n_heads, kv_dim = hs * c->n_kv_heads;
  int64_t need = vocab * dim + L * dim + L * dim * dim + 2 * L * dim * kv_dim + L * dim * dim + L * dim +
                 3 * L * hidden * dim + dim + seq * hs;
  if ((int64_t)n_floats != need) return NULL;
  or_llama *m = calloc(1, sizeof(*m));
  m->c = *c;
  const float *p = w;
  m->emb = p; p += vocab * dim;
  m->rms_att = p; p += L * dim;
  m->wq = p; p += L * dim * dim;
  m->wk = p; p += L * dim * kv_dim;
  m->wv = p; p += L * dim * kv_dim;
  m->wo = p; p += L * dim * dim;
  m->rms_ffn = p; p += L * dim;
  m->w1 = p; p += L * hidden * dim;
  m->w2 = p; p += L * dim * hidden;
  m->w3 = p; p += L * hidden * dim;
  m->rms_final = p; p += dim;
  m->fcr = p; p += seq * hs / 2;
  m->fci = p;
  m->x = calloc((size_t)dim, 4); m->xb = calloc((size_t)dim, 4); m->xb2 = calloc((size_t)dim, 4);
  m->hb = calloc((size_t)hidden, 4); m->hb2 = calloc((size_t)hidden, 4);
  m->q = calloc((size_t)dim, 4); m->k = calloc((size_t)kv_dim, 4); m->v = calloc((size_t)kv_dim, 4);
  m->att = calloc((size_t)seq, 4);
  m->key_cache = calloc((size_t)(L * seq * kv_dim), 4);
  m->value_cache = calloc((size_t)(L * seq * kv_dim), 4);
  return m;
}

void or_llama_destroy(or_llama *m) {
  if (!m) return;
  free(m->x); free(m->xb); free(m->xb2); free(m->hb); free(m->hb2); free(m->q); free(m->k);
  free(m->v); free(m->att); free(m->key_cache); free(m->value_cache); free(m);
}

/* matmul, model.go:575-586: sequential float32. */
static void llama_matmul(float *xout, const float *x, const float *w, int n, int d) {
  for (int i = 0; i < d; i++) {
    float val = 0;
    const float *row = w + (int64_t)i * n;
    for (int j = 0; j < n; j++) val += row[j] * x[j];
    xout[i] = val;
  }
}

/* rmsNorm, model.go:591-600. */
static void llama_rmsnorm(float *dest, const float *src, const float *weight, int n) {
  float ss = 0;
  for (int i = 0; i < n; i++) ss += src[i] * src[i];
  float mean = ss / (float)n + 1e-5f;
  float inv = 1.0f / (float)sqrt((double)mean);
  for (int i = 0; i < n; i++) {
    float t = inv * src[i];
    dest[i] = weight[i] * t;
  }
}

/* rotateHead, model.go:611-618. */
static void llama_rotate(float *vec, const float *fr, const float *fi, int hs) {
  for (int i = 0; i < hs; i += 2) {
    float v0 = vec[i], v1 = vec[i + 1], fcr = fr[i / 2], fci = fi[i / 2];
    float a = v0 * fcr, b = v1 * fci, c2 = v0 * fci, d2 = v1 * fcr;
    vec[i] = a - b;
    vec[i + 1] = c2 + d2;
  }
}

/* transformer, model.go:407-481. */
int or_llama_transformer(or_llama *m, int token, int pos, float *logits) {
  const or_llama_config *p = &m->c;
  int dim = p->dim, hidden = p->hidden_dim, hs = dim / p->n_heads;
  int kv_dim = hs * p->n_kv_heads, kv_mul = p->n_heads / p->n_kv_heads;
  if (token < 0 || token >= p->vocab_size || pos < 0 || pos >= p->seq_len) return -1;
  float *x = m->x;
  memcpy(x, m->emb + (int64_t)token * dim, (size_t)dim * 4);
  const float *fr = m->fcr + (int64_t)pos * hs / 2, *fi = m->fci + (int64_t)pos * hs / 2;
  float scale = (float)sqrt((double)hs);
  for (int l = 0; l < p->n_layers; l++) {
    llama_rmsnorm(m->xb, x, m->rms_att + (int64_t)l * dim, dim);
    llama_matmul(m->q, m->xb, m->wq + (int64_t)l * dim * dim, dim, dim);
    llama_matmul(m->k, m->xb, m->wk + (int64_t)l * dim * kv_dim, dim, kv_dim);
    llama_matmul(m->v, m->xb, m->wv + (int64_t)l * dim * kv_dim, dim, kv_dim);
    for (int h = 0; h < p->n_heads; h++) llama_rotate(m->q + h * hs, fr, fi, hs);
    for (int h = 0; h < p->n_kv_heads; h++) llama_rotate(m->k + h * hs, fr, fi, hs);
    int64_t loff = (int64_t)l * p->seq_len * kv_dim;
    memcpy(m->key_cache + loff + (int64_t)pos * kv_dim, m->k, (size_t)kv_dim * 4);
    memcpy(m->value_cache + loff + (int64_t)pos * kv_dim, m->v, (size_t)kv_dim * 4);
    for (int h = 0; h < p->n_heads; h++) {
      const float *q = m->q + h * hs;
      int kv_off = (h / kv_mul) * hs;
      for (int t = 0; t <= pos; t++) {
        const float *k = m->key_cache + loff + (int64_t)t * kv_dim + kv_off;
        float score = 0;
        for (int i = 0; i < hs; i++) score += q[i] * k[i];
        m->att[t] = score / scale;
      }
      or_softmax(m->att, pos + 1);
      for (int i = 0; i < hs; i++) {
        float val = 0;
        for (int t = 0; t <= pos; t++) val += m->att[t] * m->value_cache[loff + (int64_t)t * kv_dim + kv_off + i];
        m->xb[h * hs + i] = val;
      }
    }
    llama_matmul(m->xb2, m->xb, m->wo + (int64_t)l * dim * dim, dim, dim);
    for (int i = 0; i < dim; i++) x[i] += m->xb2[i];
    llama_rmsnorm(m->xb, x, m->rms_ffn + (int64_t)l * dim, dim);
    llama_matmul(m->hb, m->xb, m->w1 + (int64_t)l * dim * hidden, dim, hidden);
    llama_matmul(m->hb2, m->xb, m->w3 + (int64_t)l * dim * hidden, dim, hidden);
    for (int i = 0; i < hidden; i++) {
      float e = (float)exp(-(double)m->hb[i]);
      float den = 1.0f + e;
      float s = 1.0f / den;
      m->hb[i] = m->hb[i] * s;
      m->hb[i] = m->hb[i] * m->hb2[i];
    }
    llama_matmul(m->xb, m->hb, m->w2 + (int64_t)l * dim * hidden, hidden, dim);
    for (int i = 0; i < dim; i++) x[i] += m->xb[i];
  }
  llama_rmsnorm(x, x, m->rms_final, dim);
  llama_matmul(logits, x, m->emb, dim, p->vocab_size);
  return 0;
}
