// Launch interfaces of the gfx950 kernels. Host code (the model handles and
// the C ABI) calls only these; each returns hipSuccess or the launch error.
#pragma once

#include <hip/hip_runtime.h>

#include "formats.h"

// Per-layer weights of a StableLM block on the device (stablelm.go:113-117).
struct LayerDev {
  MatDesc q, k, v, o, gate, up, down;
  const float *ln_w, *ln_b;
};

// Shapes and constants shared by the StableLM kernels.
struct StableDims {
  int d, hd, rot, heads, kv_heads, inter, vocab;
  double eps;
  float att_scale;  // float32(sqrt(hd)), attentionScale (stablelm.go:431)
};

// KV cache of one layer: [kv_heads][cap][hd], fp32 or fp16 bits.
struct KVDev {
  void *k, *v;
  int cap;
  int half;  // 1 = fp16 storage (floatHalf rounding), 0 = fp32
};

// ---- decode (one token) ----
// Matvec launches take their grid and block size (256, 512, 640 or 1024
// threads) from the caller; blocks loop over their share of the rows.
// LayerNorm(x) -> q/k/v/gate/up with RoPE, KV append and SiLU-gate fused
// into the epilogue. pos (and token) are read from device memory. With
// `emb` (a host-side descriptor, copied), x is first set to the embedding
// row of *token (layer 0).
hipError_t launch_decode_in(const LayerDev &w, const StableDims &s, const KVDev &kv, float *x, const MatDesc *emb,
                            const int *token, const float *rope, const int *pos, float *q_out, float *m_out,
                            int grid, int threads, hipStream_t st);
// x += o * a + down * m (stablelm.go:365-377).
hipError_t launch_decode_out(const LayerDev &w, const StableDims &s, const float *a, const float *m,
                             float *x, int grid, int threads, hipStream_t st);
// Split-K flash decode with in-kernel combine for nq queries at positions
// pos0 + j (j < nq): q [nq][heads*hd] -> out [nq][heads*hd]. A block covers
// 64 * steps positions; `splits` blocks per (query, head) must cover
// max_pos + 1 positions (<= 0: derived from max_pos). partials holds
// nq * heads * splits * (hd + 2) floats; counters (nq * heads) start at 0
// and are left at 0.
hipError_t launch_attention(const StableDims &s, const KVDev &kv, const float *q, const int *pos0, int nq,
                            int max_pos, float *partials, unsigned *counters, float *out, hipStream_t st,
                            int steps = 0, int splits = 0);
int attention_steps(int max_pos, int heads);
int attention_splits(int max_pos, int steps);
// out[rows] = W * LN(x) (LN skipped when ln_w is null), for the logits head
// and single-matrix products.
hipError_t launch_ln_matvec(const MatDesc &w, const float *ln_w, const float *ln_b, double eps,
                            const float *x, float *out, int grid, int threads, hipStream_t st);
// x[n][cols] = rows ids[j] of an embedding matrix, bit-exact dequantized.
hipError_t launch_embed(const MatDesc &emb, const int *ids, int n, float *x, hipStream_t st);

// ---- prefill (n tokens) ----
hipError_t launch_layer_norm_rows(const float *x, const float *w, const float *b, double eps, int n, int d,
                                  float *out, hipStream_t st);
// out[n][rows] = x[n][cols] * W^T.
hipError_t launch_gemm(const MatDesc &w, const float *x, int n, float *out, hipStream_t st);
// RoPE on q [n][heads*hd] (in place) and k; writes k, v into the cache at
// positions pos0 + j.
hipError_t launch_rope_store(const StableDims &s, const KVDev &kv, float *q, const float *k, const float *v,
                             const float *rope, const int *pos0, int n, hipStream_t st);
hipError_t launch_silu_gate(float *g, const float *u, int64_t n, hipStream_t st);
// x = (x + p) + d elementwise (stablelm.go:375-377).
hipError_t launch_residual(float *x, const float *p, const float *d, int64_t n, hipStream_t st);
hipError_t launch_copy_row(const float *src, float *dst, int n, hipStream_t st);

// ---- weights ----
// Splits raw GGUF-encoded bytes (already in device memory) into planes.
hipError_t launch_repack(int fmt, const uint8_t *raw, int64_t rows, int64_t cols, const MatDesc &dst,
                         hipStream_t st);
hipError_t launch_read_values(const MatDesc &m, int64_t offset, int64_t n, float *out, hipStream_t st);

int device_cu_count();
