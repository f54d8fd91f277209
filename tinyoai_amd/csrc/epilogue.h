// The in-projection epilogue shared by decode (one token, fused into the
// matvec) and prefill (after the matrix-core product): a row pair of the
// fused win matrix becomes RoPE'd q, a K/V cache entry, or a SiLU-gate
// output.
#pragma once

#include "kernels.h"

// storeKV (kv_cache.go:55-65): fp32 copy, or floatHalf rounding.
__device__ __forceinline__ void kv_put(const KVDev &kv, bool key, int64_t idx, float v) {
  void *base = key ? kv.k : kv.v;
  if (kv.half)
    reinterpret_cast<uint16_t *>(base)[idx] = float_to_half(v);
  else
    reinterpret_cast<float *>(base)[idx] = v;
}

// Row pair (2u, 2u + 1) of win with dot products v0, v1 for one token at
// absolute position pos. rope_row holds cos/sin of pos as [rot/2][2].
__device__ __forceinline__ void in_pair_epilogue(const StableDims &s, const KVDev &kv, const float *rope_row, int pos,
                                                 int u, float v0, float v1, float *q_out, float *m_out) {
  const int row = 2 * u, kvw = s.kv_heads * s.hd, rh = s.rot / 2;
  if (row >= s.d + 2 * kvw) {
    m_out[(row - s.d - 2 * kvw) >> 1] = silu_gate(v0, v1);  // stablelm.go:371-373
    return;
  }
  int sec, r;  // 0 q, 1 k, 2 v
  if (row < s.d) { sec = 0; r = row; }
  else if (row < s.d + kvw) { sec = 1; r = row - s.d; }
  else { sec = 2; r = row - s.d - kvw; }
  const int head = r / s.hd, p = r - head * s.hd;
  int d0 = p, d1 = p + 1;
  if (sec != 2 && p < s.rot) {  // stableRotate (stablelm.go:309-326) on dims (j, j + rot/2)
    const int j = p >> 1;
    d0 = j;
    d1 = j + rh;
    const float cs = rope_row[2 * j], sn = rope_row[2 * j + 1];
    const float x0 = __fsub_rn(__fmul_rn(v0, cs), __fmul_rn(v1, sn));
    const float x1 = __fadd_rn(__fmul_rn(v1, cs), __fmul_rn(v0, sn));
    v0 = x0;
    v1 = x1;
  }
  if (sec == 0) {
    q_out[head * s.hd + d0] = v0;
    q_out[head * s.hd + d1] = v1;
  } else {  // head-major [kv_head][cap][hd] at the token's position
    const int64_t base = ((int64_t)head * kv.cap + pos) * s.hd;
    kv_put(kv, sec == 1, base + d0, v0);
    kv_put(kv, sec == 1, base + d1, v1);
  }
}
