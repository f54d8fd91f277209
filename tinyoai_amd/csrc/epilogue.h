// Device helpers shared by the decode kernels and the prefill epilogue:
// the in-projection epilogue (a row pair of the fused win matrix becomes
// RoPE'd q, a K/V cache entry, or a SiLU-gate output) and KV loads.
#pragma once

#include "kernels.h"

// Stores seen by other blocks of the same launch: with COH, agent-scope
// relaxed atomic stores (coherent across the XCDs' L2 caches), else plain.
template <bool COH, typename V>
__device__ __forceinline__ void put(V *p, V v) {
  if constexpr (COH)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *p = v;
}

// The layer's input normalisation of an LDS-resident row (all threads).
__device__ __forceinline__ void norm_lds(const StableDims &s, float *x, const float *w, const float *b,
                                         double *red) {
  if (s.norm) rms_norm_lds(x, s.d, w, (float)s.eps, red);
  else layer_norm_lds(x, s.d, w, b, s.eps, red);
}

// Row pair (2u, 2u + 1) of win with dot products v0, v1 for one token at
// absolute position pos. rope_row holds cos/sin of pos as [rot/2][2]. The
// outputs go through `out`: out.f32(float *, float) and, for an fp16 KV
// cache, out.f16(uint16_t *, uint16_t).
template <typename Out>
__device__ __forceinline__ void in_pair_outputs(const StableDims &s, const KVDev &kv, const float *rope_row, int pos,
                                                int u, float v0, float v1, float *q_out, float *m_out, Out &&out) {
  const int row = 2 * u, kvw = s.win_kv, rh = s.rot / 2;
  if (row >= s.win_q + 2 * kvw) {
    const int i = (row - s.win_q - 2 * kvw) >> 1;
    out.f32(m_out + i, s.silu ? silu_gate_llama(v0, v1) : silu_gate(v0, v1));
    return;
  }
  int sec, r;  // 0 q, 1 k, 2 v
  if (row < s.win_q) { sec = 0; r = row; }
  else if (row < s.win_q + kvw) { sec = 1; r = row - s.win_q; }
  else { sec = 2; r = row - s.win_q - kvw; }
  const int head = r / s.hd, p = r - head * s.hd;
  int d0 = p, d1 = p + 1;
  if (sec != 2 && p < s.rot) {  // rotate the pair by the table's cos/sin
    const int j = p >> 1;
    if (!s.rope_adjacent) {     // stableRotate: dims (j, j + rot/2), stored on adjacent rows
      d0 = j;
      d1 = j + rh;
    }
    const float cs = rope_row[2 * j], sn = rope_row[2 * j + 1];
    const float x0 = __fsub_rn(__fmul_rn(v0, cs), __fmul_rn(v1, sn));
    const float x1 = __fadd_rn(__fmul_rn(v1, cs), __fmul_rn(v0, sn));
    v0 = x0;
    v1 = x1;
  }
  if (sec == 0) {
    out.f32(q_out + head * s.hd + d0, v0);
    out.f32(q_out + head * s.hd + d1, v1);
  } else {  // head-major [kv_head][cap][hd] at the token's position (storeKV, kv_cache.go:55-65)
    const int64_t base = ((int64_t)head * kv.cap + pos) * s.hd;
    // The cache base as arithmetic on the two addresses: a choice between
    // the two fields made the compiler keep them in per-lane scratch memory
    // (stored by every thread at kernel start, read back per store).
    const uintptr_t ka = reinterpret_cast<uintptr_t>(kv.k), va = reinterpret_cast<uintptr_t>(kv.v);
    void *dst = reinterpret_cast<void *>(ka + (sec == 1 ? uintptr_t(0) : va - ka));
    if (kv.half) {
      out.f16(reinterpret_cast<uint16_t *>(dst) + base + d0, float_to_half(v0));
      out.f16(reinterpret_cast<uint16_t *>(dst) + base + d1, float_to_half(v1));
    } else {
      out.f32(reinterpret_cast<float *>(dst) + base + d0, v0);
      out.f32(reinterpret_cast<float *>(dst) + base + d1, v1);
    }
  }
}

// The same outputs stored directly (plain, or with COH agent-scope atomic
// stores).
template <bool COH>
struct DirectStores {
  __device__ void f32(float *p, float v) const { put<COH>(p, v); }
  __device__ void f16(uint16_t *p, uint16_t v) const { put<COH>(p, v); }
};

template <bool COH = false>
__device__ __forceinline__ void in_pair_epilogue(const StableDims &s, const KVDev &kv, const float *rope_row, int pos,
                                                 int u, float v0, float v1, float *q_out, float *m_out) {
  in_pair_outputs(s, kv, rope_row, pos, u, v0, v1, q_out, m_out, DirectStores<COH>{});
}

// Loads N consecutive KV values starting at element e into float registers.
template <int N, bool HALF>
__device__ __forceinline__ void load_kv(const void *base, int64_t e, float *r) {
  if constexpr (HALF) {
    const uint16_t *p = reinterpret_cast<const uint16_t *>(base) + e;
    if constexpr (N % 4 == 0) {
#pragma unroll
      for (int i = 0; i < N / 4; i++) {
        const uint2 v = reinterpret_cast<const uint2 *>(p)[i];
        r[4 * i] = hw_half((uint16_t)v.x);
        r[4 * i + 1] = hw_half((uint16_t)(v.x >> 16));
        r[4 * i + 2] = hw_half((uint16_t)v.y);
        r[4 * i + 3] = hw_half((uint16_t)(v.y >> 16));
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; i++) r[i] = hw_half(p[i]);
    }
  } else {
    const float *p = reinterpret_cast<const float *>(base) + e;
    if constexpr (N % 4 == 0) {
#pragma unroll
      for (int i = 0; i < N / 4; i++) {
        const float4 v = reinterpret_cast<const float4 *>(p)[i];
        r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
      }
    } else if constexpr (N % 2 == 0) {
#pragma unroll
      for (int i = 0; i < N / 2; i++) {
        const float2 v = reinterpret_cast<const float2 *>(p)[i];
        r[2 * i] = v.x; r[2 * i + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; i++) r[i] = p[i];
    }
  }
}

// The same with agent-scope atomic loads, for a KV entry written earlier in
// the same launch by another block.
template <int N, bool HALF>
__device__ __forceinline__ void load_kv_coherent(const void *base, int64_t e, float *r) {
  if constexpr (HALF) {
    uint16_t *p = const_cast<uint16_t *>(reinterpret_cast<const uint16_t *>(base)) + e;
#pragma unroll
    for (int i = 0; i < N; i++) r[i] = hw_half(__hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  } else {
    float *p = const_cast<float *>(reinterpret_cast<const float *>(base)) + e;
#pragma unroll
    for (int i = 0; i < N; i++) r[i] = __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
