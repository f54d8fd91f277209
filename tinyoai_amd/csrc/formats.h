// Weight formats as laid out in HBM, and the per-format arithmetic the
// kernels share.
//
// On upload every matrix is split into two planes:
//   vals: the per-value payload, each row padded to a multiple of 16 bytes,
//         so a lane streams a row with 128-bit loads (a "chunk");
//   meta: per-block metadata (Q8_0: one fp16 scale per 32 values).
// F32 / F16 / BF16 keep row-major values; Q8_0 keeps its int8 quants in
// `vals` and its fp16 block scales in `meta`. The bytes are those of the
// GGUF block {fp16 d, int8 q[32]} (dot.go:31-40), only regrouped.
#pragma once

#include <hip/hip_fp16.h>

#include "device.h"

enum : int32_t {
  FMT_F32 = 0, FMT_F16 = 1, FMT_Q5_1 = 7, FMT_Q8_0 = 8,
  FMT_Q4_K = 12, FMT_Q5_K = 13, FMT_Q6_K = 14, FMT_BF16 = 30
};

struct MatDesc {
  const uint8_t *vals;  // [rows][vstride] bytes
  const uint8_t *meta;  // [rows][mstride] bytes (Q8_0: fp16 scales)
  int64_t vstride;      // bytes per row in vals (multiple of 16)
  int64_t mstride;      // bytes per row in meta
  int32_t rows, cols;   // logical shape [out, in]
  int32_t fmt;
  int32_t chunks;       // 16-byte chunks per row = vstride / 16
};

template <int F> struct Fmt;
template <> struct Fmt<FMT_Q8_0> { static constexpr int VPC = 16; };
template <> struct Fmt<FMT_BF16> { static constexpr int VPC = 8; };
template <> struct Fmt<FMT_F16> { static constexpr int VPC = 8; };
template <> struct Fmt<FMT_F32> { static constexpr int VPC = 4; };

// Values held by one 16-byte chunk of `vals`.
__host__ __device__ inline int values_per_chunk(int fmt) {
  switch (fmt) {
    case FMT_Q8_0: return 16;
    case FMT_BF16: case FMT_F16: return 8;
    default: return 4;
  }
}

__device__ __forceinline__ float hw_half(uint16_t h) {
  return __half2float(__ushort_as_half(h));  // v_cvt_f32_f16: exact, keeps subnormals
}

// Dot product of one 16-byte chunk with the matching x values (LDS, 16-byte
// aligned), fp32 with fused multiply-adds. Q8_0 returns the unscaled sum.
template <int F>
__device__ __forceinline__ float chunk_dot(const uint4 w, const float *x);

template <>
__device__ __forceinline__ float chunk_dot<FMT_Q8_0>(const uint4 w, const float *x) {
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float4 xv = x4[k];
    const uint32_t v = ws[k];
    a = fmaf((float)(int8_t)(v), xv.x, a);
    b = fmaf((float)(int8_t)(v >> 8), xv.y, b);
    a = fmaf((float)(int8_t)(v >> 16), xv.z, a);
    b = fmaf((float)(int8_t)(v >> 24), xv.w, b);
  }
  return a + b;
}

template <>
__device__ __forceinline__ float chunk_dot<FMT_BF16>(const uint4 w, const float *x) {
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const float4 x0 = x4[0], x1 = x4[1];
  float a = __uint_as_float(w.x << 16) * x0.x;
  float b = __uint_as_float(w.x & 0xffff0000u) * x0.y;
  a = fmaf(__uint_as_float(w.y << 16), x0.z, a);
  b = fmaf(__uint_as_float(w.y & 0xffff0000u), x0.w, b);
  a = fmaf(__uint_as_float(w.z << 16), x1.x, a);
  b = fmaf(__uint_as_float(w.z & 0xffff0000u), x1.y, b);
  a = fmaf(__uint_as_float(w.w << 16), x1.z, a);
  b = fmaf(__uint_as_float(w.w & 0xffff0000u), x1.w, b);
  return a + b;
}

template <>
__device__ __forceinline__ float chunk_dot<FMT_F16>(const uint4 w, const float *x) {
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const float4 x0 = x4[0], x1 = x4[1];
  float a = hw_half((uint16_t)w.x) * x0.x;
  float b = hw_half((uint16_t)(w.x >> 16)) * x0.y;
  a = fmaf(hw_half((uint16_t)w.y), x0.z, a);
  b = fmaf(hw_half((uint16_t)(w.y >> 16)), x0.w, b);
  a = fmaf(hw_half((uint16_t)w.z), x1.x, a);
  b = fmaf(hw_half((uint16_t)(w.z >> 16)), x1.y, b);
  a = fmaf(hw_half((uint16_t)w.w), x1.z, a);
  b = fmaf(hw_half((uint16_t)(w.w >> 16)), x1.w, b);
  return a + b;
}

template <>
__device__ __forceinline__ float chunk_dot<FMT_F32>(const uint4 w, const float *x) {
  const float4 xv = *reinterpret_cast<const float4 *>(x);
  float a = __uint_as_float(w.x) * xv.x;
  float b = __uint_as_float(w.y) * xv.y;
  a = fmaf(__uint_as_float(w.z), xv.z, a);
  b = fmaf(__uint_as_float(w.w), xv.w, b);
  return a + b;
}

// Scale applied to a chunk's partial sum (Q8_0 block scale; 1 otherwise).
template <int F>
__device__ __forceinline__ float chunk_scale(const uint8_t *meta_row, int c) {
  if constexpr (F == FMT_Q8_0) {
    return hw_half(reinterpret_cast<const uint16_t *>(meta_row)[c >> 1]);
  } else {
    return 1.0f;
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// One 16-byte chunk of a weight row, streamed past the caches (each weight
// byte is read once per token).
__device__ __forceinline__ uint4 load_chunk(const uint8_t *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Wave-cooperative dot products of two row segments with LDS-resident
// vectors: segment 0 (row p0, vector x0, n0 chunks) and segment 1 (row p1,
// x1, n1 chunks), streamed as one chunk sequence so each lane keeps U loads
// in flight. Results are reduced across the wave (every lane gets them).
template <int F, int U>
__device__ __forceinline__ void seg2_dot(const uint8_t *__restrict__ v0, const uint8_t *__restrict__ m0,
                                         const float *x0, int n0,
                                         const uint8_t *__restrict__ v1, const uint8_t *__restrict__ m1,
                                         const float *x1, int n1, float &out0, float &out1) {
  constexpr int VPC = Fmt<F>::VPC;
  const int lane = threadIdx.x & 63;
  const int total = n0 + n1;
  float acc0 = 0.f, acc1 = 0.f;
  for (int base = 0; base < total; base += 64 * U) {
    uint4 w[U];
    float s[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = base + u * 64 + lane;
      const bool seg1 = c >= n0;
      const int cc = seg1 ? c - n0 : c;
      if (c < total) {
        w[u] = load_chunk((seg1 ? v1 : v0) + (int64_t)cc * 16);
        s[u] = chunk_scale<F>(seg1 ? m1 : m0, cc);
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = base + u * 64 + lane;
      const bool seg1 = c >= n0;
      const int cc = seg1 ? c - n0 : c;
      if (c < total) {
        float p = chunk_dot<F>(w[u], (seg1 ? x1 : x0) + cc * VPC);
        if constexpr (F == FMT_Q8_0) p *= s[u];
        if (seg1) acc1 += p; else acc0 += p;
      }
    }
  }
  out0 = wave_sum(acc0);
  out1 = wave_sum(acc1);
}

// Bit-exact value at (row, col): readValues (matmul.go:12-50) on the
// repacked planes.
__device__ __forceinline__ float mat_value(const MatDesc &m, int64_t row, int64_t col) {
  const uint8_t *vr = m.vals + row * m.vstride;
  switch (m.fmt) {
    case FMT_Q8_0: {
      const uint16_t d = reinterpret_cast<const uint16_t *>(m.meta + row * m.mstride)[col >> 5];
      return __fmul_rn(half_to_float(d), (float)(int8_t)vr[col]);
    }
    case FMT_BF16: return bf16_to_float(reinterpret_cast<const uint16_t *>(vr)[col]);
    case FMT_F16: return half_to_float(reinterpret_cast<const uint16_t *>(vr)[col]);
    default: return reinterpret_cast<const float *>(vr)[col];
  }
}
