// Device helpers shared by the gfx950 kernels: exact-rounding float ops,
// IEEE binary16 conversions restated bit for bit, and wave64 reductions.
//
// Every translation unit is compiled with -ffp-contract=off, so a plain
// a * b + c rounds twice. Hot reductions use fmaf() explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "expf64.h"

#define TINYOAI_WAVE 64

// halfFloat (safetensors.go:250-264): binary16 -> float32, exact for every
// pattern including subnormals, infinities and NaN payloads.
__device__ __forceinline__ float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 31u, frac = h & 1023u;
  if (exp == 0) {
    // frac * 2^-24 is exact in float32 (at most 10 significant bits).
    float v = (float)frac * 5.9604644775390625e-08f;
    return __uint_as_float(__float_as_uint(v) | sign);
  }
  if (exp == 31) return __uint_as_float(sign | 0x7f800000u | frac << 13);
  return __uint_as_float(sign | (exp + 112) << 23 | frac << 13);
}

// floatHalf (kv_cache.go:27-51): float32 -> binary16, round to nearest even.
__device__ __forceinline__ uint16_t float_to_half(float value) {
  uint32_t bits = __float_as_uint(value);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  uint32_t magnitude = bits & 0x7fffffffu;
  if (magnitude >= 0x7f800000u) return sign | (magnitude > 0x7f800000u ? 0x7e00 : 0x7c00);
  int exponent = (int)(magnitude >> 23) - 127 + 15;
  if (exponent >= 31) return sign | 0x7c00;
  if (exponent <= 0) {
    if (exponent < -10) return sign;
    uint32_t mantissa = (magnitude & 0x7fffffu) | 0x800000u;
    unsigned shift = (unsigned)(14 - exponent);
    uint32_t rounded = (mantissa + ((1u << (shift - 1)) - 1) + ((mantissa >> shift) & 1)) >> shift;
    return sign | (uint16_t)rounded;
  }
  magnitude += 0xfffu + ((magnitude >> 13) & 1u);
  return sign | (uint16_t)((magnitude >> 13) - 0x1c000u);
}

__device__ __forceinline__ float bf16_to_float(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, TINYOAI_WAVE);
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, TINYOAI_WAVE);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, TINYOAI_WAVE));
  return v;
}

// Sum over the 64 lanes of a wave as a wave-uniform value, with DPP lane
// moves instead of LDS permutes: within each 16-lane row, adjacent lanes,
// then lane pairs (quad permutes), then quads four and eight lanes apart
// (row rotations); then (row0 + row1) + (row2 + row3) from lanes 0, 16,
// 32 and 48. A fixed order, so every call on the same values gives the
// same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_total(float v) {
  v = dpp_add<0xb1>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4e>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x124>(v);  // row_ror 4
  v = dpp_add<0x128>(v);  // row_ror 8
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

// wave_total for float64: the same moves on both halves of each value.
template <int CTRL>
__device__ __forceinline__ double dpp_add_d(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, false);
  const uint32_t hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, false);
  return v + __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double lane_value_d(double v, int lane) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)b, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_total_d(double v) {
  v = dpp_add_d<0xb1>(v);
  v = dpp_add_d<0x4e>(v);
  v = dpp_add_d<0x124>(v);
  v = dpp_add_d<0x128>(v);
  return (lane_value_d(v, 0) + lane_value_d(v, 16)) + (lane_value_d(v, 32) + lane_value_d(v, 48));
}

// Block-wide sums of two float64 values per thread, the same bits in every
// thread (waves in index order). red holds 2 * waves doubles; the caller
// synchronises before reusing it. T: the block size.
template <int T>
__device__ __forceinline__ void block_sum2_d(double &a, double &b, double *red) {
  constexpr int waves = T / 64;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  a = wave_total_d(a);
  b = wave_total_d(b);
  if ((threadIdx.x & 63) == 0) {
    red[2 * wave] = a;
    red[2 * wave + 1] = b;
  }
  __syncthreads();
  a = b = 0.0;
#pragma unroll
  for (int w = 0; w < waves; w++) {
    a += red[2 * w];
    b += red[2 * w + 1];
  }
}

// The input normalisation of a row, staged in registers: norm_load issues
// the loads of a thread's float4 groups tid + j * T (j < XR4) of x and of
// the affine weights, 16 bytes per load (before a kernel issues its weight
// loads, so that waiting for them never waits for weights); norm_store
// normalises and writes the row to `out` (LDS) in one block reduction.
// Elements past 4 * XR4 * T are read from xs / w / b directly.
template <int XR4>
struct NormRegs {
  float4 x[XR4], w[XR4], b[XR4];
  float shift;  // x[0]: the float64 moments are taken about it
};

__device__ __forceinline__ float4 load4(const float *p, int i, int n) {
  if (i + 3 < n) return *reinterpret_cast<const float4 *>(p + i);
  return make_float4(i < n ? p[i] : 0.f, i + 1 < n ? p[i + 1] : 0.f, i + 2 < n ? p[i + 2] : 0.f,
                     i + 3 < n ? p[i + 3] : 0.f);
}

template <int T, int XR4>
__device__ __forceinline__ void norm_load(NormRegs<XR4> &r, const float *x, const float *w, const float *b, int n) {
  r.shift = x ? x[0] : 0.f;
#pragma unroll
  for (int j = 0; j < XR4; j++) {
    const int i = 4 * ((int)threadIdx.x + j * T);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    r.x[j] = x ? load4(x, i, n) : z;
    r.w[j] = w ? load4(w, i, n) : z;
    r.b[j] = b ? load4(b, i, n) : z;
  }
}

// kind 0: LayerNorm (stablelm.go:288-305): float64 mean and variance (here
// from moments about x[0] in one pass: the same values up to float64
// rounding), then t = x - float(mean), t *= float(1 / sqrt(var + eps)),
// t *= w, t += b, each step rounded to float32. kind 1: RMSNorm
// (model.go:591-600): ss = float32(sum of float32 squares, accumulated in
// float64), inv = 1 / float32(sqrt(ss / n + eps)), out = w * (inv * x).
// kind -1: a copy.
template <int T, int XR4>
__device__ __forceinline__ void norm_store(const NormRegs<XR4> &r, int n, int kind, double eps, const float *xs,
                                           const float *w, const float *b, float *out, double *red) {
  const int tid = threadIdx.x;
  auto vx = [&](int j, int e) { const float4 v = r.x[j]; return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; };
  auto vw = [&](int j, int e) { const float4 v = r.w[j]; return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; };
  auto vb = [&](int j, int e) { const float4 v = r.b[j]; return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; };
  const int tail = 4 * XR4 * T;  // first element past the registers
  if (kind < 0) {
#pragma unroll
    for (int j = 0; j < XR4; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = 4 * (tid + j * T) + e;
        if (i < n) out[i] = vx(j, e);
      }
    for (int i = tail + tid; i < n; i += T) out[i] = xs[i];
    return;
  }
  double s1 = 0.0, s2 = 0.0;
  const double K = kind == 0 ? (double)r.shift : 0.0;
  auto moment = [&](float v) {
    if (kind == 0) {
      const double d = (double)v - K;
      s1 += d;
      s2 += d * d;
    } else {
      s1 += (double)__fmul_rn(v, v);
    }
  };
#pragma unroll
  for (int j = 0; j < XR4; j++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (4 * (tid + j * T) + e < n) moment(vx(j, e));
  for (int i = tail + tid; i < n; i += T) moment(xs[i]);
  block_sum2_d<T>(s1, s2, red);
  if (kind == 0) {
    const double mean = K + s1 / (double)n;
    const double var = fmax((s2 - s1 * s1 / (double)n) / (double)n, 0.0);
    const float inv = (float)(1.0 / sqrt(var + eps)), fm = (float)mean;
    auto affine = [&](float x, float wi, float bi) {
      float t = __fsub_rn(x, fm);
      t = __fmul_rn(t, inv);
      t = __fmul_rn(t, wi);
      return __fadd_rn(t, bi);
    };
#pragma unroll
    for (int j = 0; j < XR4; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = 4 * (tid + j * T) + e;
        if (i < n) out[i] = affine(vx(j, e), vw(j, e), vb(j, e));
      }
    for (int i = tail + tid; i < n; i += T) out[i] = affine(xs[i], w[i], b[i]);
  } else {
    const float ss = (float)s1;
    const float mean = __fadd_rn(__fdiv_rn(ss, (float)n), (float)eps);
    const float inv = __fdiv_rn(1.0f, (float)sqrt((double)mean));
#pragma unroll
    for (int j = 0; j < XR4; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = 4 * (tid + j * T) + e;
        if (i < n) out[i] = __fmul_rn(vw(j, e), __fmul_rn(inv, vx(j, e)));
      }
    for (int i = tail + tid; i < n; i += T) out[i] = __fmul_rn(w[i], __fmul_rn(inv, xs[i]));
  }
}

// A kernel-argument pointer moved into scalar registers. Choosing between
// two such pointers with a per-lane condition then selects registers; on
// the kernel-argument fields themselves the compiler turns the choice into
// one vector load from argument memory, which a later wait must cover.
template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T *>(lo | (hi << 32));
}

// Block-wide sum in float64 with a fixed reduction tree, so every block that
// reduces the same data obtains the same bits. `red` holds >= warps doubles.
__device__ __forceinline__ double block_sum_d(double v, double *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = (blockDim.x + 63) >> 6;
  v = wave_sum_d(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double total = 0;
  for (int i = 0; i < waves; i++) total += red[i];
  return total;
}

// LayerNorm (stablelm.go:288-305) of an LDS-resident row, in place:
// float64 two-pass moments, float32 affine with separately rounded steps.
// All threads of the block participate.
__device__ __forceinline__ void layer_norm_lds(float *x, int n, const float *__restrict__ w,
                                               const float *__restrict__ b, double eps, double *red) {
  // The affine weights of this thread's first elements are loaded before the
  // moments are reduced, so their latency hides behind the reductions.
  constexpr int R = 4;
  float wr[R], br[R];
#pragma unroll
  for (int j = 0; j < R; j++) {
    const int i = threadIdx.x + j * blockDim.x;
    wr[j] = i < n ? w[i] : 0.f;
    br[j] = i < n ? b[i] : 0.f;
  }
  double s = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) s += (double)x[i];
  double mean = block_sum_d(s, red) / (double)n;
  double v = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    double d = (double)x[i] - mean;
    v += d * d;
  }
  double var = block_sum_d(v, red);
  float inv = (float)(1.0 / sqrt(var / (double)n + eps));
  float fm = (float)mean;
  __syncthreads();
  auto affine = [&](int i, float wi, float bi) {
    float t = __fsub_rn(x[i], fm);
    t = __fmul_rn(t, inv);
    t = __fmul_rn(t, wi);
    x[i] = __fadd_rn(t, bi);
  };
#pragma unroll
  for (int j = 0; j < R; j++) {
    const int i = threadIdx.x + j * blockDim.x;
    if (i < n) affine(i, wr[j], br[j]);
  }
  for (int i = threadIdx.x + R * blockDim.x; i < n; i += blockDim.x) affine(i, w[i], b[i]);
  __syncthreads();
}

// dst[i] = src[i] for i < n by all threads of the block, four loads in
// flight per thread before the first store (dst may be LDS that the
// compiler cannot tell apart from src).
__device__ __forceinline__ void copy_block(float *dst, const float *src, int n) {
  for (int i0 = threadIdx.x; i0 < n; i0 += 4 * blockDim.x) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = i0 + j * blockDim.x;
      v[j] = i < n ? src[i] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (i0 + j * blockDim.x < n) dst[i0 + j * blockDim.x] = v[j];
  }
}

// RMSNorm (model.go:591-600) of an LDS-resident row, in place: the sum of
// float32 squares (accumulated in float64, then rounded), ss / n + eps and
// 1 / float32(sqrt(.)) in float32, out = w * (inv * x).
__device__ __forceinline__ void rms_norm_lds(float *x, int n, const float *__restrict__ w, float eps, double *red) {
  double s = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) s += (double)__fmul_rn(x[i], x[i]);
  const float ss = (float)block_sum_d(s, red);
  const float mean = __fadd_rn(__fdiv_rn(ss, (float)n), eps);
  const float inv = __fdiv_rn(1.0f, (float)sqrt((double)mean));
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = __fmul_rn(w[i], __fmul_rn(inv, x[i]));
  __syncthreads();
}

// SiLU-gate (stablelm.go:371-373): (g / (1 + f32(exp(-f64(g))))) * u.
__device__ __forceinline__ float silu_gate(float g, float u) {
  float e = (float)exp_f64(-(double)g);
  float den = __fadd_rn(1.0f, e);
  return __fmul_rn(__fdiv_rn(g, den), u);
}

// The legacy Llama's SwiGLU (model.go:463-470): s = 1 / (1 + e), (g * s) * u.
__device__ __forceinline__ float silu_gate_llama(float g, float u) {
  float e = (float)exp_f64(-(double)g);
  float s = __fdiv_rn(1.0f, __fadd_rn(1.0f, e));
  return __fmul_rn(__fmul_rn(g, s), u);
}
