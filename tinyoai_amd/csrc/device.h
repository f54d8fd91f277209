// Device helpers shared by the gfx950 kernels: exact-rounding float ops,
// IEEE binary16 conversions restated bit for bit, and wave64 reductions.
//
// Every translation unit is compiled with -ffp-contract=off, so a plain
// a * b + c rounds twice. Hot reductions use fmaf() explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    float t = __fsub_rn(x[i], fm);
    t = __fmul_rn(t, inv);
    t = __fmul_rn(t, w[i]);
    x[i] = __fadd_rn(t, b[i]);
  }
  __syncthreads();
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
  float e = (float)exp(-(double)g);
  float den = __fadd_rn(1.0f, e);
  return __fmul_rn(__fdiv_rn(g, den), u);
}

// The legacy Llama's SwiGLU (model.go:463-470): s = 1 / (1 + e), (g * s) * u.
__device__ __forceinline__ float silu_gate_llama(float g, float u) {
  float e = (float)exp(-(double)g);
  float s = __fdiv_rn(1.0f, __fadd_rn(1.0f, e));
  return __fmul_rn(__fmul_rn(g, s), u);
}
