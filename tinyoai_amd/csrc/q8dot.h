// Q8_0 dequant-dot on the integer dot-product units of gfx950.
//
// The reference multiplies float32 activations by int8 quants and
// accumulates in float64 (dot.go:31-40). Here each 32-value block of the
// activation vector x is written as three int8 "limbs" over a power-of-two
// block scale s = 2^(e-7), with e the exponent of the block's largest |x|:
//     x ~= s * (a + b / 128 + c / 16384),   a, b, c in [-127, 127],
// every step an exact float32 operation with the last limb rounded to
// nearest, i.e. about 23 significant bits relative to the block maximum
// (float32 keeps 24 relative to each element). Then
//     sum_k w_k x_k = s * (sum w a + (sum w b) / 128 + (sum w c) / 16384)
// where the three inner sums are exact int32 results of v_dot4_i32_i8,
// four weights per instruction, and only one float multiply-add per
// 16 weights touches the block scale d_w * s.
#pragma once

#include "formats.h"

// LDS image of a quantized activation vector of `cols` values (multiple of 32).
struct XLimbs {
  int8_t *a, *b, *c;  // [cols] each, 16-byte aligned
  float *scale;       // [cols / 32], s per block (NaN for a non-finite block)
};

__host__ __device__ inline size_t xlimbs_bytes(int cols) { return (size_t)cols * 3 + (size_t)cols / 32 * 4 + 64; }

__device__ inline XLimbs xlimbs_at(void *base, int cols) {
  uint8_t *p = reinterpret_cast<uint8_t *>(base);
  XLimbs l;
  l.a = reinterpret_cast<int8_t *>(p);
  l.b = l.a + cols;
  l.c = l.b + cols;
  l.scale = reinterpret_cast<float *>(p + (size_t)cols * 3);
  return l;
}

// Quantizes x[0, cols) (LDS) into limbs; whole block participates, cols % 32 == 0.
__device__ inline void quantize_limbs(const float *x, int cols, XLimbs l) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const int nblocks = cols / 32;
  // Each wave takes two 32-value blocks at a time: lanes 0-31 and 32-63.
  for (int b0 = 2 * wave; b0 < nblocks; b0 += 2 * waves) {
    const int blk = b0 + (lane >> 5);
    const bool valid = blk < nblocks;
    const float v = valid ? x[blk * 32 + (lane & 31)] : 0.f;
    float m = fabsf(v);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (!valid) continue;
    int e;
    frexpf(m, &e);  // m < 2^e (m == 0 gives e == 0)
    const float s = ldexpf(1.f, e - 7), inv = ldexpf(1.f, 7 - e);
    const float t = v * inv;  // |t| < 128, exact
    float a = fminf(fmaxf(rintf(t), -127.f), 127.f);
    const float r1 = (t - a) * 128.f;
    float b = fminf(fmaxf(rintf(r1), -127.f), 127.f);
    const float r2 = (r1 - b) * 128.f;
    float c = fminf(fmaxf(rintf(r2), -127.f), 127.f);
    const int k = blk * 32 + (lane & 31);
    l.a[k] = (int8_t)(int)a;
    l.b[k] = (int8_t)(int)b;
    l.c[k] = (int8_t)(int)c;
    if ((lane & 31) == 0) l.scale[blk] = isfinite(m) ? s : __builtin_nanf("");
  }
}

// The limbs of the 16 activation values of one chunk, kept in registers.
struct XChunk {
  int4 a, b, c;
  float s;  // block scale
};

__device__ __forceinline__ XChunk load_xchunk(const XLimbs &l, int c) {
  XChunk r;
  r.a = reinterpret_cast<const int4 *>(l.a)[c];
  r.b = reinterpret_cast<const int4 *>(l.b)[c];
  r.c = reinterpret_cast<const int4 *>(l.c)[c];
  r.s = l.scale[c >> 1];
  return r;
}

// sum_k w_k x_k over one 16-weight chunk, without the weight scale.
__device__ __forceinline__ float q8_chunk_dot(const uint4 w, const XChunk &x) {
  int ia = __builtin_amdgcn_sdot4((int)w.x, x.a.x, 0, false);
  int ib = __builtin_amdgcn_sdot4((int)w.x, x.b.x, 0, false);
  int ic = __builtin_amdgcn_sdot4((int)w.x, x.c.x, 0, false);
  ia = __builtin_amdgcn_sdot4((int)w.y, x.a.y, ia, false);
  ib = __builtin_amdgcn_sdot4((int)w.y, x.b.y, ib, false);
  ic = __builtin_amdgcn_sdot4((int)w.y, x.c.y, ic, false);
  ia = __builtin_amdgcn_sdot4((int)w.z, x.a.z, ia, false);
  ib = __builtin_amdgcn_sdot4((int)w.z, x.b.z, ib, false);
  ic = __builtin_amdgcn_sdot4((int)w.z, x.c.z, ic, false);
  ia = __builtin_amdgcn_sdot4((int)w.w, x.a.w, ia, false);
  ib = __builtin_amdgcn_sdot4((int)w.w, x.b.w, ib, false);
  ic = __builtin_amdgcn_sdot4((int)w.w, x.c.w, ic, false);
  return fmaf((float)ic, 1.f / 16384.f, fmaf((float)ib, 1.f / 128.f, (float)ia));
}

// A lane's share of one Q8_0 row: chunks lane + 64 j, j < J.
template <int J>
struct Q8Row {
  uint4 w[J];
  float d[J];
};

template <int J>
__device__ __forceinline__ void q8row_issue(Q8Row<J> &r, const uint8_t *vals, const uint8_t *meta, int nchunks,
                                            int lane) {
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int c = lane + 64 * j;
    if (c < nchunks) {
      r.w[j] = load_chunk(vals + (int64_t)c * 16);
      r.d[j] = hw_half(reinterpret_cast<const uint16_t *>(meta)[c >> 1]);
    }
  }
}

template <int J>
__device__ __forceinline__ float q8row_dot(const Q8Row<J> &r, const XChunk (&x)[J], int nchunks, int lane) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (lane + 64 * j < nchunks) acc = fmaf(q8_chunk_dot(r.w[j], x[j]), r.d[j] * x[j].s, acc);
  }
  return acc;
}

template <int J>
__device__ __forceinline__ void load_xchunks(XChunk (&x)[J], const XLimbs &l, int nchunks, int lane) {
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int c = lane + 64 * j;
    if (c < nchunks) x[j] = load_xchunk(l, c);
  }
}
