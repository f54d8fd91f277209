// Weight formats as laid out in HBM, and the per-format arithmetic the
// kernels share.
//
// On upload every matrix is split into planes:
//   vals:  the per-value payload, each row padded to a multiple of 16 bytes,
//          so a lane streams a row with 128-bit loads (a "chunk");
//   meta:  per-block metadata (Q8_0: one fp16 scale per 32 values);
//   hbits: the high bits of 5- and 6-bit quants.
// F32 / F16 / BF16 keep row-major values; Q8_0 keeps its int8 quants in
// `vals` and its fp16 block scales in `meta`, the bytes of the GGUF block
// {fp16 d, int8 q[32]} (dot.go:31-40) regrouped. The 5/6-bit formats
// (decodeKBlock, quant_k.go:31-86) use chunks of 32 values: byte b of a
// chunk holds the low 4 bits of values b and b + 16; hbits holds bit 4 of
// value j at bit j (Q5_1, Q5_K: 4 bytes a chunk) or bits 4-5 at bits 2j
// (Q6_K: 8 bytes); meta keeps each block's own header bytes: Q5_1 {d, m}
// per 32 values, Q4_K / Q5_K {d, dmin, scales[12]} and Q6_K {scales[16],
// d} (padded to 32 bytes) per 256 values.
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
  const uint8_t *hbits; // [rows][hstride] bytes (Q5_1, Q5_K, Q6_K)
  int64_t hstride;
};

__host__ __device__ inline bool is_kquant(int fmt) {
  return fmt == FMT_Q5_1 || fmt == FMT_Q4_K || fmt == FMT_Q5_K || fmt == FMT_Q6_K;
}
// Bytes of hbits per chunk, and of meta per chunk (Q8_0, Q5_1) or per
// 256-value super-block (Q4_K, Q5_K, Q6_K).
__host__ __device__ inline int hbits_per_chunk(int fmt) {
  return fmt == FMT_Q6_K ? 8 : (fmt == FMT_Q5_1 || fmt == FMT_Q5_K ? 4 : 0);
}
__host__ __device__ inline int meta_per_block(int fmt) {
  switch (fmt) {
    case FMT_Q8_0: return 2;
    case FMT_Q5_1: return 4;
    case FMT_Q4_K: case FMT_Q5_K: return 16;
    case FMT_Q6_K: return 32;
    default: return 0;
  }
}
// Byte offsets of chunk c's metadata and high bits within a row.
__host__ __device__ inline int64_t meta_offset(int fmt, int64_t c) {
  switch (fmt) {
    case FMT_Q8_0: return (c >> 1) * 2;
    case FMT_Q5_1: return c * 4;
    case FMT_Q4_K: case FMT_Q5_K: return (c >> 3) * 16;
    case FMT_Q6_K: return (c >> 3) * 32;
    default: return 0;
  }
}
__host__ __device__ inline int64_t hbits_offset(int fmt, int64_t c) { return c * hbits_per_chunk(fmt); }

template <int F> struct Fmt;
template <> struct Fmt<FMT_Q8_0> { static constexpr int VPC = 16; };
template <> struct Fmt<FMT_Q5_1> { static constexpr int VPC = 32; };
template <> struct Fmt<FMT_Q4_K> { static constexpr int VPC = 32; };
template <> struct Fmt<FMT_Q5_K> { static constexpr int VPC = 32; };
template <> struct Fmt<FMT_Q6_K> { static constexpr int VPC = 32; };
template <> struct Fmt<FMT_BF16> { static constexpr int VPC = 8; };
template <> struct Fmt<FMT_F16> { static constexpr int VPC = 8; };
template <> struct Fmt<FMT_F32> { static constexpr int VPC = 4; };

// Values held by one 16-byte chunk of `vals`.
__host__ __device__ inline int values_per_chunk(int fmt) {
  switch (fmt) {
    case FMT_Q8_0: return 16;
    case FMT_BF16: case FMT_F16: return 8;
    case FMT_Q5_1: case FMT_Q4_K: case FMT_Q5_K: case FMT_Q6_K: return 32;
    default: return 4;
  }
}

__device__ __forceinline__ float hw_half(uint16_t h) {
  return __half2float(__ushort_as_half(h));  // v_cvt_f32_f16: exact, keeps subnormals
}

// ---------------------------------------------------------------- x in LDS
// The activation vector of a product is staged in LDS "transposed": for
// chunk c (VPC values) and quad q < VPC/4, the float4 of values
// x[c*VPC + 4q .. 4q + 3] sits at xq[q * nch + c]. Lanes reading chunks
// c, c+1, ... then touch consecutive 16-byte words (conflict-free), where a
// plain layout would put them VPC*4 bytes apart.
// x may live in global memory or LDS. Each thread loads four float4 before
// it stores any, so a block stages up to 4 * blockDim float4 in one memory
// round trip (a store to LDS could alias x, so the compiler would not
// overlap the iterations of a plain loop).
__device__ __forceinline__ void stage_x(float4 *xq, const float *x, int len, int nch, int vpc) {
  const int quads = vpc / 4, n = quads * nch;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  for (int i0 = threadIdx.x; i0 < n; i0 += 4 * blockDim.x) {
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = i0 + j * blockDim.x;
      const int q = i / nch, c = i % nch;
      const int k = c * vpc + 4 * q;
      if (i >= n) {
        v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      } else if (aligned && k + 3 < len) {
        v[j] = *reinterpret_cast<const float4 *>(x + k);
      } else {
        v[j].x = k < len ? x[k] : 0.f;
        v[j].y = k + 1 < len ? x[k + 1] : 0.f;
        v[j].z = k + 2 < len ? x[k + 2] : 0.f;
        v[j].w = k + 3 < len ? x[k + 3] : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (i0 + j * blockDim.x < n) xq[i0 + j * blockDim.x] = v[j];
  }
}

// Dot product of one 16-byte weight chunk with its x values (fp32, fused
// multiply-adds). Q8_0 returns the sum before the block scale.
template <int F>
__device__ __forceinline__ float chunk_dot(const uint4 w, const float4 *xq, int nch, int c);

template <>
__device__ __forceinline__ float chunk_dot<FMT_Q8_0>(const uint4 w, const float4 *xq, int nch, int c) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float4 xv = xq[k * nch + c];
    const uint32_t v = ws[k];
    a = fmaf((float)(int8_t)(v), xv.x, a);
    b = fmaf((float)(int8_t)(v >> 8), xv.y, b);
    a = fmaf((float)(int8_t)(v >> 16), xv.z, a);
    b = fmaf((float)(int8_t)(v >> 24), xv.w, b);
  }
  return a + b;
}

template <>
__device__ __forceinline__ float chunk_dot<FMT_BF16>(const uint4 w, const float4 *xq, int nch, int c) {
  const float4 x0 = xq[c], x1 = xq[nch + c];
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
__device__ __forceinline__ float chunk_dot<FMT_F16>(const uint4 w, const float4 *xq, int nch, int c) {
  const float4 x0 = xq[c], x1 = xq[nch + c];
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
__device__ __forceinline__ float chunk_dot<FMT_F32>(const uint4 w, const float4 *xq, int nch, int c) {
  const float4 xv = xq[c];
  float a = __uint_as_float(w.x) * xv.x;
  float b = __uint_as_float(w.y) * xv.y;
  a = fmaf(__uint_as_float(w.z), xv.z, a);
  b = fmaf(__uint_as_float(w.w), xv.w, b);
  return a + b;
}

// ---------------------------------------------------------------- 5/6-bit
// Per-chunk constants of the value formula, from the chunk's meta bytes
// (and, for Q6_K, its fp16 d): value = (q * a) + b for Q5_1, (q * a) - b
// for Q4_K / Q5_K, (q - 32) * (a or a2) for Q6_K (a for values 0-15, a2
// for 16-31), each step rounded as decodeKBlock rounds it.
struct KConst {
  float a, b, a2;
};

// Byte i (0..15, little-endian) of a 16-byte header held in registers. A
// selection among the four words, not a byte pointer into them: indexing
// a local array at a run-time position puts it in per-lane scratch memory.
__device__ __forceinline__ uint32_t header_byte(const uint4 mt, int i) {
  const uint32_t w = i < 8 ? (i < 4 ? mt.x : mt.y) : (i < 12 ? mt.z : mt.w);
  return (w >> (8 * (i & 3))) & 255u;
}

template <int F>
__device__ __forceinline__ KConst kquant_const(const uint4 mt, uint16_t d6, int cc) {
  KConst k{};
  if constexpr (F == FMT_Q5_1) {
    k.a = half_to_float((uint16_t)mt.x);
    k.b = half_to_float((uint16_t)(mt.x >> 16));
  } else if constexpr (F == FMT_Q4_K || F == FMT_Q5_K) {
    // the 12 scale bytes follow {d, dmin}: header bytes 4..15 (quant_k.go:69-77)
    const int g = cc & 7;
    auto sc = [&](int i) { return (int)header_byte(mt, 4 + i); };
    int scale, minimum;
    if (g < 4) {
      scale = sc(g) & 63;
      minimum = sc(g + 4) & 63;
    } else {
      scale = (sc(g + 4) & 15) | ((sc(g - 4) >> 6) << 4);
      minimum = (sc(g + 4) >> 4) | ((sc(g) >> 6) << 4);
    }
    k.a = __fmul_rn(half_to_float((uint16_t)mt.x), (float)scale);
    k.b = __fmul_rn(half_to_float((uint16_t)(mt.x >> 16)), (float)minimum);
  } else {
    const float d = half_to_float(d6);
    const int g = cc & 7;
    k.a = __fmul_rn(d, (float)(int8_t)header_byte(mt, 2 * g));
    k.a2 = __fmul_rn(d, (float)(int8_t)header_byte(mt, 2 * g + 1));
  }
  return k;
}

// The quant of value j (0..31) of a chunk: low 4 bits from the value
// bytes, high bits from hbits.
template <int F>
__device__ __forceinline__ int kquant_q(uint32_t lo_byte, int j, uint2 h) {
  const int lo = j < 16 ? (lo_byte & 15) : (lo_byte >> 4);
  if constexpr (F == FMT_Q5_1 || F == FMT_Q5_K) return lo | (int)((h.x >> j) & 1) << 4;
  if constexpr (F == FMT_Q6_K) {
    const uint32_t hw = j < 16 ? h.x : h.y;
    return lo | (int)((hw >> (2 * (j & 15))) & 3) << 4;
  }
  return lo;
}

template <int F>
__device__ __forceinline__ float kquant_value(const KConst &k, int q, int j) {
  if constexpr (F == FMT_Q5_1) return __fadd_rn(__fmul_rn(k.a, (float)q), k.b);
  if constexpr (F == FMT_Q6_K) return __fmul_rn(j < 16 ? k.a : k.a2, (float)(q - 32));
  return __fsub_rn(__fmul_rn(k.a, (float)q), k.b);
}

// Dot product of chunk cc (32 values) with its staged x (quad q of the
// chunk at xq[q * nch + c]).
template <int F>
__device__ __forceinline__ float kchunk_dot(const uint4 w, const uint2 h, const uint4 mt, uint16_t d6, int cc,
                                            const float4 *xq, int nch, int c) {
  const KConst k = kquant_const<F>(mt, d6, cc);
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int qd = 0; qd < 4; qd++) {
    const float4 xl = xq[qd * nch + c], xh = xq[(qd + 4) * nch + c];
    const float xlv[4] = {xl.x, xl.y, xl.z, xl.w}, xhv[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t byte = (ws[qd] >> (8 * e)) & 255;
      const int j = 4 * qd + e;
      a = fmaf(kquant_value<F>(k, kquant_q<F>(byte, j, h), j), xlv[e], a);
      b = fmaf(kquant_value<F>(k, kquant_q<F>(byte, j + 16, h), j + 16), xhv[e], b);
    }
  }
  return a + b;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Weights live in global memory; saying so keeps the loads global_load
// (not flat) where the compiler cannot trace a pointer back to a kernel
// argument.
#define TINYOAI_GLOBAL __attribute__((address_space(1)))

// One 16-byte chunk of a weight row, streamed past the caches (each weight
// byte is read once per token).
__device__ __forceinline__ uint4 load_chunk(const uint8_t *p) {
  const u32x4 v = __builtin_nontemporal_load((const TINYOAI_GLOBAL u32x4 *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// A 16-bit block scale, zero-extended into a 32-bit register (kept 32-bit
// in a batch: 16-bit batch fields were copied between the two batch
// buffers at the loop's back edge, each copy waiting for its load).
__device__ __forceinline__ uint32_t load_scale(const uint8_t *meta, int block) {
  return ((const TINYOAI_GLOBAL uint16_t *)meta)[block];
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Plain (cached) global loads of block headers and high bits, which
// neighbouring lanes share.
__device__ __forceinline__ uint4 load_u4(const uint8_t *p, int64_t i) {
  const u32x4 v = ((const TINYOAI_GLOBAL u32x4 *)p)[i];
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 load_u2(const uint8_t *p, int64_t i) {
  const u32x2 v = ((const TINYOAI_GLOBAL u32x2 *)p)[i];
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t load_u1(const uint8_t *p, int64_t i) {
  return ((const TINYOAI_GLOBAL uint32_t *)p)[i];
}

// ---------------------------------------------------------------- streaming
// A unit of matvec work: one or two row segments, each with its own staged
// x vector (xq0 / xq1 with n0 / n1 chunks). n1 == 0 means one segment.
struct RowPtr {
  const uint8_t *v, *m, *h;  // vals, meta, hbits of a row from some chunk on
};

// Row `row` of m from chunk c0 (a super-block boundary for Q4_K/Q5_K/Q6_K).
__host__ __device__ inline RowPtr row_ptr(const MatDesc &m, int64_t row, int64_t c0 = 0) {
  return RowPtr{m.vals + row * m.vstride + c0 * 16, m.meta + row * m.mstride + meta_offset(m.fmt, c0),
                m.hbits + row * m.hstride + hbits_offset(m.fmt, c0)};
}

struct Seg2 {
  RowPtr r0, r1;
  const float4 *x0, *x1;
  int n0, n1;
};

// One batch of U chunks per lane: the weight bytes and, for Q8_0, the raw
// fp16 block scale. Scales stay raw until the chunk is consumed: converting
// at load time would make every load wait for its predecessor.
template <int U>
struct Batch {
  uint4 w[U];
  uint32_t s[U];  // Q8_0 block scale, Q6_K d (zero-extended fp16 bits)
  uint2 h[U];     // high bits (Q5_1, Q5_K, Q6_K)
  uint4 mt[U];    // block header (Q5_1, Q4_K, Q5_K, Q6_K scales)
};

// Issues every load of a batch back to back. Lanes past the end load a
// valid chunk (the last one) whose value is never consumed, so the loads
// need no branches.
template <int F, int U>
__device__ __forceinline__ void batch_issue(Batch<U> &b, const Seg2 &g, int base, int lane) {
  const int total = g.n0 + g.n1;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int c = min(base + u * 64 + lane, total - 1);
    const bool seg1 = c >= g.n0;
    const int cc = seg1 ? c - g.n0 : c;
    const RowPtr &r = seg1 ? g.r1 : g.r0;
    b.w[u] = load_chunk(r.v + (int64_t)cc * 16);
    if constexpr (F == FMT_Q8_0) b.s[u] = load_scale(r.m, cc >> 1);
    if constexpr (F == FMT_Q5_1) {
      b.mt[u].x = load_u1(r.m, cc);
      b.h[u].x = load_u1(r.h, cc);
    }
    if constexpr (F == FMT_Q4_K || F == FMT_Q5_K) b.mt[u] = load_u4(r.m, cc >> 3);
    if constexpr (F == FMT_Q5_K) b.h[u].x = load_u1(r.h, cc);
    if constexpr (F == FMT_Q6_K) {
      b.mt[u] = load_u4(r.m, (cc >> 3) * 2);
      b.s[u] = load_scale(r.m + (cc >> 3) * 32 + 16, 0);
      b.h[u] = load_u2(r.h, cc);
    }
  }
}

// Buffer descriptors of a matrix's planes (gfx9 raw buffers: base, no
// stride, a byte count). The streaming kernels address a plane with 32-bit
// per-lane offsets; a load at an offset past the count returns zeros
// without a memory request (a lane without a chunk loads at kOffNone).
struct Planes {
  __amdgpu_buffer_rsrc_t v, m, h;
  const uint8_t *vb, *mb, *hb;
};

// Every plane below 2^31 bytes: offsets fit a signed 32-bit register and
// 2^31 lies past every plane.
__host__ __device__ inline bool planes_fit(const MatDesc &M) {
  return (int64_t)M.rows * M.vstride < 0x80000000ll && (int64_t)M.rows * M.mstride < 0x80000000ll &&
         (int64_t)M.rows * M.hstride < 0x80000000ll;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(const uint8_t *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p), (short)0, (int)(uint32_t)bytes, 0x00020000);
}

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4
// ... lds): the wave's 64 lanes fill 1 KB at LDS byte address lds_byte in
// lane order. Inline assembly, so the compiler neither tracks nor waits for
// it: the caller waits (wait_vmcnt) before any wave reads the bytes.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds_byte) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds_byte) : "memory");
}
// The same with 4 bytes per lane (buffer_load_dword ... lds): 256 bytes.
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds_byte) {
  asm volatile("buffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds_byte) : "memory");
}
// s_waitcnt with vmcnt(n) only (gfx9 encoding: vmcnt bits 3:0 and 15:14).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | 0x0f70);
}

__device__ __forceinline__ Planes make_planes(const MatDesc &M) {
  Planes P;
  P.v = plane_rsrc(M.vals, (int64_t)M.rows * M.vstride);
  P.m = plane_rsrc(M.meta, (int64_t)M.rows * M.mstride);
  P.h = plane_rsrc(M.hbits, (int64_t)M.rows * M.hstride);
  P.vb = M.vals;
  P.mb = M.meta;
  P.hb = M.hbits;
  return P;
}

// Consumes the chunks base + u * 64 + lane of a batch into acc0 (segment 0)
// and acc1 (segment 1). Branch-free: a lane past the end computes on its
// clamped (valid) chunk and contributes 0, so no per-chunk exec-mask
// branches are emitted. With SERIAL, the scheduler may not hoist the LDS
// reads of later chunks above earlier ones (bounds register use where a
// kernel keeps other state live). Only chunks with lo <= c < hi count.
template <int F, int U, bool SERIAL = false>
__device__ __forceinline__ void batch_consume_range(const Batch<U> &b, const Seg2 &g, int base, int lane, int lo,
                                                    int hi, float &acc0, float &acc1) {
  const int total = g.n0 + g.n1;
  hi = min(hi, total);
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int c = base + u * 64 + lane;
    const int cl = min(c, total - 1);
    const bool seg1 = cl >= g.n0;
    const int cc = seg1 ? cl - g.n0 : cl;
    float p;
    if constexpr (Fmt<F>::VPC == 32) {
      p = kchunk_dot<F>(b.w[u], b.h[u], b.mt[u], (uint16_t)b.s[u], cc, seg1 ? g.x1 : g.x0, seg1 ? g.n1 : g.n0, cc);
    } else {
      p = chunk_dot<F>(b.w[u], seg1 ? g.x1 : g.x0, seg1 ? g.n1 : g.n0, cc);
      if constexpr (F == FMT_Q8_0) p *= hw_half((uint16_t)b.s[u]);
    }
    p = (c >= lo && c < hi) ? p : 0.f;
    acc0 += seg1 ? 0.f : p;
    acc1 += seg1 ? p : 0.f;
    if constexpr (SERIAL) __builtin_amdgcn_sched_barrier(0);
  }
}

template <int F, int U, bool SERIAL = false>
__device__ __forceinline__ void batch_consume(const Batch<U> &b, const Seg2 &g, int base, int lane, float &acc0,
                                              float &acc1) {
  batch_consume_range<F, U, SERIAL>(b, g, base, lane, 0, g.n0 + g.n1, acc0, acc1);
}

// Value (row, col) of a 5/6-bit matrix, bit-exact with decodeKBlock.
template <int F>
__device__ __forceinline__ float kquant_at(const MatDesc &m, int64_t row, int64_t col) {
  const int64_t c = col >> 5;
  const int j = (int)(col & 31);
  const RowPtr r = row_ptr(m, row);
  const uint32_t byte = r.v[c * 16 + (j & 15)];
  uint2 h{0, 0};
  uint4 mt{0, 0, 0, 0};
  uint16_t d6 = 0;
  const uint8_t *mp = r.m + meta_offset(F, c);
  if constexpr (F == FMT_Q5_1) mt.x = *reinterpret_cast<const uint32_t *>(mp);
  else mt = *reinterpret_cast<const uint4 *>(mp);
  if constexpr (F == FMT_Q6_K) d6 = *reinterpret_cast<const uint16_t *>(mp + 16);
  if constexpr (F == FMT_Q5_1 || F == FMT_Q5_K) h.x = reinterpret_cast<const uint32_t *>(r.h)[c];
  if constexpr (F == FMT_Q6_K) h = reinterpret_cast<const uint2 *>(r.h)[c];
  return kquant_value<F>(kquant_const<F>(mt, d6, (int)c), kquant_q<F>(byte, j, h), j);
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
    case FMT_Q5_1: return kquant_at<FMT_Q5_1>(m, row, col);
    case FMT_Q4_K: return kquant_at<FMT_Q4_K>(m, row, col);
    case FMT_Q5_K: return kquant_at<FMT_Q5_K>(m, row, col);
    case FMT_Q6_K: return kquant_at<FMT_Q6_K>(m, row, col);
    default: return reinterpret_cast<const float *>(vr)[col];
  }
}
