// Products of a few activation rows with a 5/6-bit quantized matrix on the
// gfx950 matrix cores: Y[M][N] = X[M][K] * W^T for M <= 32 (the rows of a
// batched branch step), W in Q4_K, Q5_K, Q6_K or Q5_1.
//
// Every value of these formats is q * a - b (Q4_K, Q5_K), q * a + b (Q5_1)
// or (q - 32) * a (Q6_K), with a small integer q and constants a, b shared
// by a sub-block of 32 values (16 for Q6_K) (decodeKBlock,
// quant_k.go:31-86). q is exact in bf16, so each sub-block's products run
// on the matrix cores unscaled (Q6_K: over q, with -32 * xsum added),
//   t[m][n] = sum over the sub-block of x[m][k] * q[n][k],
// with x as three bf16 planes (hi + mid + lo: 24 significant bits, as
// fp32 holds), and are added to fp32 accumulators as
// acc += a * t - b * xsum, xsum[m] being the sub-block's sum of x (of
// hi + mid + lo, the values the products saw).
//
// X is converted once per product (kq_stage_kernel) into staged chunks:
// three bf16 planes of each row's 32 values and three sums per row (whole
// chunk, first and second 16 values). A block of 4 waves takes 128 matrix
// rows (32 a wave, two 16-row tiles) over one range of K, a batch of 8
// chunks (a K-quant super-block) at a time: the batch's staged chunks are
// copied into LDS, each wave reads its rows' quants straight from HBM and
// forms v_mfma_f32_16x16x32_bf16 products per 32-value chunk (two
// v_mfma_f32_16x16x16_bf16, one per 16-value sub-block, for Q6_K). The
// batches run as a software pipeline: the next batch's quants and staged
// chunks are in flight while one is computed. K ranges (splits) write
// separate partial outputs, split s at y + s * split_stride (by default
// M * ldy), which the consumer sums.
//
// Staged value order: a 16x16x32 product gives lane group g = lane / 16
// the 8 positions 8g..8g+7 of each chunk. The quants of a chunk sit as
// "byte b holds values b (low nibble) and b + 16 (high nibble)", so a
// lane reading bytes 4g..4g+3 holds values 4g..4g+3 and 16+4g..16+4g+3;
// the staged x of a chunk is permuted the same way (values 4g..4g+3 at
// positions 8g..8g+3, values 16+4g.. at 8g+4..8g+7). For Q6_K the first
// four positions of every group form sub-block 0 and the last four
// sub-block 1.
#include <algorithm>

#include "kernels.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kThreads = 256, kWaveRows = 32, kBlockRows = 128;
constexpr uint32_t kNone = 0x80000000u;  // past every plane (each < 2 GiB)
constexpr int kPlanes = 3;
constexpr int kWindow = 8;  // chunks per batch (a K-quant super-block)

// A staged chunk of R = 16 * MT rows: planes [3][R][32] bf16 (in the
// permuted value order), then sums [3][R] floats.
template <int MT>
constexpr int chunk_bytes() { return 16 * MT * (kPlanes * 64 + 3 * 4); }
// Two window buffers in LDS: one is computed while the next is filled.
template <int MT>
constexpr size_t lds_bytes() { return (size_t)2 * kWindow * chunk_bytes<MT>(); }

struct KqArgs {
  MatDesc w;
  const uint8_t *stage;  // staged chunks of X, chunk c at c * chunk_bytes (per slice of R rows)
  int M;                 // rows; slices of R rows on the grid's y dimension
  float *y;
  int ldy, ks;
  int64_t split_stride;  // floats between the K splits' outputs
};

// x [M][K] -> staged chunks. Item i: group of 4 values i % 8 of row
// (i / 8) % R and chunk i / (8 R); a chunk's 8 groups are 8 consecutive
// lanes, which form the sums by fixed-order shuffles. Slice blockIdx.y
// stages rows [R y, R y + R) at y * nch * chunk_bytes.
//
// With lw, the rows are LayerNorm'd on the way (stablelm.go:288-305, the
// arithmetic of norm_store in device.h: float64 moments about the row's
// first value in one pass, then t = x - float(mean), t *= float(1 /
// sqrt(var + eps)), t *= w, t += b, each rounded to float32). Every block
// forms the moments of its slice's rows itself (256 / R threads per row
// over contiguous spans of K, then a fixed-order shuffle tree), so no
// separate LayerNorm launch runs before the staging.
template <int MT, bool NORM>
__device__ __forceinline__ void kq_stage_body(const float *x, int ldx, int M, int K, uint8_t *stage, const float *lw,
                                              const float *lb, double eps, int bx) {
  constexpr int R = 16 * MT, TPR = 256 / R;  // threads per row for the moments
  const int nch = K / 32;
  x += (int64_t)blockIdx.y * R * ldx;
  M -= blockIdx.y * R;
  stage += (size_t)blockIdx.y * nch * chunk_bytes<MT>();
  __shared__ float s_mean[R], s_inv[R];
  // This thread's group of 4 values (and with lw its LayerNorm weight and
  // bias), loaded before the moments' loads so that they arrive with them.
  const int i = bx * 256 + threadIdx.x;
  const bool item = i < R * nch * 8;  // whole groups of 8: R * nch * 8 and the block are multiples of 8
  const int gq = i & 7, row = (i >> 3) % R, c = (i >> 3) / R, k = c * 32 + 4 * gq;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f), w4 = v, b4 = v;
  if (item && row < M) {
    v = *reinterpret_cast<const float4 *>(x + (int64_t)row * ldx + k);
    if constexpr (NORM) {
      w4 = *reinterpret_cast<const float4 *>(lw + k);
      b4 = *reinterpret_cast<const float4 *>(lb + k);
    }
  }
  if constexpr (NORM) {
    const int r = threadIdx.x / TPR, part = threadIdx.x % TPR;
    double shift = 0.0, s1 = 0.0, s2 = 0.0;
    const int span = K / TPR;  // a multiple of 4 (K % 256 == 0)
    constexpr int U = 40;      // float4 loads in flight (a 2560-value row of 16: one round)
    // Buffer loads: a load past the span gets an offset past the rows and
    // reads zeros (never added), so every load issues before any wait (a
    // conditional plain load became a branch and a wait per load).
    const __amdgpu_buffer_rsrc_t rx = plane_rsrc(reinterpret_cast<const uint8_t *>(x), (int64_t)M * ldx * 4);
    const uint32_t xs = (uint32_t)(((int64_t)min(r, M - 1) * ldx + part * span) * 4);
    for (int k0 = 0; k0 < span; k0 += 4 * U) {
      float4 t[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const uint32_t off = k0 + 4 * u < span ? xs + (uint32_t)(k0 + 4 * u) * 4 : kNone;
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0);
        t[u] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
      }
      // the moments are taken about the row's first value, which the row's
      // first thread (lanes TPR-aligned) holds first
      if (k0 == 0) shift = (double)__shfl(t[0].x, (int)(threadIdx.x & 63) & ~(TPR - 1), 64);
#pragma unroll
      for (int u = 0; u < U; u++) {
        const bool in = k0 + 4 * u < span;  // past the span: +0.0 added (a select, no branch)
        const float e[4] = {t[u].x, t[u].y, t[u].z, t[u].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const double dv = in ? (double)e[q] - shift : 0.0;
          s1 += dv;
          s2 += dv * dv;
        }
      }
    }
#pragma unroll
    for (int o = 1; o < TPR; o <<= 1) {  // the row's threads are TPR consecutive lanes
      s1 += __shfl_xor(s1, o, 64);
      s2 += __shfl_xor(s2, o, 64);
    }
    if (part == 0) {
      const double mean = shift + s1 / (double)K;
      const double var = fmax((s2 - s1 * s1 / (double)K) / (double)K, 0.0);
      s_mean[r] = (float)mean;
      s_inv[r] = (float)(1.0 / sqrt(var + eps));
    }
    __syncthreads();
  }
  if (!item) return;
  if (row < M) {
    if constexpr (NORM) {
      const float fm = s_mean[row], inv = s_inv[row];
      auto affine = [&](float xv, float wv, float bv) {
        return __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(xv, fm), inv), wv), bv);
      };
      v = make_float4(affine(v.x, w4.x, b4.x), affine(v.y, w4.y, b4.y), affine(v.z, w4.z, b4.z),
                      affine(v.w, w4.w, b4.w));
    }
  }
  const float vv[4] = {v.x, v.y, v.z, v.w};
  uint32_t pl[kPlanes][2];
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    float r = vv[e], part = 0.f;
#pragma unroll
    for (int p = 0; p < kPlanes; p++) {
      const __bf16 h = (__bf16)r;
      const uint32_t bits = __builtin_bit_cast(uint16_t, h);
      pl[p][e / 2] = e % 2 ? pl[p][e / 2] | bits << 16 : bits;
      part += (float)h;
      r -= (float)h;
    }
    s += part;
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  const float s32 = s + __shfl_xor(s, 4, 64);
  uint8_t *cb = stage + (size_t)c * chunk_bytes<MT>();
  const int pos = gq < 4 ? 8 * gq : 8 * (gq - 4) + 4;
#pragma unroll
  for (int p = 0; p < kPlanes; p++)
    *reinterpret_cast<uint2 *>(cb + ((p * R + row) * 32 + pos) * 2) = make_uint2(pl[p][0], pl[p][1]);
  float *sums = reinterpret_cast<float *>(cb + kPlanes * R * 64);
  if (gq == 0) {
    sums[row] = s32;
    sums[R + row] = s;
  } else if (gq == 4) {
    sums[2 * R + row] = s;
  }
}

// bf16 bits of an integer-valued float with |v| <= 256 (exact).
__device__ __forceinline__ uint32_t pack_exact(float a, float b) {
  return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xFFFF0000u);
}
// The four bytes of v as exact bf16 (byte conversions, then the upper
// halves). A biased form (bits 0x4300 | q = 128 + q) would save the
// conversions but put 128 * xsum into every product, whose fp32 rounding
// then exceeds the reference's tolerance where a sum nearly cancels.
__device__ __forceinline__ uint2 exact_bf16(uint32_t v) {
  // opaque to the compiler, which would otherwise fold the callers' masks
  // into a bit-field extract per value instead of v_cvt_f32_ubyteN
  asm volatile("" : "+v"(v));
  return make_uint2(pack_exact((float)(v & 255u), (float)((v >> 8) & 255u)),
                    pack_exact((float)((v >> 16) & 255u), (float)(v >> 24)));
}
// Bit e of a 4-bit x to bit 0 of byte e.
__device__ __forceinline__ uint32_t spread1(uint32_t x) {
  uint32_t t = x | (x << 7);
  t |= t << 14;
  return t & 0x01010101u;
}
// Bits 2e..2e+1 of an 8-bit x to bits 0-1 of byte e.
__device__ __forceinline__ uint32_t spread2(uint32_t x) {
  uint32_t t = x | (x << 6);
  t |= t << 12;
  return t & 0x03030303u;
}

// One batch (8 chunks) of a wave's two 16-row tiles, as loaded.
struct Quants {
  uint32_t qv[2][8], hv[2][8][2], m1[2][8];
  uint4 mt[2];
  uint32_t d6[2];
};

template <int MT, bool NORM>
__global__ __launch_bounds__(256) void kq_stage_kernel(const float *x, int ldx, int M, int K, uint8_t *stage,
                                                       const float *lw, const float *lb, double eps) {
  kq_stage_body<MT, NORM>(x, ldx, M, K, stage, lw, lb, eps, blockIdx.x);
}

// Two inputs of the same rows staged in one launch (no LayerNorm; one
// slice of rows), the second's blocks after the first's.
template <int MT>
__global__ __launch_bounds__(256) void kq_stage_pair_kernel(const float *x1, int ldx1, int K1, uint8_t *s1,
                                                            const float *x2, int ldx2, int K2, uint8_t *s2, int M,
                                                            int blocks1) {
  if ((int)blockIdx.x < blocks1)
    kq_stage_body<MT, false>(x1, ldx1, M, K1, s1, nullptr, nullptr, 0.0, blockIdx.x);
  else
    kq_stage_body<MT, false>(x2, ldx2, M, K2, s2, nullptr, nullptr, 0.0, (int)blockIdx.x - blocks1);
}

// One block's work: block bx of the product (bx = split * NB + row block).
template <int F, int MT>
__device__ __forceinline__ void kq_rows_body(const KqArgs &g, int bx, uint8_t *lds) {
  constexpr int R = 16 * MT;
  constexpr int CB = chunk_bytes<MT>();
  constexpr int kCopy = (kWindow * CB / 16 + kThreads - 1) / kThreads;  // 16-byte pieces per thread
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const MatDesc w = g.w;
  const int N = w.rows, K = w.cols, nch = (K + 31) / 32;
  const int NB = (N + kBlockRows - 1) / kBlockRows;
  const int nb = bx % NB, split = bx / NB;
  // K range of the split, in whole batches of 8 chunks
  const int batches = (nch + 7) / 8;
  const int b_lo = (int)((int64_t)batches * split / g.ks), b_hi = (int)((int64_t)batches * (split + 1) / g.ks);
  const int c_lo = b_lo * 8, c_hi = min(nch, b_hi * 8);
  // slice blockIdx.y: rows [R y, R y + R) of x, staged at y * nch * CB
  const int Ms = min(R, g.M - (int)blockIdx.y * R);
  const uint8_t *stage = g.stage + (int64_t)blockIdx.y * nch * CB;
  float *y = g.y + (int64_t)split * g.split_stride + (int64_t)blockIdx.y * R * g.ldy;

  // ---- staged chunks [c0, min(c0 + 8, c_hi)) -> window buffer buf.
  // Buffer loads: pieces past the staged chunks read zeros (stored into
  // window slots no product reads), so no lane branches.
  const __amdgpu_buffer_rsrc_t rs = plane_rsrc(stage, (int64_t)nch * CB);
  auto load_x = [&](uint4 (&xr)[kCopy], int c0) {
    const uint32_t end = (uint32_t)min(c0 + kWindow, c_hi) * CB;
#pragma unroll
    for (int j = 0; j < kCopy; j++) {
      const uint32_t off = (uint32_t)c0 * CB + (uint32_t)(tid + j * kThreads) * 16;
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(off < end ? off : kNone), 0, 0);
      xr[j] = make_uint4(v.x, v.y, v.z, v.w);
    }
  };
  auto store_x = [&](const uint4 (&xr)[kCopy], int buf) {
    uint4 *dst = reinterpret_cast<uint4 *>(lds + (size_t)buf * kWindow * CB);
#pragma unroll
    for (int j = 0; j < kCopy; j++) {
      const int i = tid + j * kThreads;
      if (kWindow * CB % (16 * kThreads) == 0 || i < kWindow * CB / 16) dst[i] = xr[j];
    }
  };

  // ---- the wave's 32 matrix rows: lane = 16 * g4 + r16 holds row r16 of
  // each 16-row tile and (after the transpose below) bytes 4 * g4 .. + 3 of
  // every chunk
  const int g4 = lane >> 4, r16 = lane & 15;
  const int row0 = nb * kBlockRows + wave * kWaveRows + r16;
  const __amdgpu_buffer_rsrc_t rv = plane_rsrc(w.vals, (int64_t)N * w.vstride);
  const __amdgpu_buffer_rsrc_t rm = plane_rsrc(w.meta, (int64_t)N * w.mstride);
  const __amdgpu_buffer_rsrc_t rh = plane_rsrc(w.hbits, (int64_t)N * w.hstride);
  uint32_t voff[2], moff[2], hoff[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int row = row0 + 16 * t;
    const bool in = row < N;
    voff[t] = in ? (uint32_t)(row * w.vstride + 16 * g4) : kNone;
    moff[t] = in ? (uint32_t)(row * w.mstride) : kNone;
    hoff[t] = in ? (uint32_t)(row * w.hstride) : kNone;
  }
  f32x4 acc[MT][2];
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int t = 0; t < 2; t++) acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Quant bytes: the four lanes of a row read 64 contiguous bytes per load
  // (lane group g: chunks c0 + g and c0 + 4 + g), then a 4 x 4 transpose
  // of dwords across the groups (v_permlane32_swap, v_permlane16_swap)
  // gives group g dword g of every chunk. High bits and block constants
  // are read whole by the four lanes of a row (one cache line).
  auto load_q = [&](Quants &q, int c0) {
#pragma unroll
    for (int t = 0; t < 2; t++) {
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const bool ok = voff[t] != kNone && c0 + 4 * i + g4 < c_hi;
        const u32x4 q4 = __builtin_amdgcn_raw_buffer_load_b128(
            rv, (int)(ok ? voff[t] + (uint32_t)(c0 + 4 * i) * 16 : kNone), 0, 0);
        uint32_t d[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const u32x2 r = __builtin_amdgcn_permlane32_swap(d[j], d[j + 2], false, false);
          d[j] = r.x;
          d[j + 2] = r.y;
        }
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
          const u32x2 r = __builtin_amdgcn_permlane16_swap(d[j], d[j + 1], false, false);
          d[j] = r.x;
          d[j + 1] = r.y;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) q.qv[t][4 * i + j] = d[j];
      }
      const bool rok = voff[t] != kNone;
      if constexpr (F == FMT_Q5_K || F == FMT_Q5_1) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const u32x4 h4 = __builtin_amdgcn_raw_buffer_load_b128(
              rh, (int)(rok ? hoff[t] + (uint32_t)(c0 + 4 * i) * 4 : kNone), 0, 0);
          q.hv[t][4 * i][0] = h4.x;
          q.hv[t][4 * i + 1][0] = h4.y;
          q.hv[t][4 * i + 2][0] = h4.z;
          q.hv[t][4 * i + 3][0] = h4.w;
        }
      }
      if constexpr (F == FMT_Q6_K) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 h4 = __builtin_amdgcn_raw_buffer_load_b128(
              rh, (int)(rok ? hoff[t] + (uint32_t)(c0 + 2 * i) * 8 : kNone), 0, 0);
          q.hv[t][2 * i][0] = h4.x;
          q.hv[t][2 * i][1] = h4.y;
          q.hv[t][2 * i + 1][0] = h4.z;
          q.hv[t][2 * i + 1][1] = h4.w;
        }
      }
      if constexpr (F == FMT_Q5_1) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const u32x4 m4 = __builtin_amdgcn_raw_buffer_load_b128(
              rm, (int)(rok ? moff[t] + (uint32_t)(c0 + 4 * i) * 4 : kNone), 0, 0);
          q.m1[t][4 * i] = m4.x;
          q.m1[t][4 * i + 1] = m4.y;
          q.m1[t][4 * i + 2] = m4.z;
          q.m1[t][4 * i + 3] = m4.w;
        }
      }
      if constexpr (F == FMT_Q4_K || F == FMT_Q5_K) {
        const u32x4 m4 = __builtin_amdgcn_raw_buffer_load_b128(
            rm, (int)(rok ? moff[t] + (uint32_t)(c0 / 8) * 16 : kNone), 0, 0);
        q.mt[t] = make_uint4(m4.x, m4.y, m4.z, m4.w);
      } else if constexpr (F == FMT_Q6_K) {
        const uint32_t mo = rok ? moff[t] + (uint32_t)(c0 / 8) * 32 : kNone;
        const u32x4 m4 = __builtin_amdgcn_raw_buffer_load_b128(rm, (int)mo, 0, 0);
        q.mt[t] = make_uint4(m4.x, m4.y, m4.z, m4.w);
        q.d6[t] = __builtin_amdgcn_raw_buffer_load_b32(rm, (int)(mo == kNone ? kNone : mo + 16), 0, 0);
      }
    }
  };

  auto compute = [&](const Quants &q, int c0, int buf) {
    const uint8_t *wb = lds + (size_t)buf * kWindow * CB;
    // Sub-block constants of the batch: acc += a * t - c * xsum per 32
    // values (c = b for q a - b, -b for q a + b), or a * (t - 32 xsum) per
    // 16 values (Q6_K, t over q). Values and roundings as decodeKBlock's
    // (a = d * scale, b = dmin * min); the 6-bit scales and mins of
    // Q4_K / Q5_K are unpacked four at a time (quant_k.go:69-77).
    float ka[2][16], kc[2][8];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      if constexpr (F == FMT_Q6_K) {
        const float d = half_to_float((uint16_t)q.d6[t]);
        const uint32_t sw[4] = {q.mt[t].x, q.mt[t].y, q.mt[t].z, q.mt[t].w};
#pragma unroll
        for (int i = 0; i < 16; i++) ka[t][i] = __fmul_rn(d, (float)(int8_t)(sw[i / 4] >> (8 * (i % 4))));
      } else if constexpr (F == FMT_Q5_1) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
          ka[t][u] = half_to_float((uint16_t)q.m1[t][u]);
          kc[t][u] = -half_to_float((uint16_t)(q.m1[t][u] >> 16));
        }
      } else {
        const float d = half_to_float((uint16_t)q.mt[t].x), dmin = half_to_float((uint16_t)(q.mt[t].x >> 16));
        const uint32_t y0 = q.mt[t].y, z0 = q.mt[t].z, w0 = q.mt[t].w;
        const uint32_t sc[2] = {y0 & 0x3F3F3F3Fu, (w0 & 0x0F0F0F0Fu) | ((y0 >> 2) & 0x30303030u)};
        const uint32_t mn[2] = {z0 & 0x3F3F3F3Fu, ((w0 >> 4) & 0x0F0F0F0Fu) | ((z0 >> 2) & 0x30303030u)};
#pragma unroll
        for (int u = 0; u < 8; u++) {
          ka[t][u] = __fmul_rn(d, (float)((sc[u / 4] >> (8 * (u % 4))) & 255u));
          kc[t][u] = __fmul_rn(dmin, (float)((mn[u / 4] >> (8 * (u % 4))) & 255u));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      if (c0 + u >= c_hi) break;
      const uint8_t *cb = wb + u * CB;
      // A operands: the staged rows of this chunk, every plane
      bf16x8 a[kPlanes][MT];
#pragma unroll
      for (int p = 0; p < kPlanes; p++)
#pragma unroll
        for (int m = 0; m < MT; m++)
          a[p][m] = *reinterpret_cast<const bf16x8 *>(cb + ((p * R + 16 * m + r16) * 32 + 8 * g4) * 2);
      const float *sums = reinterpret_cast<const float *>(cb + kPlanes * R * 64);
      f32x4 xsm[MT][2];
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if constexpr (F == FMT_Q6_K) {
          xsm[m][0] = *reinterpret_cast<const f32x4 *>(sums + R + 16 * m + 4 * g4);
          xsm[m][1] = *reinterpret_cast<const f32x4 *>(sums + 2 * R + 16 * m + 4 * g4);
        } else {
          xsm[m][0] = *reinterpret_cast<const f32x4 *>(sums + 16 * m + 4 * g4);
        }
      }
#pragma unroll
      for (int t = 0; t < 2; t++) {
        // the lane's 8 quants: values 4g..4g+3 (lo bytes) and 16+4g.. (hi)
        const uint32_t b = q.qv[t][u];
        uint32_t lo = b & 0x0F0F0F0Fu, hi = (b >> 4) & 0x0F0F0F0Fu;
        if constexpr (F == FMT_Q5_K || F == FMT_Q5_1) {
          lo |= spread1((q.hv[t][u][0] >> (4 * g4)) & 15u) << 4;
          hi |= spread1((q.hv[t][u][0] >> (16 + 4 * g4)) & 15u) << 4;
        } else if constexpr (F == FMT_Q6_K) {
          lo |= spread2((q.hv[t][u][0] >> (8 * g4)) & 255u) << 4;
          hi |= spread2((q.hv[t][u][1] >> (8 * g4)) & 255u) << 4;
        }
        const uint2 bl = exact_bf16(lo), bh = exact_bf16(hi);
        const uint4 bw = make_uint4(bl.x, bl.y, bh.x, bh.y);
        if constexpr (F == FMT_Q6_K) {
          const bf16x4 b0 = __builtin_bit_cast(bf16x4, make_uint2(bw.x, bw.y));
          const bf16x4 b1 = __builtin_bit_cast(bf16x4, make_uint2(bw.z, bw.w));
#pragma unroll
          for (int m = 0; m < MT; m++) {
            f32x4 t0 = {0.f, 0.f, 0.f, 0.f}, t1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < kPlanes; p++) {
              const uint4 av = __builtin_bit_cast(uint4, a[p][m]);
              t0 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, make_uint2(av.x, av.y)), b0,
                                                             t0, 0, 0, 0);
              t1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, make_uint2(av.z, av.w)), b1,
                                                             t1, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
              acc[m][t][v] = fmaf(ka[t][2 * u], fmaf(-32.f, xsm[m][0][v], t0[v]), acc[m][t][v]);
              acc[m][t][v] = fmaf(ka[t][2 * u + 1], fmaf(-32.f, xsm[m][1][v], t1[v]), acc[m][t][v]);
            }
          }
        } else {
          const bf16x8 bb = __builtin_bit_cast(bf16x8, bw);
#pragma unroll
          for (int m = 0; m < MT; m++) {
            f32x4 tt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < kPlanes; p++) tt = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[p][m], bb, tt, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; v++)
              acc[m][t][v] = fmaf(ka[t][u], tt[v], fmaf(-kc[t][u], xsm[m][0][v], acc[m][t][v]));
          }
        }
      }
    }
  };

  // Software pipeline over the batches: the next batch's quants and
  // staged chunks are loaded while this one is computed, then the chunks
  // go to the other window buffer before the barrier that ends the step.
  Quants qa, qb;
  uint4 xr[kCopy];
  if (c_lo < c_hi) {
    load_q(qa, c_lo);
    load_x(xr, c_lo);
    store_x(xr, 0);
  }
  __syncthreads();
  for (int c0 = c_lo; c0 < c_hi; c0 += 16) {
    const bool more = c0 + 8 < c_hi;
    if (more) {
      load_q(qb, c0 + 8);
      load_x(xr, c0 + 8);
    }
    compute(qa, c0, 0);
    if (more) store_x(xr, 1);
    __syncthreads();
    if (!more) break;
    const bool more2 = c0 + 16 < c_hi;
    if (more2) {
      load_q(qa, c0 + 16);
      load_x(xr, c0 + 16);
    }
    compute(qb, c0 + 8, 1);
    if (more2) store_x(xr, 0);
    __syncthreads();
  }
  // lane holds rows 4 * g4 + v of X tile m against matrix row row0 + 16 t
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int n = row0 + 16 * t;
    if (n >= N) continue;
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int xrow = 16 * m + 4 * g4 + v;
        if (xrow < Ms) y[(int64_t)xrow * g.ldy + n] = acc[m][t][v];
      }
  }
}

template <int F, int MT>
__global__ __launch_bounds__(kThreads) void kq_rows_kernel(KqArgs g) {
  extern __shared__ __align__(16) uint8_t lds[];
  kq_rows_body<F, MT>(g, blockIdx.x, lds);
}

// Two products of the same rows in one launch, the second's blocks after
// the first's, each block running its own product's format: their blocks
// share the device instead of running as two launches one after the other
// (each block's work and results are those of its own launch).
template <int F1, int F2, int MT>
__global__ __launch_bounds__(kThreads) void kq_rows_pair_kernel(KqArgs g1, KqArgs g2, int blocks1) {
  extern __shared__ __align__(16) uint8_t lds[];
  if ((int)blockIdx.x < blocks1)
    kq_rows_body<F1, MT>(g1, blockIdx.x, lds);
  else
    kq_rows_body<F2, MT>(g2, (int)blockIdx.x - blocks1, lds);
}

template <int F1, int F2, int MT>
hipError_t kq_pair_launch(const KqArgs &a, const KqArgs &b, hipStream_t st) {
  constexpr size_t lds = lds_bytes<MT>();
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&kq_rows_pair_kernel<F1, F2, MT>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  const int n1 = (a.w.rows + kBlockRows - 1) / kBlockRows * a.ks, n2 = (b.w.rows + kBlockRows - 1) / kBlockRows * b.ks;
  hipLaunchKernelGGL((kq_rows_pair_kernel<F1, F2, MT>), dim3(n1 + n2), dim3(kThreads), lds, st, a, b, n1);
  return hipGetLastError();
}

template <int MT>
hipError_t kq_pair_dispatch(const KqArgs &a, const KqArgs &b, hipStream_t st) {
  const int fa = a.w.fmt, fb = b.w.fmt;
  if (fa == FMT_Q6_K && fb == FMT_Q4_K) return kq_pair_launch<FMT_Q6_K, FMT_Q4_K, MT>(a, b, st);
  if (fa == FMT_Q4_K && fb == FMT_Q6_K) return kq_pair_launch<FMT_Q4_K, FMT_Q6_K, MT>(a, b, st);
  if (fa == FMT_Q4_K && fb == FMT_Q4_K) return kq_pair_launch<FMT_Q4_K, FMT_Q4_K, MT>(a, b, st);
  if (fa == FMT_Q6_K && fb == FMT_Q6_K) return kq_pair_launch<FMT_Q6_K, FMT_Q6_K, MT>(a, b, st);
  return hipErrorNotSupported;
}

template <int F, int MT>
hipError_t kq_launch(const KqArgs &g, hipStream_t st) {
  constexpr size_t lds = lds_bytes<MT>();
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&kq_rows_kernel<F, MT>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  const int NB = (g.w.rows + kBlockRows - 1) / kBlockRows;
  hipLaunchKernelGGL((kq_rows_kernel<F, MT>), dim3(NB * g.ks, (g.M + 16 * MT - 1) / (16 * MT)), dim3(kThreads), lds,
                     st, g);
  return hipGetLastError();
}

template <int MT>
hipError_t kq_dispatch(const KqArgs &g, hipStream_t st) {
  switch (g.w.fmt) {
    case FMT_Q4_K: return kq_launch<FMT_Q4_K, MT>(g, st);
    case FMT_Q5_K: return kq_launch<FMT_Q5_K, MT>(g, st);
    case FMT_Q6_K: return kq_launch<FMT_Q6_K, MT>(g, st);
    case FMT_Q5_1: return kq_launch<FMT_Q5_1, MT>(g, st);
    default: return hipErrorInvalidValue;
  }
}

template <int MT>
hipError_t kq_stage(const float *x, int ldx, int M, int K, uint8_t *stage, hipStream_t st, const float *lw = nullptr,
                    const float *lb = nullptr, double eps = 0.0) {
  const int items = 16 * MT * (K / 32) * 8;
  const dim3 grid((items + 255) / 256, (M + 16 * MT - 1) / (16 * MT));
  if (lw)
    hipLaunchKernelGGL((kq_stage_kernel<MT, true>), grid, dim3(256), 0, st, x, ldx, M, K, stage, lw, lb, eps);
  else
    hipLaunchKernelGGL((kq_stage_kernel<MT, false>), grid, dim3(256), 0, st, x, ldx, M, K, stage, lw, lb, eps);
  return hipGetLastError();
}

}  // namespace

bool kq_rows_supported(const MatDesc &w, int M) {
  return M >= 1 && M <= 32 && is_kquant(w.fmt) && w.cols % 32 == 0 && planes_fit(w) &&
         (w.fmt == FMT_Q5_1 || w.cols % 256 == 0);
}

size_t kq_rows_stage_bytes(int K, int M) {
  return (size_t)(K / 32) * (M <= 16 ? chunk_bytes<1>() : chunk_bytes<2>() * (size_t)((M + 31) / 32));
}

int kq_rows_splits(const MatDesc &w, int max_splits) {
  const int NB = (w.rows + kBlockRows - 1) / kBlockRows, batches = (w.cols / 32 + 7) / 8;
  // about 200 blocks a matrix, at least one batch per split: a branch
  // step's paired in-products (q/k/v and gate/up, 2560 + 13824 rows) then
  // fit one round of blocks at two per CU (456 blocks; the 3B K-quant
  // step 3.65-3.67 ms against 3.74-3.75 with 320 blocks a matrix and
  // 3.77-3.80 with 240, whose 564 blocks take a second round)
  return std::max(1, std::min({(200 + NB - 1) / NB, batches, max_splits}));
}

hipError_t launch_kq_stage_norm(const float *x, int ldx, int M, int K, const float *lw, const float *lb, double eps,
                                void *stage, hipStream_t st) {
  if (M < 1 || M > 32 || K < 256 || K % 256 || ldx < K || (ldx & 3) || (reinterpret_cast<uintptr_t>(x) & 15) || !lw ||
      !lb || (reinterpret_cast<uintptr_t>(lw) & 15) || (reinterpret_cast<uintptr_t>(lb) & 15) || !stage ||
      (reinterpret_cast<uintptr_t>(stage) & 15))
    return hipErrorInvalidValue;
  uint8_t *sb = static_cast<uint8_t *>(stage);
  return M <= 16 ? kq_stage<1>(x, ldx, M, K, sb, st, lw, lb, eps) : kq_stage<2>(x, ldx, M, K, sb, st, lw, lb, eps);
}

hipError_t launch_kq_rows(const MatDesc &w, const float *x, int ldx, int M, float *y, int ldy, int ks, void *stage,
                          hipStream_t st, bool staged, int64_t split_stride) {
  if (!kq_rows_supported(w, std::min(M, 32)) || M > 32 * 1024 || ks < 1 || ks > (w.cols / 32 + 7) / 8 ||
      ldx < w.cols || ldy < w.rows ||
      (reinterpret_cast<uintptr_t>(x) & 15) || (ldx & 3) || !stage || (reinterpret_cast<uintptr_t>(stage) & 15))
    return hipErrorInvalidValue;
  if (split_stride == 0) split_stride = (int64_t)M * ldy;
  if (ks > 1 && split_stride < (int64_t)M * ldy) return hipErrorInvalidValue;
  KqArgs g{w, static_cast<const uint8_t *>(stage), M, y, ldy, ks, split_stride};
  uint8_t *sb = static_cast<uint8_t *>(stage);
  if (M <= 16) {
    const hipError_t e = staged ? hipSuccess : kq_stage<1>(x, ldx, M, w.cols, sb, st);
    return e != hipSuccess ? e : kq_dispatch<1>(g, st);
  }
  const hipError_t e = staged ? hipSuccess : kq_stage<2>(x, ldx, M, w.cols, sb, st);
  return e != hipSuccess ? e : kq_dispatch<2>(g, st);
}

hipError_t launch_kq_stage_pair(const float *x1, int ldx1, int K1, void *stage1, const float *x2, int ldx2, int K2,
                                void *stage2, int M, hipStream_t st) {
  const float *xs[2] = {x1, x2};
  const int ld[2] = {ldx1, ldx2}, ks[2] = {K1, K2};
  void *ss[2] = {stage1, stage2};
  if (M < 1 || M > 32) return hipErrorInvalidValue;
  for (int i = 0; i < 2; i++)
    if (!xs[i] || ks[i] < 32 || ks[i] % 32 || ld[i] < ks[i] || (ld[i] & 3) || (reinterpret_cast<uintptr_t>(xs[i]) & 15) ||
        !ss[i] || (reinterpret_cast<uintptr_t>(ss[i]) & 15))
      return hipErrorInvalidValue;
  const int MT = M <= 16 ? 1 : 2, R = 16 * MT;
  const int b1 = (R * (K1 / 32) * 8 + 255) / 256, b2 = (R * (K2 / 32) * 8 + 255) / 256;
  uint8_t *p1 = static_cast<uint8_t *>(stage1), *p2 = static_cast<uint8_t *>(stage2);
  if (MT == 1)
    hipLaunchKernelGGL(kq_stage_pair_kernel<1>, dim3(b1 + b2), dim3(256), 0, st, x1, ldx1, K1, p1, x2, ldx2, K2, p2, M,
                       b1);
  else
    hipLaunchKernelGGL(kq_stage_pair_kernel<2>, dim3(b1 + b2), dim3(256), 0, st, x1, ldx1, K1, p1, x2, ldx2, K2, p2, M,
                       b1);
  return hipGetLastError();
}

bool kq_rows_pair_supported(int fmt1, int fmt2) {
  return (fmt1 == FMT_Q4_K || fmt1 == FMT_Q6_K) && (fmt2 == FMT_Q4_K || fmt2 == FMT_Q6_K);
}

hipError_t launch_kq_rows_pair(const KqProduct &a, const KqProduct &b, int M, hipStream_t st) {
  const KqProduct *p[2] = {&a, &b};
  KqArgs g[2];
  if (M < 1 || M > 32 || !kq_rows_pair_supported(a.w.fmt, b.w.fmt)) return hipErrorInvalidValue;
  for (int i = 0; i < 2; i++) {
    const KqProduct &q = *p[i];
    if (!kq_rows_supported(q.w, M) || q.ks < 1 || q.ks > (q.w.cols / 32 + 7) / 8 || q.ldy < q.w.rows || !q.y ||
        !q.stage || (reinterpret_cast<uintptr_t>(q.stage) & 15))
      return hipErrorInvalidValue;
    const int64_t ss = q.split_stride ? q.split_stride : (int64_t)M * q.ldy;
    if (q.ks > 1 && ss < (int64_t)M * q.ldy) return hipErrorInvalidValue;
    g[i] = KqArgs{q.w, static_cast<const uint8_t *>(q.stage), M, q.y, q.ldy, q.ks, ss};
  }
  return M <= 16 ? kq_pair_dispatch<1>(g[0], g[1], st) : kq_pair_dispatch<2>(g[0], g[1], st);
}
