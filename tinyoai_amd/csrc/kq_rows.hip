// Products of a few activation rows with a 5/6-bit quantized matrix on the
// gfx950 matrix cores: Y[M][N] = X[M][K] * W^T for M <= 32 (the rows of a
// batched branch step), W in Q4_K, Q5_K, Q6_K or Q5_1.
//
// Every value of these formats is q * a - b (Q4_K, Q5_K), q * a + b (Q5_1)
// or (q - 32) * a (Q6_K), with a small integer q and constants a, b shared
// by a sub-block of 32 values (16 for Q6_K) (decodeKBlock,
// quant_k.go:31-86). q is exact in bf16, so each sub-block's products run
// on the matrix cores unscaled,
//   t[m][n] = sum over the sub-block of x[m][k] * q[n][k],
// with x as three bf16 planes (hi + mid + lo: 24 significant bits, as
// fp32 holds), and are added to fp32 accumulators as
// acc += a * t - b * xsum, xsum[m] being the sub-block's sum of x (of
// hi + mid + lo, the values the products saw).
//
// A block of 4 waves takes 128 matrix rows (32 a wave, two 16-row tiles)
// over one range of K, in windows of up to 16 chunks (8 with 32 rows):
// the window's X is staged in LDS as bf16 planes (with the sub-block
// sums), then each wave streams its rows' quants straight from HBM and
// forms v_mfma_f32_16x16x32_bf16 products per 32-value chunk (two
// v_mfma_f32_16x16x16_bf16, one per 16-value sub-block, for Q6_K). K
// ranges (splits) write separate partial outputs, split s at
// y + s * M * ldy, which the consumer sums.
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

// Chunks (32 values) of one K range a block can stage: 16 * MT rows,
// three bf16 planes and a float sum per chunk, within 50 KB of LDS.
template <int MT>
constexpr int max_chunks() { return MT == 1 ? 16 : 8; }
template <int MT>
constexpr size_t lds_bytes() { return (size_t)max_chunks<MT>() * 16 * MT * (kPlanes * 64 + 4); }

struct KqArgs {
  MatDesc w;
  const float *x;
  int ldx, M;
  float *y;
  int ldy, ks;
};

// bf16 bits of an integer-valued float with |v| <= 256 (exact).
__device__ __forceinline__ uint32_t pack_exact(float a, float b) {
  return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xFFFF0000u);
}

template <int F, int MT>
__global__ __launch_bounds__(kThreads) void kq_rows_kernel(KqArgs g) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int R = 16 * MT;  // staged rows
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const MatDesc w = g.w;
  const int N = w.rows, K = w.cols, nch = (K + 31) / 32;
  const int NB = (N + kBlockRows - 1) / kBlockRows;
  const int nb = blockIdx.x % NB, split = blockIdx.x / NB;
  // K range of the split, in whole batches of 8 chunks (a super-block)
  const int batches = (nch + 7) / 8;
  const int b_lo = (int)((int64_t)batches * split / g.ks), b_hi = (int)((int64_t)batches * (split + 1) / g.ks);
  const int c_lo = b_lo * 8, c_hi = min(nch, b_hi * 8);
  float *y = g.y + (int64_t)split * g.M * g.ldy;
  constexpr int kWindow = max_chunks<MT>();

  uint16_t *xs = reinterpret_cast<uint16_t *>(lds);
  // ---- stage X rows [0, M) x chunks [w0, w0 + cn): planes [3][cn][R][32] bf16, sums [cn][R]
  auto stage = [&](int w0, int cn, float *xsum) {
    const int items = R * cn * 8;  // float4 groups: (row, chunk, group of 4 values)
    for (int i = tid; i < items; i += kThreads) {
      const int row = i / (cn * 8), q = i % (cn * 8), cl = q >> 3, gq = q & 7;
      const int k = (w0 + cl) * 32 + 4 * gq;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row < g.M) {
        const float *p = g.x + (int64_t)row * g.ldx + k;
        if (k + 3 < K) {
          v = *reinterpret_cast<const float4 *>(p);
        } else {
          v.x = k < K ? p[0] : 0.f;
          v.y = k + 1 < K ? p[1] : 0.f;
          v.z = k + 2 < K ? p[2] : 0.f;
          v.w = k + 3 < K ? p[3] : 0.f;
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
      // the chunk's 8 groups are 8 consecutive lanes (items and the block
      // are multiples of 8): a fixed-order sum
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      s += __shfl_xor(s, 4, 64);
      const int pos = gq < 4 ? 8 * gq : 8 * (gq - 4) + 4;
      const size_t at = ((size_t)cl * R + row) * 32 + pos;
#pragma unroll
      for (int p = 0; p < kPlanes; p++)
        *reinterpret_cast<uint2 *>(xs + (size_t)p * cn * R * 32 + at) = make_uint2(pl[p][0], pl[p][1]);
      if (gq == 0) xsum[cl * R + row] = s;
    }
  };

  // ---- stream the wave's 32 rows over the range
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
    voff[t] = in ? (uint32_t)(row * w.vstride + 4 * g4) : kNone;
    moff[t] = in ? (uint32_t)(row * w.mstride) : kNone;
    hoff[t] = in ? (uint32_t)(row * w.hstride) : kNone;
  }
  f32x4 acc[MT][2];
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int t = 0; t < 2; t++) acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int w0 = c_lo; w0 < c_hi; w0 += kWindow) {
    const int cn = min(kWindow, c_hi - w0), w1 = w0 + cn;
    float *xsum = reinterpret_cast<float *>(lds + (size_t)kPlanes * cn * R * 64);
    if (w0 > c_lo) __syncthreads();  // the previous window's reads are done
    stage(w0, cn, xsum);
    __syncthreads();
    for (int c0 = w0; c0 < w1; c0 += 8) {
      // the batch's loads: 8 chunks x 2 tiles of quant bytes, high bits and
      // block constants
      uint32_t qv[2][8], hv[2][8][2];
      uint4 mt[2];
      uint32_t d6[2];
#pragma unroll
      for (int t = 0; t < 2; t++) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
          const uint32_t off = voff[t] == kNone || c0 + u >= c_hi ? kNone : voff[t] + (uint32_t)(c0 + u) * 16;
          qv[t][u] = __builtin_amdgcn_raw_buffer_load_b32(rv, (int)off, 0, 0);
          if constexpr (F == FMT_Q5_K || F == FMT_Q5_1) {
            const uint32_t ho = hoff[t] == kNone || c0 + u >= c_hi ? kNone : hoff[t] + (uint32_t)(c0 + u) * 4;
            hv[t][u][0] = __builtin_amdgcn_raw_buffer_load_b32(rh, (int)ho, 0, 0);
          } else if constexpr (F == FMT_Q6_K) {
            const uint32_t ho = hoff[t] == kNone || c0 + u >= c_hi ? kNone : hoff[t] + (uint32_t)(c0 + u) * 8;
            const u32x2 h2 = __builtin_amdgcn_raw_buffer_load_b64(rh, (int)ho, 0, 0);
            hv[t][u][0] = h2.x;
            hv[t][u][1] = h2.y;
          }
        }
        if constexpr (F == FMT_Q4_K || F == FMT_Q5_K) {
          const u32x4 m4 = __builtin_amdgcn_raw_buffer_load_b128(rm, (int)(moff[t] == kNone ? kNone : moff[t] + (uint32_t)(c0 / 8) * 16), 0, 0);
          mt[t] = make_uint4(m4.x, m4.y, m4.z, m4.w);
        } else if constexpr (F == FMT_Q6_K) {
          const uint32_t mo = moff[t] == kNone ? kNone : moff[t] + (uint32_t)(c0 / 8) * 32;
          const u32x4 m4 = __builtin_amdgcn_raw_buffer_load_b128(rm, (int)mo, 0, 0);
          mt[t] = make_uint4(m4.x, m4.y, m4.z, m4.w);
          d6[t] = __builtin_amdgcn_raw_buffer_load_b32(rm, (int)(mo == kNone ? kNone : mo + 16), 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = c0 + u;
        if (c >= c_hi) break;
        const int cl = c - w0;
        // A operands: the staged rows of this chunk, every plane
        bf16x8 a[kPlanes][MT];
#pragma unroll
        for (int p = 0; p < kPlanes; p++)
#pragma unroll
          for (int m = 0; m < MT; m++)
            a[p][m] = *reinterpret_cast<const bf16x8 *>(xs + (size_t)p * cn * R * 32 +
                                                       ((size_t)cl * R + 16 * m + r16) * 32 + 8 * g4);
        f32x4 xsm[MT];
        if constexpr (F != FMT_Q6_K) {
#pragma unroll
          for (int m = 0; m < MT; m++) xsm[m] = *reinterpret_cast<const f32x4 *>(xsum + cl * R + 16 * m + 4 * g4);
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
          // the lane's 8 quants: values 4g..4g+3 (low nibbles), 16+4g.. (high)
          const uint32_t b = qv[t][u];
          float qf[8];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            int ql = (b >> (8 * e)) & 15, qh = (b >> (8 * e + 4)) & 15;
            if constexpr (F == FMT_Q5_K || F == FMT_Q5_1) {
              ql |= ((hv[t][u][0] >> (4 * g4 + e)) & 1) << 4;
              qh |= ((hv[t][u][0] >> (16 + 4 * g4 + e)) & 1) << 4;
            } else if constexpr (F == FMT_Q6_K) {
              ql |= ((hv[t][u][0] >> (8 * g4 + 2 * e)) & 3) << 4;
              qh |= ((hv[t][u][1] >> (8 * g4 + 2 * e)) & 3) << 4;
              ql -= 32;
              qh -= 32;
            }
            qf[e] = (float)ql;
            qf[4 + e] = (float)qh;
          }
          const uint4 bw = make_uint4(pack_exact(qf[0], qf[1]), pack_exact(qf[2], qf[3]), pack_exact(qf[4], qf[5]),
                                      pack_exact(qf[6], qf[7]));
          KConst k;
          if constexpr (F == FMT_Q5_1) {
            const uint32_t mo = moff[t] == kNone ? kNone : moff[t] + (uint32_t)c * 4;
            const uint32_t m1 = __builtin_amdgcn_raw_buffer_load_b32(rm, (int)mo, 0, 0);
            k = kquant_const<F>(make_uint4(m1, 0, 0, 0), 0, c);
          } else {
            k = kquant_const<F>(mt[t], (uint16_t)d6[t], c);
          }
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
              for (int v = 0; v < 4; v++) acc[m][t][v] = fmaf(k.a2, t1[v], fmaf(k.a, t0[v], acc[m][t][v]));
            }
          } else {
            const bf16x8 bb = __builtin_bit_cast(bf16x8, bw);
#pragma unroll
            for (int m = 0; m < MT; m++) {
              f32x4 tt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int p = 0; p < kPlanes; p++) tt = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[p][m], bb, tt, 0, 0, 0);
              const float bs = F == FMT_Q5_1 ? k.b : -k.b;
#pragma unroll
              for (int v = 0; v < 4; v++) acc[m][t][v] = fmaf(k.a, tt[v], fmaf(bs, xsm[m][v], acc[m][t][v]));
            }
          }
        }
      }
    }
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
        const int xr = 16 * m + 4 * g4 + v;
        if (xr < g.M) y[(int64_t)xr * g.ldy + n] = acc[m][t][v];
      }
  }
}

template <int F, int MT>
hipError_t kq_launch(const KqArgs &g, hipStream_t st) {
  constexpr size_t lds = lds_bytes<MT>();
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&kq_rows_kernel<F, MT>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  const int NB = (g.w.rows + kBlockRows - 1) / kBlockRows;
  hipLaunchKernelGGL((kq_rows_kernel<F, MT>), dim3(NB * g.ks), dim3(kThreads), lds, st, g);
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

}  // namespace

bool kq_rows_supported(const MatDesc &w, int M) {
  return M >= 1 && M <= 32 && is_kquant(w.fmt) && w.cols % 32 == 0 && planes_fit(w) &&
         (w.fmt == FMT_Q5_1 || w.cols % 256 == 0);
}

int kq_rows_splits(const MatDesc &w, int max_splits) {
  const int NB = (w.rows + kBlockRows - 1) / kBlockRows, batches = (w.cols / 32 + 7) / 8;
  // about two blocks per CU, at least one super-block per split
  return std::max(1, std::min({(512 + NB - 1) / NB, batches, max_splits}));
}

hipError_t launch_kq_rows(const MatDesc &w, const float *x, int ldx, int M, float *y, int ldy, int ks,
                          hipStream_t st) {
  if (!kq_rows_supported(w, M) || ks < 1 || ks > (w.cols / 32 + 7) / 8 || ldx < w.cols ||
      ldy < w.rows || (reinterpret_cast<uintptr_t>(x) & 15) || (ldx & 3))
    return hipErrorInvalidValue;
  KqArgs g{w, x, ldx, M, y, ldy, ks};
  return M <= 16 ? kq_dispatch<1>(g, st) : kq_dispatch<2>(g, st);
}
