// Prefill projections on the gfx950 matrix cores: Y[M][N] = X[M][K] * W^T
// with v_mfma_f32_16x16x32_bf16 (fp32 accumulation).
//
// Operands: X arrives as bf16 planes (split_bf16 below): with XS = 2 the
// pair hi + lo carries 16 significant bits of every activation, with XS = 1
// only hi. BF16 weights feed the cores as stored. Q8_0 quants (|q| <= 128)
// are exact in bf16; each K step of 32 is one Q8_0 block, so the block
// product is formed without scale and added as acc += d * block on the
// fp32 accumulators, which keeps the weights exact.
//
// Tiling: 128 x 128 output per 256-thread block, four waves of 64 x 64
// (4 x 4 tiles of 16 x 16), K step 32, double-buffered LDS. LDS rows are
// padded to 80 bytes so the 16-byte fragment reads of 16 consecutive rows
// cover all 64 banks once.
#include "kernels.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kBM = 128, kBN = 128, kBK = 32, kRow = 40;  // LDS row: 40 bf16 = 80 B

__device__ __forceinline__ uint32_t bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// x (fp32, rows of `k` values with stride ldx) -> bf16 hi (and lo = x - hi).
__global__ void split_bf16_kernel(const float *x, int ldx, int k, int64_t rows, uint16_t *hi, uint16_t *lo) {
  const int64_t total = rows * k;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / k, c = i % k;
    const float v = x[r * ldx + c];
    const __bf16 h = (__bf16)v;
    hi[i] = __builtin_bit_cast(uint16_t, h);
    if (lo) lo[i] = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)h));
  }
}

struct GemmArgs {
  MatDesc w;                  // N = rows, K = cols (a column view of a larger matrix is fine)
  const uint16_t *xh, *xl;    // bf16 planes [M][K]
  int M;
  float *y;
  int ldy;
};

template <int WF, int XS>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  __shared__ __align__(16) uint16_t sa[2][XS][kBM * kRow];
  __shared__ __align__(16) uint16_t sb[2][kBN * kRow];
  __shared__ float ss[2][kBN];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int K = g.w.cols, N = g.w.rows, nk = K / kBK;
  // Tile order: workgroups are dispatched round-robin over the 8 XCDs, each
  // with its own L2. Consecutive workgroups of one XCD take the M tiles of
  // one N tile, so a weight tile is fetched from HBM once and re-read from
  // that XCD's L2 by the other M tiles.
  const int MT = (g.M + kBM - 1) / kBM, NT = (N + kBN - 1) / kBN;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int nt = xcd + 8 * (slot / MT), mt = slot % MT;
  if (nt >= NT) return;  // the grid rounds NT up to a multiple of 8
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int srow = tid >> 1, shalf = tid & 1;  // staging: one row half (16 K values) per thread

  uint4 rah0, rah1, ral0, ral1, rb[2];
  uint16_t rs = 0;
  auto gload = [&](int kb) {
    const int k = kb * kBK + shalf * 16;
    const int m = m0 + srow;
    if (m < g.M) {
      const uint4 *p = reinterpret_cast<const uint4 *>(g.xh + (int64_t)m * K + k);
      rah0 = p[0];
      rah1 = p[1];
      if constexpr (XS == 2) {
        const uint4 *q = reinterpret_cast<const uint4 *>(g.xl + (int64_t)m * K + k);
        ral0 = q[0];
        ral1 = q[1];
      }
    } else {
      rah0 = rah1 = ral0 = ral1 = make_uint4(0, 0, 0, 0);
    }
    const int n = n0 + srow;
    if constexpr (WF == FMT_BF16) {
      if (n < N) {
        const uint4 *p = reinterpret_cast<const uint4 *>(g.w.vals + (int64_t)n * g.w.vstride + (int64_t)k * 2);
        rb[0] = p[0];
        rb[1] = p[1];
      } else {
        rb[0] = rb[1] = make_uint4(0, 0, 0, 0);
      }
    } else {
      rb[0] = n < N ? *reinterpret_cast<const uint4 *>(g.w.vals + (int64_t)n * g.w.vstride + k)
                    : make_uint4(0, 0, 0, 0);
      if (tid < kBN)
        rs = n0 + tid < N ? reinterpret_cast<const uint16_t *>(g.w.meta + (int64_t)(n0 + tid) * g.w.mstride)[kb] : 0;
    }
  };
  auto lstore = [&](int buf) {
    {
      uint4 *d = reinterpret_cast<uint4 *>(&sa[buf][0][srow * kRow + shalf * 16]);
      d[0] = rah0;
      d[1] = rah1;
      if constexpr (XS == 2) {
        uint4 *e = reinterpret_cast<uint4 *>(&sa[buf][XS - 1][srow * kRow + shalf * 16]);
        e[0] = ral0;
        e[1] = ral1;
      }
    }
    uint4 *d = reinterpret_cast<uint4 *>(&sb[buf][srow * kRow + shalf * 16]);
    if constexpr (WF == FMT_BF16) {
      d[0] = rb[0];
      d[1] = rb[1];
    } else {  // 16 int8 -> 16 bf16, exact
      const uint32_t ws[4] = {rb[0].x, rb[0].y, rb[0].z, rb[0].w};
      uint32_t o[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t v = ws[i];
        o[2 * i] = bf16_bits((float)(int8_t)v) | bf16_bits((float)(int8_t)(v >> 8)) << 16;
        o[2 * i + 1] = bf16_bits((float)(int8_t)(v >> 16)) | bf16_bits((float)(int8_t)(v >> 24)) << 16;
      }
      d[0] = make_uint4(o[0], o[1], o[2], o[3]);
      d[1] = make_uint4(o[4], o[5], o[6], o[7]);
      if (tid < kBN) ss[buf][tid] = hw_half(rs);
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  gload(0);
  lstore(0);
  __syncthreads();
  const int frow = lane & 15, fk = (lane >> 4) * 8;
  for (int kb = 0; kb < nk; kb++) {
    const int cur = kb & 1;
    if (kb + 1 < nk) gload(kb + 1);
    bf16x8 bfr[4];
#pragma unroll
    for (int ni = 0; ni < 4; ni++)
      bfr[ni] = *reinterpret_cast<const bf16x8 *>(&sb[cur][(wn * 64 + ni * 16 + frow) * kRow + fk]);
    float sc[4];
    if constexpr (WF == FMT_Q8_0) {
#pragma unroll
      for (int ni = 0; ni < 4; ni++) sc[ni] = ss[cur][wn * 64 + ni * 16 + frow];
    }
#pragma unroll
    for (int mi = 0; mi < 4; mi++) {
      bf16x8 ah = *reinterpret_cast<const bf16x8 *>(&sa[cur][0][(wm * 64 + mi * 16 + frow) * kRow + fk]);
      bf16x8 al;
      if constexpr (XS == 2) al = *reinterpret_cast<const bf16x8 *>(&sa[cur][XS - 1][(wm * 64 + mi * 16 + frow) * kRow + fk]);
#pragma unroll
      for (int ni = 0; ni < 4; ni++) {
        if constexpr (WF == FMT_Q8_0) {
          f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bfr[ni], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          if constexpr (XS == 2) t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bfr[ni], t, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++) acc[mi][ni][i] = fmaf(sc[ni], t[i], acc[mi][ni][i]);
        } else {
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bfr[ni], acc[mi][ni], 0, 0, 0);
          if constexpr (XS == 2) acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bfr[ni], acc[mi][ni], 0, 0, 0);
        }
      }
    }
    if (kb + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }
  // D fragment: lane holds rows 4 * (lane / 16) + i of column lane % 16.
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 4; ni++) {
      const int n = n0 + wn * 64 + ni * 16 + frow;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = m0 + wm * 64 + mi * 16 + (lane >> 4) * 4 + i;
        if (m < g.M) g.y[(int64_t)m * g.ldy + n] = acc[mi][ni][i];
      }
    }
}

template <int WF, int XS>
hipError_t gemm_launch(const GemmArgs &g, hipStream_t st) {
  const int NT = (g.w.rows + kBN - 1) / kBN, MT = (g.M + kBM - 1) / kBM;
  dim3 grid((NT + 7) / 8 * 8 * MT);
  hipLaunchKernelGGL((gemm_kernel<WF, XS>), grid, dim3(256), 0, st, g);
  return hipGetLastError();
}

}  // namespace

bool gemm_mfma_supported(const MatDesc &w) {
  return (w.fmt == FMT_Q8_0 || w.fmt == FMT_BF16) && w.cols % kBK == 0 && w.vstride % 16 == 0;
}

int gemm_planes(const MatDesc &) { return 2; }

hipError_t launch_split_bf16(const float *x, int ldx, int k, int64_t rows, uint16_t *hi, uint16_t *lo,
                             hipStream_t st) {
  const int64_t total = rows * k;
  const int grid = (int)std::min<int64_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL(split_bf16_kernel, dim3(grid), dim3(256), 0, st, x, ldx, k, rows, hi, lo);
  return hipGetLastError();
}

hipError_t launch_gemm_mfma(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int M, float *y, int ldy,
                            hipStream_t st) {
  if (!gemm_mfma_supported(w)) return hipErrorInvalidValue;
  GemmArgs g{w, xh, xl, M, y, ldy};
  if (w.fmt == FMT_Q8_0) return xl ? gemm_launch<FMT_Q8_0, 2>(g, st) : gemm_launch<FMT_Q8_0, 1>(g, st);
  return xl ? gemm_launch<FMT_BF16, 2>(g, st) : gemm_launch<FMT_BF16, 1>(g, st);
}
