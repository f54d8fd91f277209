// Prefill-path kernels (a chunk of n tokens) for gfx950: row LayerNorm, a
// vector-unit projection GEMM for formats the matrix cores do not take, the
// fused in-projection epilogue, SiLU-gate and the parallel residual.
// Follows prefill.go:33-115 step for step.
#include <algorithm>

#include "epilogue.h"

namespace {

__global__ __launch_bounds__(256) void layer_norm_rows_kernel(const float *x, const float *w, const float *b,
                                                               double eps, int d, float *out, uint16_t *oh,
                                                               uint16_t *ol, int ldo) {
  extern __shared__ __align__(16) float lds[];
  double *red = reinterpret_cast<double *>(lds + ((d + 3) & ~3));
  const int64_t row = blockIdx.x;
  for (int i = threadIdx.x; i < d; i += blockDim.x) lds[i] = x[row * d + i];
  __syncthreads();
  layer_norm_lds(lds, d, w, b, eps, red);
  for (int i = threadIdx.x; i < d; i += blockDim.x) {
    if (out) out[row * d + i] = lds[i];
    if (oh) store_bf16_split(oh, ol, row * ldo + i, lds[i]);
  }
}

// out[n][N] = x[n][K] * W[N][K]^T, fp32 SIMT tiles of 64 tokens x 64 rows,
// each thread a 4 x 4 micro-tile; weights dequantized into LDS. As mulBatch
// does (matmul.go:55-95), products accumulate in float32 within 512-column
// blocks and the block partials in float64.
constexpr int kTM = 64, kTN = 64, kTK = 32, kBlockCols = 512;

__global__ __launch_bounds__(256) void gemm_simt_kernel(MatDesc w, const float *__restrict__ x, int n,
                                                         float *__restrict__ out) {
  __shared__ float xs[kTK][kTM + 4];
  __shared__ float ws[kTK][kTN + 4];
  const int m0 = blockIdx.y * kTM, n0 = blockIdx.x * kTN;
  const int K = w.cols, N = w.rows;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  double total[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += kTK) {
    for (int e = threadIdx.x; e < kTM * kTK; e += 256) {
      const int r = e / kTK, c = e % kTK;
      const int tok = m0 + r, col = k0 + c;
      xs[c][r] = (tok < n && col < K) ? x[(int64_t)tok * K + col] : 0.f;
      const int row = n0 + r;
      ws[c][r] = (row < N && col < K) ? mat_value(w, row, col) : 0.f;
    }
    __syncthreads();
#pragma unroll 8
    for (int c = 0; c < kTK; c++) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        a[i] = xs[c][ty * 4 + i];
        b[i] = ws[c][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jj = 0; jj < 4; jj++) acc[i][jj] = fmaf(a[i], b[jj], acc[i][jj]);
    }
    __syncthreads();
    if ((k0 + kTK) % kBlockCols == 0 || k0 + kTK >= K) {
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          total[i][jj] += (double)acc[i][jj];
          acc[i][jj] = 0.f;
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int tok = m0 + ty * 4 + i;
    if (tok >= n) continue;
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      const int row = n0 + tx * 4 + jj;
      if (row < N) out[(int64_t)tok * N + row] = (float)total[i][jj];
    }
  }
}

// One block per token: the fused in-projection epilogue (RoPE on q and k,
// storeKV at the token's absolute position, SiLU-gate), as prefill.go:60-96
// applies it row by row. With mh, the SiLU-gate outputs (the units from
// mu0 on) also go out as the down projection's bf16 operand planes, and to
// m only when m is given.
// With rows, token j sits at position rows[2j] and its K and V go to slot
// rows[2j + 1] of the cache kv (a branch cache: the slot of the branch's
// suffix entry).
// One epilogue's block (token blockIdx.x, block by of its gy on the grid's
// second dimension).
__device__ __forceinline__ void in_epilogue_body(const StableDims &s, const KVDev &kv, const float *y, int ldy,
                                                 const float *rope, const int *pos0, int units, float *q, float *m,
                                                 uint16_t *mh, uint16_t *ml, const int *rows, int ys, int ldm, int by,
                                                 int gy) {
  const int j = blockIdx.x;
  const int pos = rows ? rows[2 * j] : *pos0 + j;
  const int slot = rows ? rows[2 * j + 1] : pos;
  const float *yj = y + (int64_t)j * ldy;
  const float *rope_row = rope + (int64_t)pos * s.rot;
  const int mu0 = (s.win_q + 2 * s.win_kv) / 2;
  float *qj = q + (int64_t)j * s.heads * s.hd, *mj = m ? m + (int64_t)j * s.inter : nullptr;
  const int64_t split = (int64_t)gridDim.x * ldy;
  // block by takes every gy-th group of blockDim.x units; a thread
  // loads kBatch of its units before it stores any, and the next kBatch
  // before it stores those (the stores could alias y as far as the
  // compiler knows, so loads placed after them would each wait a memory
  // round trip).
  constexpr int kBatch = 4;
  const int stride = gy * blockDim.x;
  auto load = [&](int u0, float2 (&v)[kBatch]) {
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      const int u = u0 + b * stride;
      v[b] = u < units ? *reinterpret_cast<const float2 *>(yj + 2 * u) : make_float2(0.f, 0.f);
      for (int s2 = 1; s2 < ys; s2++) {
        if (u >= units) break;
        const float2 t = *reinterpret_cast<const float2 *>(yj + s2 * split + 2 * u);
        v[b].x = __fadd_rn(v[b].x, t.x);
        v[b].y = __fadd_rn(v[b].y, t.y);
      }
    }
  };
  float2 v[kBatch], nv[kBatch];
  int u0 = by * blockDim.x + threadIdx.x;
  if (u0 < units) load(u0, v);
  for (; u0 < units; u0 += kBatch * stride) {
    const int un = u0 + kBatch * stride;
    if (un < units) load(un, nv);
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      const int u = u0 + b * stride;
      if (u >= units) break;
      if (mh && u >= mu0) {
        const float g = s.silu ? silu_gate_llama(v[b].x, v[b].y) : silu_gate(v[b].x, v[b].y);
        if (mj) mj[u - mu0] = g;
        store_bf16_split(mh, ml, (int64_t)j * ldm + (u - mu0), g);
      } else {
        in_pair_epilogue(s, kv, rope_row, slot, u, v[b].x, v[b].y, qj, mj);
      }
    }
#pragma unroll
    for (int b = 0; b < kBatch; b++) v[b] = nv[b];
  }
}

__global__ void in_epilogue_kernel(StableDims s, KVDev kv, const float *y, int ldy, const float *rope,
                                   const int *pos0, int units, float *q, float *m, uint16_t *mh, uint16_t *ml,
                                   const int *rows, int ys, int ldm) {
  in_epilogue_body(s, kv, y, ldy, rope, pos0, units, q, m, mh, ml, rows, ys, ldm, blockIdx.y, gridDim.y);
}

struct InEpiArgs {
  StableDims s;
  const float *y;
  int ldy, units, ys, gy;
  float *m;
};
// Two epilogues of the same tokens in one launch (the second's blocks after
// the first's on the grid's second dimension): the branch step's q/k/v and
// gate/up products, each with its own dims, partials and split count.
__global__ void in_epilogue_pair_kernel(InEpiArgs a, InEpiArgs b, KVDev kv, const float *rope, float *q,
                                        const int *rows) {
  if ((int)blockIdx.y < a.gy)
    in_epilogue_body(a.s, kv, a.y, a.ldy, rope, nullptr, a.units, q, a.m, nullptr, nullptr, rows, a.ys, a.s.inter,
                     blockIdx.y, a.gy);
  else
    in_epilogue_body(b.s, kv, b.y, b.ldy, rope, nullptr, b.units, q, b.m, nullptr, nullptr, rows, b.ys, b.s.inter,
                     (int)blockIdx.y - a.gy, b.gy);
}

// sum = ((v[0] + v[1]) + v[2]) + ... over s partials n apart, eight
// loads in flight before their adds (the same order as one at a time).
__device__ __forceinline__ float sum_partials(const float *v, int s, int64_t n, int64_t i) {
  constexpr int B = 8;
  float acc = v[i];
  for (int s0 = 1; s0 < s; s0 += B) {
    float t[B];
#pragma unroll
    for (int k = 0; k < B; k++) t[k] = s0 + k < s ? v[(s0 + k) * n + i] : 0.f;
#pragma unroll
    for (int k = 0; k < B; k++)
      if (s0 + k < s) acc = __fadd_rn(acc, t[k]);
  }
  return acc;
}

// The residual of a chunk's row (residual_kernel's arithmetic) and the
// next layer's LayerNorm of it (layer_norm_rows_kernel's): one block per
// row stages the new row in LDS while it stores it, so the row is read
// once for both. Two elements per thread at a time, their loads issued
// before their stores.
__global__ __launch_bounds__(256) void residual_norm_rows_kernel(float *x, const float *p, int sp, const float *dd,
                                                                 int sd, int64_t n, int d, const float *w,
                                                                 const float *b, double eps, float *out, uint16_t *oh,
                                                                 uint16_t *ol, int ldo) {
  extern __shared__ __align__(16) float lds[];
  double *red = reinterpret_cast<double *>(lds + ((d + 3) & ~3));
  const int64_t row = blockIdx.x;
  constexpr int E = 2;
  for (int i0 = threadIdx.x; i0 < d; i0 += E * blockDim.x) {
    float v[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
      const int i = i0 + e * blockDim.x;
      if (i < d) {
        const int64_t k = row * d + i;
        v[e] = __fadd_rn(__fadd_rn(x[k], sum_partials(p, sp, n, k)), sum_partials(dd, sd, n, k));
      }
    }
#pragma unroll
    for (int e = 0; e < E; e++) {
      const int i = i0 + e * blockDim.x;
      if (i < d) {
        x[row * d + i] = v[e];
        lds[i] = v[e];
      }
    }
  }
  __syncthreads();
  layer_norm_lds(lds, d, w, b, eps, red);
  for (int i = threadIdx.x; i < d; i += blockDim.x) {
    if (out) out[row * d + i] = lds[i];
    if (oh) store_bf16_split(oh, ol, row * ldo + i, lds[i]);
  }
}

__global__ void residual_kernel(float *x, const float *p, int sp, const float *d, int sd, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float o = sum_partials(p, sp, n, i), m = sum_partials(d, sd, n, i);
    x[i] = __fadd_rn(__fadd_rn(x[i], o), m);
  }
}

// out[i] = ((p[0][i] + p[1][i]) + p[2][i]) + ... over sp partials n apart.
__global__ void sum_splits_kernel(float *out, const float *p, int sp, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    out[i] = sum_partials(p, sp, n, i);
  }
}

__global__ void copy_kernel(const float *src, float *dst, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = src[i];
}

// n 32-bit words, 16 bytes per store where both ends allow it: a wide copy
// (a host-mapped destination then takes full PCIe writes).
__global__ void copy_words_kernel(const uint32_t *src, uint32_t *dst, int n) {
  const int i4 = (blockIdx.x * blockDim.x + threadIdx.x);
  const int n4 = n / 4;
  if (i4 < n4) reinterpret_cast<uint4 *>(dst)[i4] = reinterpret_cast<const uint4 *>(src)[i4];
  const int t = n4 * 4 + i4;
  if (i4 < n - n4 * 4) dst[t] = src[t];
}

int elementwise_grid(int64_t n) { return (int)std::min<int64_t>((n + 255) / 256, 4096); }

}  // namespace

hipError_t launch_residual_norm_rows(float *x, const float *p, int sp, const float *dd, int sd, int n, int d,
                                     const float *w, const float *b, double eps, float *out, uint16_t *oh,
                                     uint16_t *ol, hipStream_t st) {
  if (sp < 1 || sd < 1 || !oh != !ol || (!out && !oh)) return hipErrorInvalidValue;
  const size_t lds = (size_t)((d + 3) & ~3) * 4 + 8 * sizeof(double);
  hipLaunchKernelGGL(residual_norm_rows_kernel, dim3(n), dim3(256), lds, st, x, p, sp, dd, sd, (int64_t)n * d, d, w, b,
                     eps, out, oh, ol, d);
  return hipGetLastError();
}

hipError_t launch_layer_norm_rows(const float *x, const float *w, const float *b, double eps, int n, int d,
                                  float *out, hipStream_t st, uint16_t *oh, uint16_t *ol, int ldo) {
  if (!oh != !ol || (ldo && ldo < d)) return hipErrorInvalidValue;
  const size_t lds = (size_t)((d + 3) & ~3) * 4 + 8 * sizeof(double);
  hipLaunchKernelGGL(layer_norm_rows_kernel, dim3(n), dim3(256), lds, st, x, w, b, eps, d, out, oh, ol,
                     ldo ? ldo : d);
  return hipGetLastError();
}

hipError_t launch_gemm(const MatDesc &w, const float *x, int n, float *out, hipStream_t st) {
  dim3 grid((w.rows + kTN - 1) / kTN, (n + kTM - 1) / kTM);
  hipLaunchKernelGGL(gemm_simt_kernel, grid, dim3(256), 0, st, w, x, n, out);
  return hipGetLastError();
}

hipError_t launch_in_epilogue(const StableDims &s, const KVDev &kv, const float *y, int ldy, const float *rope,
                              const int *pos0, int n, float *q, float *m, hipStream_t st, uint16_t *mh,
                              uint16_t *ml, const int *rows, int ys, int ldm) {
  if (ldy % 2 || !mh != !ml || (!m && !mh) || s.win_q % 2 || (!rows && !pos0) || ys < 1 || (ldm && ldm < s.inter))
    return hipErrorInvalidValue;
  const int units = (s.win_q + 2 * s.win_kv + 2 * s.inter) / 2;
  // each token's units over several blocks (about 8192 blocks for a chunk)
  const int per_token = std::max(1, std::min((units + 255) / 256, 8192 / std::max(1, n)));
  hipLaunchKernelGGL(in_epilogue_kernel, dim3(n, per_token), dim3(256), 0, st, s, kv, y, ldy, rope, pos0, units, q,
                     m, mh, ml, rows, ys, ldm ? ldm : s.inter);
  return hipGetLastError();
}

hipError_t launch_in_epilogue_pair(const StableDims &sa, const float *ya, int ldya, int ysa, const StableDims &sb,
                                   const float *yb, int ldyb, int ysb, const KVDev &kv, const float *rope,
                                   const int *rows, int n, float *q, float *m, hipStream_t st) {
  const StableDims *ss[2] = {&sa, &sb};
  const int ld[2] = {ldya, ldyb}, ys[2] = {ysa, ysb};
  InEpiArgs g[2];
  if (!rows || n < 1 || !ya || !yb) return hipErrorInvalidValue;
  for (int i = 0; i < 2; i++) {
    const StableDims &s = *ss[i];
    if (ld[i] % 2 || s.win_q % 2 || ys[i] < 1 || (s.inter && !m)) return hipErrorInvalidValue;
    const int units = (s.win_q + 2 * s.win_kv + 2 * s.inter) / 2;
    const int gy = std::max(1, std::min((units + 255) / 256, 8192 / n));
    g[i] = InEpiArgs{s, i ? yb : ya, ld[i], units, ys[i], gy, m};
  }
  hipLaunchKernelGGL(in_epilogue_pair_kernel, dim3(n, g[0].gy + g[1].gy), dim3(256), 0, st, g[0], g[1], kv, rope, q,
                     rows);
  return hipGetLastError();
}

hipError_t launch_residual(float *x, const float *p, int sp, const float *d, int sd, int64_t n, hipStream_t st) {
  if (sp < 1 || sd < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(residual_kernel, dim3(elementwise_grid(n)), dim3(256), 0, st, x, p, sp, d, sd, n);
  return hipGetLastError();
}

hipError_t launch_sum_splits(float *out, const float *p, int sp, int64_t n, hipStream_t st) {
  if (sp < 1 || n < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sum_splits_kernel, dim3(elementwise_grid(n)), dim3(256), 0, st, out, p, sp, n);
  return hipGetLastError();
}

hipError_t launch_copy_words(const void *src, void *dst, int n, hipStream_t st) {
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) return hipErrorInvalidValue;
  const int threads = 256, blocks = std::max(1, (n / 4 + threads - 1) / threads);
  hipLaunchKernelGGL(copy_words_kernel, dim3(blocks), dim3(threads), 0, st, reinterpret_cast<const uint32_t *>(src),
                     reinterpret_cast<uint32_t *>(dst), n);
  return hipGetLastError();
}

hipError_t launch_copy_row(const float *src, float *dst, int n, hipStream_t st) {
  hipLaunchKernelGGL(copy_kernel, dim3(1), dim3(256), 0, st, src, dst, n);
  return hipGetLastError();
}
