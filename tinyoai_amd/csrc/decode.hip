// Decode-path kernels (one token through a StableLM layer) for gfx950.
//
// StableLM's parallel residual (stablelm.go:365-377) lets a layer run as
// three launches:
//   decode_in   LayerNorm(x) once per block into LDS, then every weight row
//               that reads it (q, k, v, gate, up) in one pass over HBM, with
//               RoPE, the KV append and SiLU-gate applied in the epilogue;
//   attention   split-K flash decode; the last block of a head combines;
//   decode_out  x = (x + o*a) + down*m over the o and down rows.
// Rows are handed out in "units" of two: a rotary pair (i, i + rot/2) of a
// q or k head, two adjacent non-rotary rows, or gate row i with up row i.
#include <algorithm>

#include "kernels.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ void store_kv(const KVDev &kv, int64_t idx, float v, bool k) {
  void *base = k ? kv.k : kv.v;
  if (kv.half)
    reinterpret_cast<uint16_t *>(base)[idx] = float_to_half(v);
  else
    reinterpret_cast<float *>(base)[idx] = v;
}

struct InArgs {
  LayerDev w;
  StableDims s;
  KVDev kv;
  const float *x, *rope;
  const int *pos;
  float *q_out, *m_out;
  int xlen;  // LDS vector length (>= d, covers padded chunks)
};

template <int FA, int FM, int U>
__global__ __launch_bounds__(kThreads) void decode_in_kernel(InArgs a) {
  extern __shared__ __align__(16) float lds[];
  double *red = reinterpret_cast<double *>(lds + ((a.xlen + 3) & ~3));
  const StableDims &s = a.s;
  for (int i = threadIdx.x; i < a.xlen; i += kThreads) lds[i] = i < s.d ? a.x[i] : 0.f;
  __syncthreads();
  layer_norm_lds(lds, s.d, a.w.ln_w, a.w.ln_b, s.eps, red);
  const int pos = *a.pos;
  const int lane = threadIdx.x & 63;
  const int half_hd = s.hd / 2, rh = s.rot / 2;
  const int nq = s.heads * half_hd, nk = s.kv_heads * half_hd;
  const int natt = nq + 2 * nk, total = natt + s.inter;
  for (int u = blockIdx.x * kWaves + (threadIdx.x >> 6); u < total; u += gridDim.x * kWaves) {
    if (u < natt) {
      int kind = u < nq ? 0 : (u < nq + nk ? 1 : 2);  // q, k, v
      const int uu = kind == 0 ? u : (kind == 1 ? u - nq : u - nq - nk);
      const int head = uu / half_hd, j = uu % half_hd;
      const MatDesc &M = kind == 0 ? a.w.q : (kind == 1 ? a.w.k : a.w.v);
      int d0, d1;
      const bool rotary = kind != 2 && j < rh;
      if (kind == 2) { d0 = 2 * j; d1 = d0 + 1; }
      else if (rotary) { d0 = j; d1 = j + rh; }
      else { d0 = s.rot + 2 * (j - rh); d1 = d0 + 1; }
      const int64_t r0 = (int64_t)head * s.hd + d0, r1 = (int64_t)head * s.hd + d1;
      float v0, v1;
      seg2_dot<FA, U>(M.vals + r0 * M.vstride, M.meta + r0 * M.mstride, lds, M.chunks,
                      M.vals + r1 * M.vstride, M.meta + r1 * M.mstride, lds, M.chunks, v0, v1);
      if (lane == 0) {
        if (rotary) {  // stableRotate (stablelm.go:309-326) with table sin/cos
          const float cs = a.rope[((int64_t)pos * rh + j) * 2], sn = a.rope[((int64_t)pos * rh + j) * 2 + 1];
          const float x0 = __fsub_rn(__fmul_rn(v0, cs), __fmul_rn(v1, sn));
          const float x1 = __fadd_rn(__fmul_rn(v1, cs), __fmul_rn(v0, sn));
          v0 = x0;
          v1 = x1;
        }
        if (kind == 0) {
          a.q_out[r0] = v0;
          a.q_out[r1] = v1;
        } else {  // storeKV (kv_cache.go:55-65), head-major [kvh][cap][hd]
          const int64_t base = ((int64_t)head * a.kv.cap + pos) * s.hd;
          store_kv(a.kv, base + d0, v0, kind == 1);
          store_kv(a.kv, base + d1, v1, kind == 1);
        }
      }
    } else {
      const int i = u - natt;
      const MatDesc &G = a.w.gate, &P = a.w.up;
      float g, up;
      seg2_dot<FM, U>(G.vals + (int64_t)i * G.vstride, G.meta + (int64_t)i * G.mstride, lds, G.chunks,
                      P.vals + (int64_t)i * P.vstride, P.meta + (int64_t)i * P.mstride, lds, P.chunks, g, up);
      if (lane == 0) a.m_out[i] = silu_gate(g, up);
    }
  }
}

struct OutArgs {
  LayerDev w;
  int d, inter, la, lm;  // la, lm: LDS lengths of a and m
  const float *a, *m;
  float *x;
};

template <int FA, int FM, int U>
__global__ __launch_bounds__(kThreads) void decode_out_kernel(OutArgs p) {
  extern __shared__ __align__(16) float lds[];
  float *xa = lds, *xm = lds + ((p.la + 3) & ~3);
  for (int i = threadIdx.x; i < p.la; i += kThreads) xa[i] = i < p.d ? p.a[i] : 0.f;
  for (int i = threadIdx.x; i < p.lm; i += kThreads) xm[i] = i < p.inter ? p.m[i] : 0.f;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const MatDesc &O = p.w.o, &D = p.w.down;
  for (int r = blockIdx.x * kWaves + (threadIdx.x >> 6); r < p.d; r += gridDim.x * kWaves) {
    float ao, ad;
    if constexpr (FA == FM) {
      seg2_dot<FA, U>(O.vals + (int64_t)r * O.vstride, O.meta + (int64_t)r * O.mstride, xa, O.chunks,
                      D.vals + (int64_t)r * D.vstride, D.meta + (int64_t)r * D.mstride, xm, D.chunks, ao, ad);
    } else {
      float unused;
      seg2_dot<FA, U>(O.vals + (int64_t)r * O.vstride, O.meta + (int64_t)r * O.mstride, xa, O.chunks,
                      nullptr, nullptr, nullptr, 0, ao, unused);
      seg2_dot<FM, U>(D.vals + (int64_t)r * D.vstride, D.meta + (int64_t)r * D.mstride, xm, D.chunks,
                      nullptr, nullptr, nullptr, 0, ad, unused);
    }
    if (lane == 0) p.x[r] = __fadd_rn(__fadd_rn(p.x[r], ao), ad);
  }
}

struct LnMvArgs {
  MatDesc w;
  const float *ln_w, *ln_b;
  double eps;
  const float *x;
  float *out;
  int xlen;
};

template <int F, int U>
__global__ __launch_bounds__(kThreads) void ln_matvec_kernel(LnMvArgs a) {
  extern __shared__ __align__(16) float lds[];
  double *red = reinterpret_cast<double *>(lds + ((a.xlen + 3) & ~3));
  const int cols = a.w.cols;
  for (int i = threadIdx.x; i < a.xlen; i += kThreads) lds[i] = i < cols ? a.x[i] : 0.f;
  __syncthreads();
  if (a.ln_w) layer_norm_lds(lds, cols, a.ln_w, a.ln_b, a.eps, red);
  const int lane = threadIdx.x & 63;
  const MatDesc &M = a.w;
  const int units = (M.rows + 1) / 2;
  for (int u = blockIdx.x * kWaves + (threadIdx.x >> 6); u < units; u += gridDim.x * kWaves) {
    const int64_t r0 = 2 * (int64_t)u, r1 = r0 + 1;
    const bool two = r1 < M.rows;
    float v0, v1;
    seg2_dot<F, U>(M.vals + r0 * M.vstride, M.meta + r0 * M.mstride, lds, M.chunks,
                   two ? M.vals + r1 * M.vstride : nullptr, two ? M.meta + r1 * M.mstride : nullptr, lds,
                   two ? M.chunks : 0, v0, v1);
    if (lane == 0) {
      a.out[r0] = v0;
      if (two) a.out[r1] = v1;
    }
  }
}

__global__ void embed_kernel(MatDesc emb, const int *ids, float *x) {
  const int j = blockIdx.x;
  const int64_t row = ids[j];
  for (int c = threadIdx.x; c < emb.cols; c += blockDim.x) x[(int64_t)j * emb.cols + c] = mat_value(emb, row, c);
}

// ---------------------------------------------------------------- attention
constexpr int kSplit = 64;  // positions per block (4 steps of 16)

struct AttArgs {
  StableDims s;
  KVDev kv;
  const float *q;
  const int *pos0;
  int max_splits;
  float *partials;
  unsigned *counters;
  float *out;
};

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

// One wave per (split, head, query). Lane = 4 * position-in-step + dim group:
// four lanes share a position, each holding hd/4 dimensions.
template <int HD, bool HALF>
__global__ __launch_bounds__(64) void attention_kernel(AttArgs a) {
  constexpr int DPL = HD / 4;
  const StableDims &s = a.s;
  const int split = blockIdx.x, h = blockIdx.y, j = blockIdx.z;
  const int pos = *a.pos0 + j;
  const int npos = pos + 1;
  const int nsplit = (npos + kSplit - 1) / kSplit;
  if (split >= nsplit) return;
  const int lane = threadIdx.x, g = lane & 3, pl = lane >> 2;
  const int kvh = h / (s.heads / s.kv_heads);
  const float *q = a.q + (int64_t)j * s.heads * HD + h * HD + g * DPL;
  float qr[DPL];
#pragma unroll
  for (int i = 0; i < DPL; i++) qr[i] = q[i];
  const int64_t head_base = (int64_t)kvh * a.kv.cap * HD;
  float score[kSplit / 16];
  float mx = -INFINITY;
#pragma unroll
  for (int st = 0; st < kSplit / 16; st++) {
    const int t = split * kSplit + st * 16 + pl;
    float p = 0.f;
    if (t < npos) {
      float kr[DPL];
      load_kv<DPL, HALF>(a.kv.k, head_base + (int64_t)t * HD + g * DPL, kr);
#pragma unroll
      for (int i = 0; i < DPL; i++) p = fmaf(qr[i], kr[i], p);
    }
    p += __shfl_xor(p, 1, 64);
    p += __shfl_xor(p, 2, 64);
    score[st] = t < npos ? __fdiv_rn(p, s.att_scale) : -INFINITY;
    mx = fmaxf(mx, score[st]);
  }
  mx = wave_max(mx);
  float o[DPL];
#pragma unroll
  for (int i = 0; i < DPL; i++) o[i] = 0.f;
  float l = 0.f;
#pragma unroll
  for (int st = 0; st < kSplit / 16; st++) {
    const int t = split * kSplit + st * 16 + pl;
    if (t < npos) {
      const float w = expf(score[st] - mx);
      if (g == 0) l += w;
      float vr[DPL];
      load_kv<DPL, HALF>(a.kv.v, head_base + (int64_t)t * HD + g * DPL, vr);
#pragma unroll
      for (int i = 0; i < DPL; i++) o[i] = fmaf(w, vr[i], o[i]);
    }
  }
  l = wave_sum(l);
#pragma unroll
  for (int i = 0; i < DPL; i++) {
    float v = o[i];
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    o[i] = v;
  }
  const int64_t qh = (int64_t)j * s.heads + h;
  float *part = a.partials + (qh * a.max_splits + split) * (HD + 2);
  if (lane == 0) { part[0] = mx; part[1] = l; }
  if (pl == 0) {
#pragma unroll
    for (int i = 0; i < DPL; i++) part[2 + g * DPL + i] = o[i];
  }
  __threadfence();
  int last = 0;
  if (lane == 0) last = atomicAdd(&a.counters[qh], 1u) == (unsigned)(nsplit - 1);
  last = __shfl(last, 0, 64);
  if (!last) return;
  __threadfence();
  // Combine the splits of this (query, head).
  const float *base = a.partials + qh * a.max_splits * (HD + 2);
  float m = -INFINITY;
  for (int sp = lane; sp < nsplit; sp += 64) m = fmaxf(m, base[sp * (HD + 2)]);
  m = wave_max(m);
  float L = 0.f;
  for (int sp = lane; sp < nsplit; sp += 64) {
    const float ms = base[sp * (HD + 2)];
    L += base[sp * (HD + 2) + 1] * expf(ms - m);
  }
  L = wave_sum(L);
  for (int dim = lane; dim < HD; dim += 64) {
    float acc = 0.f;
    for (int sp = 0; sp < nsplit; sp++) {
      const float ms = base[sp * (HD + 2)];
      acc = fmaf(base[sp * (HD + 2) + 2 + dim], expf(ms - m), acc);
    }
    a.out[(int64_t)j * s.heads * HD + h * HD + dim] = acc / L;
  }
  if (lane == 0) a.counters[qh] = 0u;
}

template <int HD>
hipError_t launch_attention_hd(const AttArgs &a, int nq, int max_pos, hipStream_t st) {
  dim3 grid((max_pos + kSplit) / kSplit, a.s.heads, nq);
  if (a.kv.half)
    hipLaunchKernelGGL((attention_kernel<HD, true>), grid, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL((attention_kernel<HD, false>), grid, dim3(64), 0, st, a);
  return hipGetLastError();
}

int round_up(int v, int m) { return (v + m - 1) / m * m; }

template <int F, int U>
hipError_t ln_matvec_launch(const LnMvArgs &a, int grid, hipStream_t st) {
  const size_t lds = (size_t)round_up(a.xlen, 4) * 4 + 8 * sizeof(double);
  hipLaunchKernelGGL((ln_matvec_kernel<F, U>), dim3(grid), dim3(kThreads), lds, st, a);
  return hipGetLastError();
}

}  // namespace

int device_cu_count() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    hipGetDevice(&dev);
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cus <= 0) cus = 256;
  }
  return cus;
}

#define TINYOAI_FMT_PAIR(FA, FM)                                                                     \
  if (w.q.fmt == FA && w.gate.fmt == FM) {                                                           \
    hipLaunchKernelGGL((decode_in_kernel<FA, FM, 4>), dim3(grid), dim3(kThreads), lds, st, a);       \
    return hipGetLastError();                                                                        \
  }

hipError_t launch_decode_in(const LayerDev &w, const StableDims &s, const KVDev &kv, const float *x,
                            const float *rope, const int *pos, float *q_out, float *m_out, int grid,
                            hipStream_t st) {
  InArgs a{w, s, kv, x, rope, pos, q_out, m_out, 0};
  a.xlen = std::max(w.q.chunks * values_per_chunk(w.q.fmt), w.gate.chunks * values_per_chunk(w.gate.fmt));
  a.xlen = std::max(a.xlen, s.d);
  const size_t lds = (size_t)round_up(a.xlen, 4) * 4 + 8 * sizeof(double);
  TINYOAI_FMT_PAIR(FMT_Q8_0, FMT_Q8_0)
  TINYOAI_FMT_PAIR(FMT_BF16, FMT_BF16)
  TINYOAI_FMT_PAIR(FMT_F32, FMT_F32)
  TINYOAI_FMT_PAIR(FMT_F16, FMT_F16)
  return hipErrorInvalidValue;
}
#undef TINYOAI_FMT_PAIR

#define TINYOAI_FMT_PAIR(FA, FM)                                                                     \
  if (w.o.fmt == FA && w.down.fmt == FM) {                                                           \
    hipLaunchKernelGGL((decode_out_kernel<FA, FM, 4>), dim3(grid), dim3(kThreads), lds, st, p);      \
    return hipGetLastError();                                                                        \
  }

hipError_t launch_decode_out(const LayerDev &w, const StableDims &s, const float *a, const float *m, float *x,
                             int grid, hipStream_t st) {
  OutArgs p{w, s.d, s.inter, 0, 0, a, m, x};
  p.la = std::max(w.o.chunks * values_per_chunk(w.o.fmt), s.d);
  p.lm = std::max(w.down.chunks * values_per_chunk(w.down.fmt), s.inter);
  const size_t lds = (size_t)(round_up(p.la, 4) + round_up(p.lm, 4)) * 4;
  TINYOAI_FMT_PAIR(FMT_Q8_0, FMT_Q8_0)
  TINYOAI_FMT_PAIR(FMT_BF16, FMT_BF16)
  TINYOAI_FMT_PAIR(FMT_F32, FMT_F32)
  TINYOAI_FMT_PAIR(FMT_F16, FMT_F16)
  return hipErrorInvalidValue;
}
#undef TINYOAI_FMT_PAIR

hipError_t launch_attention(const StableDims &s, const KVDev &kv, const float *q, const int *pos0, int nq,
                            int max_pos, float *partials, unsigned *counters, float *out, hipStream_t st) {
  AttArgs a{s, kv, q, pos0, (max_pos + kSplit) / kSplit, partials, counters, out};
  switch (s.hd) {
    case 8: return launch_attention_hd<8>(a, nq, max_pos, st);
    case 16: return launch_attention_hd<16>(a, nq, max_pos, st);
    case 32: return launch_attention_hd<32>(a, nq, max_pos, st);
    case 64: return launch_attention_hd<64>(a, nq, max_pos, st);
    case 80: return launch_attention_hd<80>(a, nq, max_pos, st);
    case 96: return launch_attention_hd<96>(a, nq, max_pos, st);
    case 128: return launch_attention_hd<128>(a, nq, max_pos, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_ln_matvec(const MatDesc &w, const float *ln_w, const float *ln_b, double eps, const float *x,
                            float *out, int grid, hipStream_t st) {
  LnMvArgs a{w, ln_w, ln_b, eps, x, out, std::max(w.chunks * values_per_chunk(w.fmt), w.cols)};
  switch (w.fmt) {
    case FMT_Q8_0: return ln_matvec_launch<FMT_Q8_0, 4>(a, grid, st);
    case FMT_BF16: return ln_matvec_launch<FMT_BF16, 4>(a, grid, st);
    case FMT_F32: return ln_matvec_launch<FMT_F32, 4>(a, grid, st);
    case FMT_F16: return ln_matvec_launch<FMT_F16, 4>(a, grid, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_embed(const MatDesc &emb, const int *ids, int n, float *x, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, st, emb, ids, x);
  return hipGetLastError();
}
