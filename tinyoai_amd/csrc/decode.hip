// Decode-path kernels (one token through a StableLM layer) for gfx950.
//
// StableLM's parallel residual (stablelm.go:365-377) lets a layer run as
// three launches over the fused matrices of LayerDev (kernels.h):
//   decode_in   LayerNorm(x) once per block into LDS, then every row of win
//               (q, k, v, gate, up) in one pass over HBM, with RoPE, the KV
//               append and SiLU-gate applied in the epilogue; layer 0 also
//               gathers the token's embedding row here;
//   attention   split-K flash decode; blocks of a head combine through the
//               last-arriving block;
//   decode_out  x = (x + o*a) + down*m, one wout row [o | down] per unit.
// decode_in hands out win rows in pairs (2u, 2u + 1): a rotary pair, two
// adjacent non-rotary dims, or gate row i with up row i. Each wave streams
// its units with the next batch of weight loads in flight (stream_units,
// formats.h).
#include <algorithm>

#include "epilogue.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct InArgs {
  LayerDev w;
  StableDims s;
  KVDev kv;
  float *x;             // residual [d]; written here when emb is set
  MatDesc emb;          // embedding table (layer 0, when use_emb)
  int use_emb;
  const int *token;     // token id (layer 0)
  const float *rope;
  const int *pos;
  float *q_out, *m_out;
};

template <int F, int U, int T>
__global__ __launch_bounds__(T) void decode_in_kernel(InArgs a) {
  extern __shared__ __align__(16) float lds[];
  constexpr int VPC = Fmt<F>::VPC;
  const MatDesc &W = a.w.win;
  const int nch = W.chunks;
  const StableDims &s = a.s;
  float4 *xq = reinterpret_cast<float4 *>(lds + ((s.d + 3) & ~3));
  double *red = reinterpret_cast<double *>(xq + (VPC / 4) * nch);
  float *rope_row = reinterpret_cast<float *>(red + 16);  // cos/sin at pos, [rot/2][2]
  const int pos = *a.pos;
  const int lane = threadIdx.x & 63;

  auto prologue = [&]() {
    if (a.use_emb) {  // embedding row (stablelm.go:338), bit-exact readValues
      const MatDesc &e = a.emb;
      const int64_t row = *a.token;
      for (int i = threadIdx.x; i < s.d; i += T) {
        const float v = mat_value(e, row, i);
        lds[i] = v;
        if (blockIdx.x == 0) a.x[i] = v;
      }
    } else {
      for (int i = threadIdx.x; i < s.d; i += T) lds[i] = a.x[i];
    }
    __syncthreads();
    norm_lds(s, lds, a.w.ln_w, a.w.ln_b, red);
    stage_x(xq, lds, s.d, nch, VPC);
    for (int i = threadIdx.x; i < s.rot; i += T) rope_row[i] = a.rope[(int64_t)pos * s.rot + i];
    __syncthreads();
  };
  auto unit = [&](int u, Seg2 &g) { g = Seg2{row_ptr(W, 2 * (int64_t)u), row_ptr(W, 2 * (int64_t)u + 1), xq, xq, nch, nch}; };
  auto done = [&](int u, float v0, float v1) {
    if (lane == 0) in_pair_epilogue(s, a.kv, rope_row, pos, u, v0, v1, a.q_out, a.m_out);
  };
  stream_units<F, U>(blockIdx.x * (T / 64) + (threadIdx.x >> 6), gridDim.x * (T / 64), W.rows / 2, prologue, unit,
                     done);
}

struct OutArgs {
  MatDesc w;
  int ka, km;  // values of the o and down parts of a wout row
  int na, nm;  // their chunks
  const float *a, *m;
  float *x;
};

template <int F, int U, int T>
__global__ __launch_bounds__(T) void decode_out_kernel(OutArgs p) {
  extern __shared__ __align__(16) float4 xq_lds[];
  constexpr int VPC = Fmt<F>::VPC;
  const MatDesc &W = p.w;
  float4 *xa = xq_lds, *xm = xq_lds + (VPC / 4) * p.na;
  const int lane = threadIdx.x & 63;
  auto prologue = [&]() {
    stage_x(xa, p.a, p.ka, p.na, VPC);
    if (p.nm) stage_x(xm, p.m, p.km, p.nm, VPC);
    __syncthreads();
  };
  auto unit = [&](int r, Seg2 &g) { g = Seg2{row_ptr(W, r), row_ptr(W, r, p.na), xa, xm, p.na, p.nm}; };
  auto done = [&](int r, float ao, float ad) {
    if (lane == 0) p.x[r] = __fadd_rn(__fadd_rn(p.x[r], ao), ad);
  };
  stream_units<F, U>(blockIdx.x * (T / 64) + (threadIdx.x >> 6), gridDim.x * (T / 64), p.w.rows, prologue, unit,
                     done);
}

struct LnMvArgs {
  MatDesc w;
  const float *ln_w, *ln_b;
  double eps;
  int norm;
  const float *x;
  float *out;
  int xlen;
};

template <int F, int U, int T>
__global__ __launch_bounds__(T) void ln_matvec_kernel(LnMvArgs a) {
  extern __shared__ __align__(16) float lds[];
  constexpr int VPC = Fmt<F>::VPC;
  const int cols = a.w.cols;
  const int lane = threadIdx.x & 63;
  const MatDesc &M = a.w;
  float4 *xq = reinterpret_cast<float4 *>(lds + ((cols + 3) & ~3));
  double *red = reinterpret_cast<double *>(xq + (VPC / 4) * M.chunks);
  auto prologue = [&]() {
    for (int i = threadIdx.x; i < cols; i += T) lds[i] = a.x[i];
    __syncthreads();
    if (a.ln_w) {
      if (a.norm) rms_norm_lds(lds, cols, a.ln_w, (float)a.eps, red);
      else layer_norm_lds(lds, cols, a.ln_w, a.ln_b, a.eps, red);
    }
    stage_x(xq, lds, cols, M.chunks, VPC);
    __syncthreads();
  };
  auto unit = [&](int u, Seg2 &g) {
    const int64_t r0 = 2 * (int64_t)u, r1 = r0 + 1;
    const bool two = r1 < M.rows;
    g = Seg2{row_ptr(M, r0), row_ptr(M, two ? r1 : r0), xq, xq, M.chunks, two ? M.chunks : 0};
  };
  auto done = [&](int u, float v0, float v1) {
    if (lane != 0) return;
    a.out[2 * (int64_t)u] = v0;
    if (2 * u + 1 < M.rows) a.out[2 * (int64_t)u + 1] = v1;
  };
  stream_units<F, U>(blockIdx.x * (T / 64) + (threadIdx.x >> 6), gridDim.x * (T / 64), (M.rows + 1) / 2, prologue,
                     unit, done);
}

__global__ void embed_kernel(MatDesc emb, const int *ids, float *x) {
  const int j = blockIdx.x;
  const int64_t row = ids[j];
  for (int c = threadIdx.x; c < emb.cols; c += blockDim.x) x[(int64_t)j * emb.cols + c] = mat_value(emb, row, c);
}

// ---------------------------------------------------------------- attention
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

// Agent-scope relaxed atomic store of a partial result.
__device__ __forceinline__ void publish(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One block of 4 waves per (split, head, query); a split covers
// 4 * STEPS * 16 positions. Lane = 4 * position-in-step + dim group: four
// lanes share a position, each holding hd/4 dimensions. Online-softmax
// partials combine across the waves in LDS, then across the splits of a
// (query, head) in the last block to finish (the others exit).
template <int HD, bool HALF, int STEPS>
__global__ __launch_bounds__(kThreads) void attention_kernel(AttArgs a) {
  constexpr int DPL = HD / 4;
  constexpr int SPLIT = kWaves * STEPS * 16;
  __shared__ float s_m[kWaves], s_l[kWaves], s_o[kWaves][HD];
  __shared__ float s_e[512];
  __shared__ int s_last;
  const StableDims &s = a.s;
  const int split = blockIdx.x, h = blockIdx.y, j = blockIdx.z;
  const int pos = *a.pos0 + j;
  const int npos = pos + 1;
  const int nsplit = (npos + SPLIT - 1) / SPLIT;
  if (split >= nsplit) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane & 3, pl = lane >> 2;
  const int kvh = h / (s.heads / s.kv_heads);
  const float *q = a.q + (int64_t)j * s.heads * HD + h * HD + g * DPL;
  float qr[DPL];
#pragma unroll
  for (int i = 0; i < DPL; i++) qr[i] = q[i];
  const int64_t head_base = (int64_t)kvh * a.kv.cap * HD;
  const int t0 = split * SPLIT + wave * STEPS * 16 + pl;
  // Narrow blocks issue the V loads with the K loads (one memory round
  // trip); wide ones load V after the scores to bound register use.
  constexpr bool kEarlyV = STEPS <= 2;
  float kr[STEPS][DPL], vr[STEPS][DPL];
#pragma unroll
  for (int st = 0; st < STEPS; st++)
    if (t0 + st * 16 < npos) {
      load_kv<DPL, HALF>(a.kv.k, head_base + (int64_t)(t0 + st * 16) * HD + g * DPL, kr[st]);
      if constexpr (kEarlyV)
        load_kv<DPL, HALF>(a.kv.v, head_base + (int64_t)(t0 + st * 16) * HD + g * DPL, vr[st]);
    }
  float score[STEPS];
  float mx = -INFINITY;
#pragma unroll
  for (int st = 0; st < STEPS; st++) {
    const int t = t0 + st * 16;
    float p = 0.f;
    if (t < npos) {
#pragma unroll
      for (int i = 0; i < DPL; i++) p = fmaf(qr[i], kr[st][i], p);
    }
    p += __shfl_xor(p, 1, 64);
    p += __shfl_xor(p, 2, 64);
    score[st] = t < npos ? __fdiv_rn(p, s.att_scale) : -INFINITY;
    mx = fmaxf(mx, score[st]);
  }
  mx = wave_max(mx);
  if constexpr (!kEarlyV) {
#pragma unroll
    for (int st = 0; st < STEPS; st++)
      if (t0 + st * 16 < npos) load_kv<DPL, HALF>(a.kv.v, head_base + (int64_t)(t0 + st * 16) * HD + g * DPL, vr[st]);
  }
  float o[DPL];
#pragma unroll
  for (int i = 0; i < DPL; i++) o[i] = 0.f;
  float l = 0.f;
#pragma unroll
  for (int st = 0; st < STEPS; st++) {
    if (t0 + st * 16 < npos) {
      const float w = expf(score[st] - mx);
      if (g == 0) l += w;
#pragma unroll
      for (int i = 0; i < DPL; i++) o[i] = fmaf(w, vr[st][i], o[i]);
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
  if (lane == 0) { s_m[wave] = mx; s_l[wave] = l; }
  if (pl == 0) {
#pragma unroll
    for (int i = 0; i < DPL; i++) s_o[wave][g * DPL + i] = o[i];
  }
  __syncthreads();
  // combine the waves (a wave with no valid position has m = -inf, l = 0)
  float M = s_m[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) M = fmaxf(M, s_m[w]);
  float L = 0.f, ew[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; w++) {
    ew[w] = expf(s_m[w] - M);
    L = fmaf(s_l[w], ew[w], L);
  }
  const int64_t qh = (int64_t)j * s.heads + h;
  float *outp = a.out + (int64_t)j * s.heads * HD + h * HD;
  if (nsplit == 1) {
    for (int d = tid; d < HD; d += kThreads) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; w++) acc = fmaf(s_o[w][d], ew[w], acc);
      outp[d] = acc / L;
    }
    return;
  }
  // Cross-block combine. Partials are written with agent-scope relaxed
  // atomic stores (write-through, visible across the XCDs' L2 caches) and
  // ordered before the arrival increment by waiting for the stores; an
  // agent-scope fence would write back and invalidate the whole L2 instead.
  // Each (query, head) owns a 256-byte aligned region that only its last
  // block reads, once, after every store to it: no cache holds a stale copy
  // of those lines, so plain (pipelined) loads are safe there.
  float *region = a.partials + qh * partial_region(a.max_splits, HD);
  float *part = region + split * (HD + 2);
  if (tid == 0) {
    publish(part, M);
    publish(part + 1, L);
  }
  for (int d = tid; d < HD; d += kThreads) {
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) acc = fmaf(s_o[w][d], ew[w], acc);
    publish(part + 2 + d, acc);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores have completed
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(&a.counters[qh], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (unsigned)(nsplit - 1);
  __syncthreads();
  if (!s_last) return;
  // Last block of this (query, head): every other split has published.
  const float *base = region;
  float m = -INFINITY;
  for (int sp = tid; sp < nsplit; sp += kThreads) m = fmaxf(m, base[sp * (HD + 2)]);
  m = wave_max(m);
  if (lane == 0) s_m[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
  float lsum = 0.f;
  for (int sp = tid; sp < nsplit; sp += kThreads) {
    const float e = expf(base[sp * (HD + 2)] - m);
    s_e[sp] = e;
    lsum = fmaf(base[sp * (HD + 2) + 1], e, lsum);
  }
  lsum = wave_sum(lsum);
  __syncthreads();
  if (lane == 0) s_l[wave] = lsum;
  __syncthreads();
  const float Ltot = (s_l[0] + s_l[1]) + (s_l[2] + s_l[3]);
  for (int d = tid; d < HD; d += kThreads) {
    float acc = 0.f;
#pragma unroll 8
    for (int sp = 0; sp < nsplit; sp++) acc = fmaf(base[sp * (HD + 2) + 2 + d], s_e[sp], acc);
    outp[d] = acc / Ltot;
  }
  if (tid == 0) __hip_atomic_store(&a.counters[qh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD, bool HALF>
hipError_t launch_attention_hd(const AttArgs &a, int nq, int splits, int steps, hipStream_t st) {
  dim3 grid(splits, a.s.heads, nq);
  switch (steps) {
    case 1: hipLaunchKernelGGL((attention_kernel<HD, HALF, 1>), grid, dim3(kThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL((attention_kernel<HD, HALF, 2>), grid, dim3(kThreads), 0, st, a); break;
    case 4: hipLaunchKernelGGL((attention_kernel<HD, HALF, 4>), grid, dim3(kThreads), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int HD>
hipError_t launch_attention_kv(const AttArgs &a, int nq, int splits, int steps, hipStream_t st) {
  return a.kv.half ? launch_attention_hd<HD, true>(a, nq, splits, steps, st)
                   : launch_attention_hd<HD, false>(a, nq, splits, steps, st);
}

int round_up(int v, int m) { return (v + m - 1) / m * m; }

// Batch width U (chunks per lane per batch): the smallest instantiated
// value that covers a whole unit, else 8 with several batches per unit.
int pick_u(int chunks_per_unit) {
  static const int us[] = {1, 2, 4, 5, 8, 10};
  for (int u : us)
    if (64 * u >= chunks_per_unit) return u;
  return 8;
}

#define TINYOAI_DISPATCH_U(U, LAUNCH) \
  switch (U) {                        \
    case 1: LAUNCH(1); break;         \
    case 2: LAUNCH(2); break;         \
    case 4: LAUNCH(4); break;         \
    case 5: LAUNCH(5); break;         \
    case 8: LAUNCH(8); break;         \
    case 10: LAUNCH(10); break;       \
  }

#define TINYOAI_DISPATCH_T(T, LAUNCH)                   \
  switch (T) {                                          \
    case 256: TINYOAI_DISPATCH_U(U, LAUNCH##256) break; \
    case 512: TINYOAI_DISPATCH_U(U, LAUNCH##512) break; \
    case 640: TINYOAI_DISPATCH_U(U, LAUNCH##640) break; \
    case 1024: TINYOAI_DISPATCH_U(U, LAUNCH##1024) break; \
    default: return hipErrorInvalidValue;               \
  }

template <int F>
hipError_t ln_matvec_launch(const LnMvArgs &a, int grid, int threads, hipStream_t st) {
  const size_t lds = (size_t)round_up(a.w.cols, 4) * 4 + (size_t)a.w.chunks * Fmt<F>::VPC * 4 + 16 * sizeof(double);
  const int U = pick_u(2 * a.w.chunks);
#define L256(U_) hipLaunchKernelGGL((ln_matvec_kernel<F, U_, 256>), dim3(grid), dim3(256), lds, st, a)
#define L512(U_) hipLaunchKernelGGL((ln_matvec_kernel<F, U_, 512>), dim3(grid), dim3(512), lds, st, a)
#define L640(U_) hipLaunchKernelGGL((ln_matvec_kernel<F, U_, 640>), dim3(grid), dim3(640), lds, st, a)
#define L1024(U_) hipLaunchKernelGGL((ln_matvec_kernel<F, U_, 1024>), dim3(grid), dim3(1024), lds, st, a)
  TINYOAI_DISPATCH_T(threads, L)
#undef L256
#undef L512
#undef L640
#undef L1024
  return hipGetLastError();
}

template <int F>
hipError_t decode_in_launch(const InArgs &a, int grid, int threads, hipStream_t st) {
  const size_t lds = (size_t)round_up(a.s.d, 4) * 4 + (size_t)a.w.win.chunks * Fmt<F>::VPC * 4 +
                     16 * sizeof(double) + (size_t)a.s.rot * 4;
  const int U = pick_u(2 * a.w.win.chunks);
#define L256(U_) hipLaunchKernelGGL((decode_in_kernel<F, U_, 256>), dim3(grid), dim3(256), lds, st, a)
#define L512(U_) hipLaunchKernelGGL((decode_in_kernel<F, U_, 512>), dim3(grid), dim3(512), lds, st, a)
#define L640(U_) hipLaunchKernelGGL((decode_in_kernel<F, U_, 640>), dim3(grid), dim3(640), lds, st, a)
#define L1024(U_) hipLaunchKernelGGL((decode_in_kernel<F, U_, 1024>), dim3(grid), dim3(1024), lds, st, a)
  TINYOAI_DISPATCH_T(threads, L)
#undef L256
#undef L512
#undef L640
#undef L1024
  return hipGetLastError();
}

template <int F>
hipError_t decode_out_launch(OutArgs p, int grid, int threads, hipStream_t st) {
  constexpr int VPC = Fmt<F>::VPC;
  // The down part starts a new quant block (and super-block).
  const int align = F == FMT_Q8_0 || F == FMT_Q5_1 ? 32 : (is_kquant(F) ? 256 : 1);
  if (p.ka % align) return hipErrorInvalidValue;
  p.na = (p.ka + VPC - 1) / VPC;
  p.nm = p.w.chunks - p.na;
  if (p.nm < 0 || (p.km == 0) != (p.nm == 0) || (int64_t)p.nm * VPC < p.km) return hipErrorInvalidValue;
  const size_t lds = (size_t)p.w.chunks * VPC * 4;
  const int U = pick_u(p.w.chunks);
#define L256(U_) hipLaunchKernelGGL((decode_out_kernel<F, U_, 256>), dim3(grid), dim3(256), lds, st, p)
#define L512(U_) hipLaunchKernelGGL((decode_out_kernel<F, U_, 512>), dim3(grid), dim3(512), lds, st, p)
#define L640(U_) hipLaunchKernelGGL((decode_out_kernel<F, U_, 640>), dim3(grid), dim3(640), lds, st, p)
#define L1024(U_) hipLaunchKernelGGL((decode_out_kernel<F, U_, 1024>), dim3(grid), dim3(1024), lds, st, p)
  TINYOAI_DISPATCH_T(threads, L)
#undef L256
#undef L512
#undef L640
#undef L1024
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

hipError_t launch_decode_in(const LayerDev &w, const StableDims &s, const KVDev &kv, float *x, const MatDesc *emb,
                            const int *token, const float *rope, const int *pos, float *q_out, float *m_out, int grid,
                            int threads, hipStream_t st) {
  InArgs a{w, s, kv, x, emb ? *emb : MatDesc{}, emb != nullptr, token, rope, pos, q_out, m_out};
  if (w.win.rows % 2) return hipErrorInvalidValue;
  switch (w.win.fmt) {
    case FMT_Q8_0: return decode_in_launch<FMT_Q8_0>(a, grid, threads, st);
    case FMT_BF16: return decode_in_launch<FMT_BF16>(a, grid, threads, st);
    case FMT_F32: return decode_in_launch<FMT_F32>(a, grid, threads, st);
    case FMT_F16: return decode_in_launch<FMT_F16>(a, grid, threads, st);
    case FMT_Q5_1: return decode_in_launch<FMT_Q5_1>(a, grid, threads, st);
    case FMT_Q4_K: return decode_in_launch<FMT_Q4_K>(a, grid, threads, st);
    case FMT_Q5_K: return decode_in_launch<FMT_Q5_K>(a, grid, threads, st);
    case FMT_Q6_K: return decode_in_launch<FMT_Q6_K>(a, grid, threads, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_decode_out(const MatDesc &wout, int ka, int km, const float *a, const float *m, float *x,
                             int grid, int threads, hipStream_t st) {
  OutArgs p{wout, ka, km, 0, 0, a, m, x};
  switch (wout.fmt) {
    case FMT_Q8_0: return decode_out_launch<FMT_Q8_0>(p, grid, threads, st);
    case FMT_BF16: return decode_out_launch<FMT_BF16>(p, grid, threads, st);
    case FMT_F32: return decode_out_launch<FMT_F32>(p, grid, threads, st);
    case FMT_F16: return decode_out_launch<FMT_F16>(p, grid, threads, st);
    case FMT_Q5_1: return decode_out_launch<FMT_Q5_1>(p, grid, threads, st);
    case FMT_Q4_K: return decode_out_launch<FMT_Q4_K>(p, grid, threads, st);
    case FMT_Q5_K: return decode_out_launch<FMT_Q5_K>(p, grid, threads, st);
    case FMT_Q6_K: return decode_out_launch<FMT_Q6_K>(p, grid, threads, st);
  }
  return hipErrorInvalidValue;
}

int attention_steps(int max_pos, int heads) {
  // Positions per block (64 * steps): two steps (V loaded with K, one
  // memory round trip) measured fastest on gfx950 at 512-768 positions;
  // narrower blocks when that leaves fewer than 64 blocks.
  const int npos = max_pos + 1;
  int steps = 2;
  while (steps > 1 && (npos + 64 * steps - 1) / (64 * steps) * heads < 64) steps /= 2;
  return steps;
}

int attention_splits(int max_pos, int steps) { return (max_pos + 64 * steps) / (64 * steps); }

hipError_t launch_attention(const StableDims &s, const KVDev &kv, const float *q, const int *pos0, int nq,
                            int max_pos, float *partials, unsigned *counters, float *out, hipStream_t st, int steps,
                            int splits) {
  if (steps <= 0) steps = attention_steps(max_pos, s.heads);
  if (splits <= 0) splits = attention_splits(max_pos, steps);
  if (splits > 512) return hipErrorInvalidValue;  // combine scratch holds 512 splits
  AttArgs a{s, kv, q, pos0, splits, partials, counters, out};
  switch (s.hd) {
    case 8: return launch_attention_kv<8>(a, nq, splits, steps, st);
    case 16: return launch_attention_kv<16>(a, nq, splits, steps, st);
    case 32: return launch_attention_kv<32>(a, nq, splits, steps, st);
    case 64: return launch_attention_kv<64>(a, nq, splits, steps, st);
    case 80: return launch_attention_kv<80>(a, nq, splits, steps, st);
    case 96: return launch_attention_kv<96>(a, nq, splits, steps, st);
    case 128: return launch_attention_kv<128>(a, nq, splits, steps, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_ln_matvec(const MatDesc &w, const float *ln_w, const float *ln_b, double eps, int norm,
                            const float *x, float *out, int grid, int threads, hipStream_t st) {
  LnMvArgs a{w, ln_w, ln_b, eps, norm, x, out, std::max(w.chunks * values_per_chunk(w.fmt), w.cols)};
  switch (w.fmt) {
    case FMT_Q8_0: return ln_matvec_launch<FMT_Q8_0>(a, grid, threads, st);
    case FMT_BF16: return ln_matvec_launch<FMT_BF16>(a, grid, threads, st);
    case FMT_F32: return ln_matvec_launch<FMT_F32>(a, grid, threads, st);
    case FMT_F16: return ln_matvec_launch<FMT_F16>(a, grid, threads, st);
    case FMT_Q5_1: return ln_matvec_launch<FMT_Q5_1>(a, grid, threads, st);
    case FMT_Q4_K: return ln_matvec_launch<FMT_Q4_K>(a, grid, threads, st);
    case FMT_Q5_K: return ln_matvec_launch<FMT_Q5_K>(a, grid, threads, st);
    case FMT_Q6_K: return ln_matvec_launch<FMT_Q6_K>(a, grid, threads, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_embed(const MatDesc &emb, const int *ids, int n, float *x, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, st, emb, ids, x);
  return hipGetLastError();
}
