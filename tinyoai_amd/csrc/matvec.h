// Streaming matrix-vector kernels of the decode path (one token), for
// gfx950, shared by the per-format translation units matvec_<format>.hip
// (each instantiates the kernels of one weight format, so the build
// compiles the formats in parallel):
//   decode_in   LayerNorm(x) once per block into LDS, then every row of win
//               (q, k, v, gate, up) in one pass over HBM, with RoPE, the KV
//               append and SiLU-gate applied in the epilogue; layer 0 also
//               gathers the token's embedding row here;
//   decode_out  x = (x + o*a) + down*m, one wout row [o | down] per unit;
//   ln_matvec   an optional LayerNorm / RMSNorm of x, then out = W x (the
//               classifier, and the legacy Llama's projections).
// decode_in hands out win rows in pairs (2u, 2u + 1): a rotary pair, two
// adjacent non-rotary dims, or gate row i with up row i. Each wave streams
// its units with the next batch of weight loads in flight (stream_units,
// formats.h).
#pragma once

#include <algorithm>

#include "epilogue.h"
#include "rowstream.h"

struct InArgs {
  LayerDev w;
  StableDims s;
  KVDev kv;
  float *x;             // residual [d]; written here when emb is set
  MatDesc emb;          // embedding table (layer 0, when use_emb)
  int use_emb;
  const int *token;     // token id (layer 0)
  const float *rope;    // the token's rotary row [rot]
  const int *pos;
  float *q_out, *m_out;
};

struct OutArgs {
  MatDesc w;
  int ka, km;  // values of the o and down parts of a wout row
  int na, nm;  // their chunks
  const float *a, *m;
  float *x;
};

struct LnMvArgs {
  MatDesc w;
  const float *ln_w, *ln_b;
  double eps;
  int norm;
  const float *x;
  float *out;
  int xlen;
};

template <int F> hipError_t run_decode_in(const InArgs &a, int grid, int threads, hipStream_t st);
template <int F> hipError_t run_decode_out(OutArgs p, int grid, int threads, hipStream_t st);
template <int F> hipError_t run_ln_matvec(const LnMvArgs &a, int grid, int threads, hipStream_t st);

#define TINYOAI_MATVEC_DECLARE(F)                                                              \
  template <> hipError_t run_decode_in<F>(const InArgs &, int, int, hipStream_t);             \
  template <> hipError_t run_decode_out<F>(OutArgs, int, int, hipStream_t);                   \
  template <> hipError_t run_ln_matvec<F>(const LnMvArgs &, int, int, hipStream_t);
TINYOAI_MATVEC_DECLARE(FMT_Q8_0)
TINYOAI_MATVEC_DECLARE(FMT_BF16)
TINYOAI_MATVEC_DECLARE(FMT_F32)
TINYOAI_MATVEC_DECLARE(FMT_F16)
TINYOAI_MATVEC_DECLARE(FMT_Q5_1)
TINYOAI_MATVEC_DECLARE(FMT_Q4_K)
TINYOAI_MATVEC_DECLARE(FMT_Q5_K)
TINYOAI_MATVEC_DECLARE(FMT_Q6_K)

namespace tinyoai_matvec {

// Chunks per lane of a wave's column slice: a lane keeps CPL * VPC x
// values in registers (48 for Q8_0, 40 for BF16 / F16, 20 for F32, 64 for
// the 32-value chunks), so the 3B rows (2560 columns) fit one slice except
// in F32 (two), and a 3B wout row (2560 + 6912 columns) at most eight.
template <int F>
constexpr int cpl_for() {
  return F == FMT_Q8_0 ? 3 : (F == FMT_BF16 || F == FMT_F16 || F == FMT_F32) ? 5 : 2;
}

__host__ __device__ inline int round_up(int v, int m) { return (v + m - 1) / m * m; }

// The VPC x values of chunk c of a vector of `len` floats (zeros past it).
template <int VPC>
__device__ __forceinline__ void x_chunk(const float *src, int len, int c, float *out) {
  const int base = c * VPC;
  if (base + VPC <= len) {
#pragma unroll
    for (int v = 0; v < VPC; v += 4) {
      const float4 t = *reinterpret_cast<const float4 *>(src + base + v);
      out[v] = t.x;
      out[v + 1] = t.y;
      out[v + 2] = t.z;
      out[v + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int v = 0; v < VPC; v++) out[v] = base + v < len ? src[base + v] : 0.f;
  }
}

// The slice partials' LDS (floats) of a launch: units_per_block * slot
// when the rows span more than one slice.
template <int F>
inline size_t slice_lds(int chunks, int split, int n_units, int grid, int R) {
  const SliceShape sh = slice_shape(chunks, split, cpl_for<F>());
  if (sh.S == 1) return 0;
  const int per_block = (n_units + grid - 1) / grid;
  return (size_t)per_block * (sh.S * R * 2 + R);
}

// float4 groups of the normalised row a thread stages in registers (rows
// up to 4 * kNormRegs * threads; longer ones read the rest directly).
constexpr int kNormRegs = 3;

template <int F, int T>
__global__ __launch_bounds__(T) void decode_in_kernel(InArgs a) {
  // LDS: pending stores | x [d] | 32 doubles | rotary row [rot] | slice partials
  extern __shared__ __align__(16) float lds_raw[];
  PendingStore *pend = reinterpret_cast<PendingStore *>(lds_raw);
  float *lds = lds_raw + (T / 64) * kPendingPerWave * 4;
  constexpr int VPC = Fmt<F>::VPC;
  const MatDesc &W = a.w.win;
  const StableDims &s = a.s;
  double *red = reinterpret_cast<double *>(lds + round_up(s.d, 4));
  float *rope_row = reinterpret_cast<float *>(red + 32);  // cos/sin at pos, [rot/2][2]
  float *part = rope_row + round_up(s.rot, 4);
  const int pos = *a.pos;
  KVDev kv = a.kv;
  kv.k = uniform_ptr(kv.k);
  kv.v = uniform_ptr(kv.v);
  NormRegs<kNormRegs> nr;
  float rv;
  const float *xs = a.x;  // where norm_store reads elements past the registers
  auto pre = [&]() {
    rv = (int)threadIdx.x < s.rot ? a.rope[threadIdx.x] : 0.f;
    norm_load<T>(nr, a.use_emb ? nullptr : a.x, a.w.ln_w, s.norm ? nullptr : a.w.ln_b, s.d);
    if (a.use_emb) {
      // Layer 0: the embedding row (stablelm.go:338), bit-exact readValues,
      // gathered before any weight load (its registers do not meet the
      // batches').
      const MatDesc &e = a.emb;
      const int64_t row = *a.token;
      for (int i = threadIdx.x; i < s.d; i += T) {
        const float v = mat_value(e, row, i);
        lds[i] = v;
        if (blockIdx.x == 0) a.x[i] = v;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kNormRegs; j++) nr.x[j] = load4(lds, 4 * ((int)threadIdx.x + j * T), s.d);
      nr.shift = lds[0];
      xs = lds;
    }
  };
  auto prologue = [&]() {
    for (int i = threadIdx.x; i < s.rot; i += T) rope_row[i] = i == (int)threadIdx.x ? rv : a.rope[i];
    norm_store<T>(nr, s.d, s.norm, s.eps, xs, a.w.ln_w, a.w.ln_b, lds, red);
    __syncthreads();
  };
  auto rows = [&](int u, int (&row)[2]) {
    row[0] = 2 * u;
    row[1] = 2 * u + 1;
  };
  auto xload = [&](int c, float *out) { x_chunk<VPC>(lds, s.d, c, out); };
  auto noaux = [](int) { return 0.f; };
  auto done = [&](int u, const float (&r)[2][2], const float (&)[2], const auto &out) {
    in_pair_outputs(s, kv, rope_row, pos, u, r[0][0], r[1][0], a.q_out, a.m_out, out);
  };
  stream_rows<F, T, cpl_for<F>(), 2, false, true, 1, false>(W, W.rows / 2, W.chunks, part, pend, rows, xload, noaux,
                                                            pre, prologue, done);
}

// x = (x + o*a) + down*m: a wout row is [o | down], the down part from
// chunk na on.
template <int F, int T>
__global__ __launch_bounds__(T) void decode_out_kernel(OutArgs p) {
  // LDS: pending stores | slice partials
  extern __shared__ __align__(16) float lds_raw[];
  PendingStore *pend = reinterpret_cast<PendingStore *>(lds_raw);
  float *part = lds_raw + (T / 64) * kPendingPerWave * 4;
  constexpr int VPC = Fmt<F>::VPC;
  const MatDesc &W = p.w;
  auto rows = [&](int u, int (&row)[2]) {
    row[0] = 2 * u;
    row[1] = min(2 * u + 1, W.rows - 1);
  };
  auto xload = [&](int c, float *out) {
    if (c < p.na) x_chunk<VPC>(p.a, p.ka, c, out);
    else x_chunk<VPC>(p.m, p.km, c - p.na, out);
  };
  // The residual x[r] is loaded with the unit's batch, not in done().
  auto aux = [&](int r) { return p.x[r]; };
  auto done = [&](int u, const float (&r)[2][2], const float (&x0)[2], const auto &out) {
    out.f32(p.x + 2 * u, __fadd_rn(__fadd_rn(x0[0], r[0][0]), r[0][1]));
    if (2 * u + 1 < W.rows) out.f32(p.x + 2 * u + 1, __fadd_rn(__fadd_rn(x0[1], r[1][0]), r[1][1]));
  };
  stream_rows<F, T, cpl_for<F>(), 2, true, false, 0, true>(W, (W.rows + 1) / 2, p.na, part, pend, rows, xload, aux,
                                                           [] {}, [] {}, done);
}

template <int F, int T>
__global__ __launch_bounds__(T) void ln_matvec_kernel(LnMvArgs a) {
  // LDS: pending stores | x [cols] | 32 doubles | slice partials
  extern __shared__ __align__(16) float lds_raw[];
  PendingStore *pend = reinterpret_cast<PendingStore *>(lds_raw);
  float *lds = lds_raw + (T / 64) * kPendingPerWave * 4;
  constexpr int VPC = Fmt<F>::VPC;
  const int cols = a.w.cols;
  const MatDesc &M = a.w;
  double *red = reinterpret_cast<double *>(lds + round_up(cols, 4));
  float *part = reinterpret_cast<float *>(red + 32);
  NormRegs<kNormRegs> nr;
  auto pre = [&]() { norm_load<T>(nr, a.x, a.ln_w, a.ln_w && !a.norm ? a.ln_b : nullptr, cols); };
  auto prologue = [&]() {
    norm_store<T>(nr, cols, a.ln_w ? a.norm : -1, a.eps, a.x, a.ln_w, a.ln_b, lds, red);
    __syncthreads();
  };
  auto rows = [&](int u, int (&row)[2]) {
    row[0] = 2 * u;
    row[1] = min(2 * u + 1, M.rows - 1);
  };
  auto xload = [&](int c, float *out) { x_chunk<VPC>(lds, cols, c, out); };
  auto noaux = [](int) { return 0.f; };
  auto done = [&](int u, const float (&r)[2][2], const float (&)[2], const auto &out) {
    out.f32(a.out + 2 * (int64_t)u, r[0][0]);
    if (2 * u + 1 < M.rows) out.f32(a.out + 2 * (int64_t)u + 1, r[1][0]);
  };
  stream_rows<F, T, cpl_for<F>(), 2, false, true, 1, false>(M, (M.rows + 1) / 2, M.chunks, part, pend, rows, xload,
                                                            noaux, pre, prologue, done);
}

// LDS bytes of the blocks' pending result stores.
inline size_t pending_lds(int threads) { return (size_t)(threads / 64) * kPendingPerWave * sizeof(PendingStore); }

// Block size of a row-streaming launch: the caller's 256 or 512 threads
// (a lane keeps its x slice and its batches in registers, more than a few
// waves per SIMD allow), raised to 512 when a row spans more column slices
// than the block has waves; 0 when it spans more than 8.
template <int F>
int fit_threads(int chunks, int split, int threads) {
  const int need = 64 * slice_shape(chunks, split, cpl_for<F>()).S;
  if ((threads != 256 && threads != 512) || need > 512) return 0;
  return need > threads ? 512 : threads;
}

#define TINYOAI_LAUNCH_T(KERNEL, ARGS)                                                                  \
  switch (threads) {                                                                                    \
    case 256: TINYOAI_TIMED_LAUNCH((KERNEL<F, 256>), dim3(grid), dim3(256), lds, st, ARGS); break;       \
    case 512: TINYOAI_TIMED_LAUNCH((KERNEL<F, 512>), dim3(grid), dim3(512), lds, st, ARGS); break;       \
    default: return hipErrorInvalidValue;                                                               \
  }

template <int F>
hipError_t ln_matvec_launch(const LnMvArgs &a, int grid, int threads, hipStream_t st) {
  threads = fit_threads<F>(a.w.chunks, a.w.chunks, threads);
  const size_t lds = pending_lds(threads) + (size_t)round_up(a.w.cols, 4) * 4 + 32 * sizeof(double) +
                     slice_lds<F>(a.w.chunks, a.w.chunks, (a.w.rows + 1) / 2, grid, 2) * 4;
  if (!threads || lds > 65536) return hipErrorInvalidValue;
  TINYOAI_LAUNCH_T(ln_matvec_kernel, a)
  return hipGetLastError();
}

template <int F>
hipError_t decode_in_launch(const InArgs &a, int grid, int threads, hipStream_t st) {
  threads = fit_threads<F>(a.w.win.chunks, a.w.win.chunks, threads);
  const size_t lds = pending_lds(threads) + (size_t)round_up(a.s.d, 4) * 4 + 32 * sizeof(double) +
                     (size_t)round_up(a.s.rot, 4) * 4 +
                     slice_lds<F>(a.w.win.chunks, a.w.win.chunks, a.w.win.rows / 2, grid, 2) * 4;
  if (!threads || lds > 65536) return hipErrorInvalidValue;
  TINYOAI_LAUNCH_T(decode_in_kernel, a)
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
  threads = fit_threads<F>(p.w.chunks, p.na, threads);
  const size_t lds = pending_lds(threads) + slice_lds<F>(p.w.chunks, p.na, (p.w.rows + 1) / 2, grid, 2) * 4;
  if (!threads || lds > 65536) return hipErrorInvalidValue;
  TINYOAI_LAUNCH_T(decode_out_kernel, p)
  return hipGetLastError();
}

#undef TINYOAI_LAUNCH_T

}  // namespace tinyoai_matvec

// The three launchers of format F, for its translation unit.
#define TINYOAI_MATVEC_DEFINE(F)                                                                  \
  template <>                                                                                     \
  hipError_t run_decode_in<F>(const InArgs &a, int grid, int threads, hipStream_t st) {           \
    return tinyoai_matvec::decode_in_launch<F>(a, grid, threads, st);                             \
  }                                                                                               \
  template <>                                                                                     \
  hipError_t run_decode_out<F>(OutArgs p, int grid, int threads, hipStream_t st) {                \
    return tinyoai_matvec::decode_out_launch<F>(p, grid, threads, st);                            \
  }                                                                                               \
  template <>                                                                                     \
  hipError_t run_ln_matvec<F>(const LnMvArgs &a, int grid, int threads, hipStream_t st) {         \
    return tinyoai_matvec::ln_matvec_launch<F>(a, grid, threads, st);                             \
  }
