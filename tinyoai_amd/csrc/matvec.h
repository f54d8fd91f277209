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

#include "attention.h"
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

// The input side and the attention of a decode layer in one launch: the
// attention's arguments, and how its blocks learn that the q/k/v rows are
// stored (see decode_in_att_kernel).
// Arrivals are counted in a tree: the waves of a block in LDS, the blocks
// of group b % kFuseGroups (kernels.h) on that group's counter, the groups
// on the top counter; each counter line is 32 words.
struct FuseArgs {
  unsigned *ctr;        // the layer's top counter line, then its kFuseGroups group counter lines
  unsigned *go;         // per head, 32 words apart: the launch number the attention may start on
  const int *epoch;     // launches completed on ctr (in the parameter block)
  unsigned waves;       // streaming waves of the launch
  int blocks;           // streaming blocks; the attention blocks follow them
  int qkv_units;        // units (row pairs) of win's q, k and v sections
  unsigned *err;        // set to nonzero when a wait times out
  unsigned spin_limit;  // polls per wait
};

template <int F> hipError_t run_decode_in(const InArgs &a, int grid, int threads, hipStream_t st);
template <int F>
hipError_t run_decode_in_att(const InArgs &a, const AttArgs &att, const FuseArgs &fz, int steps, hipStream_t st);
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
template <>
hipError_t run_decode_in_att<FMT_Q8_0>(const InArgs &, const AttArgs &, const FuseArgs &, int, hipStream_t);
template <>
hipError_t run_decode_in_att<FMT_BF16>(const InArgs &, const AttArgs &, const FuseArgs &, int, hipStream_t);

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

// decode_in's work for one of `blocks` blocks (COH: outputs stored at
// agent scope; hook as stream_rows takes it).
template <int F, int T, bool COH, typename Hook>
__device__ __forceinline__ void decode_in_body(const InArgs &a, float *lds_raw, Hook hook, int blocks) {
  // LDS: pending stores | x [d] | 32 doubles | rotary row [rot] | slice partials
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
  stream_rows<F, T, cpl_for<F>(), 2, false, true, 1, false, COH, COH>(W, W.rows / 2, W.chunks, part, pend, rows,
                                                                  xload, noaux, pre, prologue, done, hook, blocks);
}

template <int F, int T>
__global__ __launch_bounds__(T) void decode_in_kernel(InArgs a) {
  extern __shared__ __align__(16) float lds_raw[];
  decode_in_body<F, T, false>(a, lds_raw, [](int) {}, (int)gridDim.x);
}

__device__ __forceinline__ unsigned poll_counter(unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// decode_in and the layer's split-K attention in one launch. Blocks
// [0, fz.blocks) stream win as decode_in_kernel does, storing the query and
// the K/V entry at agent scope; a wave's units come in increasing order, so
// once the next unit it would take lies past the q/k/v sections, its q/k/v
// results are stored: it waits for its stores and arrives (with 512 blocks
// of four waves and groups of two units, right after its first group).
// The last wave of a block to arrive adds the block to its group's
// counter, the last block of a group adds the group to the top counter,
// and the last group raises every head's go flag to the launch number
// (counters grow by a fixed amount per launch, so nothing is reset between
// launches). The blocks after the streaming ones run the attention of
// (split idx % splits, head idx / splits). Where the kernel fits 168 VGPRs
// (fused_waves), three blocks share a CU, so with up to 256 attention
// blocks beside 512 streaming ones every block is resident from the start
// (elsewhere attention blocks start as streaming blocks retire); an
// attention block issues
// its older positions' K/V loads at once, waits for its head's flag, then
// reads the query and the token's own entry, so the attention overlaps
// the gate/up rows' stream. A single counter for every wave made each wave
// stall behind thousands of atomics to one address; the tree keeps one
// wave per block on a global atomic and a head's few blocks on a flag
// line. An attention block waits only for blocks before it in dispatch
// order, which have all started when it runs; the wait is still bounded,
// and a time-out sets *fz.err (every waiting block then leaves).
// Waves per SIMD the fused kernel is compiled for: three where its
// registers fit 168 VGPRs without spilling (Q8_0 rows with at most 160
// attention values per lane step), else two.
template <int F, int HD, int STEPS>
constexpr int fused_waves() {
  return F == FMT_Q8_0 && HD * STEPS <= 160 ? 3 : 2;
}

template <int F, int T, int HD, bool HALF, int STEPS>
__global__ __launch_bounds__(T, (fused_waves<F, HD, STEPS>())) void decode_in_att_kernel(InArgs a, AttArgs att,
                                                                                       FuseArgs fz) {
  static_assert(T == 256, "attention blocks are four waves");
  extern __shared__ __align__(16) float lds_raw[];
  __shared__ unsigned s_arrived;
  const unsigned launch = (unsigned)*fz.epoch + 1;
  if ((int)blockIdx.x >= fz.blocks) {
    __shared__ int s_ok;
    const int idx = (int)blockIdx.x - fz.blocks, splits = att.max_splits, h = idx / splits;
    auto wait = [&]() {
      if (threadIdx.x == 0) {
        unsigned *flag = fz.go + h * 32;
        int ok = 1;
        for (unsigned it = 0; (int)(poll_counter(flag) - launch) < 0; it++) {
          if (it >= fz.spin_limit || ((it & 15) == 15 && poll_counter(fz.err) != 0)) {
            ok = 0;
            break;
          }
          __builtin_amdgcn_s_sleep(4);
        }
        if (!ok) __hip_atomic_store(fz.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_ok = ok;
      }
      __syncthreads();
      return s_ok != 0;
    };
    attention_block<HD, HALF, STEPS, 4, false, true>(att, idx % splits, h, 0, wait);
    return;
  }
  if (threadIdx.x == 0) s_arrived = 0;  // the prologue's barrier orders this before any arrival
  bool signaled = false;  // wave-uniform
  auto hook = [&](int next_unit) {
    if (signaled || next_unit < fz.qkv_units) return;
    signaled = true;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's q/k/v stores have completed
    const int lane = threadIdx.x & 63;
    unsigned last = 0;
    if (lane == 0 && atomicAdd(&s_arrived, 1u) == T / 64 - 1) {
      const int g = blockIdx.x % kFuseGroups;
      const unsigned in_group = (unsigned)(fz.blocks - g + kFuseGroups - 1) / kFuseGroups;
      const unsigned groups = (unsigned)min(fz.blocks, kFuseGroups);
      if (__hip_atomic_fetch_add(fz.ctr + 32 * (1 + g), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              launch * in_group - 1 &&
          __hip_atomic_fetch_add(fz.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == launch * groups - 1)
        last = 1;
    }
    if (__builtin_amdgcn_readfirstlane(last))  // every q/k/v row of the launch is stored
      for (int h = lane; h < a.s.heads; h += 64)
        __hip_atomic_store(fz.go + h * 32, launch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  decode_in_body<F, T, true>(a, lds_raw, hook, fz.blocks);
}

// x = (x + o*a) + down*m: a wout row is [o | down], the down part from
// chunk na on. Q8_0: no batch carried past a group, which fits three waves
// per SIMD (measured faster at the 3B shape than two with the carry).
template <int F, int T>
__global__ __launch_bounds__(T, (F == FMT_Q8_0 ? 3 : 2)) void decode_out_kernel(OutArgs p) {
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
  stream_rows<F, T, cpl_for<F>(), 2, true, false, 0, true, false, false, F == FMT_Q8_0>(
      W, (W.rows + 1) / 2, p.na, part, pend, rows, xload, aux, [] {}, [] {}, done);
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

// The fused launch: 256-thread blocks, rows within one column slice.
template <int F>
inline bool decode_in_att_fits(const InArgs &a) {
  return slice_shape(a.w.win.chunks, a.w.win.chunks, cpl_for<F>()).S == 1;
}

template <int F, int HD, bool HALF>
hipError_t decode_in_att_launch_hd(const InArgs &a, const AttArgs &att, const FuseArgs &fz, int steps,
                                   hipStream_t st) {
  constexpr int T = 256;
  const size_t lds = pending_lds(T) + (size_t)round_up(a.s.d, 4) * 4 + 32 * sizeof(double) +
                     (size_t)round_up(a.s.rot, 4) * 4;
  if (!decode_in_att_fits<F>(a) || lds > 65536 || fz.blocks < 1) return hipErrorInvalidValue;
  const dim3 grid(fz.blocks + att.max_splits * a.s.heads);
  switch (steps) {
    case 1: TINYOAI_TIMED_LAUNCH((decode_in_att_kernel<F, T, HD, HALF, 1>), grid, dim3(T), lds, st, a, att, fz); break;
    case 2: TINYOAI_TIMED_LAUNCH((decode_in_att_kernel<F, T, HD, HALF, 2>), grid, dim3(T), lds, st, a, att, fz); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int F>
hipError_t decode_in_att_launch(const InArgs &a, const AttArgs &att, const FuseArgs &fz, int steps, hipStream_t st) {
  const bool half = att.kv.half != 0;
  switch (a.s.hd) {
    case 64: return half ? decode_in_att_launch_hd<F, 64, true>(a, att, fz, steps, st)
                         : decode_in_att_launch_hd<F, 64, false>(a, att, fz, steps, st);
    case 80: return half ? decode_in_att_launch_hd<F, 80, true>(a, att, fz, steps, st)
                         : decode_in_att_launch_hd<F, 80, false>(a, att, fz, steps, st);
    case 128: return half ? decode_in_att_launch_hd<F, 128, true>(a, att, fz, steps, st)
                          : decode_in_att_launch_hd<F, 128, false>(a, att, fz, steps, st);
  }
  return hipErrorInvalidValue;
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

// The fused input-side + attention launcher of format F (the formats the
// decode workloads stream: Q8_0 and BF16).
#define TINYOAI_MATVEC_DEFINE_FUSED(F)                                                           \
  template <>                                                                                    \
  hipError_t run_decode_in_att<F>(const InArgs &a, const AttArgs &att, const FuseArgs &fz, int steps, \
                                  hipStream_t st) {                                              \
    return tinyoai_matvec::decode_in_att_launch<F>(a, att, fz, steps, st);                       \
  }

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
