// Decode-path attention and embedding kernels for gfx950, and the format
// dispatch of the streaming matrix-vector kernels (matvec.h).
//
// StableLM's parallel residual (stablelm.go:365-377) lets a layer run as
// three launches over the fused matrices of LayerDev (kernels.h):
// decode_in (matvec.h), attention (here: split-K flash decode; blocks of a
// head combine through the last-arriving block) and decode_out (matvec.h).
#include <algorithm>

#include "matvec.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

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
  // Branches (BR): query j sits at position rows[2j] with its own K/V at
  // slot rows[2j + 1] of the branch cache sfx; positions below `prefix`
  // come from kv (the shared prefix), position t >= prefix from slot
  // rows[2j + 1] - rows[2j] + t of sfx.
  KVDev sfx;
  int prefix;
  const int *rows;
};

// Agent-scope relaxed atomic store of a partial result, and the matching
// load: both go to the device's coherence point, past the XCDs' L2 caches.
__device__ __forceinline__ void publish(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float collect(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Dimension held in register r by lane group g of a position's four lanes.
// When hd/4 is a multiple of 4, the lanes interleave 4-value chunks
// (group g holds chunks g, g + 4, ...), so one load instruction reads 4
// adjacent chunks of each position: 64 contiguous bytes of an fp32 row
// (32 of an fp16 row) instead of four pieces a quarter-row apart.
template <int DPL>
__device__ __forceinline__ constexpr int att_dim(int g, int r) {
  return DPL % 4 == 0 ? ((r >> 2) * 4 + g) * 4 + (r & 3) : g * DPL + r;
}

// Loads the DPL values of lane group g from the row at element e.
template <int DPL, bool HALF>
__device__ __forceinline__ void load_kv_lanes(const void *base, int64_t e, int g, float *r) {
  if constexpr (DPL % 4 == 0) {
#pragma unroll
    for (int c = 0; c < DPL / 4; c++) load_kv<4, HALF>(base, e + att_dim<DPL>(g, 4 * c), r + 4 * c);
  } else {
    load_kv<DPL, HALF>(base, e + g * DPL, r);
  }
}

// One block of WAVES waves per (split, head, query); a split covers
// WAVES * STEPS * 16 positions. Lane = 4 * position-in-step + dim group:
// four lanes share a position, each holding hd/4 dimensions. Online-softmax
// partials combine across the waves in LDS, then across the splits of a
// (query, head) in the last block to finish (the others exit). With 16
// waves a block covers up to 1024 positions, so a short context needs one
// block per head and no cross-block combine at all.
template <int HD, bool HALF, int STEPS, int WAVES = kWaves, bool BR = false>
__global__ __launch_bounds__(WAVES * 64) void attention_kernel(AttArgs a) {
  constexpr int kWaves = WAVES, kThreads = WAVES * 64;
  constexpr int DPL = HD / 4;
  constexpr int SPLIT = kWaves * STEPS * 16;
  __shared__ float s_m[kWaves], s_l[kWaves], s_o[kWaves][HD];
  __shared__ float s_e[512];
  __shared__ int s_last;
  const StableDims &s = a.s;
  const int split = blockIdx.x, h = blockIdx.y, j = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane & 3, pl = lane >> 2;
  const int kvh = h / (s.heads / s.kv_heads);
  const float *q = a.q + (int64_t)j * s.heads * HD + h * HD;
  float qr[DPL];
#pragma unroll
  for (int i = 0; i < DPL; i++) qr[i] = q[att_dim<DPL>(g, i)];
  const int64_t head_base = (int64_t)kvh * a.kv.cap * HD;
  // BR: the query's position, and its suffix as element offsets: position
  // t >= prefix at sfx_base + t * HD (t clamped to the query's position).
  const int qpos = BR ? a.rows[2 * j] : 0;
  const int64_t sfx_base = BR ? ((int64_t)kvh * a.sfx.cap + a.rows[2 * j + 1] - qpos) * HD : 0;
  const int t0 = split * SPLIT + wave * STEPS * 16 + pl;
  // Element offset of position t (clamped into its region) and whether it
  // lies in the branch cache. The base is chosen by address arithmetic on
  // the two caches (as in_pair_outputs does), not by a pointer select.
  auto where = [&](int t, int64_t &e) -> bool {
    if constexpr (BR) {
      if (t >= a.prefix) {
        e = sfx_base + (int64_t)min(t, qpos) * HD;
        return true;
      }
      e = head_base + (int64_t)t * HD;
      return false;
    } else {
      e = head_base + (int64_t)min(t, a.kv.cap - 1) * HD;
      return false;
    }
  };
  const uintptr_t kbase = reinterpret_cast<uintptr_t>(a.kv.k), vbase = reinterpret_cast<uintptr_t>(a.kv.v);
  const uintptr_t kdelta = BR ? reinterpret_cast<uintptr_t>(a.sfx.k) - kbase : 0;
  const uintptr_t vdelta = BR ? reinterpret_cast<uintptr_t>(a.sfx.v) - vbase : 0;
  // The block's K (and V) entries are loaded before the query position
  // arrives, so the loads do not wait for it: positions are clamped to the
  // cache, and entries past the query's position are masked below.
  // Narrow blocks issue the V loads with the K loads (one memory round
  // trip); wide ones load V after the scores to bound register use.
  constexpr bool kEarlyV = STEPS <= 2;
  float kr[STEPS][DPL], vr[STEPS][DPL];
#pragma unroll
  for (int st = 0; st < STEPS; st++) {
    int64_t e;
    const bool b = where(t0 + st * 16, e);
    load_kv_lanes<DPL, HALF>(reinterpret_cast<const void *>(kbase + (b ? kdelta : 0)), e, g, kr[st]);
    if constexpr (kEarlyV) load_kv_lanes<DPL, HALF>(reinterpret_cast<const void *>(vbase + (b ? vdelta : 0)), e, g, vr[st]);
  }
  const int pos = BR ? qpos : *a.pos0 + j;
  const int npos = pos + 1;
  const int nsplit = (npos + SPLIT - 1) / SPLIT;
  if (split >= nsplit) return;
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
      if (t0 + st * 16 < npos) {
        int64_t e;
        const bool b = where(t0 + st * 16, e);
        load_kv_lanes<DPL, HALF>(reinterpret_cast<const void *>(vbase + (b ? vdelta : 0)), e, g, vr[st]);
      }
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
    for (int i = 0; i < DPL; i++) s_o[wave][att_dim<DPL>(g, i)] = o[i];
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
  // atomic stores, and each thread waits for its stores to complete
  // (vmcnt(0)) before the block's arrival increment; an agent-scope
  // release fence would write back the whole L2 instead. The last block
  // learns that it is last from the value its increment returns, so its
  // loads of the partials issue after every other block's stores have
  // completed; they are agent-scope atomic loads, which read the coherence
  // point rather than a line an XCD's L2 may hold from earlier.
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
  for (int sp = tid; sp < nsplit; sp += kThreads) m = fmaxf(m, collect(base + sp * (HD + 2)));
  m = wave_max(m);
  if (lane == 0) s_m[wave] = m;
  __syncthreads();
  m = s_m[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) m = fmaxf(m, s_m[w]);
  float lsum = 0.f;
  for (int sp = tid; sp < nsplit; sp += kThreads) {
    const float e = expf(collect(base + sp * (HD + 2)) - m);
    s_e[sp] = e;
    lsum = fmaf(collect(base + sp * (HD + 2) + 1), e, lsum);
  }
  lsum = wave_sum(lsum);
  __syncthreads();
  if (lane == 0) s_l[wave] = lsum;
  __syncthreads();
  float Ltot = 0.f;
  if constexpr (kWaves == 4) {
    Ltot = (s_l[0] + s_l[1]) + (s_l[2] + s_l[3]);
  } else {
#pragma unroll
    for (int w = 0; w < kWaves; w++) Ltot += s_l[w];
  }
  for (int d = tid; d < HD; d += kThreads) {
    float acc = 0.f;
#pragma unroll 8
    for (int sp = 0; sp < nsplit; sp++) acc = fmaf(collect(base + sp * (HD + 2) + 2 + d), s_e[sp], acc);
    outp[d] = acc / Ltot;
  }
  if (tid == 0) __hip_atomic_store(&a.counters[qh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD, bool HALF>
hipError_t launch_attention_hd(const AttArgs &a, int nq, int splits, int steps, hipStream_t st) {
  // `steps` = positions per block / 64: 1, 2 and 4 on 4-wave blocks, 8 and
  // 16 on 16-wave blocks (2 and 4 positions of 16 per wave).
  dim3 grid(splits, a.s.heads, nq);
  switch (steps) {
    case 1: TINYOAI_TIMED_LAUNCH((attention_kernel<HD, HALF, 1>), grid, dim3(kThreads), 0, st, a); break;
    case 2: TINYOAI_TIMED_LAUNCH((attention_kernel<HD, HALF, 2>), grid, dim3(kThreads), 0, st, a); break;
    case 4: TINYOAI_TIMED_LAUNCH((attention_kernel<HD, HALF, 4>), grid, dim3(kThreads), 0, st, a); break;
    case 8:
    case 16:
      // 16-wave blocks hold at most 128 VGPRs per lane: wider heads would spill.
      if constexpr (HD <= 80) {
        if (steps == 8) TINYOAI_TIMED_LAUNCH((attention_kernel<HD, HALF, 2, 16>), grid, dim3(1024), 0, st, a);
        else TINYOAI_TIMED_LAUNCH((attention_kernel<HD, HALF, 4, 16>), grid, dim3(1024), 0, st, a);
        break;
      }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int HD, bool HALF>
hipError_t launch_branch_attention_hd(const AttArgs &a, int nq, int splits, int steps, hipStream_t st) {
  dim3 grid(splits, a.s.heads, nq);
  switch (steps) {
    case 1: hipLaunchKernelGGL((attention_kernel<HD, HALF, 1, kWaves, true>), grid, dim3(kThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL((attention_kernel<HD, HALF, 2, kWaves, true>), grid, dim3(kThreads), 0, st, a); break;
    case 4: hipLaunchKernelGGL((attention_kernel<HD, HALF, 4, kWaves, true>), grid, dim3(kThreads), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int HD>
hipError_t launch_attention_kv(const AttArgs &a, int nq, int splits, int steps, hipStream_t st) {
  return a.kv.half ? launch_attention_hd<HD, true>(a, nq, splits, steps, st)
                   : launch_attention_hd<HD, false>(a, nq, splits, steps, st);
}

}  // namespace

int device_cu_count() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  return cus;
}

hipError_t launch_decode_in(const LayerDev &w, const StableDims &s, const KVDev &kv, float *x, const MatDesc *emb,
                            const int *token, const float *rope, const int *pos, float *q_out, float *m_out, int grid,
                            int threads, hipStream_t st) {
  InArgs a{w, s, kv, x, emb ? *emb : MatDesc{}, emb != nullptr, token, rope, pos, q_out, m_out};
  if (w.win.rows % 2 || !planes_fit(w.win)) return hipErrorInvalidValue;
  switch (w.win.fmt) {
    case FMT_Q8_0: return run_decode_in<FMT_Q8_0>(a, grid, threads, st);
    case FMT_BF16: return run_decode_in<FMT_BF16>(a, grid, threads, st);
    case FMT_F32: return run_decode_in<FMT_F32>(a, grid, threads, st);
    case FMT_F16: return run_decode_in<FMT_F16>(a, grid, threads, st);
    case FMT_Q5_1: return run_decode_in<FMT_Q5_1>(a, grid, threads, st);
    case FMT_Q4_K: return run_decode_in<FMT_Q4_K>(a, grid, threads, st);
    case FMT_Q5_K: return run_decode_in<FMT_Q5_K>(a, grid, threads, st);
    case FMT_Q6_K: return run_decode_in<FMT_Q6_K>(a, grid, threads, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_decode_out(const MatDesc &wout, int ka, int km, const float *a, const float *m, float *x,
                             int grid, int threads, hipStream_t st) {
  OutArgs p{wout, ka, km, 0, 0, a, m, x};
  if (!planes_fit(wout)) return hipErrorInvalidValue;
  switch (wout.fmt) {
    case FMT_Q8_0: return run_decode_out<FMT_Q8_0>(p, grid, threads, st);
    case FMT_BF16: return run_decode_out<FMT_BF16>(p, grid, threads, st);
    case FMT_F32: return run_decode_out<FMT_F32>(p, grid, threads, st);
    case FMT_F16: return run_decode_out<FMT_F16>(p, grid, threads, st);
    case FMT_Q5_1: return run_decode_out<FMT_Q5_1>(p, grid, threads, st);
    case FMT_Q4_K: return run_decode_out<FMT_Q4_K>(p, grid, threads, st);
    case FMT_Q5_K: return run_decode_out<FMT_Q5_K>(p, grid, threads, st);
    case FMT_Q6_K: return run_decode_out<FMT_Q6_K>(p, grid, threads, st);
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

hipError_t launch_branch_attention(const StableDims &s, const KVDev &kv, const KVDev &sfx, int prefix,
                                   const float *q, const int *rows, int nq, int max_pos, float *partials,
                                   unsigned *counters, float *out, int max_splits, hipStream_t st) {
  const int steps = std::min(attention_steps(max_pos, s.heads), 4), splits = attention_splits(max_pos, steps);
  if (splits > 512 || splits > max_splits || prefix < 0 || prefix > kv.cap || nq < 1 || !rows ||
      kv.half != sfx.half)
    return hipErrorInvalidValue;
  AttArgs a{s, kv, q, nullptr, max_splits, partials, counters, out, sfx, prefix, rows};
  switch (s.hd) {
    case 64: return kv.half ? launch_branch_attention_hd<64, true>(a, nq, splits, steps, st)
                            : launch_branch_attention_hd<64, false>(a, nq, splits, steps, st);
    case 80: return kv.half ? launch_branch_attention_hd<80, true>(a, nq, splits, steps, st)
                            : launch_branch_attention_hd<80, false>(a, nq, splits, steps, st);
    case 8: return kv.half ? launch_branch_attention_hd<8, true>(a, nq, splits, steps, st)
                           : launch_branch_attention_hd<8, false>(a, nq, splits, steps, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_ln_matvec(const MatDesc &w, const float *ln_w, const float *ln_b, double eps, int norm,
                            const float *x, float *out, int grid, int threads, hipStream_t st) {
  LnMvArgs a{w, ln_w, ln_b, eps, norm, x, out, std::max(w.chunks * values_per_chunk(w.fmt), w.cols)};
  if (!planes_fit(w)) return hipErrorInvalidValue;
  switch (w.fmt) {
    case FMT_Q8_0: return run_ln_matvec<FMT_Q8_0>(a, grid, threads, st);
    case FMT_BF16: return run_ln_matvec<FMT_BF16>(a, grid, threads, st);
    case FMT_F32: return run_ln_matvec<FMT_F32>(a, grid, threads, st);
    case FMT_F16: return run_ln_matvec<FMT_F16>(a, grid, threads, st);
    case FMT_Q5_1: return run_ln_matvec<FMT_Q5_1>(a, grid, threads, st);
    case FMT_Q4_K: return run_ln_matvec<FMT_Q4_K>(a, grid, threads, st);
    case FMT_Q5_K: return run_ln_matvec<FMT_Q5_K>(a, grid, threads, st);
    case FMT_Q6_K: return run_ln_matvec<FMT_Q6_K>(a, grid, threads, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_embed(const MatDesc &emb, const int *ids, int n, float *x, hipStream_t st) {
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, st, emb, ids, x);
  return hipGetLastError();
}
