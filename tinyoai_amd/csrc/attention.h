// Split-K flash decode attention (attendHeads, stablelm.go:391-431, with
// softmax as model.go:552-570) for gfx950: the block body shared by the
// standalone decode attention launch (decode.hip) and the input-side launch
// that also runs the attention (matvec.h).
#pragma once

#include "epilogue.h"

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
  // Branches after a shared-prefix pass (BR): positions below t_begin were
  // attended by that pass, whose pre_splits partial records lead each
  // (query, head) region; this launch's splits cover [t_begin, position]
  // and write their records after them, and the last of them combines all.
  int t_begin = 0, pre_splits = 0;
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

// The same with agent-scope atomic loads (an entry stored in this launch).
template <int DPL, bool HALF>
__device__ __forceinline__ void load_kv_lanes_coherent(const void *base, int64_t e, int g, float *r) {
  if constexpr (DPL % 4 == 0) {
#pragma unroll
    for (int c = 0; c < DPL / 4; c++) load_kv_coherent<4, HALF>(base, e + att_dim<DPL>(g, 4 * c), r + 4 * c);
  } else {
    load_kv_coherent<DPL, HALF>(base, e + g * DPL, r);
  }
}

// The wait of a block whose inputs are ready at launch.
struct NoWait {
  __device__ bool operator()() const { return true; }
};

// One block of WAVES waves per (split, head, query); a split covers
// WAVES * STEPS * 16 positions. Lane = 4 * position-in-step + dim group:
// four lanes share a position, each holding hd/4 dimensions. Online-softmax
// partials combine across the waves in LDS, then across the splits of a
// (query, head) in the last block to finish (the others exit). With 16
// waves a block covers up to 1024 positions, so a short context needs one
// block per head and no cross-block combine at all.
//
// FUSED: the block runs inside the launch that writes this token's query
// and K/V entry. It issues the loads of the older positions' K/V, then
// calls wait() (block-uniform: true once the query and the entry are
// stored, false to give up), then reads the query and the entry at the
// token's own position with agent-scope atomic loads, which see the other
// blocks' stores.
template <int HD, bool HALF, int STEPS, int WAVES, bool BR, bool FUSED, typename Wait = NoWait>
__device__ __forceinline__ void attention_block(const AttArgs &a, const int split, const int h, const int j,
                                                Wait wait = Wait{}) {
  static_assert(!(FUSED && BR), "the fused launch runs single-sequence decode");
  constexpr int kWaves = WAVES, kThreads = WAVES * 64;
  constexpr int DPL = HD / 4;
  constexpr int SPLIT = kWaves * STEPS * 16;
  __shared__ float s_m[kWaves], s_l[kWaves], s_o[kWaves][HD];
  __shared__ float s_e[512];
  __shared__ int s_last;
  const StableDims &s = a.s;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane & 3, pl = lane >> 2;
  const int kvh = h / (s.heads / s.kv_heads);
  const float *q = a.q + (int64_t)j * s.heads * HD + h * HD;
  float qr[DPL];
  if constexpr (!FUSED) {
#pragma unroll
    for (int i = 0; i < DPL; i++) qr[i] = q[att_dim<DPL>(g, i)];
  }
  const int64_t head_base = (int64_t)kvh * a.kv.cap * HD;
  // BR: the query's position, and its suffix as element offsets: position
  // t >= prefix at sfx_base + t * HD (t clamped to the query's position).
  const int qpos = BR ? a.rows[2 * j] : 0;
  const int64_t sfx_base = BR ? ((int64_t)kvh * a.sfx.cap + a.rows[2 * j + 1] - qpos) * HD : 0;
  const int tb = BR ? a.t_begin : 0, pre = BR ? a.pre_splits : 0;
  const int t0 = tb + split * SPLIT + wave * STEPS * 16 + pl;
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
  // FUSED: the token's own entry was stored in this launch.
  const int fpos = FUSED ? *a.pos0 + j : -1;
#pragma unroll
  for (int st = 0; st < STEPS; st++) {
    int64_t e;
    const bool b = where(t0 + st * 16, e);
    const void *kp = reinterpret_cast<const void *>(kbase + (b ? kdelta : 0));
    const void *vp = reinterpret_cast<const void *>(vbase + (b ? vdelta : 0));
    if (!FUSED || t0 + st * 16 != fpos) {
      load_kv_lanes<DPL, HALF>(kp, e, g, kr[st]);
      if constexpr (kEarlyV) load_kv_lanes<DPL, HALF>(vp, e, g, vr[st]);
    }
  }
  const int pos = BR ? qpos : *a.pos0 + j;
  const int npos = pos + 1;
  const int nsplit = (npos - tb + SPLIT - 1) / SPLIT;  // this launch's splits
  if (split >= nsplit) return;
  if constexpr (FUSED) {
    if (!wait()) return;
#pragma unroll
    for (int i = 0; i < DPL; i++) qr[i] = collect(q + att_dim<DPL>(g, i));
#pragma unroll
    for (int st = 0; st < STEPS; st++)
      if (t0 + st * 16 == fpos) {
        int64_t e;
        where(t0 + st * 16, e);
        load_kv_lanes_coherent<DPL, HALF>(a.kv.k, e, g, kr[st]);
        if constexpr (kEarlyV) load_kv_lanes_coherent<DPL, HALF>(a.kv.v, e, g, vr[st]);
      }
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
      if (t0 + st * 16 < npos) {
        int64_t e;
        const bool b = where(t0 + st * 16, e);
        const void *vp = reinterpret_cast<const void *>(vbase + (b ? vdelta : 0));
        if (FUSED && t0 + st * 16 == fpos) load_kv_lanes_coherent<DPL, HALF>(vp, e, g, vr[st]);
        else load_kv_lanes<DPL, HALF>(vp, e, g, vr[st]);
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
  if (nsplit == 1 && pre == 0) {
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
  float *part = region + (pre + split) * (HD + 2);
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
  // Last block of this (query, head): every other split has published (and
  // the shared-prefix records were written by an earlier launch). The
  // records are staged in LDS kRec at a time by independent loads (one
  // memory round trip per kRec records) and combined from there: with
  // M = max m_r, e_r = exp(m_r - M), out[d] = sum o_r[d] e_r / sum l_r e_r,
  // rescaled from one staged chunk to the next. Every thread forms the same
  // M and L from the same LDS values.
  // (FUSED: 4 KiB of LDS, so the input-side launch that runs these blocks
  // keeps three blocks per CU; else 16 KiB, which holds a branch query's
  // shared-prefix records and suffix splits in one round.)
  constexpr int RS = HD + 2, kRec = (FUSED ? 1024 : 4096) / RS;
  static_assert(HD <= kThreads && kRec <= 512, "one output dimension per thread; weights in s_e");
  __shared__ float s_rec[kRec * RS];
  const int total = pre + nsplit;
  float m_run = -INFINITY, l_run = 0.f, acc = 0.f;
  for (int c0 = 0; c0 < total; c0 += kRec) {
    const int nr = min(kRec, total - c0);
    for (int i = tid; i < nr * RS; i += kThreads) s_rec[i] = collect(region + (int64_t)c0 * RS + i);
    __syncthreads();
    float mc = m_run;
    for (int r = 0; r < nr; r++) mc = fmaxf(mc, s_rec[r * RS]);
    for (int r = tid; r < nr; r += kThreads) s_e[r] = expf(s_rec[r * RS] - mc);
    __syncthreads();
    const float scale = expf(m_run - mc);  // 0 for the first chunk
    float lc = 0.f;
    for (int r = 0; r < nr; r++) lc = fmaf(s_rec[r * RS + 1], s_e[r], lc);
    l_run = fmaf(l_run, scale, lc);
    if (tid < HD) {
      float ac = 0.f;
      for (int r = 0; r < nr; r++) ac = fmaf(s_rec[r * RS + 2 + tid], s_e[r], ac);
      acc = fmaf(acc, scale, ac);
    }
    m_run = mc;
    __syncthreads();  // the next chunk reuses s_rec and s_e
  }
  if (tid < HD) outp[tid] = acc / l_run;
  if (tid == 0) __hip_atomic_store(&a.counters[qh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
