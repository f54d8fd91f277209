// Persistent decode: one token through every StableLM layer and the logits
// head in a single cooperative launch, one 1024-thread block per CU
// (StableLM.forward, stablelm.go:332-387).
//
// Each layer runs the work of decode_in, attention and decode_out as three
// phases separated by grid-wide dependency counters instead of kernel
// boundaries. Weight rows do not depend on the previous phase, so every
// wave issues the loads of its first unit before it waits: the wait, the
// LayerNorm and the activation staging overlap the HBM stream. The o/down
// phase consumes the down half of its row (needs only SiLU-gate outputs)
// before it waits for attention.
//
// Visibility across XCDs (each has its own L2):
//  - values read by other blocks in the same launch are written with
//    agent-scope atomic stores, and a block signals a counter only after
//    its waves' stores have completed (s_waitcnt);
//  - counters are polled with agent-scope atomic loads;
//  - handoff buffers are distinct per layer (xs, qs, ms, as) and start on
//    256-byte boundaries, so no block caches one of their lines before it
//    is written in this launch (plain loads can return such a stale line);
//  - KV loads issued before a wait end before the 256-byte line that holds
//    the current position (written during the wait); the rest are issued
//    after it, so they too find no stale line;
//  - attention partials are distinct per layer and read after the arrivals.
//
// Counters: bar_in[l] and bar_out[l] (one arrival per block) and
// att_done[l] (one per head) grow by a fixed amount per launch, so a wait
// targets (epoch + 1) * amount and nothing is reset between launches;
// att_arrive[l][h] is reset by the wave that combines head h. Every wait is
// bounded: on time-out a block sets the error word and leaves, and waiting
// blocks leave as soon as they see it.
#include <algorithm>

#include "epilogue.h"

namespace {

constexpr int kT = 1024, kWavesPerBlock = kT / 64;
constexpr int kLine = 32;  // counter spacing in words (128 bytes)

struct SyncMap {
  unsigned *base;
  int L, heads;
  __device__ unsigned *bar_in(int l) const { return base + (1 + l) * kLine; }
  __device__ unsigned *bar_out(int l) const { return base + (1 + L + l) * kLine; }
  __device__ unsigned *att_done(int l) const { return base + (1 + 2 * L + l) * kLine; }
  __device__ unsigned *att_arrive(int l, int h) const { return base + (1 + 3 * L + l * heads + h) * kLine; }
};

__device__ __forceinline__ unsigned poll(unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-uniform wait until *ctr reaches target (wrapping compare). Returns
// false after `limit` polls or when another block has reported an error.
__device__ bool block_wait(unsigned *ctr, unsigned target, unsigned *err, unsigned limit, int *flag) {
  if (threadIdx.x == 0) {
    int ok = 1;
    for (unsigned it = 0; (int)(poll(ctr) - target) < 0; it++) {
      if (it >= limit || ((it & 63) == 63 && poll(err) != 0)) {
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (!ok) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = ok;
  }
  __syncthreads();
  const int ok = *flag;
  __syncthreads();
  return ok != 0;
}

// Signals *ctr once every wave of the block has completed its stores.
__device__ __forceinline__ void block_arrive(unsigned *ctr) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Batches after the first of one unit.
template <int F, int U>
__device__ __forceinline__ void stream_rest(Batch<U> &b, const Seg2 &g, int lane, float &a0, float &a1) {
  for (int base = 64 * U; base < g.n0 + g.n1; base += 64 * U) {
    batch_issue<F, U>(b, g, base, lane);
    batch_consume<F, U, true>(b, g, base, lane, a0, a1);
  }
}

// Streams units u0, u0 + stride, ... (< n) through one wave. The first
// unit's first batch is already in (b, g), issued before the caller's wait;
// each following unit's first batch is issued before the current unit is
// consumed, so two batches are in flight.
// Streams units u0, u0 + stride, ... (< n) through one wave; the first
// unit's first batch is already in (b, g), issued before the caller's wait.
template <int F, int U, typename UnitFn, typename Done>
__device__ __forceinline__ void stream_units_from(int u0, int stride, int n, Batch<U> &b, Seg2 &g, int lane,
                                                  UnitFn unit, Done done) {
  for (int u = u0; u < n; u += stride) {
    if (u != u0) {
      unit(u, g);
      batch_issue<F, U>(b, g, 0, lane);
    }
    float a0 = 0.f, a1 = 0.f;
    batch_consume<F, U, true>(b, g, 0, lane, a0, a1);
    stream_rest<F, U>(b, g, lane, a0, a1);
    done(u, wave_sum(a0), wave_sum(a1));
  }
}

template <int F, int U, typename UnitFn, typename Done>
__device__ __forceinline__ void stream_units_db(int u0, int stride, int n, Batch<U> &b, Seg2 &g, int lane,
                                                UnitFn unit, Done done) {
  for (int u = u0; u < n; u += stride) {
    Batch<U> bn;
    Seg2 gn{};
    const bool more = u + stride < n;
    if (more) {
      unit(u + stride, gn);
      batch_issue<F, U>(bn, gn, 0, lane);
    }
    float a0 = 0.f, a1 = 0.f;
    batch_consume<F, U, true>(b, g, 0, lane, a0, a1);
    stream_rest<F, U>(b, g, lane, a0, a1);
    done(u, wave_sum(a0), wave_sum(a1));
    if (more) {
      b = bn;
      g = gn;
    }
  }
}

template <int F, int UI, int UO, int HD, bool HALF>
__global__ __launch_bounds__(kT) void persistent_decode_kernel(PersistentDecode a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int s_flag;
  constexpr int VPC = Fmt<F>::VPC;
  constexpr int DPL = HD / 4;  // attention: four lanes per position
  constexpr int ES = HALF ? 2 : 4;
  const StableDims s = a.s;
  const int d = s.d, I = s.inter, HQ = s.heads * HD;
  const int tid = threadIdx.x, lane0 = tid & 63;
  const int gw = blockIdx.x * kWavesPerBlock + (tid >> 6), NW = gridDim.x * kWavesPerBlock;
  const int pos = a.params[1];
  const SyncMap sy{a.sync, a.L, s.heads};
  unsigned *err = a.err;
  const unsigned tgt_blocks = (a.epoch + 1u) * gridDim.x, tgt_heads = (a.epoch + 1u) * (unsigned)s.heads;
  uint64_t *stamp = a.stamps ? a.stamps + (int64_t)blockIdx.x * persistent_stamps(a.L) : nullptr;
  auto mark = [&](int k) {
    if (stamp && tid == 0) stamp[k] = __builtin_amdgcn_s_memrealtime();
  };
  mark(0);

  // LDS: LayerNorm row, its staged chunks, reduction scratch, RoPE row, and
  // the staged attention output and SiLU-gate vectors of the o/down phase.
  const int na = (d + VPC - 1) / VPC;
  float *xl = lds;
  float4 *xq = reinterpret_cast<float4 *>(xl + ((d + 3) & ~3));
  double *red = reinterpret_cast<double *>(xq + (VPC / 4) * na);
  float *rope_row = reinterpret_cast<float *>(red + 16);
  float4 *xa = reinterpret_cast<float4 *>(rope_row + ((s.rot + 3) & ~3));
  float4 *xm = xa + (VPC / 4) * na;

  for (int l = 0; l < a.L; l++) {
    // An opaque copy of the lane index per layer: without it the compiler
    // hoists every lane-dependent load offset of all three phases out of the
    // layer loop and spills them.
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const LayerDev w = a.layers[l];
    const KVDev kv = a.kv[l];
    float *x_in = a.xs + (int64_t)l * persistent_stride(d), *x_out = x_in + persistent_stride(d);
    float *q = a.qs + (int64_t)l * persistent_stride(HQ), *att = a.as + (int64_t)l * persistent_stride(HQ);
    float *m = a.ms + (int64_t)l * persistent_stride(I);

    // ---- LayerNorm + win rows, epilogue RoPE / KV append / SiLU-gate
    {
      const MatDesc &W = w.win;
      const int units = W.rows >> 1, nch = W.chunks;
      auto unit = [&](int u, Seg2 &g) {
        g = Seg2{row_ptr(W, 2 * (int64_t)u), row_ptr(W, 2 * (int64_t)u + 1), xq, xq, nch, nch};
      };
      auto done = [&](int u, float v0, float v1) {
        if (lane == 0) in_pair_epilogue<true>(s, kv, rope_row, pos, u, v0, v1, q, m);
      };
      Batch<UI> b;
      Seg2 g{};
      if (gw < units) {
        unit(gw, g);
        batch_issue<F, UI>(b, g, 0, lane);
      }
      if (l > 0 && !block_wait(sy.bar_out(l - 1), tgt_blocks, err, a.spin_limit, &s_flag)) return;
      mark(1 + 6 * l);
      if (l == 0) {  // embedding row (stablelm.go:338), bit-exact readValues
        const int64_t row = a.params[0];
        for (int i = tid; i < d; i += kT) {
          const float v = mat_value(a.emb, row, i);
          xl[i] = v;
          if (blockIdx.x == 0) put<true>(x_in + i, v);
        }
      } else {
        for (int i = tid; i < d; i += kT) xl[i] = x_in[i];
      }
      __syncthreads();
      norm_lds(s, xl, w.ln_w, w.ln_b, red);
      stage_x(xq, xl, d, nch, VPC);
      for (int i = tid; i < s.rot; i += kT) rope_row[i] = a.rope[(int64_t)pos * s.rot + i];
      __syncthreads();
      stream_units_from<F, UI>(gw, NW, units, b, g, lane, unit, done);
      block_arrive(sy.bar_in(l));
      mark(2 + 6 * l);
    }

    // ---- attention: one wave per (head, 16 positions); the last wave of a
    // head to finish combines its partials (attendHeads, stablelm.go:391-431)
    {
      const int nsplit = (pos + 16) / 16;
      const int n_att = s.heads * nsplit, aw0 = NW - 1 - gw;
      const int g4 = lane & 3, pl = lane >> 2, grp = s.heads / s.kv_heads;
      // Partials of this layer, one 256-byte aligned region per head: fresh
      // lines in every launch, each read once by the head's last wave.
      float *parts = a.partials + (int64_t)l * s.heads * partial_region(a.max_splits, HD);
      // Loads issued before the wait must end before the 256-byte line that
      // holds this token's entry (written during the wait); with rows that
      // are not whole lines, nothing is loaded early.
      const bool lines = ((int64_t)kv.cap * HD * ES) % 256 == 0;
      float kr[DPL];
      int h = 0, sp = 0, t = 0;
      int64_t off = 0;
      bool early = false;
      auto locate = [&](int au) {
        h = au / nsplit;
        sp = au - h * nsplit;
        t = sp * 16 + pl;
        const int64_t row = (int64_t)(h / grp) * kv.cap;
        off = (row + t) * HD + g4 * DPL;
        const int64_t fence = ((row + pos) * HD * ES) & ~(int64_t)255;
        early = lines && t < pos && (off + DPL) * ES <= fence;
        if (early) load_kv<DPL, HALF>(kv.k, off, kr);
      };
      if (aw0 < n_att) locate(aw0);
      if (!block_wait(sy.bar_in(l), tgt_blocks, err, a.spin_limit, &s_flag)) return;
      mark(3 + 6 * l);
      for (int au = aw0; au < n_att; au += NW) {
        if (au != aw0) locate(au);
        if (!early && t <= pos) load_kv<DPL, HALF>(kv.k, off, kr);
        const float *qp = q + h * HD + g4 * DPL;
        float p = 0.f;
        if (t <= pos) {
#pragma unroll
          for (int i = 0; i < DPL; i++) p = fmaf(qp[i], kr[i], p);
        }
        p += __shfl_xor(p, 1, 64);
        p += __shfl_xor(p, 2, 64);
        const float sc = t <= pos ? __fdiv_rn(p, s.att_scale) : -INFINITY;
        const float mx = wave_max(sc);
        const float e = t <= pos ? expf(sc - mx) : 0.f;
        const float lsum = wave_sum(g4 == 0 ? e : 0.f);
        float vr[DPL];
        if (t <= pos) load_kv<DPL, HALF>(kv.v, off, vr);
        float o[DPL];
#pragma unroll
        for (int i = 0; i < DPL; i++) {
          float v = t <= pos ? e * vr[i] : 0.f;
          v += __shfl_xor(v, 4, 64);
          v += __shfl_xor(v, 8, 64);
          v += __shfl_xor(v, 16, 64);
          v += __shfl_xor(v, 32, 64);
          o[i] = v;
        }
        float *part = parts + (int64_t)h * partial_region(a.max_splits, HD) + sp * (HD + 2);
        if (lane == 0) {
          put<true>(part, mx);
          put<true>(part + 1, lsum);
        }
        if (pl == 0) {
#pragma unroll
          for (int i = 0; i < DPL; i++) put<true>(part + 2 + g4 * DPL + i, o[i]);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(sy.att_arrive(l, h), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0, 64);
        if (old != (unsigned)(nsplit - 1)) continue;
        // Last split of head h: every other split has published.
        const float *base = parts + (int64_t)h * partial_region(a.max_splits, HD);
        float M = -INFINITY;
        for (int j = lane; j < nsplit; j += 64) M = fmaxf(M, base[(int64_t)j * (HD + 2)]);
        M = wave_max(M);
        float ereg[8], L = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
          const int j = k * 64 + lane;
          ereg[k] = j < nsplit ? expf(base[(int64_t)j * (HD + 2)] - M) : 0.f;
          if (j < nsplit) L = fmaf(base[(int64_t)j * (HD + 2) + 1], ereg[k], L);
        }
        L = wave_sum(L);
        for (int d0 = 0; d0 < HD; d0 += 64) {
          const int dd = min(d0 + lane, HD - 1);
          float acc = 0.f;
#pragma unroll
          for (int k = 0; k < 8; k++) {
            if (k * 64 >= nsplit) break;
            const int jn = min(64, nsplit - k * 64);
            const float *col = base + (int64_t)k * 64 * (HD + 2) + 2 + dd;
#pragma unroll 8
            for (int j = 0; j < jn; j++) acc = fmaf(col[(int64_t)j * (HD + 2)], __shfl(ereg[k], j, 64), acc);
          }
          if (d0 + lane < HD) put<true>(att + h * HD + dd, acc / L);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0) {
          __hip_atomic_store(sy.att_arrive(l, h), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_fetch_add(sy.att_done(l), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }

    // ---- wout rows: x = (x + o*a) + down*m (stablelm.go:365-377)
    {
      const MatDesc &W = w.wout;
      const int nm = W.chunks - na;
      const int r0 = gw;
      auto unit = [&](int r, Seg2 &g) { g = Seg2{row_ptr(W, r), row_ptr(W, r, na), xa, xm, na, nm}; };
      auto done = [&](int r, float ao, float ad) {
        if (lane == 0) put<true>(x_out + r, __fadd_rn(__fadd_rn(x_in[r], ao), ad));
      };
      Batch<UO> b;
      Seg2 g{};
      if (r0 < d) {
        unit(r0, g);
        batch_issue<F, UO>(b, g, 0, lane);
      }
      mark(4 + 6 * l);
      stage_x(xm, m, I, nm, VPC);  // complete: every block has passed bar_in
      __syncthreads();
      float ao = 0.f, ad = 0.f;
      if (r0 < d) batch_consume_range<F, UO, true>(b, g, 0, lane, na, na + nm, ao, ad);
      if (!block_wait(sy.att_done(l), tgt_heads, err, a.spin_limit, &s_flag)) return;
      mark(5 + 6 * l);
      stage_x(xa, att, d, na, VPC);
      __syncthreads();
      if (r0 < d) {
        batch_consume_range<F, UO, true>(b, g, 0, lane, 0, na, ao, ad);
        stream_rest<F, UO>(b, g, lane, ao, ad);
        done(r0, wave_sum(ao), wave_sum(ad));
        for (int r = r0 + NW; r < d; r += NW) {  // rows beyond one per wave
          unit(r, g);
          batch_issue<F, UO>(b, g, 0, lane);
          float x0 = 0.f, x1 = 0.f;
          batch_consume<F, UO, true>(b, g, 0, lane, x0, x1);
          stream_rest<F, UO>(b, g, lane, x0, x1);
          done(r, wave_sum(x0), wave_sum(x1));
        }
      }
      block_arrive(sy.bar_out(l));
      mark(6 + 6 * l);
    }
  }

  // ---- final LayerNorm + logits head
  if (!a.want_logits) return;
  {
    const int lane = lane0;
    const MatDesc &H = a.head;
    const int units = (H.rows + 1) >> 1, hch = H.chunks;
    auto unit = [&](int u, Seg2 &g) {
      const int64_t r0 = 2 * (int64_t)u;
      const bool two = r0 + 1 < H.rows;
      g = Seg2{row_ptr(H, r0), row_ptr(H, two ? r0 + 1 : r0), xq, xq, hch, two ? hch : 0};
    };
    auto done = [&](int u, float v0, float v1) {
      if (lane == 0) {
        a.logits[2 * (int64_t)u] = v0;
        if (2 * u + 1 < H.rows) a.logits[2 * (int64_t)u + 1] = v1;
      }
    };
    Batch<UI> b;
    Seg2 g{};
    if (gw < units) {
      unit(gw, g);
      batch_issue<F, UI>(b, g, 0, lane);
    }
    if (!block_wait(sy.bar_out(a.L - 1), tgt_blocks, err, a.spin_limit, &s_flag)) return;
    mark(1 + 6 * a.L);
    const float *xf = a.xs + (int64_t)a.L * persistent_stride(d);
    for (int i = tid; i < d; i += kT) xl[i] = xf[i];
    __syncthreads();
    norm_lds(s, xl, a.norm_w, a.norm_b, red);
    stage_x(xq, xl, d, hch, VPC);
    __syncthreads();
    stream_units_from<F, UI>(gw, NW, units, b, g, lane, unit, done);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    mark(2 + 6 * a.L);
  }
}

using KernelFn = void (*)(PersistentDecode);

struct Variant {
  int fmt, ui, uo, hd, half;
  KernelFn fn;
};

#define TINYOAI_VARIANT(F, UI, UO, HD)                                       \
  {F, UI, UO, HD, 0, persistent_decode_kernel<F, UI, UO, HD, false>},       \
  {F, UI, UO, HD, 1, persistent_decode_kernel<F, UI, UO, HD, true>}

// Shapes with an instantiation: the 3B StableLM in Q8_0 and BF16, and the
// small test models.
const Variant kVariants[] = {
    TINYOAI_VARIANT(FMT_Q8_0, 5, 10, 80), TINYOAI_VARIANT(FMT_BF16, 10, 10, 80),
    TINYOAI_VARIANT(FMT_BF16, 1, 1, 8),   TINYOAI_VARIANT(FMT_F32, 1, 1, 8),
    TINYOAI_VARIANT(FMT_Q8_0, 1, 2, 8),
};

int pick_batch(int chunks) {
  static const int us[] = {1, 2, 5, 10};
  for (int u : us)
    if (64 * u >= chunks) return u;
  return 10;
}

const Variant *find_variant(const PersistentDecode &a, const LayerDev &l0) {
  const int fmt = l0.win.fmt;
  if (l0.wout.fmt != fmt || a.head.fmt != fmt || a.head.cols != a.s.d) return nullptr;
  const int ui = pick_batch(2 * l0.win.chunks), uo = pick_batch(l0.wout.chunks);
  for (const Variant &v : kVariants)
    if (v.fmt == fmt && v.ui == ui && v.uo == uo && v.hd == a.s.hd && v.half == a.half_kv) return &v;
  return nullptr;
}

size_t lds_bytes(const PersistentDecode &a, const LayerDev &l0) {
  const int vpc = values_per_chunk(l0.win.fmt);
  const int na = (a.s.d + vpc - 1) / vpc;
  return (size_t)((a.s.d + 3) & ~3) * 4 + (size_t)l0.win.chunks * vpc * 4 + 16 * sizeof(double) +
         (size_t)((a.s.rot + 3) & ~3) * 4 + (size_t)na * vpc * 4 + (size_t)(l0.wout.chunks - na) * vpc * 4;
}

}  // namespace

size_t persistent_sync_words(int layers, int heads) { return (size_t)(1 + 3 * layers + layers * heads) * kLine; }

int persistent_decode_grid(const PersistentDecode &a, const LayerDev &layer0) {
  const Variant *v = find_variant(a, layer0);
  if (!v || a.s.heads % a.s.kv_heads || (a.cap_max + 15) / 16 > 512) return 0;
  int dev = 0, coop = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) return 0;
  const size_t lds = lds_bytes(a, layer0);
  if (lds > 64 * 1024) return 0;
  if (lds > 48 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void *>(v->fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(v->fn), kT, lds) !=
          hipSuccess ||
      per_cu < 1)
    return 0;
  return device_cu_count();
}

hipError_t launch_persistent_decode(const PersistentDecode &a, const LayerDev &layer0, int grid, hipStream_t st) {
  const Variant *v = find_variant(a, layer0);
  if (!v || grid <= 0) return hipErrorInvalidValue;
  if (a.max_splits < (a.cap_max + 15) / 16 || (a.cap_max + 15) / 16 > 512) return hipErrorInvalidValue;
  PersistentDecode arg = a;
  void *args[] = {&arg};
  return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(v->fn), dim3(grid), dim3(kT), args,
                                    lds_bytes(a, layer0), st);
}
