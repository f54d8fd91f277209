// Row streaming for the decode matrix-vector products (one activation
// vector, every row of a matrix once), for gfx950.
//
// Lanes own columns, rows stream past them. A wave owns a column slice of
// the matrix; lane l of the wave owns the chunks c0 + j*64 + l (j < CPL) of
// every row it processes, so it loads its part of x into registers once and
// then, per row, issues CPL buffer loads whose per-lane offsets never change
// (the row's offset rides in a scalar register). The consume of a chunk is
// the value decode and fused multiply-adds against registers: no LDS
// traffic, no per-chunk address arithmetic. Rows longer than one wave's
// 64 * CPL chunks are split into S column slices taken by S waves of the
// block; their partial sums meet in LDS and are added in slice order, so
// the result does not depend on timing.
//
// Work comes in units of R rows. Block b takes units b, b + G, b + 2G, ...
// (G blocks), so the grid reads one advancing window of the matrix; its
// waves form W / S row groups that take the block's units in turn. A wave
// runs its units as fully unrolled groups of up to kRowGroup batches (one
// batch = one unit's rows), an instance per group size, so every batch has
// registers of its own (a batch carried around a loop is copied at the
// back edge, and the copy waits for the loads just issued) and no load is
// issued past the wave's last unit. kAhead batches are in flight beyond
// the one being consumed; within a group every issue is unconditional,
// which keeps the compiler's vector-memory wait counts exact. The units'
// results are handed out after the group's last consume and stored
// together (PendingStore).
#pragma once

#include <climits>
#include <type_traits>

#include "epilogue.h"  // put<COH>
#include "formats.h"

// Batches per unrolled group, and how many batches a wave keeps in flight
// ahead of the one it consumes. Groups of two with one batch ahead keep a
// row-streaming wave within 168 VGPRs, so three waves fit a SIMD (twelve
// per CU hold ~130 KiB of 5.5 KiB batches in flight); measured on the 3B
// decode matrices, groups of four with two batches ahead (two waves per
// SIMD) were slower in every kernel.
constexpr int kRowGroup = 2;
// Result stores a wave holds back per group (two per unit).
constexpr int kPendingPerWave = 2 * kRowGroup;

// A store of a unit's result, held in LDS until the wave writes its group's
// results together: stores made one by one make each result wait for the
// previous stores to complete before their registers are reused.
struct PendingStore {
  uint64_t addr;
  uint32_t bits;
  uint32_t half;  // 1: a 16-bit store
};

// The output sink handed to done(): f32 / f16 record a store.
template <typename Rec>
struct PendingSink {
  Rec &rec;
  __device__ void f32(float *p, float v) const { rec(p, __float_as_uint(v), 0u); }
  __device__ void f16(uint16_t *p, uint16_t v) const { rec(p, (uint32_t)v, 1u); }
};
constexpr int kAhead = 1;
// Batches of the next group issued before a group's result code: one for
// the 16-byte-value formats; none for the 5/6-bit formats, whose batches
// carry block headers and high bits as well.
template <int F>
constexpr int carry_for() {
  return F == FMT_Q5_1 || F == FMT_Q4_K || F == FMT_Q5_K || F == FMT_Q6_K ? 0 : 1;
}
static_assert(kAhead >= 1 && kAhead + 1 <= kRowGroup, "the first group issues kAhead + 1 batches");
constexpr uint32_t kOffNone = 0x80000000u;  // a buffer offset past every plane (planes_fit)

// The byte offsets, within a row, of a lane's chunks (kOffNone where the
// lane has no chunk j) and their chunk indices.
template <int CPL>
struct LaneChunks {
  uint32_t vo[CPL], mo[CPL], ho[CPL];
  int cc[CPL];
  bool valid[CPL];
};

template <int F, int CPL>
__device__ __forceinline__ LaneChunks<CPL> lane_chunks(int c0, int width, int lane) {
  LaneChunks<CPL> L;
#pragma unroll
  for (int j = 0; j < CPL; j++) {
    const int rel = j * 64 + lane, c = c0 + rel;
    const bool ok = rel < width;
    L.valid[j] = ok;
    L.cc[j] = ok ? c : 0;
    L.vo[j] = ok ? (uint32_t)c * 16 : kOffNone;
    L.mo[j] = ok ? (uint32_t)meta_offset(F, c) : kOffNone;
    L.ho[j] = ok ? (uint32_t)hbits_offset(F, c) : kOffNone;
  }
  return L;
}

template <int CPL, int R>
struct RowBatch {
  uint4 w[R][CPL];
  uint32_t s[R][CPL];  // Q8_0 block scale, Q6_K d (fp16 bits)
  uint2 h[R][CPL];     // high bits (Q5_1, Q5_K, Q6_K)
  uint4 mt[R][CPL];    // block header (Q5_1, Q4_K, Q5_K, Q6_K)
};

// Calls f(integral_constant<n>) for the wave-uniform n in [1, N].
template <int N, typename Fn>
__device__ __forceinline__ void group_of_size(int n, Fn &&f) {
  if constexpr (N >= 1) {
    if (n == N) f(std::integral_constant<int, N>{});
    else group_of_size<N - 1>(n, f);
  }
}

// Issues the loads of rows row[0..R). Row offsets are wave-uniform.
template <int F, int CPL, int R>
__device__ __forceinline__ void rows_issue(RowBatch<CPL, R> &b, const LaneChunks<CPL> &L, const Planes &P,
                                           const MatDesc &M, const int (&row)[R]) {
  constexpr int kNT = 2;  // cache policy bit: nontemporal (each weight byte is read once)
  const __amdgpu_buffer_rsrc_t rv = P.v, rm = P.m, rh = P.h;
#pragma unroll
  for (int i = 0; i < R; i++) {
    const int sv = __builtin_amdgcn_readfirstlane((int)(row[i] * M.vstride));
    const int sm = __builtin_amdgcn_readfirstlane((int)(row[i] * M.mstride));
    const int sh = __builtin_amdgcn_readfirstlane((int)(row[i] * M.hstride));
#pragma unroll
    for (int j = 0; j < CPL; j++) {
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rv, (int)L.vo[j], sv, kNT);
      b.w[i][j] = make_uint4(w.x, w.y, w.z, w.w);
      if constexpr (F == FMT_Q8_0) b.s[i][j] = __builtin_amdgcn_raw_buffer_load_b16(rm, (int)L.mo[j], sm, 0);
      if constexpr (F == FMT_Q5_1) {
        b.mt[i][j].x = __builtin_amdgcn_raw_buffer_load_b32(rm, (int)L.mo[j], sm, 0);
        b.h[i][j].x = __builtin_amdgcn_raw_buffer_load_b32(rh, (int)L.ho[j], sh, 0);
      }
      if constexpr (F == FMT_Q4_K || F == FMT_Q5_K || F == FMT_Q6_K) {
        const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rm, (int)L.mo[j], sm, 0);
        b.mt[i][j] = make_uint4(t.x, t.y, t.z, t.w);
      }
      if constexpr (F == FMT_Q5_K) b.h[i][j].x = __builtin_amdgcn_raw_buffer_load_b32(rh, (int)L.ho[j], sh, 0);
      if constexpr (F == FMT_Q6_K) {
        b.s[i][j] = __builtin_amdgcn_raw_buffer_load_b16(rm, (int)(L.mo[j] + 16), sm, 0);
        const u32x2 hh = __builtin_amdgcn_raw_buffer_load_b64(rh, (int)L.ho[j], sh, 0);
        b.h[i][j] = make_uint2(hh.x, hh.y);
      }
    }
  }
}

// Adds one chunk's products with its x values in registers to acc: one
// chain of fused multiply-adds per row (Q8_0: the chunk's sum times its
// block scale, fused into acc).
template <int F>
__device__ __forceinline__ float reg_chunk_acc(const uint4 w, uint32_t s, uint2 h, const uint4 mt, int cc,
                                               const float *x, float acc) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  if constexpr (F == FMT_Q8_0) {
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t v = ws[k];
      a = fmaf((float)(int8_t)(v), x[4 * k], a);
      a = fmaf((float)(int8_t)(v >> 8), x[4 * k + 1], a);
      a = fmaf((float)(int8_t)(v >> 16), x[4 * k + 2], a);
      a = fmaf((float)(int8_t)(v >> 24), x[4 * k + 3], a);
    }
    return fmaf(a, hw_half((uint16_t)s), acc);
  } else if constexpr (F == FMT_BF16) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      acc = fmaf(__uint_as_float(ws[k] << 16), x[2 * k], acc);
      acc = fmaf(__uint_as_float(ws[k] & 0xffff0000u), x[2 * k + 1], acc);
    }
    return acc;
  } else if constexpr (F == FMT_F16) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      acc = fmaf(hw_half((uint16_t)ws[k]), x[2 * k], acc);
      acc = fmaf(hw_half((uint16_t)(ws[k] >> 16)), x[2 * k + 1], acc);
    }
    return acc;
  } else if constexpr (F == FMT_F32) {
#pragma unroll
    for (int k = 0; k < 4; k++) acc = fmaf(__uint_as_float(ws[k]), x[k], acc);
    return acc;
  } else {
    const KConst k = kquant_const<F>(mt, (uint16_t)s, cc);
#pragma unroll
    for (int qd = 0; qd < 4; qd++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t byte = (ws[qd] >> (8 * e)) & 255;
        const int j = 4 * qd + e;
        acc = fmaf(kquant_value<F>(k, kquant_q<F>(byte, j, h), j), x[j], acc);
        acc = fmaf(kquant_value<F>(k, kquant_q<F>(byte, j + 16, h), j + 16), x[j + 16], acc);
      }
    }
    return acc;
  }
}

// Adds the batch's rows' products to acc[row].
template <int F, int CPL, int R>
__device__ __forceinline__ void rows_consume(const RowBatch<CPL, R> &b, const LaneChunks<CPL> &L,
                                             const float (&x)[CPL][Fmt<F>::VPC], float (&acc)[R]) {
#pragma unroll
  for (int i = 0; i < R; i++)
#pragma unroll
    for (int j = 0; j < CPL; j++)
      acc[i] = reg_chunk_acc<F>(b.w[i][j], b.s[i][j], b.h[i][j], b.mt[i][j], L.cc[j], x[j], acc[i]);
}

// Column slices of a row of `nch` chunks split in two parts at chunk
// `split` (split == nch: one part): S0 slices of width w0 over the first
// part, then S - S0 slices of width w1 over the second, each at most
// 64 * CPL chunks, so no slice mixes the parts.
struct SliceShape {
  int S, S0, w0, w1;
};
__host__ __device__ inline SliceShape slice_shape(int nch, int split, int cpl) {
  const int span = 64 * cpl, n1 = nch - split;
  const int S0 = (split + span - 1) / span, S1 = (n1 + span - 1) / span;
  return SliceShape{S0 + S1, S0, S0 ? (split + S0 - 1) / S0 : 0, S1 ? (n1 + S1 - 1) / S1 : 0};
}
// First chunk and width of slice s.
__host__ __device__ inline void slice_range(const SliceShape &sh, int nch, int split, int s, int &c0, int &width) {
  if (s < sh.S0) {
    c0 = s * sh.w0;
    width = min(sh.w0, split - c0);
  } else {
    c0 = split + (s - sh.S0) * sh.w1;
    width = min(sh.w1, nch - c0);
  }
}

// Streams n_units units of R rows (unit u: rows unit_rows(u, row[]), row
// indices < M.rows) through the block; each row's sum comes in two parts,
// chunks before `split` and from it on (split == M.chunks: one part).
// Order of work: with XFIRST, `x_load(c, out)` fills the VPC x values of
// each of the lane's chunks (zeros past the vector); `pre()` issues the
// loads the prologue needs, and with PREWAIT the wave waits for them
// before any weight load goes out (they are not queued behind the weight
// stream); the first PRE batches (at most a group); `prologue()`
// (block-wide staging, with barriers); without XFIRST the x load; then the
// groups, which first bring the batches in flight up to kAhead. With AUX,
// `aux_load(row)` is issued with each batch (a per-row operand for done,
// e.g. the residual). `done(u, r, aux, out)` receives unit u's sums
// r[R][2] and aux[R] (wave-uniform; every lane calls it) and hands its
// results to out.f32 / out.f16 (at most two per unit). red: LDS of
// units_per_block * (S * R * 2 + R) floats when the rows span S > 1
// slices; pend: LDS of (T / 64) * kPendingPerWave PendingStores.
// With COH the results are stored with agent-scope atomic stores (other
// blocks of the launch read them); `hook(next)` runs on the wave after
// each group's results are stored, with the next unit the wave takes
// (INT_MAX when none), and once more with INT_MAX at the end. `blocks` is
// the number of blocks sharing the units (blocks 0 .. blocks - 1 of the
// launch; 0 = the whole grid). With DRAIN_FIRST the first group issues
// none of the next group's batches, so a hook that waits for the wave's
// stores after it waits for nothing else; with NOCARRY no group does (a
// kernel held to fewer registers).
template <int F, int T, int CPL, int R, bool XFIRST, bool PREWAIT, int PRE, bool AUX, bool COH = false,
          bool DRAIN_FIRST = false, bool NOCARRY = false, typename Rows, typename XLoad, typename AuxLoad, typename Pre, typename Prologue, typename Done,
          typename Hook = void (*)(int)>
__device__ __forceinline__ void stream_rows(const MatDesc &M, int n_units, int split, float *red, PendingStore *pend,
                                            Rows unit_rows, XLoad x_load, AuxLoad aux_load, Pre pre, Prologue prologue,
                                            Done done, Hook hook = [](int) {}, int blocks = 0) {
  constexpr int VPC = Fmt<F>::VPC, K = kRowGroup;
  // The wave index in a scalar register: everything per wave below (slice,
  // row group, units, whether a batch is real) is then scalar, and so is
  // the choice of buffer descriptor (a per-lane choice would make the
  // compiler loop over the lanes' descriptors around every load).
  constexpr int W = T / 64;
  static_assert(PRE >= 0 && PRE <= kRowGroup, "batches before the prologue: at most a group");
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const SliceShape sh = slice_shape(M.chunks, split, CPL);
  const int S = sh.S, RG = W / S;
  const int s = wave % S, rg = wave / S;  // rg == RG for waves left over (W % S)
  const int part = s >= sh.S0;            // which part of the row this wave's slice sums
  int c0, width;
  slice_range(sh, M.chunks, split, s, c0, width);
  // The block's units, by local index j < nj: unit_of(j) = blockIdx.x + j * G.
  // Interleaving the blocks' units keeps the whole grid reading one advancing
  // window of the matrix (contiguous ranges per block had every block open
  // its own DRAM rows).
  const int G = blocks > 0 ? blocks : (int)gridDim.x, b0 = blockIdx.x;
  const int nj = n_units > b0 ? (n_units - b0 + G - 1) / G : 0;
  auto unit_of = [&](int j) { return b0 + j * G; };
  const int slot = S * R * 2 + R;  // LDS floats per unit (S > 1)
  PendingStore *pw = pend + wave * kPendingPerWave;
  int np = 0;  // pending stores (wave-uniform)
  auto flush = [&]() {
    if (lane < np) {
      const PendingStore e = pw[lane];
      if (e.half) put<COH>(reinterpret_cast<uint16_t *>(e.addr), (uint16_t)e.bits);
      else put<COH>(reinterpret_cast<uint32_t *>(e.addr), e.bits);
    }
    np = 0;
  };
  auto record = [&](void *p, uint32_t bits, uint32_t half) {
    if (np == kPendingPerWave) flush();
    if (lane == 0) pw[np] = PendingStore{reinterpret_cast<uint64_t>(p), bits, half};
    np++;
  };
  const PendingSink<decltype(record)> sink{record};
  const Planes P = make_planes(M);
  const LaneChunks<CPL> L = lane_chunks<F, CPL>(c0, width, lane);
  float x[CPL][VPC];
  auto load_x = [&]() {
#pragma unroll
    for (int j = 0; j < CPL; j++) {
      if (L.valid[j]) {
        x_load(L.cc[j], x[j]);
      } else {
#pragma unroll
        for (int v = 0; v < VPC; v++) x[j][v] = 0.f;
      }
    }
  };
  // This wave's units: local indices rg, rg + RG, ... below nj (wave-uniform
  // count nb). Every batch issued is a real one: a group of N batches is a
  // separately unrolled instance for each N <= K, so no load is issued past
  // the wave's last unit (such loads complete behind the grid's traffic,
  // and code that reuses their registers waits for them).
  const int nb = rg < RG && nj > rg ? (nj - rg + RG - 1) / RG : 0;
  RowBatch<CPL, R> b[K];
  float aux[K][R];
  int first_j = rg;  // local index of the group's first unit
  // Batch k of the group starting at local index j0.
  auto issue_at = [&](int j0, int k) {
    int row[R];
    unit_rows(unit_of(j0 + k * RG), row);
    if constexpr (AUX) {
#pragma unroll
      for (int i = 0; i < R; i++) aux[k][i] = aux_load(row[i]);
    }
    rows_issue<F, CPL, R>(b[k], L, P, M, row);
  };
  auto issue = [&](int k) { issue_at(first_j, k); };
  if constexpr (XFIRST) load_x();
  pre();
  if constexpr (PREWAIT) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // One group of N batches, P0 of them already issued; step k issues the
  // batches up to k + kAhead, then consumes batch k; the units' results
  // follow the last consume (result code between the consumes reuses
  // registers and makes the wave wait for the batches in flight). After
  // the last consume the first min(kCarry, n_next) batches of the next
  // group (n_next units) are issued into the consumed batches' registers,
  // so the wave's loads stay in flight through the result code.
  constexpr int kCarry = NOCARRY ? 0 : carry_for<F>();
  auto group = [&](auto n_tag, auto p0_tag, int n_next) {
    constexpr int N = decltype(n_tag)::value, P0 = decltype(p0_tag)::value;
    int r[N][R];  // float bits, wave-uniform (scalar registers)
#pragma unroll
    for (int k = 0; k < N; k++) {
#pragma unroll
      for (int t = (k == 0 ? P0 : k + kAhead); t < N && t <= k + kAhead; t++) issue(t);
      // every load of the new batches is issued before any wait for this one
      __builtin_amdgcn_sched_barrier(0);
      float acc[R];
#pragma unroll
      for (int i = 0; i < R; i++) acc[i] = 0.f;
      rows_consume<F, CPL, R>(b[k], L, x, acc);
#pragma unroll
      for (int i = 0; i < R; i++) r[k][i] = __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, wave_total(acc[i])));
    }
    float ax[N][R];  // this group's per-row operands (their slots take the next group's)
#pragma unroll
    for (int k = 0; k < N; k++)
#pragma unroll
      for (int i = 0; i < R; i++) ax[k][i] = AUX ? aux[k][i] : 0.f;
    if constexpr (kCarry > 0) {
      group_of_size<kCarry>(min(n_next, kCarry), [&](auto pn_tag) {
        constexpr int PN = decltype(pn_tag)::value;
#pragma unroll
        for (int t = 0; t < PN; t++) issue_at(first_j + N * RG, t);
      });
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < N; k++) {
      float rk[R][2];
#pragma unroll
      for (int i = 0; i < R; i++) {
        const float v = __builtin_bit_cast(float, r[k][i]);
        rk[i][0] = part ? 0.f : v;
        rk[i][1] = part ? v : 0.f;
      }
      const int j = first_j + k * RG;
      if (S == 1) {
        done(unit_of(j), rk, ax[k], sink);
        __builtin_amdgcn_sched_barrier(0);  // one unit's result code at a time
      } else if (lane == 0) {
        float *dst = red + j * slot;
#pragma unroll
        for (int i = 0; i < R; i++) {
          dst[s * R * 2 + 2 * i] = rk[i][0];
          dst[s * R * 2 + 2 * i + 1] = rk[i][1];
          if (s == 0) dst[S * R * 2 + i] = ax[k][i];
        }
      }
    }
    flush();
    // the next group's loads are not hoisted into the result code
    __builtin_amdgcn_sched_barrier(0);
    first_j += N * RG;
    hook(first_j < nj ? unit_of(first_j) : INT_MAX);
  };
  // The first group issues its first min(N, PRE) batches before the
  // prologue (older than every later load, so later wait counts stay
  // exact); a wave with no units still runs the prologue (its barriers).
  auto first = [&](auto n_tag, int n_next) {
    constexpr int N = decltype(n_tag)::value, PI = N < PRE ? N : PRE;
#pragma unroll
    for (int t = 0; t < PI; t++) issue(t);
    prologue();
    if constexpr (!XFIRST) load_x();
    group(n_tag, std::integral_constant<int, PI>{}, DRAIN_FIRST ? 0 : n_next);
  };
  int left = nb;
  auto peek = [&]() { return min(left, K); };
  auto take = [&]() {
    const int n = peek();
    left -= n;
    return n;
  };
  // Groups after the first find min(kCarry, N) of their batches issued by
  // the group before.
  auto rest = [&](auto n_tag, int n_next) {
    constexpr int N = decltype(n_tag)::value;
    group(n_tag, std::integral_constant<int, (N < kCarry ? N : kCarry)>{}, n_next);
  };
  if (left > 0) {
    const int n = take(), nn = peek();
    group_of_size<K>(n, [&](auto n_tag) { first(n_tag, nn); });
    if constexpr (DRAIN_FIRST) {  // the second group issues all of its batches
      if (left > 0) {
        const int n2 = take(), nn2 = peek();
        group_of_size<K>(n2, [&](auto n_tag) { group(n_tag, std::integral_constant<int, 0>{}, nn2); });
      }
    }
  } else {
    prologue();
    if constexpr (!XFIRST) load_x();
  }
  while (left > 0) {
    const int n = take(), nn = peek();
    group_of_size<K>(n, [&](auto n_tag) { rest(n_tag, nn); });
  }
  if (S == 1) {
    hook(INT_MAX);
    return;
  }
  __syncthreads();  // every slice's partial sums are in LDS
  for (int j = wave; j < nj; j += W) {
    float r[R][2], a[R];
    const float *src = red + j * slot;
#pragma unroll
    for (int i = 0; i < R; i++) {
      r[i][0] = r[i][1] = 0.f;
      for (int t = 0; t < S; t++) {
        r[i][0] += src[t * R * 2 + 2 * i];
        r[i][1] += src[t * R * 2 + 2 * i + 1];
      }
      a[i] = src[S * R * 2 + i];
    }
    done(unit_of(j), r, a, sink);
  }
  flush();
  hook(INT_MAX);
}
