// Causal attention of a prefill chunk on the matrix cores (attendBatch,
// attention.go:6-45; per head as attendHeads, stablelm.go:391-431): n
// queries at positions pos0 .. pos0 + n - 1 against cache positions
// 0 .. pos0 + n - 1, online softmax in fp32.
//
// With an fp32 cache the fp32 operands are carried as fp16 hi + lo (x =
// hi + lo to ~22 bits): queries, softmax weights, K and V. With an fp16
// cache K and V are exact as stored, and the queries and weights are
// rounded to fp16 (to nearest), the precision the cache keeps K and V in:
// one product per operand pair instead of two. Products accumulate in fp32.
#include "kernels.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

namespace {

constexpr int kTile = 64;   // cache positions per iteration
// Scores are kept in base 2 (s / scale * log2 e): the softmax weights are
// then single v_exp_f32 (2^x) instructions; exp(v - m) = 2^((v - m) log2 e).
constexpr float kLog2e = 1.4426950408889634f;

struct FlashArgs {
  StableDims s;
  KVDev kv;
  const float *q;  // [n][heads][hd]
  const int *pos0;
  int n;
  float *out;      // [n][heads][hd] (may be null)
  uint16_t *oh, *ol;  // the same as bf16 operand planes (null: none)
  // Branch rows (BR instances): cache positions t >= prefix come from slot
  // sfx_slot0 + (t - prefix) of the branch cache sfx.
  KVDev sfx;
  int prefix, sfx_slot0;
  // Shared prefix (SH instances): block x attends cache positions
  // [x * split_keys, min(prefix, (x + 1) * split_keys)) for all n queries
  // (branch rows, each past the prefix, so no causal mask) and writes the
  // unnormalised record {m, l, o[hd]} (m in natural-log units, o and l
  // weighted by exp(score - m)) at partials + (j * heads + h) * region +
  // x * (hd + 2), the split-K decode attention's partial layout.
  float *partials;
  int64_t region;
  int split_keys;
  int64_t ld_o;  // values between the query rows of oh, ol (0: heads * hd)
  // Key splits (prefill, ksplit > 1): block z of a query tile attends the
  // key tiles of split z (key_split_tiles) and writes its record {m, l,
  // o[hd]} at partials + (j * heads + h) * region + z * (hd + 2), as the
  // shared-prefix pass does; flash_combine_kernel forms the output.
  int ksplit;
  // Branch runs in one launch (BR instances): segment blockIdx.z is
  // segs[3z..3z+2] = (first row a0, rows, slot of its first position): its
  // queries are rows a0.. of q / out and its positions and slots rows a0..
  // of pos0 (pairs); n is the longest run.
  const int *segs;
};

// x = hi + lo to about 2^-22. The empty asm pins x as one fp32 value: when x
// is a product, the compiler otherwise forms hi once by a fused
// multiply-convert (one rounding) for the residual and once by converting the
// rounded product for the operand, and the two can differ by an fp16 ulp.
__device__ __forceinline__ void split_half(float x, _Float16 &hi, _Float16 &lo) {
  asm volatile("" : "+v"(x));
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

// One block of 4 waves per (128 queries, head) on v_mfma_f32_32x32x16_f16;
// each wave owns 32 queries and every 64-key tile of K and V^T is staged in
// LDS once for all of them.
//   S^T = K Q^T: two 32-key halves x 32 queries, k = 16 head dims per step
//   (hd / 16 steps, no padding). Lane l then holds, for query l % 32, the
//   keys (v / 4) * 8 + (l / 32) * 4 + v % 4 (v < 16) of each half.
//   O += P V: 32 queries x 32 dims per tile, k = 16 keys per step. Step kk
//   takes keys base + g * 4 + {0..3} and base + 8 + g * 4 + {0..3} (g = l /
//   32, base = 16 kk), exactly the scores lane l holds as values
//   (kk % 2) * 8 .. + 8 of half kk / 2, so P needs no lane exchange; V^T is
//   read with the same key order. O rows are queries ((v / 4) * 8 + g * 4 +
//   v % 4), so each lane fetches the softmax factors of its 16 rows.
constexpr int kQ32 = 128;  // queries per block
constexpr int kSharedKeys = 256;  // cache positions per block of the shared-prefix pass

// Key splits of a query tile whose first query sits at position `first`:
// the key tiles 0 .. first / kTile (each starts at or before every query of
// the tile, so every query sees a key of every split) are cut in at most
// `ks` runs of `per` tiles; the last split also takes the tiles past them
// (the diagonal). Returns the number of splits.
__host__ __device__ inline int key_split_tiles(int first, int ks, int &per) {
  const int d = first / kTile + 1;
  per = (d + ks - 1) / ks;
  return (d + per - 1) / per;
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int HD, bool HALF, bool BR, bool SH = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void flash32_kernel(FlashArgs a) {
  static_assert(HD % 16 == 0, "head width in 16-dim k-steps");
  constexpr int KS = HD / 16;         // k-steps over head dims
  constexpr int KP = HD + 8;          // LDS pitch of a K row (halves)
  constexpr int DT = (HD + 31) / 32;  // 32-wide output tiles over head dims (zero padded)
  constexpr int VP = kTile + 4;       // LDS pitch of a V^T row (halves): 16 rows of 8 bytes span all banks
  constexpr int NPL = HALF ? 1 : 2;   // fp16 planes of K and V
  constexpr float kRescale = 8.f;     // reference moves only when a score exceeds it by 2^8
  // With head dims padded to DT * 32, V^T row HD holds ones: that output
  // column accumulates the softmax denominator from the very P fed to the
  // matrix cores.
  constexpr bool ONES = DT * 32 > HD;
  __shared__ __align__(16) _Float16 ks[NPL][kTile * KP];
  __shared__ __align__(16) _Float16 vt[NPL][DT * 32 * VP];

  const StableDims &s = a.s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.y, kvh = h / (s.heads / s.kv_heads);
  if (BR && a.segs) {
    const int *sg = a.segs + 3 * blockIdx.z;
    const int a0 = sg[0];
    a.n = sg[1];
    a.sfx_slot0 = sg[2];
    a.q += (int64_t)a0 * s.heads * HD;
    a.pos0 += 2 * a0;
    if (a.out) a.out += (int64_t)a0 * s.heads * HD;
  }
  const int p0 = SH ? 0 : *a.pos0;
  // Query tiles run in reverse order for the second half of the heads:
  // workgroups k and k + grid / 2 share a CU when the grid fills two per
  // CU, and the reversal pairs a long causal range with a short one there.
  // SH: one query tile; blockIdx.x is the key range.
  const int qt = SH ? 0 : blockIdx.y >= (gridDim.y + 1) / 2 ? gridDim.x - 1 - blockIdx.x : blockIdx.x;
  if (BR && a.segs && qt * kQ32 >= a.n) return;      // past this run's queries (the whole block)
  const int qb = qt * kQ32;                          // first query of the block
  const int qw = qb + wave * 32;                     // first query of the wave
  const int col = lane & 31, g = lane >> 5;          // S^T column (query) / B row, lane group
  const int myq = qw + col;                          // this lane's query as an S^T column
  const int k_lo = SH ? blockIdx.x * a.split_keys : 0;
  const int k_hi = SH ? min(a.prefix, k_lo + a.split_keys) : 0;
  // the last key a query sees (SH: every key of the range)
  const int myq_pos = SH ? k_hi - 1 : p0 + min(myq, a.n - 1);
  const int last_pos = SH ? k_hi - 1 : p0 + min(qb + kQ32, a.n) - 1;  // causal bound of the block
  const float qscale = kLog2e / s.att_scale;          // Q pre-scaled: scores come out in base 2

  // Q^T as B operands: column = query, k = dims 16 * step + 8 * g .. + 8.
  f16x8 qh[KS], ql[KS];
  {
    const float *qp = a.q + ((int64_t)min(myq, a.n - 1) * s.heads + h) * HD;
    // every value loaded before the first conversion (split_half's empty
    // asm keeps later loads behind it: one memory round trip per value)
    float qv[KS][8];
#pragma unroll
    for (int k = 0; k < KS; k++) {
      const float4 a0 = *reinterpret_cast<const float4 *>(qp + k * 16 + g * 8);
      const float4 a1 = *reinterpret_cast<const float4 *>(qp + k * 16 + g * 8 + 4);
      qv[k][0] = a0.x, qv[k][1] = a0.y, qv[k][2] = a0.z, qv[k][3] = a0.w;
      qv[k][4] = a1.x, qv[k][5] = a1.y, qv[k][6] = a1.z, qv[k][7] = a1.w;
    }
#pragma unroll
    for (int k = 0; k < KS; k++)
#pragma unroll
      for (int i = 0; i < 8; i++) {
        _Float16 hi, lo;
        if constexpr (HALF) {
          hi = (_Float16)(qv[k][i] * qscale);
          lo = (_Float16)0.f;
        } else {
          split_half(qv[k][i] * qscale, hi, lo);
        }
        qh[k][i] = hi;
        ql[k][i] = lo;
      }
  }
  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; t++)
#pragma unroll
    for (int v = 0; v < 16; v++) o[t][v] = 0.f;
  // Softmax state of query `col` (same in both lane groups). Weights are
  // 2^(score - ref); ref is the exact max of the first tile and then moves
  // only when a score exceeds it by more than kRescale, so the weights stay
  // in [0, 2^8] and O is rescaled rarely. The accumulators of S start at
  // -ref, which applies the reference for free.
  float ref = 0.f, l_run = 0.f;

  if constexpr (ONES) {  // V^T rows HD .. DT * 32: row HD ones, the rest zero
    constexpr int PAD = (DT * 32 - HD) * VP;
    for (int e = tid; e < NPL * PAD; e += 256)
      vt[e / PAD][HD * VP + e % PAD] = (_Float16)(e < VP ? 1.f : 0.f);
  }
  const int64_t head_base = (int64_t)kvh * a.kv.cap * HD;
  // BR: the branch's suffix, position t >= prefix at element sfx_base + (t - prefix) * HD.
  const int64_t sfx_base = BR ? ((int64_t)kvh * a.sfx.cap + a.sfx_slot0) * HD : 0;
  int ntiles = last_pos / kTile + 1, tile0 = k_lo / kTile;
  if (!SH && !BR && a.ksplit > 1) {  // block-uniform
    int per;
    const int splits = key_split_tiles(p0 + qb, a.ksplit, per), z = blockIdx.z;
    if (z >= splits) return;
    tile0 = z * per;
    if (z + 1 < splits) ntiles = tile0 + per;
  }
  // fp16 cache: a tile is loaded into registers while the previous one is
  // computed. Buffer loads read zeros past the block's last position.
  constexpr int KC = kTile * (HD / 8), KPT = (KC + 255) / 256;  // 16-byte K pieces
  // V: each of VB threads moves 4 keys x 8 dims; the key group runs fastest
  // over lanes so the transposed 8-byte stores of one dim fill all banks.
  constexpr int VB = (kTile / 4) * (HD / 8);
  static_assert(VB <= 256, "one V block per thread");
  constexpr uint32_t kNone = 0x80000000u;
  uint4 kreg[KPT], vreg[4];
  // The model cache holds positions [0, min(last_pos + 1, prefix)) (all of
  // them without BR); with BR the branch cache the rest. A piece whose key
  // lies in the other region reads at kNone (zeros, no memory request) from
  // this one, so OR-ing the two loads gives the piece.
  const int n_model = BR ? min(last_pos + 1, a.prefix) : last_pos + 1;
  const __amdgpu_buffer_rsrc_t rk = plane_rsrc(
      reinterpret_cast<const uint8_t *>(a.kv.k) + head_base * 2, (int64_t)n_model * HD * 2);
  const __amdgpu_buffer_rsrc_t rv = plane_rsrc(
      reinterpret_cast<const uint8_t *>(a.kv.v) + head_base * 2, (int64_t)n_model * HD * 2);
  const int n_sfx = BR ? max(last_pos + 1 - a.prefix, 0) : 0;
  const __amdgpu_buffer_rsrc_t rk2 = plane_rsrc(
      reinterpret_cast<const uint8_t *>(BR ? a.sfx.k : a.kv.k) + sfx_base * 2, (int64_t)n_sfx * HD * 2);
  const __amdgpu_buffer_rsrc_t rv2 = plane_rsrc(
      reinterpret_cast<const uint8_t *>(BR ? a.sfx.v : a.kv.v) + sfx_base * 2, (int64_t)n_sfx * HD * 2);
  auto ld16 = [](__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
  };
  // The 16-byte piece at dims [c8, c8 + 8) of key t (t < kNone / 2 / HD).
  auto piece = [&](__amdgpu_buffer_rsrc_t r, __amdgpu_buffer_rsrc_t r2, bool ok, int t, int c8) {
    if constexpr (BR) {
      const uint32_t o1 = ok && t < a.prefix ? (uint32_t)((t * HD + c8) * 2) : kNone;
      const uint32_t o2 = ok && t >= a.prefix ? (uint32_t)(((t - a.prefix) * HD + c8) * 2) : kNone;
      const uint4 x = ld16(r, o1), y = ld16(r2, o2);
      return make_uint4(x.x | y.x, x.y | y.y, x.z | y.z, x.w | y.w);
    } else {
      return ld16(r, ok ? (uint32_t)((t * HD + c8) * 2) : kNone);
    }
  };
  auto hload = [&](int t0) {
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int e = tid + 256 * i;
      kreg[i] = piece(rk, rk2, e < KC, t0 + e / (HD / 8), (e % (HD / 8)) * 8);
    }
    const int kg = tid % (kTile / 4), dg = tid / (kTile / 4);
#pragma unroll
    for (int i = 0; i < 4; i++) vreg[i] = piece(rv, rv2, tid < VB, t0 + kg * 4 + i, dg * 8);
  };
  auto hstore = [&]() {
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int e = tid + 256 * i, key = e / (HD / 8), c = e % (HD / 8);
      if (KC % 256 == 0 || e < KC) *reinterpret_cast<uint4 *>(&ks[0][key * KP + c * 8]) = kreg[i];
    }
    if (tid < VB) {  // V^T: 8 dims x 4 keys, one 8-byte row piece per dim
      const int kg = tid % (kTile / 4), dg = tid / (kTile / 4);
      const uint32_t w[4][4] = {{vreg[0].x, vreg[0].y, vreg[0].z, vreg[0].w},
                                {vreg[1].x, vreg[1].y, vreg[1].z, vreg[1].w},
                                {vreg[2].x, vreg[2].y, vreg[2].z, vreg[2].w},
                                {vreg[3].x, vreg[3].y, vreg[3].z, vreg[3].w}};
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int sh = 16 * (j & 1);
        const uint32_t k0 = (w[0][j >> 1] >> sh) & 0xffffu, k1 = (w[1][j >> 1] >> sh) & 0xffffu;
        const uint32_t k2 = (w[2][j >> 1] >> sh) & 0xffffu, k3 = (w[3][j >> 1] >> sh) & 0xffffu;
        *reinterpret_cast<uint2 *>(&vt[0][(dg * 8 + j) * VP + kg * 4]) = make_uint2(k0 | (k1 << 16), k2 | (k3 << 16));
      }
    }
  };
  // fp32 cache: 16-byte pieces of 4 values of key t at dims [d0, d0 + 4),
  // read by buffer loads (zeros past the block's last position) as pieces of
  // the fp16 cache are, so a tile's loads all issue before any is used.
  const __amdgpu_buffer_rsrc_t rk4 = plane_rsrc(
      reinterpret_cast<const uint8_t *>(a.kv.k) + head_base * 4, HALF ? 0 : (int64_t)n_model * HD * 4);
  const __amdgpu_buffer_rsrc_t rv4 = plane_rsrc(
      reinterpret_cast<const uint8_t *>(a.kv.v) + head_base * 4, HALF ? 0 : (int64_t)n_model * HD * 4);
  const __amdgpu_buffer_rsrc_t rk4s = plane_rsrc(
      reinterpret_cast<const uint8_t *>(BR ? a.sfx.k : a.kv.k) + sfx_base * 4, HALF ? 0 : (int64_t)n_sfx * HD * 4);
  const __amdgpu_buffer_rsrc_t rv4s = plane_rsrc(
      reinterpret_cast<const uint8_t *>(BR ? a.sfx.v : a.kv.v) + sfx_base * 4, HALF ? 0 : (int64_t)n_sfx * HD * 4);
  auto piece4 = [&](__amdgpu_buffer_rsrc_t r, __amdgpu_buffer_rsrc_t r2, bool ok, int t, int d0) {
    if constexpr (BR) {
      const uint32_t o1 = ok && t < a.prefix ? (uint32_t)((t * HD + d0) * 4) : kNone;
      const uint32_t o2 = ok && t >= a.prefix ? (uint32_t)(((t - a.prefix) * HD + d0) * 4) : kNone;
      const uint4 x = ld16(r, o1), y = ld16(r2, o2);
      return make_uint4(x.x | y.x, x.y | y.y, x.z | y.z, x.w | y.w);
    } else {
      return ld16(r, ok ? (uint32_t)((t * HD + d0) * 4) : kNone);
    }
  };
  if constexpr (HALF) hload(tile0 * kTile);
  for (int tile = tile0; tile < ntiles; tile++) {
    const int t0 = tile * kTile;
    __syncthreads();
    if constexpr (HALF) {
      hstore();
      if (tile + 1 < ntiles) hload(t0 + kTile);
    } else {
      // fp32 cache: hi and lo planes, 4 values per 16-byte load, every load
      // of the tile issued before the first is used
      constexpr int KE4 = kTile * (HD / 4), KI = (KE4 + 255) / 256;
      uint4 kw4[KI], vw4[KI];
#pragma unroll
      for (int i = 0; i < KI; i++) {
        const int e = tid + 256 * i, key = e / (HD / 4), d0 = (e % (HD / 4)) * 4;
        const bool ok = e < KE4 && t0 + key <= last_pos;
        kw4[i] = piece4(rk4, rk4s, ok, t0 + key, d0);
        vw4[i] = piece4(rv4, rv4s, ok, t0 + key, d0);
      }
#pragma unroll
      for (int i = 0; i < KI; i++) {
        const int e = tid + 256 * i, key = e / (HD / 4), d0 = (e % (HD / 4)) * 4;
        if (KE4 % 256 != 0 && e >= KE4) continue;
        const float kx[4] = {__uint_as_float(kw4[i].x), __uint_as_float(kw4[i].y), __uint_as_float(kw4[i].z),
                             __uint_as_float(kw4[i].w)};
        const float vx[4] = {__uint_as_float(vw4[i].x), __uint_as_float(vw4[i].y), __uint_as_float(vw4[i].z),
                             __uint_as_float(vw4[i].w)};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          _Float16 kh, kl, vh, vl;
          split_half(kx[j], kh, kl);
          split_half(vx[j], vh, vl);
          ks[0][key * KP + d0 + j] = kh;
          ks[NPL - 1][key * KP + d0 + j] = kl;
          vt[0][(d0 + j) * VP + key] = vh;
          vt[NPL - 1][(d0 + j) * VP + key] = vl;
        }
      }
    }
    __syncthreads();
    if (qw >= a.n || (!SH && t0 > p0 + qw + 31)) continue;  // nothing for this wave in this tile

    // ---- S^T - ref (two 32-key halves; the Q hi/lo parts chain into one accumulator)
    f32x16 sc[2];
#pragma unroll
    for (int kh = 0; kh < 2; kh++)
#pragma unroll
      for (int v = 0; v < 16; v++) sc[kh][v] = -ref;
#pragma unroll
    for (int k = 0; k < KS; k++)
#pragma unroll
      for (int kh = 0; kh < 2; kh++) {
        const int r = (kh * 32 + col) * KP + k * 16 + g * 8;
        const f16x8 ka = *reinterpret_cast<const f16x8 *>(&ks[0][r]);
        sc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[k], sc[kh], 0, 0, 0);
        if constexpr (!HALF) sc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, ql[k], sc[kh], 0, 0, 0);
        if constexpr (!HALF) {
          const f16x8 kl = *reinterpret_cast<const f16x8 *>(&ks[NPL - 1][r]);
          sc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[k], sc[kh], 0, 0, 0);
        }
      }
    if (SH ? t0 + kTile > k_hi : t0 + kTile - 1 > p0 + qw) {  // tile reaches past a visible key: mask
#pragma unroll
      for (int kh = 0; kh < 2; kh++)
#pragma unroll
        for (int v = 0; v < 16; v++)
          if (t0 + kh * 32 + (v >> 2) * 8 + g * 4 + (v & 3) > myq_pos) sc[kh][v] = -INFINITY;
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kh = 0; kh < 2; kh++)
#pragma unroll
      for (int v = 0; v < 16; v++) tmax = fmaxf(tmax, sc[kh][v]);
    // finite: the first key of the first tile is visible to every query
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    if (tile == tile0 || __ballot(tmax > kRescale)) {
      const float d = tile == tile0 ? tmax : fmaxf(tmax, 0.f);  // reference shift of this lane's query
      ref += d;
#pragma unroll
      for (int kh = 0; kh < 2; kh++)
#pragma unroll
        for (int v = 0; v < 16; v++) sc[kh][v] -= d;
      if (tile > tile0) {
        const float corr = __builtin_amdgcn_exp2f(-d);
        if constexpr (!ONES) l_run *= corr;
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const float rc = __shfl(corr, (v >> 2) * 8 + g * 4 + (v & 3), 64);
#pragma unroll
          for (int t = 0; t < DT; t++) o[t][v] *= rc;
        }
      }
    }
    // Weights 2^(score - ref) in [0, 2^8] (masked: 2^-inf = 0) as fp16 hi + lo
    // (both truncated: the residual p - hi is exact in fp32); with an fp16
    // cache one fp16 part, rounded to nearest (the ones row of V^T then
    // sums the same rounded weights).
    f16x8 ph[4], pl[4];  // A operands of the four 16-key steps
    float psum = 0.f;
#pragma unroll
    for (int kh = 0; kh < 2; kh++)
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const float p0v = __builtin_amdgcn_exp2f(sc[kh][v]), p1v = __builtin_amdgcn_exp2f(sc[kh][v + 1]);
        if constexpr (HALF) {
          const _Float16 h0 = (_Float16)p0v, h1 = (_Float16)p1v;
          if constexpr (!ONES) psum += (float)h0 + (float)h1;
          ph[kh * 2 + (v >> 3)][v & 7] = h0;
          ph[kh * 2 + (v >> 3)][(v & 7) + 1] = h1;
        } else {
          if constexpr (!ONES) psum += p0v + p1v;
          const auto hi = __builtin_amdgcn_cvt_pkrtz(p0v, p1v);
          const auto lo = __builtin_amdgcn_cvt_pkrtz(p0v - (float)hi[0], p1v - (float)hi[1]);
          ph[kh * 2 + (v >> 3)][v & 7] = hi[0];
          ph[kh * 2 + (v >> 3)][(v & 7) + 1] = hi[1];
          pl[kh * 2 + (v >> 3)][v & 7] = lo[0];
          pl[kh * 2 + (v >> 3)][(v & 7) + 1] = lo[1];
        }
      }
    if constexpr (!ONES) l_run += psum + __shfl_xor(psum, 32, 64);
    // ---- O += P V
#pragma unroll
    for (int kk = 0; kk < 4; kk++)
#pragma unroll
      for (int t = 0; t < DT; t++) {
        const int base = kk * 16 + g * 4;
        const _Float16 *v0 = &vt[0][(t * 32 + col) * VP + base];
        const uint2 a4 = *reinterpret_cast<const uint2 *>(v0), b4 = *reinterpret_cast<const uint2 *>(v0 + 8);
        const f16x8 vb = __builtin_bit_cast(f16x8, make_uint4(a4.x, a4.y, b4.x, b4.y));
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph[kk], vb, o[t], 0, 0, 0);
        if constexpr (!HALF) o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl[kk], vb, o[t], 0, 0, 0);
        if constexpr (!HALF) {
          const _Float16 *v1 = &vt[NPL - 1][(t * 32 + col) * VP + base];
          const uint2 c4 = *reinterpret_cast<const uint2 *>(v1), d4 = *reinterpret_cast<const uint2 *>(v1 + 8);
          const f16x8 vl = __builtin_bit_cast(f16x8, make_uint4(c4.x, c4.y, d4.x, d4.y));
          o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph[kk], vl, o[t], 0, 0, 0);
        }
      }
  }
  // ---- normalise and store: lane holds queries (v / 4) * 8 + g * 4 + v % 4, dim t * 32 + col
  if (SH || (!BR && a.ksplit > 1)) {  // the record of this key range
    constexpr float kLn2 = 0.6931471805599453f;
    const int slot = SH ? blockIdx.x : blockIdx.z;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int src = (v >> 2) * 8 + g * 4 + (v & 3);
      const float lq = ONES ? __shfl(o[DT - 1][v], g * 32 + HD % 32, 64) : __shfl(l_run, src, 64);
      const float mq = __shfl(ref, src, 64) * kLn2;
      const int qi = qw + src;
      if (qi >= a.n) continue;
      float *part = a.partials + ((int64_t)qi * s.heads + h) * a.region + (int64_t)slot * (HD + 2);
      if (col == 0) {
        part[0] = mq;
        part[1] = lq;
      }
#pragma unroll
      for (int t = 0; t < DT; t++) {
        const int dd = t * 32 + col;
        if (dd < HD) part[2 + dd] = o[t][v];
      }
    }
    return;
  }
#pragma unroll
  for (int v = 0; v < 16; v++) {
    const float lq = ONES ? __shfl(o[DT - 1][v], g * 32 + HD % 32, 64)
                          : __shfl(l_run, (v >> 2) * 8 + g * 4 + (v & 3), 64);
    const int qi = qw + (v >> 2) * 8 + g * 4 + (v & 3);
    if (qi >= a.n) continue;
    const int64_t ob = ((int64_t)qi * s.heads + h) * HD;
    const int64_t obp = a.ld_o ? (int64_t)qi * a.ld_o + h * HD : ob;
#pragma unroll
    for (int t = 0; t < DT; t++) {
      const int dd = t * 32 + col;
      if (dd < HD) {
        const float r = o[t][v] / lq;
        if (a.out) a.out[ob + dd] = r;
        if (a.oh) store_bf16_split(a.oh, a.ol, obp + dd, r);
      }
    }
  }
}

// The output of query j, head h (block j * heads + h, thread = dim) from
// the records of its tile's key splits, in split order: with M the largest
// m, out = sum o_z e_z / sum l_z e_z, e_z = exp(m_z - M).
template <int HD>
__global__ __launch_bounds__(128) void flash_combine_kernel(FlashArgs a) {
  const StableDims &s = a.s;
  const int qi = blockIdx.x / s.heads, h = blockIdx.x % s.heads, d = threadIdx.x;
  if (d >= HD) return;
  int per;
  const int splits = key_split_tiles(*a.pos0 + qi / kQ32 * kQ32, a.ksplit, per);
  const float *rec = a.partials + ((int64_t)qi * s.heads + h) * a.region;
  float m = rec[0];
  for (int z = 1; z < splits; z++) m = fmaxf(m, rec[z * (HD + 2)]);
  float l = 0.f, acc = 0.f;
  for (int z = 0; z < splits; z++) {
    const float *r = rec + z * (HD + 2);
    const float e = expf(r[0] - m);
    l = fmaf(r[1], e, l);
    acc = fmaf(r[2 + d], e, acc);
  }
  const float v = acc / l;
  const int64_t ob = ((int64_t)qi * s.heads + h) * HD;
  if (a.out) a.out[ob + d] = v;
  if (a.oh) store_bf16_split(a.oh, a.ol, (a.ld_o ? (int64_t)qi * a.ld_o + h * HD : ob) + d, v);
}

template <int HD, bool BR>
hipError_t flash32_launch(const FlashArgs &a, int nseg, hipStream_t st) {
  dim3 grid((a.n + kQ32 - 1) / kQ32, a.s.heads, nseg);
  if (a.kv.half)
    hipLaunchKernelGGL((flash32_kernel<HD, true, BR>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((flash32_kernel<HD, false, BR>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int HD>
hipError_t flash32_dispatch(const FlashArgs &a, bool br, int nseg, hipStream_t st) {
  if (br) return flash32_launch<HD, true>(a, nseg, st);
  if (a.ksplit <= 1) return flash32_launch<HD, false>(a, 1, st);
  hipError_t e = flash32_launch<HD, false>(a, a.ksplit, st);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(flash_combine_kernel<HD>, dim3(a.n * a.s.heads), dim3(128), 0, st, a);
  return hipGetLastError();
}

template <int HD>
hipError_t flash32_shared(const FlashArgs &a, int splits, hipStream_t st) {
  dim3 grid(splits, a.s.heads);
  if (a.kv.half)
    hipLaunchKernelGGL((flash32_kernel<HD, true, false, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((flash32_kernel<HD, false, false, true>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace

bool flash_prefill_supported(int hd) { return hd == 64 || hd == 80 || hd == 96 || hd == 128; }

int shared_prefix_splits(int prefix) { return (prefix + kSharedKeys - 1) / kSharedKeys; }

hipError_t launch_shared_prefix_attention(const StableDims &s, const KVDev &kv, int prefix, const float *q, int nq,
                                          float *partials, int64_t region, hipStream_t st) {
  if (nq < 1 || nq > kQ32 || prefix < 1 || prefix > kv.cap || !flash_prefill_supported(s.hd) ||
      region < (int64_t)shared_prefix_splits(prefix) * (s.hd + 2))
    return hipErrorInvalidValue;
  FlashArgs a{s, kv, q, nullptr, nq, nullptr, nullptr, nullptr, KVDev{}, prefix, 0, partials, region, kSharedKeys, 0, 0,
              nullptr};
  const int splits = shared_prefix_splits(prefix);
  switch (s.hd) {
    case 64: return flash32_shared<64>(a, splits, st);
    case 80: return flash32_shared<80>(a, splits, st);
    case 96: return flash32_shared<96>(a, splits, st);
    case 128: return flash32_shared<128>(a, splits, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_flash_prefill(const StableDims &s, const KVDev &kv, const float *q, const int *pos0, int n,
                                float *out, hipStream_t st, uint16_t *oh, uint16_t *ol, const KVDev *sfx, int prefix,
                                int sfx_slot0, int64_t ld_o, const int *segs, int nseg, float *work,
                                int64_t work_floats, int last_pos) {
  if (!oh != !ol || (!out && !oh) || n < 1 || (ld_o && ld_o < (int64_t)s.heads * s.hd)) return hipErrorInvalidValue;
  if (sfx && (sfx->half != kv.half || prefix < 0 || prefix > kv.cap || sfx_slot0 < 0)) return hipErrorInvalidValue;
  if (segs && (!sfx || oh || nseg < 1 || nseg > 65535)) return hipErrorInvalidValue;
  FlashArgs a{s, kv, q, pos0, n, out, oh, ol, sfx ? *sfx : KVDev{}, prefix, sfx_slot0, nullptr, 0, 0, ld_o, 0, segs};
  // Key splits where the query tiles alone leave CUs idle (a few hundred
  // queries against a long cache): about 512 blocks, the records in `work`.
  const int blocks = (n + kQ32 - 1) / kQ32 * s.heads;
  if (!sfx && work && blocks < 256 && last_pos >= 256) {
    int ks = std::min(8, (512 + blocks - 1) / blocks);
    while (ks > 1 && (int64_t)n * s.heads * ks * (s.hd + 2) > work_floats) ks--;
    if (ks > 1) {
      a.ksplit = ks;
      a.partials = work;
      a.region = (int64_t)ks * (s.hd + 2);
    }
  }
  const bool br = sfx != nullptr;
  const int z = segs ? nseg : 1;
  switch (s.hd) {
    case 64: return flash32_dispatch<64>(a, br, z, st);
    case 80: return flash32_dispatch<80>(a, br, z, st);
    case 96: return flash32_dispatch<96>(a, br, z, st);
    case 128: return flash32_dispatch<128>(a, br, z, st);
  }
  return hipErrorInvalidValue;
}
