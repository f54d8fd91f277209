// Causal attention of a prefill chunk on the matrix cores (attendBatch,
// attention.go:6-45; per head as attendHeads, stablelm.go:391-431): n
// queries at positions pos0 .. pos0 + n - 1 against cache positions
// 0 .. pos0 + n - 1, online softmax in fp32.
//
// One block of 4 waves per (64 queries, head); each wave owns 16 queries.
// Per tile of 64 cache positions the block stages K [key][dim] and V
// transposed [dim][key] in LDS as fp16, and each wave computes
//   S^T = K Q^T  with v_mfma_f32_16x16x32_f16 (keys x queries), so that
//   P = exp(S - m) already sits in the A-operand layout of
//   O += P V     (queries x dims), again 16x16x32 f16.
// fp32 operands are carried as fp16 hi + lo (x = hi + lo to ~22 bits):
// queries and probabilities always, K and V when the cache is fp32. With
// an fp16 cache K and V are exact as stored. Products accumulate in fp32.
#include "kernels.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kTile = 64;   // cache positions per iteration
constexpr int kQ = 64;      // queries per block
// Scores are kept in base 2 (s / scale * log2 e): the softmax weights are
// then single v_exp_f32 (2^x) instructions; exp(v - m) = 2^((v - m) log2 e).
constexpr float kLog2e = 1.4426950408889634f;

struct FlashArgs {
  StableDims s;
  KVDev kv;
  const float *q;  // [n][heads][hd]
  const int *pos0;
  int n;
  float *out;      // [n][heads][hd]
};

__device__ __forceinline__ void split_half(float x, _Float16 &hi, _Float16 &lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

template <int HD, bool HALF>
__global__ __launch_bounds__(256) void flash_prefill_kernel(FlashArgs a) {
  constexpr int KS = (HD + 31) / 32;  // 32-wide k-steps over head dims (zero padded)
  constexpr int KP = KS * 32 + 8;     // LDS pitch of a K row (halves), padded against bank conflicts
  constexpr int VP = kTile + 8;       // LDS pitch of a V^T row (halves)
  constexpr int NPL = HALF ? 1 : 2;   // fp16 planes of K and V
  constexpr int DT = (HD + 15) / 16;  // 16-wide output tiles over head dims
  __shared__ __align__(16) _Float16 ks[NPL][kTile * KP];
  __shared__ __align__(16) _Float16 vt[NPL][DT * 16 * VP];

  const StableDims &s = a.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y, kvh = h / (s.heads / s.kv_heads);
  const int p0 = *a.pos0;
  const int qb = blockIdx.x * kQ;                  // first query of the block
  const int qw = qb + wave * 16;                   // first query of the wave
  const int qcol = lane & 15, grp = lane >> 4;     // S^T column (query) and lane group
  const int myq = qw + qcol;                       // this lane's query (as an S^T column)
  const int myq_pos = p0 + min(myq, a.n - 1);
  const int last_pos = p0 + min(qb + kQ, a.n) - 1;  // causal bound of the block

  // Q^T as B operands: column = query, k = dims 8 * grp .. + 8 of each step.
  f16x8 qh[KS], ql[KS];
  {
    const float *qp = a.q + ((int64_t)min(myq, a.n - 1) * s.heads + h) * HD;
#pragma unroll
    for (int k = 0; k < KS; k++)
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int dd = k * 32 + grp * 8 + i;
        _Float16 hi = 0, lo = 0;
        if (dd < HD) split_half(qp[dd], hi, lo);
        qh[k][i] = hi;
        ql[k][i] = lo;
      }
  }
  f32x4 o[DT], ol[DT];
#pragma unroll
  for (int t = 0; t < DT; t++) o[t] = ol[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // per query column (replicated over lane groups)

  // Padding dims of K (HD .. KS * 32) and V^T rows HD .. DT * 16 stay zero.
  for (int e = tid; e < NPL * kTile * (KS * 32 - HD); e += 256) {
    const int pl = e / (kTile * (KS * 32 - HD)), r = e % (kTile * (KS * 32 - HD));
    ks[pl][(r / (KS * 32 - HD)) * KP + HD + r % (KS * 32 - HD)] = (_Float16)0.f;
  }
  for (int e = tid; e < NPL * (DT * 16 - HD) * VP; e += 256) {
    const int pl = e / ((DT * 16 - HD) * VP), r = e % ((DT * 16 - HD) * VP);
    vt[pl][HD * VP + r] = (_Float16)0.f;
  }
  const int64_t head_base = (int64_t)kvh * a.kv.cap * HD;
  const int ntiles = last_pos / kTile + 1;
  // fp16 cache: a tile is loaded into registers while the previous one is
  // computed (K rows as stored, 16 bytes a load; V in blocks of 8 keys x 8
  // dims that are transposed in registers, so every LDS store is 16 bytes
  // wide). Positions past the block's last query load as zeros.
  constexpr int KC = kTile * (HD / 8), KPT = (KC + 255) / 256;  // K chunks of a tile, per thread
  constexpr int VB = (kTile / 8) * (HD / 8);                      // V blocks of a tile (<= 256)
  static_assert(VB <= 256, "one V block per thread");
  uint4 kreg[KPT];
  uint32_t vreg[8][4];
  const _Float16 *kp = reinterpret_cast<const _Float16 *>(a.kv.k) + head_base;
  const _Float16 *vp = reinterpret_cast<const _Float16 *>(a.kv.v) + head_base;
  auto hload = [&](int t0) {
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int e = tid + 256 * i, key = e / (HD / 8), c = e % (HD / 8), t = t0 + key;
      kreg[i] = e < KC && t <= last_pos ? *reinterpret_cast<const uint4 *>(kp + (int64_t)t * HD + c * 8)
                                        : make_uint4(0, 0, 0, 0);
    }
    if (tid < VB) {
      const int kg = tid / (HD / 8), dg = tid % (HD / 8);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int t = t0 + kg * 8 + i;
        const uint4 v = t <= last_pos ? *reinterpret_cast<const uint4 *>(vp + (int64_t)t * HD + dg * 8)
                                      : make_uint4(0, 0, 0, 0);
        vreg[i][0] = v.x;
        vreg[i][1] = v.y;
        vreg[i][2] = v.z;
        vreg[i][3] = v.w;
      }
    }
  };
  auto hstore = [&]() {
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const int e = tid + 256 * i, key = e / (HD / 8), c = e % (HD / 8);
      if (e < KC) *reinterpret_cast<uint4 *>(&ks[0][key * KP + c * 8]) = kreg[i];
    }
    if (tid < VB) {
      const int kg = tid / (HD / 8), dg = tid % (HD / 8);
#pragma unroll
      for (int j = 0; j < 8; j++) {  // dim dg * 8 + j: keys kg * 8 .. + 8
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const uint32_t lo = (vreg[2 * q][j >> 1] >> (16 * (j & 1))) & 0xffffu;
          const uint32_t hi = (vreg[2 * q + 1][j >> 1] >> (16 * (j & 1))) & 0xffffu;
          w[q] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4 *>(&vt[0][(dg * 8 + j) * VP + kg * 8]) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  };
  if constexpr (HALF) hload(0);
  for (int tile = 0; tile < ntiles; tile++) {
    const int t0 = tile * kTile;
    // ---- stage K [key][dim] and V^T [dim][key] as fp16 (hi, lo planes for
    // fp32). Positions past the block's last query stage as zeros.
    __syncthreads();
    if constexpr (HALF) {
      hstore();
      if (tile + 1 < ntiles) hload(t0 + kTile);
    } else {
    constexpr int VPL = 4;        // values per 16-byte load
    constexpr int LPR = HD / VPL;  // loads per key row
    for (int e = tid; e < kTile * LPR; e += 256) {
      const int key = e / LPR, d0 = (e % LPR) * VPL;
      const int t = t0 + key;
      const int64_t idx = head_base + (int64_t)t * HD + d0;
      float kx[VPL], vx[VPL];
      if (t <= last_pos) {
        const float4 kw = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.kv.k) + idx);
        const float4 vw = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.kv.v) + idx);
        kx[0] = kw.x; kx[1] = kw.y; kx[2] = kw.z; kx[3] = kw.w;
        vx[0] = vw.x; vx[1] = vw.y; vx[2] = vw.z; vx[3] = vw.w;
      } else {
#pragma unroll
        for (int j = 0; j < VPL; j++) kx[j] = vx[j] = 0.f;
      }
#pragma unroll
      for (int j = 0; j < VPL; j++) {
        _Float16 kh, kl, vh, vl;
        split_half(kx[j], kh, kl);
        split_half(vx[j], vh, vl);
        ks[0][key * KP + d0 + j] = kh;
        vt[0][(d0 + j) * VP + key] = vh;
        ks[NPL - 1][key * KP + d0 + j] = kl;
        vt[NPL - 1][(d0 + j) * VP + key] = vl;
      }
    }
    }
    __syncthreads();
    if (qw >= a.n || t0 > p0 + qw + 15) continue;  // nothing for this wave in this tile (uniform per wave)

    // ---- S^T: 4 sub-tiles of 16 keys x 16 queries
    // Two accumulators per sub-tile (query hi and lo parts) and the k-steps
    // outermost: eight independent MFMA chains instead of four long ones.
    f32x4 st[4], sl[4];
#pragma unroll
    for (int sub = 0; sub < 4; sub++) st[sub] = sl[sub] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KS; k++)
#pragma unroll
      for (int sub = 0; sub < 4; sub++) {
        const int krow = sub * 16 + qcol;  // A operand row: key
        const f16x8 kah = *reinterpret_cast<const f16x8 *>(&ks[0][krow * KP + k * 32 + grp * 8]);
        st[sub] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kah, qh[k], st[sub], 0, 0, 0);
        sl[sub] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kah, ql[k], sl[sub], 0, 0, 0);
        if constexpr (!HALF) {
          const f16x8 kal = *reinterpret_cast<const f16x8 *>(&ks[NPL - 1][krow * KP + k * 32 + grp * 8]);
          sl[sub] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kal, qh[k], sl[sub], 0, 0, 0);
        }
      }
#pragma unroll
    for (int sub = 0; sub < 4; sub++) st[sub] += sl[sub];
    // Scale (to base 2), causal mask (key position > query position),
    // running max.
    // Lane holds keys sub * 16 + 4 * grp + i for query qcol.
    float tmax = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < 4; sub++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = t0 + sub * 16 + grp * 4 + i;
        const float v = t <= myq_pos ? __fmul_rn(__fdiv_rn(st[sub][i], s.att_scale), kLog2e) : -INFINITY;
        st[sub][i] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float corr = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.f;
    // P as A operands of P V: row = query, k slots = keys {4 grp + i, 16 + 4 grp + i}
    // of each 32-key half; V^T is read with the same key order.
    f16x8 ph[2], pl[2];
#pragma unroll
    for (int sub = 0; sub < 4; sub++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float p = st[sub][i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st[sub][i] - m_new);
        psum += p;
        _Float16 hi, lo;
        split_half(p, hi, lo);
        ph[sub >> 1][(sub & 1) * 4 + i] = hi;
        pl[sub >> 1][(sub & 1) * 4 + i] = lo;
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = fmaf(l_run, corr, psum);
    m_run = m_new;
    // Rescale O rows (queries 4 grp + i of the wave) by their query's factor.
    float rc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) rc[i] = __shfl(corr, grp * 4 + i, 64);
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        o[t][i] *= rc[i];
        ol[t][i] *= rc[i];
      }
    // ---- O += P V: per 32-key half and 16-dim tile; the lo parts go to a
    // second accumulator (independent MFMA chains), added at the end.
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
      for (int t = 0; t < DT; t++) {
        const int vrow = t * 16 + qcol;  // B operand column: dim
        const _Float16 *v0 = &vt[0][vrow * VP + half * 32 + grp * 4];
        f16x8 vb;
        const uint2 lo4 = *reinterpret_cast<const uint2 *>(v0);
        const uint2 hi4 = *reinterpret_cast<const uint2 *>(v0 + 16);
        vb = __builtin_bit_cast(f16x8, make_uint4(lo4.x, lo4.y, hi4.x, hi4.y));
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[half], vb, o[t], 0, 0, 0);
        ol[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[half], vb, ol[t], 0, 0, 0);
        if constexpr (!HALF) {
          const _Float16 *v1 = &vt[NPL - 1][vrow * VP + half * 32 + grp * 4];
          const uint2 a4 = *reinterpret_cast<const uint2 *>(v1);
          const uint2 b4 = *reinterpret_cast<const uint2 *>(v1 + 16);
          const f16x8 vl = __builtin_bit_cast(f16x8, make_uint4(a4.x, a4.y, b4.x, b4.y));
          ol[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[half], vl, ol[t], 0, 0, 0);
        }
      }
  }
#pragma unroll
  for (int t = 0; t < DT; t++) o[t] += ol[t];
  // ---- normalise and store: D lane holds queries 4 grp + i, dim t * 16 + qcol
  float linv[4];
#pragma unroll
  for (int i = 0; i < 4; i++) linv[i] = __shfl(l_run, grp * 4 + i, 64);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int qi = qw + grp * 4 + i;
    if (qi >= a.n) continue;
    float *op = a.out + ((int64_t)qi * s.heads + h) * HD;
#pragma unroll
    for (int t = 0; t < DT; t++) {
      const int dd = t * 16 + qcol;
      if (dd < HD) op[dd] = o[t][i] / linv[i];
    }
  }
}

template <int HD>
hipError_t flash_launch(const FlashArgs &a, hipStream_t st) {
  dim3 grid((a.n + kQ - 1) / kQ, a.s.heads);
  if (a.kv.half)
    hipLaunchKernelGGL((flash_prefill_kernel<HD, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((flash_prefill_kernel<HD, false>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace

bool flash_prefill_supported(int hd) { return hd == 64 || hd == 80 || hd == 96 || hd == 128; }

hipError_t launch_flash_prefill(const StableDims &s, const KVDev &kv, const float *q, const int *pos0, int n,
                                float *out, hipStream_t st) {
  FlashArgs a{s, kv, q, pos0, n, out};
  switch (s.hd) {
    case 64: return flash_launch<64>(a, st);
    case 80: return flash_launch<80>(a, st);
    case 96: return flash_launch<96>(a, st);
    case 128: return flash_launch<128>(a, st);
  }
  return hipErrorInvalidValue;
}
