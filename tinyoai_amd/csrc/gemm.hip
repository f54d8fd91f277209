// Prefill projections on the gfx950 matrix cores: Y[M][N] = X[M][K] * W^T
// with v_mfma_f32_32x32x16_bf16 (fp32 accumulation).
//
// Operands: X arrives as bf16 planes (split_bf16 below, or written so by the
// producing kernel): with XS = 2 the pair hi + lo carries 16 significant
// bits of every activation, with XS = 1 only hi (the products with BF16
// weights, see gemm_planes). BF16 weights feed the cores as stored. Q8_0 quants (|q| <= 128) are exact in bf16; each quant
// block's product is formed without scale and added as acc += d * block on
// the fp32 accumulators, which keeps the weights exact.
//
// The in-projection can finish in the kernel itself: with EPI the output
// pairs of win go through the fused epilogue (RoPE, KV append, SiLU-gate)
// instead of being stored.
#include <algorithm>

#include "gemm_wide.h"

using namespace tinyoai_gemm;

typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kKAlign = 32;  // K of the matrix-core products: a multiple of 32 (one Q8_0 block)


// x (fp32, rows of `k` values with stride ldx) -> bf16 hi (and lo = x - hi).
__global__ void split_bf16_kernel(const float *x, int ldx, int k, int64_t rows, uint16_t *hi, uint16_t *lo) {
  const int64_t total = rows * k;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / k, c = i % k;
    const float v = x[r * ldx + c];
    const __bf16 h = (__bf16)v;
    hi[i] = __builtin_bit_cast(uint16_t, h);
    if (lo) lo[i] = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)h));
  }
}

struct GemmArgs {
  MatDesc w;                  // N = rows, K = cols (a column view of a larger matrix is fine)
  const uint16_t *xh, *xl;    // bf16 planes [M][K]
  int M;
  float *y;
  int ldy;
  int ksplit;                 // K ranges summed separately: split s writes y + s * M * ldy
  InEpilogue e;               // the fused in-projection epilogue (EPI instances)
};

// The K steps of split s of `splits` (nk steps in all): [k_lo, k_hi).
__device__ __forceinline__ void split_range(int nk, int splits, int s, int &k_lo, int &k_hi) {
  k_lo = (int)((int64_t)nk * s / splits);
  k_hi = (int)((int64_t)nk * (s + 1) / splits);
}

// ------------------------------------------------------------ large tiles
// 128 (M) x 256 (N) per 512-thread block, eight waves of 64 x 64 (2 x 2
// tiles of 32 x 32, v_mfma_f32_32x32x16_bf16), K step 64 (four MFMA
// k-steps), double-buffered LDS with rows of 64 bf16 padded to 144 bytes
// (16 consecutive rows of a 16-byte fragment read cover all 64 banks once).
// Two waves per SIMD: one's LDS reads and barrier waits overlap the
// other's MFMAs. The 32 x 32 products run at about twice the rate of the
// 16 x 16 ones on gfx950 (measured 2.1-2.4 against 0.8-1.4 PFLOP/s).
// Q8_0: a K step holds two quant blocks; each block's products are formed
// without scale (exact) and added as acc += d * block.
constexpr int kLM = 128, kLN = 256, kLK = 64, kLRow = 72;  // LDS row: 72 bf16 = 144 B
constexpr int kLThreads = 512;


template <int WF, int XS, bool EPI = false>
constexpr size_t gemm_large_lds() {
  // staging (two K steps); with EPI also the block's fp32 output tile
  const size_t stage = (size_t)2 * (XS * kLM * kLRow + kLN * kLRow + (WF == FMT_Q8_0 ? 2 * kLN * 2 : 0)) * 2;
  const size_t tile = (size_t)kLM * (kLN + 4) * 4;
  return EPI && tile > stage ? tile : stage;
}

template <int WF, int XS, bool EPI>
__global__ __launch_bounds__(kLThreads) void gemm_large_kernel(GemmArgs g) {
  extern __shared__ __align__(16) uint16_t lds16[];
  // per stage: A planes [XS][kLM][kLRow], B [kLN][kLRow], scales [2][kLN] floats (Q8_0)
  constexpr int kA = kLM * kLRow, kB = kLN * kLRow;
  constexpr int kStage = XS * kA + kB + (WF == FMT_Q8_0 ? 2 * kLN * 2 : 0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;  // 2 x 4 waves of 64 x 64
  const int K = g.w.cols, N = g.w.rows, nk = (K + kLK - 1) / kLK;
  const int MT = (g.M + kLM - 1) / kLM, NT = (N + kLN - 1) / kLN;
  // Workgroups go round-robin to the 8 XCDs (one L2 each): consecutive
  // workgroups of an XCD take the M tiles of one N tile, so its weight
  // tile comes from HBM once.
  const int per_split = (NT + 7) / 8 * 8 * MT, b = blockIdx.x % per_split, split = blockIdx.x / per_split;
  const int xcd = b & 7, slot = b >> 3;
  const int nt = xcd + 8 * (slot / MT), mt = slot % MT;
  if (nt >= NT) return;
  const int m0 = mt * kLM, n0 = nt * kLN;
  int k_lo, k_hi;
  split_range(nk, g.ksplit, split, k_lo, k_hi);
  float *y = g.y + (int64_t)split * g.M * g.ldy;

  // Staging: A chunk q = tid + 512 i (i < 2) of a plane is row q / 8,
  // 8-value column group q % 8; B (BF16) chunk q = tid + 512 i (i < 4)
  // likewise; B (Q8_0, 16 int8 a chunk) chunk q = tid + 512 i (i < 2): row
  // q / 4, 16-value group q % 4, and the scale pair of row tid / 2. Buffer
  // loads: an offset past the operand (rows past M or N, columns past K)
  // reads zeros, with no branch.
  constexpr int NB = WF == FMT_BF16 ? 4 : 2;
  struct Stage {
    uint4 a[XS][2], b[NB];
    uint32_t s;
  };
  constexpr uint32_t kNone = 0x80000000u;  // past every operand (each < 2 GiB)
  const __amdgpu_buffer_rsrc_t rxh = plane_rsrc(reinterpret_cast<const uint8_t *>(g.xh), (int64_t)g.M * K * 2);
  const __amdgpu_buffer_rsrc_t rxl =
      plane_rsrc(reinterpret_cast<const uint8_t *>(XS == 2 ? g.xl : g.xh), (int64_t)g.M * K * 2);
  const __amdgpu_buffer_rsrc_t rw = plane_rsrc(g.w.vals, (int64_t)N * g.w.vstride);
  auto ld16 = [](__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
  };
  auto gload = [&](int kb, Stage &r) {
    const int k0 = kb * kLK;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int q = tid + kLThreads * i, row = q >> 3, kc = k0 + (q & 7) * 8;
      const uint32_t off = m0 + row < g.M && kc < K ? (uint32_t)(((m0 + row) * K + kc) * 2) : kNone;
      r.a[0][i] = ld16(rxh, off);
      if constexpr (XS == 2) r.a[1][i] = ld16(rxl, off);
    }
    if constexpr (WF == FMT_BF16) {
#pragma unroll
      for (int i = 0; i < NB; i++) {
        const int q = tid + kLThreads * i, row = q >> 3, kc = k0 + (q & 7) * 8;
        r.b[i] = ld16(rw, n0 + row < N && kc < K ? (uint32_t)((n0 + row) * g.w.vstride + kc * 2) : kNone);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NB; i++) {
        const int q = tid + kLThreads * i, row = q >> 2, kc = k0 + (q & 3) * 16;
        r.b[i] = ld16(rw, n0 + row < N && kc < K ? (uint32_t)((n0 + row) * g.w.vstride + kc) : kNone);
      }
      const int n = n0 + (tid >> 1), kq = k0 + (tid & 1) * 32;
      r.s = n < N && kq < K ? reinterpret_cast<const uint16_t *>(g.w.meta + (int64_t)n * g.w.mstride)[kq / 32] : 0;
    }
  };
  auto lstore = [&](int buf, const Stage &r) {
    uint16_t *st = lds16 + buf * kStage;
#pragma unroll
    for (int p = 0; p < XS; p++)
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int q = tid + kLThreads * i, row = q >> 3, c = (q & 7) * 8;
        *reinterpret_cast<uint4 *>(st + p * kA + row * kLRow + c) = r.a[p][i];
      }
    uint16_t *sb = st + XS * kA;
    if constexpr (WF == FMT_BF16) {
#pragma unroll
      for (int i = 0; i < NB; i++) {
        const int q = tid + kLThreads * i, row = q >> 3, c = (q & 7) * 8;
        *reinterpret_cast<uint4 *>(sb + row * kLRow + c) = r.b[i];
      }
    } else {  // 16 int8 -> 16 bf16, exact
#pragma unroll
      for (int i = 0; i < NB; i++) {
        const int q = tid + kLThreads * i, row = q >> 2, c = (q & 3) * 16;
        const uint32_t ws[4] = {r.b[i].x, r.b[i].y, r.b[i].z, r.b[i].w};
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint32_t v = ws[j];
          o[2 * j] = bf16_bits((float)(int8_t)v) | bf16_bits((float)(int8_t)(v >> 8)) << 16;
          o[2 * j + 1] = bf16_bits((float)(int8_t)(v >> 16)) | bf16_bits((float)(int8_t)(v >> 24)) << 16;
        }
        uint4 *d = reinterpret_cast<uint4 *>(sb + row * kLRow + c);
        d[0] = make_uint4(o[0], o[1], o[2], o[3]);
        d[1] = make_uint4(o[4], o[5], o[6], o[7]);
      }
      float *ss = reinterpret_cast<float *>(sb + kB);  // [block of the step][row]
      ss[(tid & 1) * kLN + (tid >> 1)] = hw_half((uint16_t)r.s);
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;
  const int frow = lane & 31, fk = (lane >> 5) * 8;
  // The products of the K step in LDS buffer buf.
  auto compute = [&](int buf) {
    const uint16_t *st = lds16 + buf * kStage;
    const uint16_t *sb = st + XS * kA;
    f32x16 t[2][2];  // Q8_0: the current quant block's products
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      bf16x8 afr[XS][2], bfr[2];
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
        bfr[ni] = *reinterpret_cast<const bf16x8 *>(sb + (wn * 64 + ni * 32 + frow) * kLRow + ks * 16 + fk);
#pragma unroll
      for (int p = 0; p < XS; p++)
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
          afr[p][mi] = *reinterpret_cast<const bf16x8 *>(st + p * kA + (wm * 64 + mi * 32 + frow) * kLRow + ks * 16 + fk);
      // One plane's 4 products before the other's: consecutive MFMAs write
      // different accumulators.
      if constexpr (WF == FMT_Q8_0) {
        if (ks % 2 == 0) {
#pragma unroll
          for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int ni = 0; ni < 2; ni++)
#pragma unroll
              for (int v = 0; v < 16; v++) t[mi][ni][v] = 0.f;
        }
#pragma unroll
        for (int p = 0; p < XS; p++)
#pragma unroll
          for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int ni = 0; ni < 2; ni++)
              t[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr[p][mi], bfr[ni], t[mi][ni], 0, 0, 0);
        if (ks % 2 == 1) {
          const float *ss = reinterpret_cast<const float *>(sb + kB) + (ks / 2) * kLN;
#pragma unroll
          for (int ni = 0; ni < 2; ni++) {
            const float sc = ss[wn * 64 + ni * 32 + frow];
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
              for (int v = 0; v < 16; v++) acc[mi][ni][v] = fmaf(sc, t[mi][ni][v], acc[mi][ni][v]);
          }
        }
      } else {
#pragma unroll
        for (int p = 0; p < XS; p++)
#pragma unroll
          for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int ni = 0; ni < 2; ni++)
              acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr[p][mi], bfr[ni], acc[mi][ni], 0, 0, 0);
      }
    }
  };
  if constexpr (WF == FMT_BF16) {
    // Loads run two K steps ahead of the products through two register
    // stages: step kb issues the loads of kb + 2, computes kb, then stores
    // kb + 1 (loaded during step kb - 1) to the other LDS buffer.
    Stage r0, r1;
    if (k_lo < k_hi) {
      gload(k_lo, r0);
      lstore(0, r0);
    }
    if (k_lo + 1 < k_hi) gload(k_lo + 1, r1);
    __syncthreads();
    for (int kb = k_lo; kb < k_hi; kb += 2) {
      if (kb + 2 < k_hi) gload(kb + 2, r0);
      compute(0);
      if (kb + 1 < k_hi) lstore(1, r1);
      __syncthreads();
      if (kb + 1 >= k_hi) break;
      if (kb + 3 < k_hi) gload(kb + 3, r1);
      compute(1);
      if (kb + 2 < k_hi) lstore(0, r0);
      __syncthreads();
    }
  } else {
    // Q8_0 holds each quant block's products besides the accumulators:
    // one register stage (loads one K step ahead) keeps it within 256
    // registers.
    Stage r;
    if (k_lo < k_hi) {
      gload(k_lo, r);
      lstore(0, r);
    }
    __syncthreads();
    for (int kb = k_lo; kb < k_hi; kb++) {
      const int cur = (kb - k_lo) & 1;
      if (kb + 1 < k_hi) gload(kb + 1, r);
      compute(cur);
      if (kb + 1 < k_hi) lstore(cur ^ 1, r);
      __syncthreads();
    }
  }
  // D fragment: lane holds column lane % 32 of rows (v / 4) * 8 + (lane / 32) * 4 + v % 4.
  if constexpr (EPI) {
    // The block's output tile goes to LDS (free once every wave's last
    // products are formed), then threads take (token, row pair of win)
    // items in order through the in-projection epilogue, as
    // in_epilogue_kernel does per token: neighbouring threads store
    // neighbouring outputs.
    constexpr int kPitch = kLN + 4;  // floats: the lane groups' rows fall on different banks
    static_assert(kLM * kPitch * 4 <= gemm_large_lds<WF, XS, EPI>(), "output tile fits the block's LDS");
    float *tile = reinterpret_cast<float *>(lds16);
    __syncthreads();
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int v = 0; v < 16; v++)
          tile[(wm * 64 + mi * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3)) * kPitch + wn * 64 + ni * 32 + frow] =
              acc[mi][ni][v];
    __syncthreads();
    // Values, not references into the kernel arguments (a reference makes
    // the compiler copy the argument block to per-lane scratch).
    const StableDims es = g.e.s;
    const KVDev ekv = g.e.kv;
    const float *rope = g.e.rope;
    float *eq = g.e.q, *em = g.e.m;
    uint16_t *emh = g.e.mh, *eml = g.e.ml;
    const int p0 = *g.e.pos0, mu0 = (es.win_q + 2 * es.win_kv) / 2;
    for (int it = tid; it < kLM * (kLN / 2); it += kLThreads) {
      const int r = it / (kLN / 2), c = 2 * (it % (kLN / 2)), m = m0 + r, n = n0 + c, u = n >> 1;
      if (m >= g.M || n >= N) continue;
      const float2 pv = *reinterpret_cast<const float2 *>(tile + r * kPitch + c);
      if (u >= mu0) {
        const float gv = es.silu ? silu_gate_llama(pv.x, pv.y) : silu_gate(pv.x, pv.y);
        const int64_t i = (int64_t)m * es.inter + (u - mu0);
        if (em) em[i] = gv;
        store_bf16_split(emh, eml, i, gv);
      } else {
        const int pos = p0 + m;
        in_pair_epilogue(es, ekv, rope + (int64_t)pos * es.rot, pos, u, pv.x, pv.y,
                         eq + (int64_t)m * es.heads * es.hd, nullptr);
      }
    }
    return;
  }
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
      const int n = n0 + wn * 64 + ni * 32 + frow;
      if (n >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = m0 + wm * 64 + mi * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (m < g.M) y[(int64_t)m * g.ldy + n] = acc[mi][ni][v];
      }
    }
}

// ------------------------------------------------------------ loads direct to LDS
// Both operands are loaded straight into LDS (buffer_load_dwordx4 ...
// lds): no staging registers, so each wave holds a step's fragments for
// both k halves and the compiler keeps the LDS reads ahead of the
// products. (Staging through registers with coalesced loads kept the
// matrix cores 41% busy at best, most wave time waiting on loads.) A
// ring of three LDS stages: step kb waits for its own loads of stage kb
// (the count of loads in flight is exact: every wave issues the same
// loads every step, past the operands reading zeros), meets the block
// barrier (every wave's loads of kb landed, and every wave is done with
// stage kb - 1), issues the loads of kb + 2 into kb - 1's slot and forms
// the products of kb. Each wave load writes 1 KB of LDS (16 rows of a
// step, 64 lane x 16 bytes in lane order); the chunk swizzle of the
// fragment reads is applied on the global side: lane l fetches logical
// chunk (l % 4) ^ ((row >> 2) & 3) of row l / 4.
//
// The loads are inline assembly: the compiler's own handling of LDS DMA
// waits for every load in flight before any LDS read, which would leave
// one step to hide the memory latency. The kernel waits for its loads
// itself (s_waitcnt vmcnt) and issues no other vector memory load in the
// loop.

template <int XS, int MF, int NF>
constexpr int dma_slot_bytes() {
  return XS * 128 * MF * 64 + 256 * 64;  // activation planes, then 256 weight rows (the tile's, then padding)
}
template <int XS, int MF, int NF, bool EPI>
constexpr size_t gemm_dma_lds() {
  const size_t ring = (size_t)3 * dma_slot_bytes<XS, MF, NF>();
  const size_t rows = (size_t)4 * 32 * (NF * 32 + 4) * 4;
  return EPI && rows > ring ? rows : ring;
}

template <int XS, int MF, int NF, bool EPI>
__global__ __launch_bounds__(kWThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_dma_kernel(WideArgs g) {
  constexpr int BM = 4 * 32 * MF, BN = 32 * NF;
  static_assert(BN <= 256, "weight rows of a slot");
  constexpr int kSlot = dma_slot_bytes<XS, MF, NF>(), kAPlane = BM * 64, kB0 = XS * kAPlane;
  constexpr int NA = BM / 64;   // wave loads per activation plane and step
  constexpr int NBW = 4;        // wave loads of the weight rows per step (256 rows)
  constexpr int kPerStep = XS * NA + NBW;
  extern __shared__ __align__(16) uint16_t lds16[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  int b = blockIdx.x, pi = 0;
  {
    const WideProduct &p0 = g.p[0];
    const int tiles0 = ((g.M + BM - 1) / BM) * ((p0.w.rows + BN - 1) / BN);
    const int nb0 = (tiles0 * p0.ksplit + 7) / 8 * 8;
    if (g.nprod > 1 && b >= nb0) {
      b -= nb0;
      pi = 1;
    }
  }
  const WideProduct &P = g.p[pi];
  const int K = P.w.cols, N = P.w.rows, nk = K / kWK;
  const int MT = (g.M + BM - 1) / BM, NT = (N + BN - 1) / BN, tiles = MT * NT;
  const int total = tiles * P.ksplit, per = (total + 7) / 8;
  const int t = (b & 7) * per + (b >> 3);
  if (t >= total) return;
  const int split = t / tiles, tt = t - split * tiles, nt = tt / MT, mt = tt - nt * MT;
  const int m0 = mt * BM, n0 = nt * BN;
  const int k_lo = (int)((int64_t)nk * split / P.ksplit), k_hi = (int)((int64_t)nk * (split + 1) / P.ksplit);

  constexpr uint32_t kNone = 0x80000000u, kPast = 0x40000000u;
  const __amdgpu_buffer_rsrc_t rxh = plane_rsrc(reinterpret_cast<const uint8_t *>(P.xh), (int64_t)g.M * P.lda * 2);
  const __amdgpu_buffer_rsrc_t rxl =
      plane_rsrc(reinterpret_cast<const uint8_t *>(XS == 2 ? P.xl : P.xh), (int64_t)g.M * P.lda * 2);
  const __amdgpu_buffer_rsrc_t rw = plane_rsrc(P.w.vals, (int64_t)N * P.w.vstride);

  // Lane offsets of this wave's loads at k = 0 (the LDS side is the wave's
  // 1 KB piece: row (16 j + lane / 4), position lane % 4).
  const int lrow = lane >> 2, lc = (lane & 3) ^ ((lrow >> 2) & 3);
  uint32_t aoff[NA], boff[NBW];
#pragma unroll
  for (int i = 0; i < NA; i++) {
    const int row = (wave + 4 * i) * 16 + lrow;
    aoff[i] = m0 + row < g.M ? (uint32_t)(((m0 + row) * P.lda + lc * 8) * 2) : kNone;
  }
#pragma unroll
  for (int i = 0; i < NBW; i++) {
    const int row = (wave + 4 * i) * 16 + lrow;
    boff[i] = row < BN && n0 + row < N ? (uint32_t)((n0 + row) * P.w.vstride + lc * 16) : kNone;
  }
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)lds16;
  const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](int kb, int slot) {
    const uint32_t k2 = kb < k_hi ? (uint32_t)(kb * kWK * 2) : kPast;
    const uint32_t sb = lds_base + slot * kSlot + wave_u * 1024;
#pragma unroll
    for (int p = 0; p < XS; p++)
#pragma unroll
      for (int i = 0; i < NA; i++) lds_dma16(p ? rxl : rxh, aoff[i] + k2, sb + p * kAPlane + i * 4096);
#pragma unroll
    for (int i = 0; i < NBW; i++) lds_dma16(rw, boff[i] + k2, sb + kB0 + i * 4096);
  };

  f32x16 acc[MF][NF];
#pragma unroll
  for (int f = 0; f < MF; f++)
#pragma unroll
    for (int j = 0; j < NF; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[f][j][v] = 0.f;
  const int arow = wave * 32 * MF + (lane & 31), brow = lane & 31;
  auto frag = [&](const uint16_t *base, int row, int s) {
    return *reinterpret_cast<const bf16x8 *>(base + swz(row, 2 * (lane >> 5) + s));
  };
  auto compute = [&](int slot) {
    const uint16_t *st = lds16 + slot * (kSlot / 2);
    bf16x8 af[2][MF][XS], bf[2][NF];
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
      for (int j = 0; j < NF; j++) bf[s][j] = frag(st + kB0 / 2, j * 32 + brow, s);
#pragma unroll
      for (int f = 0; f < MF; f++)
#pragma unroll
        for (int p = 0; p < XS; p++) af[s][f][p] = frag(st + p * (kAPlane / 2), arow + f * 32, s);
    }
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int f = 0; f < MF; f++)
#pragma unroll
        for (int p = 0; p < XS; p++)
#pragma unroll
          for (int j = 0; j < NF; j++)
            acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][f][p], bf[s][j], acc[f][j], 0, 0, 0);
  };
  auto step = [&](int kb, int slot) {
    wait_vmcnt<kPerStep>();  // this wave's loads of kb (those of kb + 1 may be in flight)
    __syncthreads();
    issue(kb + 2, (slot + 2) % 3);
    compute(slot);
  };
  issue(k_lo, 0);
  issue(k_lo + 1, 1);
  int kb = k_lo;
  for (; kb + 3 <= k_hi; kb += 3) {
    step(kb, 0);
    step(kb + 1, 1);
    step(kb + 2, 2);
  }
  if (kb < k_hi) step(kb, 0);
  if (kb + 1 < k_hi) step(kb + 1, 1);
  wait_vmcnt<0>();  // no load may land in LDS after this point
  __syncthreads();

  wide_finish<MF, NF, EPI>(g, P, acc, reinterpret_cast<float *>(lds16), split, m0, n0, N, wave, lane);
}

template <int XS, int MF, int NF, bool EPI>
hipError_t gemm_wide_launch(const WideArgs &g, hipStream_t st) {
  constexpr int BM = 4 * 32 * MF, BN = 32 * NF;
  int blocks = 0;
  for (int i = 0; i < g.nprod; i++) {
    const int tiles = ((g.M + BM - 1) / BM) * ((g.p[i].w.rows + BN - 1) / BN);
    blocks += (tiles * g.p[i].ksplit + 7) / 8 * 8;
  }
  constexpr size_t lds = gemm_dma_lds<XS, MF, NF, EPI>();
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_dma_kernel<XS, MF, NF, EPI>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((gemm_dma_kernel<XS, MF, NF, EPI>), dim3(blocks), dim3(kWThreads), lds, st, g);
  return hipGetLastError();
}

template <int WF, int XS, bool EPI = false>
hipError_t gemm_large_launch(const GemmArgs &g, hipStream_t st) {
  constexpr size_t lds = gemm_large_lds<WF, XS, EPI>();
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void *>(&gemm_large_kernel<WF, XS, EPI>), hipFuncAttributeMaxDynamicSharedMemorySize,
      (int)lds);
  if (attr != hipSuccess) return attr;
  const int NT = (g.w.rows + kLN - 1) / kLN, MT = (g.M + kLM - 1) / kLM;
  dim3 grid((NT + 7) / 8 * 8 * MT * g.ksplit);
  hipLaunchKernelGGL((gemm_large_kernel<WF, XS, EPI>), grid, dim3(kLThreads), lds, st, g);
  return hipGetLastError();
}

}  // namespace

bool gemm_mfma_supported(const MatDesc &w) {
  return (w.fmt == FMT_Q8_0 || w.fmt == FMT_BF16) && w.cols % kKAlign == 0 && w.vstride % 16 == 0;
}

// Activation planes a product takes: two (16 significant bits, the fp32
// paths' accuracy), or one (bf16 activations) for BF16 weights where the
// caller asks for the bf16 path (within its 2e-2 of the logit range,
// measured 1.4e-3 over two layers at 8K positions).
int gemm_planes(const MatDesc &w, bool bf16_path) { return bf16_path && w.fmt == FMT_BF16 ? 1 : 2; }

hipError_t launch_split_bf16(const float *x, int ldx, int k, int64_t rows, uint16_t *hi, uint16_t *lo,
                             hipStream_t st) {
  const int64_t total = rows * k;
  const int grid = (int)std::min<int64_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL(split_bf16_kernel, dim3(grid), dim3(256), 0, st, x, ldx, k, rows, hi, lo);
  return hipGetLastError();
}

int gemm_splits(const MatDesc &w, int M, int max_splits) {
  const int NT = (w.rows + kLN - 1) / kLN, MT = (M + kLM - 1) / kLM, nk = (w.cols + kLK - 1) / kLK;
  // about two blocks per CU, at least 4 K steps per split
  int s = std::max(1, 512 / std::max(1, NT * MT));
  s = std::min({s, max_splits, std::max(1, nk / 4)});
  return s;
}

hipError_t launch_gemm_mfma(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int M, float *y, int ldy,
                            hipStream_t st, int ksplit) {
  if (!gemm_mfma_supported(w) || ksplit < 1) return hipErrorInvalidValue;
  GemmArgs g{w, xh, xl, M, y, ldy, ksplit, {}};
  if (w.fmt == FMT_Q8_0) return xl ? gemm_large_launch<FMT_Q8_0, 2>(g, st) : gemm_large_launch<FMT_Q8_0, 1>(g, st);
  return xl ? gemm_large_launch<FMT_BF16, 2>(g, st) : gemm_large_launch<FMT_BF16, 1>(g, st);
}

hipError_t launch_gemm_in_epilogue(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int M,
                                   const InEpilogue &e, hipStream_t st) {
  if (!gemm_mfma_supported(w) || (!xl && w.fmt != FMT_BF16) || !e.mh || !e.ml || !e.q || !e.rope || !e.pos0 ||
      w.rows % 2 || e.s.win_q % 2)
    return hipErrorInvalidValue;
  GemmArgs g{w, xh, xl, M, nullptr, 0, 1, e};
  if (w.fmt == FMT_Q8_0) return gemm_large_launch<FMT_Q8_0, 2, true>(g, st);
  return xl ? gemm_large_launch<FMT_BF16, 2, true>(g, st) : gemm_large_launch<FMT_BF16, 1, true>(g, st);
}

namespace {

template <int XS, bool EPI>
hipError_t gemm_wide_dispatch(const WideArgs &g, int mf, int nf, hipStream_t st) {
  if (mf == 2 && nf == 7) return gemm_wide_launch<XS, 2, 7, EPI>(g, st);
  if (mf == 2 && nf == 8) return gemm_wide_launch<XS, 2, 8, EPI>(g, st);
  if (mf == 1 && nf == 8) return gemm_wide_launch<XS, 1, 8, EPI>(g, st);
  if (mf == 1 && nf == 7) return gemm_wide_launch<XS, 1, 7, EPI>(g, st);
  return hipErrorInvalidValue;
}

template <bool EPI>
hipError_t gemm_wide_fmt(const WideArgs &g, int mf, int nf, bool two, hipStream_t st) {
  if (g.p[0].w.fmt == FMT_Q8_0) {  // two planes
    if (!two) return hipErrorInvalidValue;
    return launch_gemm_wideq(g, mf, nf, EPI, st);
  }
  return two ? gemm_wide_dispatch<2, EPI>(g, mf, nf, st) : gemm_wide_dispatch<1, EPI>(g, mf, nf, st);
}

bool wide_operand_ok(const MatDesc &w, const uint16_t *xh, int lda, int M) {
  constexpr int64_t kGiB = int64_t(1) << 30;  // the kernel's offset sentinels need operands below 1 GiB
  return gemm_mfma_supported(w) && xh && lda >= w.cols && lda % 8 == 0 && (reinterpret_cast<uintptr_t>(xh) & 15) == 0 &&
         (w.fmt != FMT_Q8_0 || wide_q8_ok(w)) &&
         (int64_t)M * lda * 2 < kGiB && (int64_t)w.rows * w.vstride < kGiB && (int64_t)w.rows * w.mstride < kGiB;
}

}  // namespace

bool gemm_wide_shape(int fmt, int mf, int nf) {
  if (fmt == FMT_Q8_0) return (mf == 1 || mf == 2) && (nf == 6 || nf == 8);
  return fmt == FMT_BF16 && (nf == 7 || nf == 8) && (mf == 1 || mf == 2);
}

hipError_t launch_gemm_wide(const WideGemm *p, int nprod, int M, int mf, int nf, hipStream_t st) {
  if (nprod < 1 || nprod > 2 || M < 1 || !gemm_wide_shape(p[0].w.fmt, mf, nf)) return hipErrorInvalidValue;
  WideArgs g{};
  g.nprod = nprod;
  g.M = M;
  const bool two = p[0].xl != nullptr;
  for (int i = 0; i < nprod; i++) {
    const WideGemm &q = p[i];
    if (!wide_operand_ok(q.w, q.xh, q.lda, M) || (q.xl != nullptr) != two || q.w.fmt != p[0].w.fmt || q.ksplit < 1 ||
        q.ksplit > q.w.cols / kWK || (q.xl && (reinterpret_cast<uintptr_t>(q.xl) & 15)) || !q.y ||
        (q.ksplit > 1 && q.split_stride < (int64_t)M * q.ldy))
      return hipErrorInvalidValue;
    g.p[i] = WideProduct{q.w, q.xh, q.xl, q.lda, q.y, q.ldy, q.ksplit, q.split_stride};
  }
  return gemm_wide_fmt<false>(g, mf, nf, two, st);
}

hipError_t launch_gemm_wide_in_epilogue(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int lda, int M,
                                        const InEpilogue &e, int mf, int nf, hipStream_t st) {
  if (!wide_operand_ok(w, xh, lda, M) || M < 1 || !gemm_wide_shape(w.fmt, mf, nf) || !e.mh || !e.ml || !e.q || !e.rope ||
      !e.pos0 || w.rows % 2 || e.s.win_q % 2 || (xl && (reinterpret_cast<uintptr_t>(xl) & 15)))
    return hipErrorInvalidValue;
  WideArgs g{};
  g.nprod = 1;
  g.M = M;
  g.p[0] = WideProduct{w, xh, xl, lda, nullptr, 0, 1, 0};
  g.e = e;
  return gemm_wide_fmt<true>(g, mf, nf, xl != nullptr, st);
}
