// Prefill projections with Q8_0 weights on the wide tiles of the
// matrix cores (v_mfma_f32_32x32x16_bf16, fp32 accumulation); see
// gemm_wide.h. Built as a translation unit of its own: its matrix-core
// results stay in ordinary vector registers (the accumulators take a
// multiply-add per quant block), where the BF16 kernels keep theirs in
// the accumulation registers.
#include "gemm_wide.h"

namespace tinyoai_gemm {
namespace {

constexpr int kQThreads = 512;  // eight waves: 4 (rows) x 2 (column halves)

// ------------------------------------------------------------ Q8_0 on the ring
// Q8_0 weights on wide tiles: 128 * WM rows x 32 * NF columns, two
// activation planes, eight waves of 32 * WM rows x 16 * NF columns, two
// per SIMD (one wave's vector work, the scales and the conversion below,
// runs beside the other's matrix products). A K step is 32 values, one
// quant block: the step's activation planes, quants (32 bytes a row) and
// the dword of fp16 block scales holding its scale (blocks 2i and 2i + 1
// of a row share one) land in an LDS ring of SLOTS stages by
// buffer_load ... lds, with no staging registers. The quants are converted to bf16 once per block,
// not once per wave: while the products of step kb run, each thread
// converts 16 quants of step kb + 1 (exact: |q| <= 128) into one of two
// bf16 weight buffers, and the scale of each row to fp32. Step kb's
// barrier certifies everything one step needs: every wave's loads of
// kb + 1 landed, and every wave finished step kb - 1 (its products, which
// read the other bf16 buffer and the ring slot refilled next, and its
// conversion of kb). Each quant block's products are formed without scale
// (the block's first product takes a zero accumulator) and added as
// acc += d * block on the fp32 accumulators, which keeps the weights exact.
//
// LDS quant rows are 32 bytes as two 16-byte halves, half h of row r at
// position h ^ ((r >> 3) & 1), so the 16 rows a conversion pass reads in a
// cycle hit distinct banks; the swizzle is applied on the global side
// (lane l of a wave load fetches logical half (l % 2) ^ ((row >> 3) & 1) of
// row l / 2). The bf16 buffers use the activation rows' layout (swz).
template <int WM>
constexpr int dmaq_slot_bytes() {
  return 2 * 128 * WM * 64 + 256 * 32 + 512 * 4;  // activation planes, quant rows, scale dwords (64 rows a wave)
}
// Ring stages: four for 128-row tiles, three (all the LDS) for 256 rows.
template <int WM>
constexpr int dmaq_slots() {
  return WM == 1 ? 4 : 3;
}
template <int NF>
constexpr int dmaq_bf_bytes() {
  return 32 * NF * 64;  // one bf16 weight buffer
}
template <int WM, int NF, bool EPI>
constexpr size_t gemm_dmaq_lds() {
  const size_t ring = (size_t)dmaq_slots<WM>() * dmaq_slot_bytes<WM>() + 2 * (size_t)dmaq_bf_bytes<NF>() + 2 * 256 * 4;
  const size_t rows = (size_t)8 * 32 * (NF * 16 + 4) * 4;
  return EPI && rows > ring ? rows : ring;
}

template <int WM, int NF, bool EPI>
__global__ __launch_bounds__(kQThreads) void gemm_dmaq_kernel(WideArgs g) {
  constexpr int XS = 2, BM = 128 * WM, BN = 32 * NF, NW = NF / 2;  // NW weight tiles a wave
  constexpr int SLOTS = dmaq_slots<WM>();
  static_assert(NF % 2 == 0 && BN <= 256 && (WM == 1 || WM == 2), "column halves; quant rows of a slot");
  constexpr int kSlot = dmaq_slot_bytes<WM>(), kAPlane = BM * 64, kB0 = XS * kAPlane, kS0 = kB0 + 256 * 32;
  constexpr int kBF = SLOTS * kSlot, kBFBytes = dmaq_bf_bytes<NF>(), kSC = kBF + 2 * kBFBytes;
  // a wave's loads per step: 16 * WM rows of each plane, 32 quant rows, 64 scale dwords
  constexpr int kPerStep = XS * WM + 2;
  static_assert((SLOTS - 2) * kPerStep < 64, "vmcnt range");
  extern __shared__ __align__(16) uint16_t lds16[];
  uint8_t *lds8 = reinterpret_cast<uint8_t *>(lds16);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave & 3, wn = wave >> 2;

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
  const __amdgpu_buffer_rsrc_t rxl = plane_rsrc(reinterpret_cast<const uint8_t *>(P.xl), (int64_t)g.M * P.lda * 2);
  const __amdgpu_buffer_rsrc_t rw = plane_rsrc(P.w.vals, (int64_t)N * P.w.vstride);
  const __amdgpu_buffer_rsrc_t rs = plane_rsrc(P.w.meta, (int64_t)N * P.w.mstride);

  // Lane offsets at k = 0. Wave w loads activation rows (w + 8 i) * 16 ..
  // + 15 of each plane (lane l: row l / 4, chunk as swz), quant rows w * 32
  // .. + 31 (lane l: row l / 2) and the scale dwords of rows w * 64 .. + 63.
  uint32_t aoff[WM];
#pragma unroll
  for (int i = 0; i < WM; i++) {
    const int row = (wave + 8 * i) * 16 + (lane >> 2), lc = (lane & 3) ^ ((row >> 2) & 3);
    aoff[i] = m0 + row < g.M ? (uint32_t)(((m0 + row) * P.lda + lc * 8) * 2) : kNone;
  }
  const int brow0 = wave * 32 + (lane >> 1), bh = (lane & 1) ^ ((brow0 >> 3) & 1);
  const uint32_t boff = brow0 < BN && n0 + brow0 < N ? (uint32_t)((n0 + brow0) * P.w.vstride + bh * 16) : kNone;
  const int srow = wave * 64 + lane;
  const uint32_t soff = srow < BN && n0 + srow < N ? (uint32_t)((n0 + srow) * P.w.mstride) : kNone;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)lds16;
  const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);
  // Step kb's loads into ring slot `slot` (past k_hi they read zeros, so
  // every wave issues kPerStep loads every step and the wait counts stay
  // exact).
  auto issue = [&](int kb, int slot) {
    const bool in = kb < k_hi;
    const uint32_t ka = in ? (uint32_t)(kb * kWK * 2) : kPast, kq = in ? (uint32_t)(kb * kWK) : kPast;
    const uint32_t ks = in ? (uint32_t)((kb >> 1) * 4) : kPast;
    const uint32_t sb = lds_base + slot * kSlot + wave_u * 1024;
#pragma unroll
    for (int i = 0; i < WM; i++) {
      lds_dma16(rxh, aoff[i] + ka, sb + i * 8192);
      lds_dma16(rxl, aoff[i] + ka, sb + kAPlane + i * 8192);
    }
    lds_dma16(rw, boff + kq, sb + kB0);
    lds_dma4(rs, soff + ks, lds_base + slot * kSlot + kS0 + wave_u * 256);
  };
  // The quants of step kb (ring slot `slot`) -> bf16 buffer bb, and each
  // row's scale -> fp32. Thread item: (row, half) of 16 values; threads
  // past the items (NF = 6) repeat the last row's (the same bytes to the
  // same places), so the conversion has no branch and schedules among the
  // products. A quant's fp32 value has zero low 16 bits (|q| <= 128), so
  // its bf16 is the high half, and two go to a dword with one permute.
  auto convert = [&](int kb, int slot, int bb) {
    const int row = min(tid >> 1, BN - 1), h = tid & 1;
    const uint8_t *q = lds8 + slot * kSlot + kB0;
    const uint32_t *sd = reinterpret_cast<const uint32_t *>(lds8 + slot * kSlot + kS0);
    uint16_t *wb = lds16 + (kBF + bb * kBFBytes) / 2;
    float *sc = reinterpret_cast<float *>(lds8 + kSC) + bb * 256;
    const uint4 w = *reinterpret_cast<const uint4 *>(q + row * 32 + ((h ^ ((row >> 3) & 1)) << 4));
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    auto pair = [](uint32_t v, int sh) {
      const uint32_t lo = __float_as_uint((float)(int8_t)(v >> sh)), hi = __float_as_uint((float)(int8_t)(v >> (sh + 8)));
      return __builtin_amdgcn_perm(hi, lo, 0x07060302u);  // hi[31:16] : lo[31:16]
    };
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      o[2 * j] = pair(ws[j], 0);
      o[2 * j + 1] = pair(ws[j], 16);
    }
    *reinterpret_cast<uint4 *>(wb + swz(row, 2 * h)) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4 *>(wb + swz(row, 2 * h + 1)) = make_uint4(o[4], o[5], o[6], o[7]);
    const uint32_t dw = sd[row];
    sc[row] = hw_half((uint16_t)((kb & 1) ? dw >> 16 : dw));
  };

  f32x16 acc[WM][NW];
#pragma unroll
  for (int f = 0; f < WM; f++)
#pragma unroll
    for (int j = 0; j < NW; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[f][j][v] = 0.f;
  const int arow = wm * 32 * WM + (lane & 31), brow = lane & 31;
  auto frag = [&](const uint16_t *base, int row, int s) {
    return *reinterpret_cast<const bf16x8 *>(base + swz(row, 2 * (lane >> 5) + s));
  };
  const f32x16 zero = {};
  // The products of the step in ring slot `slot` with bf16 buffer bb.
  auto compute = [&](int slot, int bb) {
    const uint16_t *st = lds16 + slot * (kSlot / 2);
    const uint16_t *wb = lds16 + (kBF + bb * kBFBytes) / 2;
    const float *sc = reinterpret_cast<const float *>(lds8 + kSC) + bb * 256;
    bf16x8 af[2][WM][XS];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int f = 0; f < WM; f++)
#pragma unroll
        for (int p = 0; p < XS; p++) af[s][f][p] = frag(st + p * (kAPlane / 2), arow + f * 32, s);
    // two products at a time (two weight tiles, or one tile's two row
    // tiles): consecutive matrix-core ops write different accumulators
    constexpr int JU = WM == 1 ? 2 : 1;
#pragma unroll
    for (int j0 = 0; j0 < NW; j0 += JU) {
      f32x16 tb[JU][WM];
      float d[JU];
#pragma unroll
      for (int u = 0; u < JU; u++) {
        if (j0 + u >= NW) continue;
        const int col = (wn * NW + j0 + u) * 32 + brow;
        const bf16x8 b0 = frag(wb, col, 0), b1 = frag(wb, col, 1);
        d[u] = sc[col];
#pragma unroll
        for (int f = 0; f < WM; f++) {
          tb[u][f] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0][f][0], b0, zero, 0, 0, 0);
          tb[u][f] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0][f][1], b0, tb[u][f], 0, 0, 0);
          tb[u][f] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][f][0], b1, tb[u][f], 0, 0, 0);
          tb[u][f] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][f][1], b1, tb[u][f], 0, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < JU; u++) {
        if (j0 + u >= NW) continue;
#pragma unroll
        for (int f = 0; f < WM; f++)
#pragma unroll
          for (int v = 0; v < 16; v++) acc[f][j0 + u][v] = fmaf(d[u], tb[u][f][v], acc[f][j0 + u][v]);
      }
    }
  };
  // Prologue: steps k_lo .. k_lo + SLOTS - 2 in flight; the first one's
  // quants converted.
#pragma unroll
  for (int i = 0; i < SLOTS - 1; i++) issue(k_lo + i, i);
  wait_vmcnt<(SLOTS - 2) * kPerStep>();
  __syncthreads();
  convert(k_lo, 0, 0);
  // Step kb (slot kb % SLOTS, bf16 buffer kb % 2, relative to k_lo): wait
  // for kb + 1's loads (kb + 2 .. kb + SLOTS - 2 may be in flight), meet
  // the barrier, refill the slot of kb - 1 with kb + SLOTS - 1, convert
  // kb + 1, form the products of kb.
  int slot = 0;
#pragma unroll 1
  for (int kb = k_lo; kb < k_hi; kb++) {
    wait_vmcnt<(SLOTS - 3) * kPerStep>();
    __syncthreads();
    issue(kb + SLOTS - 1, slot == 0 ? SLOTS - 1 : slot - 1);
    const int next = slot + 1 == SLOTS ? 0 : slot + 1, r = kb - k_lo;
    convert(kb + 1, next, (r + 1) & 1);  // past k_hi: zeros (kPast loads), never read
    compute(slot, r & 1);
    slot = next;
  }
  wait_vmcnt<0>();  // no load may land in LDS after this point
  __syncthreads();

  // D fragment: lane holds column lane % 32 of rows (v / 4) * 8 + (lane / 32) * 4 + v % 4.
  const int r0 = m0 + wm * 32 * WM, c0 = n0 + wn * (BN / 2);
  if constexpr (EPI) {
    constexpr int kPitch = BN / 2 + 4;
    float *tile = reinterpret_cast<float *>(lds16) + wave * 32 * kPitch;
#pragma unroll
    for (int f = 0; f < WM; f++) {
#pragma unroll
      for (int j = 0; j < NW; j++)
#pragma unroll
        for (int v = 0; v < 16; v++)
          tile[((v >> 2) * 8 + (lane >> 5) * 4 + (v & 3)) * kPitch + j * 32 + (lane & 31)] = acc[f][j][v];
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      wide_epilogue_rows(g, tile, kPitch, BN / 2, r0 + f * 32, c0, N, lane);
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    return;
  }
  float *y = P.y + (int64_t)split * P.split_stride;
#pragma unroll
  for (int f = 0; f < WM; f++)
#pragma unroll
    for (int j = 0; j < NW; j++) {
      const int n = c0 + j * 32 + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = r0 + f * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (m < g.M) y[(int64_t)m * P.ldy + n] = acc[f][j][v];
      }
    }
}

template <int WM, int NF, bool EPI>
hipError_t gemm_wideq_launch(const WideArgs &g, hipStream_t st) {
  constexpr int BM = 128 * WM, BN = 32 * NF;
  int blocks = 0;
  for (int i = 0; i < g.nprod; i++) {
    const int tiles = ((g.M + BM - 1) / BM) * ((g.p[i].w.rows + BN - 1) / BN);
    blocks += (tiles * g.p[i].ksplit + 7) / 8 * 8;
  }
  constexpr size_t lds = gemm_dmaq_lds<WM, NF, EPI>();
  static_assert(lds <= 160 * 1024, "LDS of a CU");
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_dmaq_kernel<WM, NF, EPI>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((gemm_dmaq_kernel<WM, NF, EPI>), dim3(blocks), dim3(kQThreads), lds, st, g);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_wideq(const WideArgs &g, int mf, int nf, bool epi, hipStream_t st) {
  if (mf == 1 && nf == 8) return epi ? gemm_wideq_launch<1, 8, true>(g, st) : gemm_wideq_launch<1, 8, false>(g, st);
  if (mf == 1 && nf == 6) return epi ? gemm_wideq_launch<1, 6, true>(g, st) : gemm_wideq_launch<1, 6, false>(g, st);
  if (mf == 2 && nf == 8) return epi ? gemm_wideq_launch<2, 8, true>(g, st) : gemm_wideq_launch<2, 8, false>(g, st);
  if (mf == 2 && nf == 6) return epi ? gemm_wideq_launch<2, 6, true>(g, st) : gemm_wideq_launch<2, 6, false>(g, st);
  return hipErrorInvalidValue;
}

}  // namespace tinyoai_gemm
