// Wide-tile matrix-core products shared by the BF16 (gemm.hip) and Q8_0
// (gemm_q8.hip) kernels: the launch arguments, the LDS row layout of the
// operand fragments, the fused in-projection epilogue and the tile store.
#pragma once

#include "epilogue.h"

namespace tinyoai_gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// ------------------------------------------------------------ wide tiles
// BF16 weights. One wave per SIMD: four waves of a 256-thread block own
// 32 * MF rows each (block rows BM = 128 * MF) and all BN = 32 * NF columns
// of the block's tile, as MF x NF tiles of v_mfma_f32_32x32x16_bf16; per
// k16 a wave reads MF * XS activation and NF weight fragments from LDS for
// XS * MF * NF products (MF = 2, NF = 7, two planes: 11 fragment reads for
// 28 products). A K step is 32 values.
//
// LDS rows are 64 bytes (32 bf16) as four 16-byte chunks, chunk c of row r
// at position c ^ ((r >> 2) & 3): the 16 lanes of a fragment read that
// share a chunk index hit 16 distinct bank groups. Lane l of a fragment
// holds the 16 consecutive values 16 * (l / 32) .. + 15 of its row's step,
// the first 8 for the step's first product and the rest for its second;
// activation and weight fragments use the same k order, so each step is
// covered exactly once.
//
// Blocks map onto the 8 XCDs in runs: XCD x takes tiles [x * per, (x + 1)
// * per) (M tiles fastest), so the blocks resident on one XCD share their
// weight tiles through its L2.
struct WideProduct {
  MatDesc w;                // N = rows, K = cols (a column view of a larger matrix is fine)
  const uint16_t *xh, *xl;  // bf16 planes, rows lda values apart
  int lda;
  float *y;                 // split s at y + s * split_stride, rows ldy floats apart
  int ldy;
  int ksplit;
  int64_t split_stride;
};
struct WideArgs {
  WideProduct p[2];  // one launch may carry two products of the same tile shape
  int nprod;
  int M;
  InEpilogue e;      // EPI: the fused in-projection epilogue (one product, no split)
};

constexpr int kWThreads = 256, kWK = 32;

__device__ __forceinline__ int swz(int row, int c) { return row * kWK + ((c ^ ((row >> 2) & 3)) << 3); }

// The in-projection epilogue of 32 output rows staged in LDS (row r of
// the wave's band at tile + r * pitch, bn columns from n0): the wave's
// lanes take (row, output pair) items in order, four at a time so that
// their float64 exp chains and stores overlap (one wave per SIMD runs
// this part).
__device__ __forceinline__ void wide_epilogue_rows(const WideArgs &g, const float *tile, int pitch, int bn, int r0,
                                                   int n0, int N, int lane) {
  const StableDims es = g.e.s;
  const KVDev ekv = g.e.kv;
  const float *rope = g.e.rope;
  float *eq = g.e.q, *em = g.e.m;
  uint16_t *emh = g.e.mh, *eml = g.e.ml;
  const int ldm = g.e.ldm ? g.e.ldm : es.inter;
  const int p0 = *g.e.pos0, mu0 = (es.win_q + 2 * es.win_kv) / 2;
  const int half = bn / 2, items = 32 * half;
  for (int it0 = lane; it0 < items; it0 += 4 * 64) {
    float2 pv[4];
    int m[4], u[4];
    bool ok[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int it = it0 + b * 64, r = it / half, c = 2 * (it - r * half);
      m[b] = r0 + r;
      u[b] = (n0 + c) >> 1;
      ok[b] = it < items && m[b] < g.M && n0 + c < N;
      pv[b] = ok[b] ? *reinterpret_cast<const float2 *>(tile + r * pitch + c) : make_float2(0.f, 0.f);
    }
#pragma unroll
    for (int b = 0; b < 4; b++) {
      if (!ok[b]) continue;
      if (u[b] >= mu0) {
        const float gv = es.silu ? silu_gate_llama(pv[b].x, pv[b].y) : silu_gate(pv[b].x, pv[b].y);
        if (em) em[(int64_t)m[b] * es.inter + (u[b] - mu0)] = gv;
        store_bf16_split(emh, eml, (int64_t)m[b] * ldm + (u[b] - mu0), gv);
      } else {
        const int pos = p0 + m[b];
        in_pair_epilogue(es, ekv, rope + (int64_t)pos * es.rot, pos, u[b], pv[b].x, pv[b].y,
                         eq + (int64_t)m[b] * es.heads * es.hd, nullptr);
      }
    }
  }
}

// The end of a wide-tile block: with EPI its output rows go through the
// in-projection epilogue (staged in LDS, which the caller has released:
// no load may still land there), else the tile (split `split`) is stored.
template <int MF, int NF, bool EPI>
__device__ __forceinline__ void wide_finish(const WideArgs &g, const WideProduct &P, const f32x16 (&acc)[MF][NF],
                                            float *lds, int split, int m0, int n0, int N, int wave, int lane) {
  constexpr int BN = 32 * NF;
  if constexpr (EPI) {
    constexpr int kPitch = BN + 4;
    float *tile = lds + wave * 32 * kPitch;
#pragma unroll
    for (int f = 0; f < MF; f++) {
#pragma unroll
      for (int j = 0; j < NF; j++)
#pragma unroll
        for (int v = 0; v < 16; v++)
          tile[((v >> 2) * 8 + (lane >> 5) * 4 + (v & 3)) * kPitch + j * 32 + (lane & 31)] = acc[f][j][v];
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int r0w = m0 + (wave * MF + f) * 32;
      wide_epilogue_rows(g, tile, kPitch, BN, r0w, n0, N, lane);
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    return;
  }
  float *y = P.y + (int64_t)split * P.split_stride;
#pragma unroll
  for (int f = 0; f < MF; f++)
#pragma unroll
    for (int j = 0; j < NF; j++) {
      const int n = n0 + j * 32 + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = m0 + (wave * MF + f) * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (m < g.M) y[(int64_t)m * P.ldy + n] = acc[f][j][v];
      }
    }
}

// The Q8_0 products on wide tiles (128 * mf x 32 * nf, two activation planes).
hipError_t launch_gemm_wideq(const WideArgs &g, int mf, int nf, bool epi, hipStream_t st);

}  // namespace tinyoai_gemm
