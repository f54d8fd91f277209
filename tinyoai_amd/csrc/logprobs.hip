// Log probabilities of a forward's rows on the device (ForwardWithLogprobs,
// mlx.go:53-57 / mlx_native.go:300-311, with the arithmetic of
// summarizeLogits, logprobs.go:60-95): for each row of logits, the target's
// log probability and the `count` largest entries (descending, ties to the
// lower id), all normalised over the whole vocabulary:
//   best = max_i v_i; total = sum_i exp(v_i - best) in float64;
//   z = best + log(total); logprob(i) = v_i - z in float64.
//
// One 1024-thread block per row. The count-th largest key is found by a
// radix select over order-preserving 32-bit keys (four passes of 8-bit
// digits, histograms in LDS; -0 keys as +0, which compares equal to it);
// the entries above it are taken, and of those equal to it the lowest ids,
// found by a prefix scan over the threads' contiguous id ranges; the
// candidates are then ranked by (value desc, id asc): in LDS for up to
// 1024 of them, else as 64-bit words (key, then the complement of the id)
// bitonic-sorted in global scratch. The float64 sum differs from the
// reference's sequential one only in summation order.
//
// A row holding NaN sets the error word (to row + 1): the reference's
// float64 max then propagates NaN into every value, and its shortlist
// appends NaN entries wherever its comparisons all fail; the library
// refuses such rows instead.
#include <algorithm>

#include "kernels.h"

namespace {

constexpr int kT = 1024;
constexpr int kMaxCount = 1024;   // candidates ranked in LDS
constexpr int kLargeBlocks = 64;  // blocks (rows at a time) of the global-scratch ranking

// Order-preserving key of a float: larger float -> larger unsigned key;
// -0 takes +0's key (the two compare equal).
__device__ __forceinline__ uint32_t float_key(float v) {
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0;
  return b & 0x80000000u ? ~b : b | 0x80000000u;
}

__device__ __forceinline__ double block_sum_d(double v, double *red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < kT / 64; i++) t += red[i];  // fixed order
  return t;
}

// LARGE: more than kMaxCount candidates, ranked in `sorted` (P words per
// block, P a power of two >= count); the grid's blocks then step through
// the rows.
template <bool LARGE>
__global__ __launch_bounds__(kT) void logprob_kernel(const float *logits, int64_t ld, int rows, int V,
                                                     const int *targets, int count, double *chosen, int *top_ids,
                                                     double *top_lp, uint64_t *sorted, int P, int *bad) {
  __shared__ uint32_t hist[256];
  __shared__ double red[kT / 64];
  __shared__ float fred[kT / 64];
  __shared__ uint32_t s_prefix, s_need;
  __shared__ int s_scan[kT];
  __shared__ int s_ncand, s_nan;
  __shared__ float cval[LARGE ? 1 : kMaxCount];
  __shared__ int cid[LARGE ? 1 : kMaxCount];
  const int tid = threadIdx.x;
  uint64_t *srt = LARGE ? sorted + (int64_t)blockIdx.x * P : nullptr;
  for (int row = blockIdx.x; row < rows; row += gridDim.x) {
  const float *v = logits + (int64_t)row * ld;
  // NaN check, then the max
  if (tid == 0) s_nan = 0;
  __syncthreads();
  bool nan = false;
  for (int i = tid; i < V; i += kT) nan |= v[i] != v[i];
  if (nan) s_nan = 1;
  __syncthreads();
  if (s_nan) {  // uniform across the block
    if (tid == 0) atomicMax(bad, row + 1);
    __syncthreads();
    continue;
  }
  float mx = -INFINITY;
  for (int i = tid; i < V; i += kT) mx = fmaxf(mx, v[i]);
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((tid & 63) == 0) fred[tid >> 6] = mx;
  __syncthreads();
  float best = fred[0];
  for (int i = 1; i < kT / 64; i++) best = fmaxf(best, fred[i]);
  // float64 normaliser
  double total = 0.0;
  for (int i = tid; i < V; i += kT) total += exp((double)v[i] - (double)best);
  total = block_sum_d(total, red);
  const double z = (double)best + log(total);
  // radix select of the count-th largest key
  uint32_t prefix = 0, need = (uint32_t)count;  // keys above the prefix already taken: count - need
  for (int pass = 0; pass < 4; pass++) {
    const int shift = 24 - 8 * pass;
    const uint32_t hi_mask = pass == 0 ? 0u : 0xFFFFFFFFu << (shift + 8);
    for (int i = tid; i < 256; i += kT) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < V; i += kT) {
      const uint32_t k = float_key(v[i]);
      if ((k & hi_mask) == (prefix & hi_mask)) atomicAdd(&hist[(k >> shift) & 255], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t above = 0;
      int digit = 255;
      for (; digit > 0; digit--) {
        if (above + hist[digit] >= need) break;
        above += hist[digit];
      }
      s_prefix = (prefix & hi_mask) | ((uint32_t)digit << shift);
      s_need = need - above;
    }
    __syncthreads();
    prefix = s_prefix;
    need = s_need;
    __syncthreads();
  }
  // prefix: the count-th largest key; need: how many entries equal to it
  // are taken (the lowest ids). Each thread owns ids [tid * per, ...).
  const int per = (V + kT - 1) / kT, lo = tid * per, hi = min(V, lo + per);
  int eq = 0;
  for (int i = lo; i < hi; i++) eq += float_key(v[i]) == prefix;
  s_scan[tid] = eq;
  if (tid == 0) s_ncand = 0;
  __syncthreads();
  for (int o = 1; o < kT; o <<= 1) {  // inclusive scan
    const int add = tid >= o ? s_scan[tid - o] : 0;
    __syncthreads();
    s_scan[tid] += add;
    __syncthreads();
  }
  int rank_eq = s_scan[tid] - eq;  // equal keys before this thread's range
  for (int i = lo; i < hi; i++) {
    const uint32_t k = float_key(v[i]);
    bool take = k > prefix;
    if (k == prefix) take = (uint32_t)rank_eq++ < need;
    if (take) {
      const int slot = atomicAdd(&s_ncand, 1);
      if constexpr (LARGE) {
        srt[slot] = (uint64_t)k << 32 | (uint32_t)~i;
      } else {
        cval[slot] = v[i];
        cid[slot] = i;
      }
    }
  }
  __syncthreads();
  const int nc = s_ncand;  // == count
  if constexpr (LARGE) {
    // Pad to P with zeros (below every entry's word: keys of non-NaN
    // values are at least 0x007FFFFF), then a bitonic sort, descending.
    for (int c = nc + tid; c < P; c += kT) srt[c] = 0;
    __syncthreads();
    for (int k2 = 2; k2 <= P; k2 <<= 1)
      for (int j = k2 >> 1; j > 0; j >>= 1) {
        for (int p = tid; p < P / 2; p += kT) {
          const int i = (p / j) * 2 * j + p % j, l = i + j;
          const uint64_t a = srt[i], b = srt[l];
          const bool desc = (i & k2) == 0;
          if (desc ? a < b : a > b) {
            srt[i] = b;
            srt[l] = a;
          }
        }
        __syncthreads();
      }
    for (int r = tid; r < nc; r += kT) {
      const int id = (int)~(uint32_t)srt[r];
      top_ids[(int64_t)row * count + r] = id;
      top_lp[(int64_t)row * count + r] = (double)v[id] - z;
    }
  } else {
    for (int c = tid; c < nc; c += kT) {
      const float cv = cval[c];
      const int ci = cid[c];
      int r = 0;
      for (int j = 0; j < nc; j++) r += cval[j] > cv || (cval[j] == cv && cid[j] < ci);
      top_ids[(int64_t)row * count + r] = ci;
      top_lp[(int64_t)row * count + r] = (double)cv - z;
    }
  }
  if (tid == 0) chosen[row] = (double)v[targets[row]] - z;
  __syncthreads();
  }
}

}  // namespace

size_t logprob_scratch_bytes(int count) {
  if (count <= kMaxCount) return 256;
  size_t p = 1;
  while (p < (size_t)count) p <<= 1;
  return 256 + (size_t)kLargeBlocks * p * 8;
}

hipError_t launch_logprobs(const float *logits, int64_t ld, int rows, int vocab, const int *targets, int count,
                           double *chosen, int *top_ids, double *top_lp, void *scratch, hipStream_t st) {
  if (rows < 1 || vocab < 1 || count < 1 || count > vocab || ld < vocab || !scratch) return hipErrorInvalidValue;
  int *bad = reinterpret_cast<int *>(scratch);
  if (count <= kMaxCount) {
    hipLaunchKernelGGL(logprob_kernel<false>, dim3(rows), dim3(kT), 0, st, logits, ld, rows, vocab, targets, count,
                       chosen, top_ids, top_lp, nullptr, 0, bad);
  } else {
    int P = 1;
    while (P < count) P <<= 1;
    uint64_t *sorted = reinterpret_cast<uint64_t *>(reinterpret_cast<char *>(scratch) + 256);
    hipLaunchKernelGGL(logprob_kernel<true>, dim3(std::min(rows, kLargeBlocks)), dim3(kT), 0, st, logits, ld, rows,
                       vocab, targets, count, chosen, top_ids, top_lp, sorted, P, bad);
  }
  return hipGetLastError();
}
