// Decode-path attention and embedding kernels for gfx950, and the format
// dispatch of the streaming matrix-vector kernels (matvec.h).
//
// StableLM's parallel residual (stablelm.go:365-377) lets a layer run as
// three launches over the fused matrices of LayerDev (kernels.h):
// decode_in (matvec.h), attention (here: split-K flash decode; blocks of a
// head combine through the last-arriving block) and decode_out (matvec.h).
#include <algorithm>

#include "attention.h"
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
template <int HD, bool HALF, int STEPS, int WAVES = kWaves, bool BR = false>
__global__ __launch_bounds__(WAVES * 64) void attention_kernel(AttArgs a) {
  attention_block<HD, HALF, STEPS, WAVES, BR, false>(a, blockIdx.x, blockIdx.y, blockIdx.z);
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

bool decode_in_att_supported(const LayerDev &w, const StableDims &s, int threads, int steps) {
  if (threads != 256 || (steps != 1 && steps != 2) || w.win2.rows || w.win.rows % 2 || !planes_fit(w.win) ||
      (s.hd != 64 && s.hd != 80 && s.hd != 128) || s.win_q + 2 * s.win_kv > w.win.rows)
    return false;
  InArgs a{w, s};
  switch (w.win.fmt) {
    case FMT_Q8_0: return tinyoai_matvec::decode_in_att_fits<FMT_Q8_0>(a);
    case FMT_BF16: return tinyoai_matvec::decode_in_att_fits<FMT_BF16>(a);
  }
  return false;
}

hipError_t launch_decode_in_att(const LayerDev &w, const StableDims &s, const KVDev &kv, float *x, const MatDesc *emb,
                                const int *token, const float *rope, const int *pos, float *q_out, float *m_out,
                                int grid, int steps, int splits, float *partials, unsigned *counters, float *att_out,
                                unsigned *fuse_ctr, const int *epoch, unsigned *err, hipStream_t st) {
  if (!decode_in_att_supported(w, s, 256, steps) || splits < 1 || splits > 512 || grid < 1)
    return hipErrorInvalidValue;
  InArgs a{w, s, kv, x, emb ? *emb : MatDesc{}, emb != nullptr, token, rope, pos, q_out, m_out};
  AttArgs att{s, kv, q_out, pos, splits, partials, counters, att_out, KVDev{}, 0, nullptr};
  FuseArgs fz{fuse_ctr, fuse_ctr + 32 * (1 + kFuseGroups), epoch, (unsigned)grid * 4u, grid,
              (s.win_q + 2 * s.win_kv) / 2, err, 1u << 20};
  switch (w.win.fmt) {
    case FMT_Q8_0: return run_decode_in_att<FMT_Q8_0>(a, att, fz, steps, st);
    case FMT_BF16: return run_decode_in_att<FMT_BF16>(a, att, fz, steps, st);
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

int decode_attention_steps(int pos, int heads, int hd) {
  // Measured at the 3B shapes (Q8_0 with fp32 KV, BF16 with fp16 KV), tok/s
  // of the whole decode step: two steps inside the decode_in launch lead up
  // to ~1500 positions (869 against 798 at 640, Q8_0); four steps as a
  // launch of its own lead from ~2000 (BF16 at 4096: 550 against 476);
  // 1024 positions per 16-wave block beyond ~5000 (BF16 at 8000: 512
  // against 475 with four steps and 360 fused).
  const int npos = pos + 1;
  if (npos <= 1800) return attention_steps(pos, heads);
  if (npos <= 5000 || hd > 80) return 4;
  return 16;
}

int attention_splits(int max_pos, int steps) { return (max_pos + 64 * steps) / (64 * steps); }

hipError_t launch_attention(const StableDims &s, const KVDev &kv, const float *q, const int *pos0, int nq,
                            int max_pos, float *partials, unsigned *counters, float *out, hipStream_t st, int steps,
                            int splits) {
  if (steps <= 0) steps = attention_steps(max_pos, s.heads);
  if (splits <= 0) splits = attention_splits(max_pos, steps);
  if (splits > 512) return hipErrorInvalidValue;  // combine scratch holds 512 splits
  AttArgs a{s, kv, q, pos0, splits, partials, counters, out, KVDev{}, 0, nullptr};
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

namespace {
// The shared-prefix pass applies: a prefix, a head width the matrix-core
// attention takes, and at most one query tile of it.
bool branch_shared(const StableDims &s, int prefix, int nq) {
  return prefix > 0 && nq <= 128 && flash_prefill_supported(s.hd);
}
// Suffix blocks' positions / 64 and their count after a shared pass.
void suffix_splits(const StableDims &s, int prefix, int max_pos, int &steps, int &splits) {
  const int span = max_pos - prefix + 1;
  steps = std::min(attention_steps(span - 1, s.heads), 4);
  splits = attention_splits(span - 1, steps);
}
}  // namespace

int branch_attention_records(const StableDims &s, int prefix, int max_pos, int nq) {
  if (branch_shared(s, prefix, nq)) {
    int steps, splits;
    suffix_splits(s, prefix, max_pos, steps, splits);
    return shared_prefix_splits(prefix) + splits;
  }
  return attention_splits(max_pos, std::min(attention_steps(max_pos, s.heads), 4));
}

int branch_attention_shape(const StableDims &s, int prefix, int max_pos, int nq) {
  int steps = std::min(attention_steps(max_pos, s.heads), 4), splits = attention_splits(max_pos, steps);
  if (branch_shared(s, prefix, nq)) suffix_splits(s, prefix, max_pos, steps, splits);
  return steps * 4096 + splits;
}

hipError_t launch_branch_attention(const StableDims &s, const KVDev &kv, const KVDev &sfx, int prefix,
                                   const float *q, const int *rows, int nq, int max_pos, float *partials,
                                   unsigned *counters, float *out, int max_splits, hipStream_t st) {
  if (prefix < 0 || prefix > kv.cap || nq < 1 || !rows || kv.half != sfx.half || max_pos < prefix)
    return hipErrorInvalidValue;
  int steps = std::min(attention_steps(max_pos, s.heads), 4), splits = attention_splits(max_pos, steps);
  AttArgs a{s, kv, q, nullptr, max_splits, partials, counters, out, sfx, prefix, rows};
  if (branch_shared(s, prefix, nq)) {
    // One matrix-core pass reads the prefix once for every query and leaves
    // its records first in each region; the suffix splits follow.
    suffix_splits(s, prefix, max_pos, steps, splits);
    a.t_begin = prefix;
    a.pre_splits = shared_prefix_splits(prefix);
    if (a.pre_splits + splits > 512 || a.pre_splits + splits > max_splits) return hipErrorInvalidValue;
    const hipError_t e =
        launch_shared_prefix_attention(s, kv, prefix, q, nq, partials, partial_region(max_splits, s.hd), st);
    if (e != hipSuccess) return e;
  } else if (splits > 512 || splits > max_splits) {
    return hipErrorInvalidValue;
  }
  switch (s.hd) {
    case 64: return kv.half ? launch_branch_attention_hd<64, true>(a, nq, splits, steps, st)
                            : launch_branch_attention_hd<64, false>(a, nq, splits, steps, st);
    case 80: return kv.half ? launch_branch_attention_hd<80, true>(a, nq, splits, steps, st)
                            : launch_branch_attention_hd<80, false>(a, nq, splits, steps, st);
    case 8: return kv.half ? launch_branch_attention_hd<8, true>(a, nq, splits, steps, st)
                           : launch_branch_attention_hd<8, false>(a, nq, splits, steps, st);
    case 128: return kv.half ? launch_branch_attention_hd<128, true>(a, nq, splits, steps, st)
                             : launch_branch_attention_hd<128, false>(a, nq, splits, steps, st);
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
