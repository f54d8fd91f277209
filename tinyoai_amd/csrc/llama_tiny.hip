// Decode tokens of the stories260K-shaped legacy Llama (llama2.c: dim 64,
// 8 query / 4 kv heads of width 8, MLP 172, up to 8 layers and 512
// positions) in one launch: Model.transformer (model.go:407-481) for each
// token of a forward, from the embedding row to the classifier's logits.
//
// The model is about 1 MB of fp32 weights, so a token is bound by the
// latency of its dependent steps, not by bandwidth; one kernel per step
// spends most of a token in launch gaps. Here one workgroup of 1024
// threads runs every token of the call in order and keeps the activations
// in LDS:
//   per layer: RMSNorm (model.go:591-600) -> the fused [wq | wk | wv] rows
//   -> the adjacent-pair rotation (model.go:611-618), K/V stored at the
//   token's position -> attention over positions 0..pos (model.go:432-461,
//   softmax model.go:552-570) -> x += wo * att -> RMSNorm -> w1/w3 rows
//   (interleaved) and SwiGLU (model.go:463-470) -> x += w2 * h;
//   then the final RMSNorm and the tied classifier (model.go:476-479).
// Matrix rows: 16 lanes (one DPP row) per matrix row, lane t holding the
// row's 16-byte chunks t, t + 16, ... in registers; a layer's weights are
// loaded while the previous layer runs (the registers of a matrix are
// refilled with the next layer's rows as soon as they have been used), so
// only the first layer of a call waits for memory. The 16 partial sums of
// a row are added with DPP lane moves in a fixed order, and lane 0 of the
// row's lanes keeps the result. Rotation and SwiGLU pair rows 2j and
// 2j + 1, which sit in adjacent DPP rows of one wave (v_permlane16_swap).
// RMSNorm: every wave forms the float64 sum of float32 squares of x itself
// (no barrier), then ss / n + eps and 1 / float32(sqrt(.)) in float32.
// Attention: 256 threads per kv head, each holding positions p and p + 256
// for both query heads of the head; a wave forms its maximum, exp(s - m)
// weights, their sum and the weighted V, reduced across lanes with lane
// swaps and DPP moves; the four waves of a kv head are combined as
// M = max m_w, out = sum o_w e^(m_w - M) / sum l_w e^(m_w - M).
#include "kernels.h"

namespace {

constexpr int kT = 1024;
constexpr int D = kTinyDim, HS = 8, NH = 8, NKV = 4, KVD = NKV * HS, QKV = D + 2 * KVD;
constexpr int HID = kTinyHidden, HROWS = 2 * HID, HCH = HID / 4;
constexpr int kPerKv = kT / NKV;  // attention threads per kv head
static_assert(D == 64 && HID % 4 == 0 && HCH <= 48, "one chunk of x per lane, up to three of h");
static_assert(kTinyMaxSeq == 2 * kPerKv, "two positions per attention thread");
constexpr int kW13 = (HROWS + 63) / 64;  // w1/w3 rows per DPP row
constexpr int kW2 = (HCH + 15) / 16;     // w2 chunks per lane
constexpr int kHeadRows = kTinyMaxVocab / 64;
constexpr int kRec = 12;                 // attention record: m, l, -, -, o[8]

using f4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot4(f4 a, f4 b, float acc) {
  acc = fmaf(a.x, b.x, acc);
  acc = fmaf(a.y, b.y, acc);
  acc = fmaf(a.z, b.z, acc);
  return fmaf(a.w, b.w, acc);
}
// Sum of the 16 lanes of a DPP row, the same bits in every lane of the row:
// adjacent lanes, lane pairs, quads (row_half_mirror pairs quad 0 with 1 and
// 2 with 3), then half rows (row_ror 8); each step adds two values that
// both lanes of a pair hold.
__device__ __forceinline__ float row_total(float v) {
  v = dpp_add<0xb1>(v);   // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4e>(v);   // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  return dpp_add<0x128>(v);  // row_ror 8
}
template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf,
                                                                        0xf, false)));
}
__device__ __forceinline__ float row_max(float v) {
  v = dpp_max<0xb1>(v);
  v = dpp_max<0x4e>(v);
  v = dpp_max<0x124>(v);
  return dpp_max<0x128>(v);
}
// v_permlane16_swap exchanges the odd DPP rows of a with the even rows of b,
// so swap16(v, w) leaves an even row's lanes their own v in a and the next
// row's v in b; v_permlane32_swap exchanges the upper 32 lanes of a with
// the lower 32 of b. The two operands must be different values (given the
// same value twice, the two results share one register).
__device__ __forceinline__ void swap16(float &a, float &b) {
  const u32x2 r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                   false, false);
  const uint32_t x = r.x, y = r.y;  // (bit_cast of a vector element reads element 0)
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
__device__ __forceinline__ void swap32(float &a, float &b) {
  const u32x2 r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                   false, false);
  const uint32_t x = r.x, y = r.y;  // (bit_cast of a vector element reads element 0)
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}

// RMSNorm scale of the LDS row xs[0..64) (rms_norm_lds's arithmetic), formed
// by the calling wave alone.
__device__ __forceinline__ float rms_scale(const float *xs) {
  const float v = xs[threadIdx.x & 63];
  const float ss = (float)wave_total_d((double)__fmul_rn(v, v));
  const float mean = __fadd_rn(__fdiv_rn(ss, (float)D), 1e-5f);
  return __fdiv_rn(1.0f, (float)sqrt((double)mean));
}
__device__ __forceinline__ f4 rms_apply(f4 x, f4 w, float inv) {
  return f4{__fmul_rn(w.x, __fmul_rn(inv, x.x)), __fmul_rn(w.y, __fmul_rn(inv, x.y)),
            __fmul_rn(w.z, __fmul_rn(inv, x.z)), __fmul_rn(w.w, __fmul_rn(inv, x.w))};
}

// SwiGLU of one w1/w3 pair. Not inlined: inside the layer loop the
// compiler would keep exp_f64's constants in registers across the whole
// loop.
__device__ __attribute__((noinline)) float swiglu(float g, float u) { return silu_gate_llama(g, u); }

// A layer's weights in one lane's registers.
struct Regs {
  f4 qkv[2], wo, w13[kW13], w2[kW2];
};

// 16 bytes at byte voff + soff of a buffer (zeros past its end).
__device__ __forceinline__ f4 bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mat_rsrc(const uint8_t *p, int rows, int cols) {
  return plane_rsrc(p, (int64_t)rows * cols * 4);
}
constexpr uint32_t kFar = 0x80000000u;  // an offset past every buffer

// Lane offsets: vo = row grp, chunk t of a 64-column matrix (rows grp + 64u
// at + 16384u); vo2 = row grp, chunk t of w2 (chunk t + 16u at + 256u;
// chunks past the row read as zeros).
__device__ __forceinline__ void load_qkv(Regs &r, const TinyLlamaArgs &a, int l, uint32_t vo) {
  const auto rs = mat_rsrc(a.w[l][0], QKV, D);
#pragma unroll
  for (int u = 0; u < 2; u++) r.qkv[u] = bload(rs, vo, 16384u * u);
}
__device__ __forceinline__ void load_wo(Regs &r, const TinyLlamaArgs &a, int l, uint32_t vo) {
  r.wo = bload(mat_rsrc(a.w[l][1], D, D), vo, 0);
}
__device__ __forceinline__ void load_w13(Regs &r, const TinyLlamaArgs &a, int l, uint32_t vo) {
  const auto rs = mat_rsrc(a.w[l][2], HROWS, D);
#pragma unroll
  for (int u = 0; u < kW13; u++) r.w13[u] = bload(rs, vo, 16384u * u);
}
__device__ __forceinline__ void load_w2(Regs &r, const TinyLlamaArgs &a, int l, uint32_t vo2) {
  const auto rs = mat_rsrc(a.w[l][3], D, HID);
#pragma unroll
  for (int u = 0; u < kW2; u++) r.w2[u] = bload(rs, vo2, 256u * u);
}

// K/V of positions [0, count) of layer l (every kv head) into LDS: kv head
// h's keys at kvs[h][p][8], values at kvs[NKV + h][p][8]. Streams of 1 KB
// (32 positions), spread over the waves; a stream reaching past a head's
// positions brings bytes that no lane reads.
__device__ __forceinline__ void kv_to_lds(const TinyLlamaArgs &a, int l, int count, const float *kvs, int wave,
                                          int lane) {
  const int nch = (count + 31) / 32;
  const int64_t bytes = (int64_t)NKV * a.cap * HS * 4;
  const auto rk = plane_rsrc(reinterpret_cast<const uint8_t *>(a.k[l]), bytes);
  const auto rv = plane_rsrc(reinterpret_cast<const uint8_t *>(a.v[l]), bytes);
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)kvs;
  for (int i = wave; i < 2 * NKV * nch; i += kT / 64) {
    const int stream = i % (2 * NKV), c = i / (2 * NKV), h = stream % NKV;
    lds_dma16(stream < NKV ? rk : rv, (uint32_t)(h * a.cap * HS * 4 + c * 1024 + lane * 16),
              base + (uint32_t)((stream * kTinyMaxSeq + c * 32) * HS * 4));
  }
}

__global__ __launch_bounds__(kT) void tiny_llama_kernel(TinyLlamaArgs a) {
  __shared__ __align__(16) float kvs[2 * NKV * kTinyMaxSeq * HS];  // cached K/V of the layer
  __shared__ __align__(16) float xs[D];            // residual stream
  __shared__ __align__(16) float qkv[QKV];         // rotated q | k | v of the token
  __shared__ __align__(16) float hb[HCH * 4 + 4];  // SwiGLU output
  __shared__ __align__(16) float rec[kT / 64][2][kRec];
  __shared__ __align__(16) float rmsw[2 * kTinyMaxLayers + 1][D];
  __shared__ __align__(16) float lg[kTinyMaxVocab];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = tid >> 4, t = tid & 15;
  const int L = a.layers;

  kv_to_lds(a, 0, a.prefix, kvs, wave, lane);
  for (int i = tid; i < L * D; i += kT) {
    rmsw[i / D][i % D] = a.rms_att[i];
    rmsw[kTinyMaxLayers + i / D][i % D] = a.rms_ffn[i];
  }
  if (tid < D) rmsw[2 * kTinyMaxLayers][tid] = a.rms_final[tid];

  const uint32_t vo = (uint32_t)grp * (D * 4) + 16 * t;
  const uint32_t vo2 = (uint32_t)grp * (HID * 4) + 16 * t;
  Regs r;
  load_qkv(r, a, 0, vo);
  load_wo(r, a, 0, vo);
  load_w13(r, a, 0, vo);
  load_w2(r, a, 0, vo2);
  // attention lanes: kv head, positions p0 and p0 + 256
  const int kvh = tid / kPerKv, p0 = tid % kPerKv;
  const float scale = a.att_scale;

  for (int j = 0; j < a.n; j++) {
    const int pos = a.prefix + j, token = a.tokens[j];
    const float2 cs = *reinterpret_cast<const float2 *>(a.rope + (int64_t)pos * HS + 2 * ((grp % HS) >> 1));
    if (tid < D) xs[tid] = reinterpret_cast<const float *>(a.emb + (int64_t)token * (D * 4))[tid];
    __syncthreads();

    for (int l = 0; l < L; l++) {
      const bool more = l + 1 < L || j + 1 < a.n;  // a layer follows in this launch
      const int nl = l + 1 < L ? l + 1 : 0;
      // RMSNorm, then q | k | v rows grp and grp + 64
      float kv0, kv1;  // even rows, lane t == 0: the K or V pair of rows grp + 64, grp + 65
      {
        const float inv = rms_scale(xs);
        const f4 xn = rms_apply(reinterpret_cast<const f4 *>(xs)[t], reinterpret_cast<const f4 *>(rmsw[l])[t], inv);
        float v[2];
#pragma unroll
        for (int u = 0; u < 2; u++) v[u] = row_total(dot4(r.qkv[u], xn, 0.f));
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const int row = grp + 64 * u;
          float x0 = v[u], x1 = 0.f;
          swap16(x0, x1);  // even rows: rows 2j and 2j + 1 of the pair
          if (row < D + KVD) {
            const float e0 = x0, e1 = x1;
            x0 = __fsub_rn(__fmul_rn(e0, cs.x), __fmul_rn(e1, cs.y));
            x1 = __fadd_rn(__fmul_rn(e1, cs.x), __fmul_rn(e0, cs.y));
          }
          if (t == 0 && !(grp & 1)) *reinterpret_cast<float2 *>(qkv + row) = float2{x0, x1};
          if (u == 1) {
            kv0 = x0;
            kv1 = x1;
          }
        }
      }
      wait_vmcnt<0>();  // this wave's K/V streams into LDS have landed
      __syncthreads();
      if (t == 0 && !(grp & 1)) {  // storeKV at the token's position: rows grp + 64, grp + 65
        const int row = grp + 64;
        const bool is_k = row < D + KVD;
        const int rr = row - D - (is_k ? 0 : KVD);
        *reinterpret_cast<float2 *>((is_k ? a.k[l] : a.v[l]) + ((int64_t)(rr / HS) * a.cap + pos) * HS + rr % HS) =
            float2{kv0, kv1};
      }
      // attention of query heads 2 kvh and 2 kvh + 1
      {
        const f4 *q4 = reinterpret_cast<const f4 *>(qkv + 2 * kvh * HS);
        float s[2][2];
        bool ok[2];
        const f4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const int p = p0 + i * kPerKv;
          ok[i] = p <= pos;
          const f4 *kp = reinterpret_cast<const f4 *>(p == pos ? qkv + D + kvh * HS : kvs + (kvh * kTinyMaxSeq + p) * HS);
          const f4 k0 = ok[i] ? kp[0] : zero, k1 = ok[i] ? kp[1] : zero;
#pragma unroll
          for (int g = 0; g < 2; g++) {
            const float d = dot4(q4[2 * g + 1], k1, dot4(q4[2 * g], k0, 0.f));
            s[g][i] = ok[i] ? __fdiv_rn(d, scale) : -INFINITY;
          }
        }
        // per-wave maximum of each head: lanes < 32 reduce head 0, >= 32 head 1
        float ma = fmaxf(s[0][0], s[0][1]), mb = fmaxf(s[1][0], s[1][1]);
        swap32(ma, mb);
        float mx = row_max(fmaxf(ma, mb)), m2 = -INFINITY;
        swap16(mx, m2);
        mx = fmaxf(mx, m2);  // row 0: head 0; row 2: head 1
        const int mbits = __builtin_bit_cast(int, mx);
        const float m[2] = {__builtin_bit_cast(float, __builtin_amdgcn_readlane(mbits, 0)),
                            __builtin_bit_cast(float, __builtin_amdgcn_readlane(mbits, 32))};
        float o[2][HS], lsum[2] = {0.f, 0.f};
#pragma unroll
        for (int g = 0; g < 2; g++)
#pragma unroll
          for (int d = 0; d < HS; d++) o[g][d] = 0.f;
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const int p = p0 + i * kPerKv;
          const f4 *vp = reinterpret_cast<const f4 *>(p == pos ? qkv + D + KVD + kvh * HS
                                                              : kvs + ((NKV + kvh) * kTinyMaxSeq + p) * HS);
          const f4 v0 = ok[i] ? vp[0] : zero, v1 = ok[i] ? vp[1] : zero;
#pragma unroll
          for (int g = 0; g < 2; g++) {
            const float e = ok[i] ? expf(s[g][i] - m[g]) : 0.f;
            lsum[g] += e;
#pragma unroll
            for (int d = 0; d < 4; d++) {
              o[g][d] = fmaf(e, v0[d], o[g][d]);
              o[g][d + 4] = fmaf(e, v1[d], o[g][d + 4]);
            }
          }
        }
        // lanes i and i + 32, then rows 2r and 2r + 1, then the 16 lanes of a row
#pragma unroll
        for (int d = 0; d < HS; d++) {
          swap32(o[0][d], o[1][d]);
          o[0][d] += o[1][d];
        }
        swap32(lsum[0], lsum[1]);
        float ls = lsum[0] + lsum[1], ls2 = 0.f;
#pragma unroll
        for (int d = 0; d < 4; d++) {
          swap16(o[0][d], o[0][d + 4]);
          o[0][d] = row_total(o[0][d] + o[0][d + 4]);
        }
        swap16(ls, ls2);
        ls = row_total(ls + ls2);  // rows 0 and 2: the sums of heads 0 and 1
        // row rw of the wave: head rw >> 1, dims 4 (rw & 1) .. + 4
        const int rw = lane >> 4;
        if ((lane & 15) == 0) {
          float *rc = rec[wave][rw >> 1];
          *reinterpret_cast<f4 *>(rc + 4 + 4 * (rw & 1)) = f4{o[0][0], o[0][1], o[0][2], o[0][3]};
          if ((rw & 1) == 0) {
            rc[0] = m[rw >> 1];
            rc[1] = ls;
          }
        }
      }
      // the next layer's K/V may replace this one's once every wave is past
      // its reads; a one-layer model's next token reads the position just
      // stored, so that store must have completed first
      if (L == 1) wait_vmcnt<0>();
      __syncthreads();
      if (more) {
        kv_to_lds(a, nl, l + 1 < L ? pos : pos + 1, kvs, wave, lane);
        load_qkv(r, a, nl, vo);
      }
      // x += wo * att: lane t's chunk is dims 4 (t & 1) .. of head t >> 1
      {
        const int h = t >> 1, w0 = (h >> 1) * 4, g = h & 1;
        float mw[4], M = -INFINITY;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          mw[k] = rec[w0 + k][g][0];
          M = fmaxf(M, mw[k]);
        }
        float Lw = 0.f;
        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float e = expf(mw[k] - M);
          Lw = fmaf(rec[w0 + k][g][1], e, Lw);
          const f4 ov = *reinterpret_cast<const f4 *>(&rec[w0 + k][g][4 + 4 * (t & 1)]);
          acc = f4{fmaf(ov.x, e, acc.x), fmaf(ov.y, e, acc.y), fmaf(ov.z, e, acc.z), fmaf(ov.w, e, acc.w)};
        }
        const f4 att = {acc.x / Lw, acc.y / Lw, acc.z / Lw, acc.w / Lw};
        const float v = row_total(dot4(r.wo, att, 0.f));
        if (more) load_wo(r, a, nl, vo);
        if (t == 0) xs[grp] = __fadd_rn(xs[grp], v);
      }
      __syncthreads();
      // RMSNorm, w1/w3 row pairs and SwiGLU
      {
        const float inv = rms_scale(xs);
        const f4 xn = rms_apply(reinterpret_cast<const f4 *>(xs)[t],
                                reinterpret_cast<const f4 *>(rmsw[kTinyMaxLayers + l])[t], inv);
        float v[kW13];
#pragma unroll
        for (int u = 0; u < kW13; u++) v[u] = row_total(dot4(r.w13[u], xn, 0.f));
        if (more) load_w13(r, a, nl, vo);
        // lane t of an even row computes h for its row grp + 64 t
        float gv = 0.f, uv = 0.f;
#pragma unroll
        for (int u = 0; u < kW13; u++) {
          float ev = v[u], od = 0.f;
          swap16(ev, od);
          gv = t == u ? ev : gv;
          uv = t == u ? od : uv;
        }
        const int row = grp + 64 * t;
        if (t < kW13 && !(grp & 1) && row < HROWS) hb[row >> 1] = swiglu(gv, uv);
      }
      __syncthreads();
      // x += w2 * h
      {
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < kW2; u++) {
          const int c = t + 16 * u;
          if (c < HCH) acc = dot4(r.w2[u], reinterpret_cast<const f4 *>(hb)[c], acc);
        }
        const float v = row_total(acc);
        if (more) load_w2(r, a, nl, vo2);
        if (t == 0) xs[grp] = __fadd_rn(xs[grp], v);
      }
      __syncthreads();
    }

    const bool want = a.all || (a.last && j + 1 == a.n);
    if (want) {
      const float inv = rms_scale(xs);
      const f4 xn = rms_apply(reinterpret_cast<const f4 *>(xs)[t],
                              reinterpret_cast<const f4 *>(rmsw[2 * kTinyMaxLayers])[t], inv);
      f4 e[kHeadRows];
      const auto re = mat_rsrc(a.emb, a.vocab, D);
#pragma unroll
      for (int u = 0; u < kHeadRows; u++) e[u] = bload(re, vo, 16384u * u);
#pragma unroll
      for (int u = 0; u < kHeadRows; u++) {
        const int row = grp + 64 * u;
        const float v = row_total(dot4(e[u], xn, 0.f));
        if (t == 0 && row < a.vocab) lg[row] = v;
      }
      __syncthreads();
      float *out = a.out + (int64_t)(a.all ? j : 0) * a.vocab;
      for (int i = tid; i < a.vocab; i += kT) out[i] = lg[i];
    }
    __syncthreads();
  }
  wait_vmcnt<0>();  // no stream may land in LDS after the workgroup ends
}

}  // namespace

bool tiny_llama_supported(int dim, int hidden, int heads, int kv_heads, int layers, int vocab, int seq) {
  return dim == D && hidden == HID && heads == NH && kv_heads == NKV && layers >= 1 && layers <= kTinyMaxLayers &&
         vocab >= 1 && vocab <= kTinyMaxVocab && seq >= 1 && seq <= kTinyMaxSeq;
}

hipError_t launch_tiny_llama(const TinyLlamaArgs &a, hipStream_t st) {
  if (a.n < 1 || a.n > kTinyMaxTokens || a.layers < 1 || a.layers > kTinyMaxLayers || a.vocab < 1 ||
      a.vocab > kTinyMaxVocab || a.prefix < 0 || a.prefix + a.n > a.cap || a.cap > kTinyMaxSeq)
    return hipErrorInvalidValue;
  for (int j = 0; j < a.n; j++)
    if (a.tokens[j] < 0 || a.tokens[j] >= a.vocab) return hipErrorInvalidValue;
  TINYOAI_TIMED_LAUNCH(tiny_llama_kernel, dim3(1), dim3(kT), 0, st, a);
  return hipGetLastError();
}
