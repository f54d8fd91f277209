// Decode tokens of the stories260K-shaped legacy Llama (llama2.c: dim 64,
// 8 query / 4 kv heads of width 8, MLP 172, up to 8 layers and 512
// positions) in one launch: Model.transformer (model.go:407-481) for each
// token of a forward, from the embedding row to the classifier's logits.
//
// The model is about 1 MB of fp32 weights, so a token is bound by the
// latency of its dependent steps and by instruction issue, not by
// bandwidth; one kernel per step spends most of a token in launch gaps.
// Here one workgroup of 512 threads (8 waves, two per SIMD) runs every
// token of the call in order and keeps the activations in LDS:
//   per layer: RMSNorm (model.go:591-600) -> the fused [wq | wk | wv] rows
//   -> the adjacent-pair rotation (model.go:611-618), K/V stored at the
//   token's position -> attention over positions 0..pos (model.go:432-461,
//   softmax model.go:552-570) -> x += wo * att -> RMSNorm -> w1/w3 rows
//   (interleaved) and SwiGLU (model.go:463-470) -> x += w2 * h;
//   then the final RMSNorm and the tied classifier (model.go:476-479).
// Matrix rows: 16 lanes (one DPP row) per matrix row, 32 such groups; lane
// t holds chunk t (t + 16, t + 32 for w2) of each of its group's rows in
// registers. A layer's weights are loaded while the previous layer runs
// (a matrix's registers are refilled with the next layer's rows as soon as
// they have been used), and the layer's cached K/V stream into LDS (loads
// straight to LDS) while the previous layer's MLP runs, so only a call's
// first layer waits for memory. The 16 partial sums of a row are added
// with DPP lane moves in a fixed order (every lane of the row obtains the
// same bits). Rotation and SwiGLU pair rows 2j and 2j + 1, which sit in
// adjacent DPP rows of one wave (v_permlane16_swap).
// RMSNorm: every wave forms the float64 sum of float32 squares of x itself
// (no barrier), then ss / n + eps and 1 / float32(sqrt(.)) in float32.
// Attention: wave h is query head h; lane l holds positions l, l + 64, ...
// up to pos; scores, the wave's maximum, exp(s - m) weights, their sum and
// the weighted V, reduced across lanes with lane swaps and DPP moves, then
// out = o / l into LDS.
#include "kernels.h"

namespace {

constexpr int kT = 512, kG = kT / 16;  // threads; 16-lane row groups
constexpr int D = kTinyDim, HS = 8, NH = 8, NKV = 4, KVD = NKV * HS, QKV = D + 2 * KVD;
constexpr int HID = kTinyHidden, HROWS = 2 * HID, HCH = HID / 4;
static_assert(D == 64 && D / 4 == 16, "one 16-byte chunk of x per lane of a row group");
static_assert(NH == kT / 64, "one wave per query head");
static_assert(HID % 4 == 0 && HCH <= 48, "up to three 16-byte chunks of h per lane");
constexpr int kQkv = QKV / kG, kWo = D / kG;  // rows per group
constexpr int kW13 = (HROWS + kG - 1) / kG;
constexpr int kW2 = (HCH + 15) / 16;           // w2 chunks per lane and row
constexpr int kHeadRows = kTinyMaxVocab / kG;
constexpr int kMaxBlocks = kTinyMaxSeq / 64;   // attention positions per lane
// weight loads of a layer issued after its q/k/v rows (wo, w1/w3, w2)
constexpr int kAfterQkv = kWo + kW13 + kWo * kW2;
static_assert(kAfterQkv < 64, "vmcnt range");

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
  v = dpp_add<0xb1>(v);      // quad_perm [1, 0, 3, 2]
  v = dpp_add<0x4e>(v);      // quad_perm [2, 3, 0, 1]
  v = dpp_add<0x141>(v);     // row_half_mirror
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
  v = dpp_max<0x141>(v);
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
  const uint32_t x = r.x, y = r.y;
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
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

// A layer's weights in one lane's registers: row grp + 32 u of each matrix.
struct Regs {
  f4 qkv[kQkv], wo[kWo], w13[kW13], w2[kWo][kW2];
};

// 16 bytes at byte voff + soff of a buffer. (The range check covers voff
// only: every read here stays inside its buffer, the padded ones included.)
__device__ __forceinline__ f4 bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

// Lane offsets: vo = row grp, chunk t of a 64-column matrix (row grp + 32 u
// at + 8192 u); vo2 = row grp, chunk t of w2 (row grp + 32 u at + 22016 u,
// chunk t + 16 v at + 256 v). Reads past a matrix (w1/w3 rows 344-351, w2
// chunks 43-47) land in the next matrix or the padding; their products are
// never used.
__device__ __forceinline__ uint32_t layer_off(int l) { return (uint32_t)(l * kTinyLayerBytes); }
__device__ __forceinline__ void load_qkv(Regs &r, __amdgpu_buffer_rsrc_t rw, int l, uint32_t vo) {
#pragma unroll
  for (int u = 0; u < kQkv; u++) r.qkv[u] = bload(rw, vo, layer_off(l) + kTinyQkvOff + kG * D * 4 * u);
}
__device__ __forceinline__ void load_wo(Regs &r, __amdgpu_buffer_rsrc_t rw, int l, uint32_t vo) {
#pragma unroll
  for (int u = 0; u < kWo; u++) r.wo[u] = bload(rw, vo, layer_off(l) + kTinyWoOff + kG * D * 4 * u);
}
__device__ __forceinline__ void load_w13(Regs &r, __amdgpu_buffer_rsrc_t rw, int l, uint32_t vo) {
#pragma unroll
  for (int u = 0; u < kW13; u++) r.w13[u] = bload(rw, vo, layer_off(l) + kTinyW13Off + kG * D * 4 * u);
}
__device__ __forceinline__ void load_w2(Regs &r, __amdgpu_buffer_rsrc_t rw, int l, uint32_t vo2) {
#pragma unroll
  for (int u = 0; u < kWo; u++)
#pragma unroll
    for (int v = 0; v < kW2; v++)
      r.w2[u][v] = bload(rw, vo2, layer_off(l) + kTinyW2Off + kG * HID * 4 * u + 256 * v);
}

// K/V of positions [0, count) of layer l (every kv head) into LDS: kv head
// h's keys at kvs[h][p][8], values at kvs[NKV + h][p][8]. Streams of 1 KB
// (32 positions), spread over the waves; a stream reaching past a head's
// positions (at most into the buffer's padding) brings bytes that no lane
// reads.
__device__ __forceinline__ void kv_to_lds(const TinyLlamaArgs &a, __amdgpu_buffer_rsrc_t rkv, int l, int count,
                                          const float *kvs, int wave, int lane) {
  const int nch = (count + 31) / 32;
  const uint32_t head = (uint32_t)a.cap * HS * 4, kvsz = NKV * head;
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)kvs;
  for (int i = wave; i < 2 * NKV * nch; i += kT / 64) {
    const int stream = i % (2 * NKV), c = i / (2 * NKV);
    lds_dma16(rkv, (2 * l + stream / NKV) * kvsz + (stream % NKV) * head + c * 1024 + lane * 16,
              base + (uint32_t)((stream * kTinyMaxSeq + c * 32) * HS * 4));
  }
}

__global__ __launch_bounds__(kT) void tiny_llama_kernel(TinyLlamaArgs a) {
  __shared__ __align__(16) float kvs[2 * NKV * kTinyMaxSeq * HS];  // cached K/V of the layer
  __shared__ __align__(16) float xs[D];            // residual stream
  __shared__ __align__(16) float qkv[QKV];         // rotated q | k | v of the token
  __shared__ __align__(16) float att[D];           // attention output
  __shared__ __align__(16) float hb[HCH * 4 + 4];  // SwiGLU output
  __shared__ __align__(16) float rmsw[2 * kTinyMaxLayers + 1][D];
  __shared__ __align__(16) float lg[kTinyMaxVocab];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = tid >> 4, t = tid & 15;
  const int L = a.layers;

  // The first token's embedding value (lanes < 64) and rotary pair; later
  // tokens' are loaded during the previous token.
  const int jrow = (grp % HS) >> 1;
  float x_in = tid < D ? reinterpret_cast<const float *>(a.emb + (int64_t)a.tokens[0] * (D * 4))[tid] : 0.f;
  float2 cs_in = *reinterpret_cast<const float2 *>(a.rope + (int64_t)a.prefix * HS + 2 * jrow);
  for (int i = tid; i < L * D; i += kT) {
    rmsw[i / D][i % D] = a.rms_att[i];
    rmsw[kTinyMaxLayers + i / D][i % D] = a.rms_ffn[i];
  }
  if (tid < D) rmsw[2 * kTinyMaxLayers][tid] = a.rms_final[tid];

  const uint32_t vo = (uint32_t)grp * (D * 4) + 16 * t;
  const uint32_t vo2 = (uint32_t)grp * (HID * 4) + 16 * t;
  const auto rw = plane_rsrc(a.w, (int64_t)L * kTinyLayerBytes + kTinyPad);
  const int64_t kv_floats = (int64_t)NKV * a.cap * HS;  // one layer's K (or V)
  const auto rkv = plane_rsrc(reinterpret_cast<const uint8_t *>(a.kv), 2 * L * kv_floats * 4 + kTinyPad);
  Regs r;
  load_qkv(r, rw, 0, vo);
  kv_to_lds(a, rkv, 0, a.prefix, kvs, wave, lane);
  load_wo(r, rw, 0, vo);
  load_w13(r, rw, 0, vo);
  load_w2(r, rw, 0, vo2);
  const float scale = a.att_scale;
  const int kvh = wave / (NH / NKV);  // attention: query head `wave`

  for (int j = 0; j < a.n; j++) {
    const int pos = a.prefix + j;
    const float2 cs = cs_in;
    if (tid < D) xs[tid] = x_in;
    __syncthreads();

    for (int l = 0; l < L; l++) {
      const bool more = l + 1 < L || j + 1 < a.n;  // a layer follows in this launch
      const int nl = l + 1 < L ? l + 1 : 0;
      // RMSNorm, then q | k | v rows grp + 32 u; even groups keep the pair
      // (rows 2j, 2j + 1) and write it
      float kv0[2], kv1[2];  // rows >= 64 (u >= 2): the K or V pair to store
      {
        const float inv = rms_scale(xs);
        const f4 xn = rms_apply(reinterpret_cast<const f4 *>(xs)[t], reinterpret_cast<const f4 *>(rmsw[l])[t], inv);
#pragma unroll
        for (int u = 0; u < kQkv; u++) {
          const int row = grp + kG * u;
          float x0 = row_total(dot4(r.qkv[u], xn, 0.f)), x1 = 0.f;
          swap16(x0, x1);
          if (row < D + KVD) {
            const float e0 = x0, e1 = x1;
            x0 = __fsub_rn(__fmul_rn(e0, cs.x), __fmul_rn(e1, cs.y));
            x1 = __fadd_rn(__fmul_rn(e1, cs.x), __fmul_rn(e0, cs.y));
          }
          if (t == 0 && !(grp & 1)) *reinterpret_cast<float2 *>(qkv + row) = float2{x0, x1};
          if (u >= 2) {
            kv0[u - 2] = x0;
            kv1[u - 2] = x1;
          }
        }
      }
      // This wave's K/V streams into LDS have landed: they were issued
      // before this layer's wo, w1/w3 and w2 loads, and memory operations
      // complete in order.
      wait_vmcnt<kAfterQkv>();
      __syncthreads();
      if (t == 0 && !(grp & 1)) {  // storeKV at the token's position: K rows grp, grp + 1, V the same
#pragma unroll
        for (int u = 0; u < 2; u++)
          *reinterpret_cast<float2 *>(a.kv + (2 * l + u) * kv_floats + ((int64_t)(grp / HS) * a.cap + pos) * HS +
                                      grp % HS) = float2{kv0[u], kv1[u]};
      }
      // attention of query head `wave` over positions 0..pos
      {
        const f4 *q4 = reinterpret_cast<const f4 *>(qkv + wave * HS);
        const f4 q0 = q4[0], q1 = q4[1];
        const f4 zero = {0.f, 0.f, 0.f, 0.f};
        const int nb = pos / 64 + 1;  // position blocks
        float s[kMaxBlocks];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < kMaxBlocks; i++) {
          s[i] = -INFINITY;
          if (i < nb) {
            const int p = lane + 64 * i;
            const bool ok = p <= pos;
            const f4 *kp = reinterpret_cast<const f4 *>(p == pos ? qkv + D + kvh * HS
                                                                 : kvs + (kvh * kTinyMaxSeq + p) * HS);
            const f4 k0 = ok ? kp[0] : zero, k1 = ok ? kp[1] : zero;
            const float d = dot4(q1, k1, dot4(q0, k0, 0.f));
            s[i] = ok ? __fdiv_rn(d, scale) : -INFINITY;
            mx = fmaxf(mx, s[i]);
          }
        }
        // the wave's maximum: rows, then the four row maxima
        mx = row_max(mx);
        const float m =
            fmaxf(fmaxf(lane_value(mx, 0), lane_value(mx, 16)), fmaxf(lane_value(mx, 32), lane_value(mx, 48)));
        float o[HS], lsum = 0.f;
#pragma unroll
        for (int d = 0; d < HS; d++) o[d] = 0.f;
#pragma unroll
        for (int i = 0; i < kMaxBlocks; i++) {
          if (i < nb) {
            const int p = lane + 64 * i;
            const bool ok = p <= pos;
            const f4 *vp = reinterpret_cast<const f4 *>(p == pos ? qkv + D + KVD + kvh * HS
                                                                 : kvs + ((NKV + kvh) * kTinyMaxSeq + p) * HS);
            const f4 v0 = ok ? vp[0] : zero, v1 = ok ? vp[1] : zero;
            const float e = ok ? expf(s[i] - m) : 0.f;
            lsum += e;
#pragma unroll
            for (int d = 0; d < 4; d++) {
              o[d] = fmaf(e, v0[d], o[d]);
              o[d + 4] = fmaf(e, v1[d], o[d + 4]);
            }
          }
        }
        // o: lanes i and i + 32 (lanes < 32 keep dims 0-3, the rest 4-7),
        // then rows 2r and 2r + 1 (row r keeps dims 2r, 2r + 1), then the 16
        // lanes of a row; l: the same with zeros as partners, row 0 ends
        // with the total
#pragma unroll
        for (int d = 0; d < 4; d++) {
          swap32(o[d], o[d + 4]);
          o[d] += o[d + 4];
        }
#pragma unroll
        for (int d = 0; d < 2; d++) {
          swap16(o[d], o[d + 2]);
          o[d] = row_total(o[d] + o[d + 2]);
        }
        float lz = 0.f;
        swap32(lsum, lz);
        lsum = row_total(lsum + lz);
        lz = 0.f;
        swap16(lsum, lz);
        const float lt = lane_value(lsum + lz, 0);
        if ((lane & 15) == 0)
          *reinterpret_cast<float2 *>(att + wave * HS + 2 * (lane >> 4)) = float2{o[0] / lt, o[1] / lt};
      }
      // the next layer's K/V may replace this one's once every wave is past
      // its reads; a one-layer model's next token reads the position just
      // stored, so that store must have completed first
      if (L == 1) wait_vmcnt<0>();
      __syncthreads();
      if (more) {
        kv_to_lds(a, rkv, nl, l + 1 < L ? pos : pos + 1, kvs, wave, lane);
        load_qkv(r, rw, nl, vo);
        if (l + 1 == L) {  // the next token's inputs
          if (tid < D) x_in = reinterpret_cast<const float *>(a.emb + (int64_t)a.tokens[j + 1] * (D * 4))[tid];
          cs_in = *reinterpret_cast<const float2 *>(a.rope + (int64_t)(pos + 1) * HS + 2 * jrow);
        }
      }
      // x += wo * att
      {
        const f4 av = reinterpret_cast<const f4 *>(att)[t];
        float v[kWo];
#pragma unroll
        for (int u = 0; u < kWo; u++) v[u] = row_total(dot4(r.wo[u], av, 0.f));
        if (more) load_wo(r, rw, nl, vo);
        if (t == 0) {
#pragma unroll
          for (int u = 0; u < kWo; u++) xs[grp + kG * u] = __fadd_rn(xs[grp + kG * u], v[u]);
        }
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
        if (more) load_w13(r, rw, nl, vo);
        // lane t of an even group computes h for its row grp + 32 t
        float gv = 0.f, uv = 0.f;
#pragma unroll
        for (int u = 0; u < kW13; u++) {
          float ev = v[u], od = 0.f;
          swap16(ev, od);
          gv = t == u ? ev : gv;
          uv = t == u ? od : uv;
        }
        const int row = grp + kG * t;
        if (t < kW13 && !(grp & 1) && row < HROWS) hb[row >> 1] = swiglu(gv, uv);
      }
      __syncthreads();
      // x += w2 * h
      {
        f4 h4[kW2];
#pragma unroll
        for (int c = 0; c < kW2; c++)
          h4[c] = t + 16 * c < HCH ? reinterpret_cast<const f4 *>(hb)[t + 16 * c] : f4{0.f, 0.f, 0.f, 0.f};
        float v[kWo];
#pragma unroll
        for (int u = 0; u < kWo; u++) {
          float acc = 0.f;
#pragma unroll
          for (int c = 0; c < kW2; c++)
            if (t + 16 * c < HCH) acc = dot4(r.w2[u][c], h4[c], acc);
          v[u] = row_total(acc);
        }
        if (more) load_w2(r, rw, nl, vo2);
        if (t == 0) {
#pragma unroll
          for (int u = 0; u < kWo; u++) xs[grp + kG * u] = __fadd_rn(xs[grp + kG * u], v[u]);
        }
      }
      __syncthreads();
    }

    const bool want = a.all || (a.last && j + 1 == a.n);
    if (want) {
      const float inv = rms_scale(xs);
      const f4 xn = rms_apply(reinterpret_cast<const f4 *>(xs)[t],
                              reinterpret_cast<const f4 *>(rmsw[2 * kTinyMaxLayers])[t], inv);
      f4 e[kHeadRows];
      const auto re = plane_rsrc(a.emb, (int64_t)a.vocab * D * 4);  // rows past the vocabulary read as zeros
#pragma unroll
      for (int u = 0; u < kHeadRows; u++) e[u] = bload(re, vo + kG * D * 4 * u, 0);
#pragma unroll
      for (int u = 0; u < kHeadRows; u++) {
        const int row = grp + kG * u;
        const float v = row_total(dot4(e[u], xn, 0.f));
        if (t == 0 && row < a.vocab) lg[row] = v;
      }
      __syncthreads();
      float *out = a.out + (int64_t)(a.all ? j : 0) * a.vocab;
      for (int i = tid; i < a.vocab; i += kT) out[i] = lg[i];
    }
    __syncthreads();
  }
  if (a.done) {  // every thread's rows are visible system-wide before the word
    __threadfence_system();
    __syncthreads();
    if (tid == 0) __hip_atomic_store(a.done, a.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
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
