// The legacy Llama (llama2.c checkpoints) behind the llamaMLXForwarder
// contract (mlx_llama.go:27-35; nativeLlamaMLX.Forward,
// mlx_llama_native.go:119-175), computed by the decode kernels of the
// StableLM path: per layer RMSNorm + fused q/k/v rows with the adjacent-pair
// rotation and KV store in the epilogue, split-K attention, x += wo * att,
// RMSNorm + interleaved w1/w3 rows with SwiGLU in the epilogue, x += w2 * h
// (Model.transformer, model.go:407-481).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>

#include "kernels.h"
#include "model.h"

namespace tinyoai {

#define TRY_HIP(expr, what)                             \
  do {                                                  \
    hipError_t e_ = (expr);                             \
    if (e_ != hipSuccess) return hip_fail(e_, what);    \
  } while (0)

LlamaModel::~LlamaModel() {
  for (auto &g : graphs) hipGraphExecDestroy(g.second);
  if (kv_base) hipFree(kv_base);
  for (void *p : buffers) hipFree(p);
  if (h_pinned) hipHostFree(h_pinned);
  if (out_host) hipHostFree(out_host);
  if (done_host) hipHostFree(done_host);
  if (params_copied) hipEventDestroy(params_copied);
  if (stream) hipStreamDestroy(stream);
}

int LlamaModel::alloc(void **p, size_t bytes) {
  hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 256));
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  buffers.push_back(*p);
  return TINYOAI_OK;
}

static int grid_for(int units, int threads) {
  const int waves = threads / 64;
  return std::max(1, std::min(device_cu_count() * 2, (units + waves - 1) / waves));
}

// Weights in readWeights order (model.go:129-166): embeddings, rms_att,
// wq, wk, wv, wo, rms_ffn, w1, w2, w3, rms_final, freq_cis_real,
// freq_cis_imag.
int LlamaModel::init(const tinyoai_llama_config &c, const float *w, uint64_t n_floats) {
  cfg = c;
  if (c.dim <= 0 || c.hidden_dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
      c.vocab_size <= 0 || c.seq_len <= 0 || c.dim % c.n_heads || c.n_heads % c.n_kv_heads)
    return fail(TINYOAI_EINVAL, "invalid Llama dimensions");
  const int64_t dim = c.dim, hidden = c.hidden_dim, L = c.n_layers, vocab = c.vocab_size, seq = c.seq_len;
  const int hs = c.dim / c.n_heads, kv_dim = hs * c.n_kv_heads;
  if (hs % 2 || (hs != 8 && hs != 16 && hs != 32 && hs != 64 && hs != 80 && hs != 96 && hs != 128))
    return fail(TINYOAI_EINVAL, "head width %d is not supported by the attention kernels", hs);
  const uint64_t need = vocab * dim + L * dim + L * dim * dim + 2 * L * dim * kv_dim + L * dim * dim + L * dim +
                        3 * L * hidden * dim + dim + seq * hs;
  if (!w || n_floats != need)
    return fail(TINYOAI_EINVAL, "checkpoint holds %llu floats, the config needs %llu", (unsigned long long)n_floats,
                (unsigned long long)need);
  att = StableDims{c.dim, hs, hs, c.n_heads, c.n_kv_heads, c.hidden_dim, c.vocab_size, 1e-5,
                   (float)std::sqrt((double)hs), /*norm=*/1, /*rope_adjacent=*/1, /*silu=*/1, c.dim, kv_dim};
  mlp = att;
  mlp.win_q = mlp.win_kv = 0;  // every win row of the MLP half is a w1/w3 pair
  TRY_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");

  const float *p = w;
  const float *emb = p; p += vocab * dim;
  const float *rms_att = p; p += L * dim;
  const float *wq = p; p += L * dim * dim;
  const float *wk = p; p += L * dim * kv_dim;
  const float *wv = p; p += L * dim * kv_dim;
  const float *wo = p; p += L * dim * dim;
  const float *rms_ffn = p; p += L * dim;
  const float *w1 = p; p += L * hidden * dim;
  const float *w2 = p; p += L * dim * hidden;
  const float *w3 = p; p += L * hidden * dim;
  const float *rms_fin = p; p += dim;
  const float *fcr = p; p += seq * hs / 2;
  const float *fci = p;

  int rc;
  if ((rc = embed.upload(FMT_F32, vocab, dim, emb, vocab * dim * 4, stream))) return rc;
  auto vec = [&](const float *src, int64_t n, float **dst) -> int {
    int r = alloc((void **)dst, n * 4);
    if (r) return r;
    TRY_HIP(hipMemcpyAsync(*dst, src, n * 4, hipMemcpyHostToDevice, stream), "weight upload");
    return TINYOAI_OK;
  };
  float *rms_att_dev, *rms_ffn_dev;
  if ((rc = vec(rms_att, L * dim, &rms_att_dev)) || (rc = vec(rms_ffn, L * dim, &rms_ffn_dev)) ||
      (rc = vec(rms_fin, dim, &rms_final)))
    return rc;
  mats.resize(L * 4);
  att_layers.resize(L);
  mlp_layers.resize(L);
  const RowMap ident{ROWMAP_IDENTITY, 0, 0, 0, 0};
  for (int64_t l = 0; l < L; l++) {
    DevMatrix *m = &mats[l * 4];
    const uint64_t qb = dim * dim * 4, kb = (uint64_t)kv_dim * dim * 4, hb = hidden * dim * 4;
    if ((rc = m[0].create(FMT_F32, dim + 2 * kv_dim, dim, stream)) ||
        (rc = m[0].place(FMT_F32, dim, dim, wq + l * dim * dim, qb, ident, 0, stream)) ||
        (rc = m[0].place(FMT_F32, kv_dim, dim, wk + l * dim * kv_dim, kb, RowMap{ROWMAP_IDENTITY, dim, 0, 0, 0}, 0,
                         stream)) ||
        (rc = m[0].place(FMT_F32, kv_dim, dim, wv + l * dim * kv_dim, kb,
                         RowMap{ROWMAP_IDENTITY, dim + kv_dim, 0, 0, 0}, 0, stream)) ||
        (rc = m[1].upload(FMT_F32, dim, dim, wo + l * dim * dim, qb, stream)) ||
        (rc = m[2].create(FMT_F32, 2 * hidden, dim, stream)) ||
        (rc = m[2].place(FMT_F32, hidden, dim, w1 + l * hidden * dim, hb, RowMap{ROWMAP_INTERLEAVE, 0, 0, 0, 0}, 0,
                         stream)) ||
        (rc = m[2].place(FMT_F32, hidden, dim, w3 + l * hidden * dim, hb, RowMap{ROWMAP_INTERLEAVE, 0, 0, 0, 1}, 0,
                         stream)) ||
        (rc = m[3].upload(FMT_F32, dim, hidden, w2 + l * dim * hidden, hb, stream)))
      return rc;
    att_layers[l] = LayerDev{m[0].desc, m[1].desc, rms_att_dev + l * dim, nullptr};
    mlp_layers[l] = LayerDev{m[2].desc, m[3].desc, rms_ffn_dev + l * dim, nullptr};
  }
  // Rotation table [pos][hs/2][cos, sin] from the checkpoint's tables.
  std::vector<float> &rt = rope_host;
  rt.assign((size_t)seq * hs, 0.f);
  for (int64_t t = 0; t < seq; t++)
    for (int i = 0; i < hs / 2; i++) {
      rt[(size_t)t * hs + 2 * i] = fcr[t * (hs / 2) + i];
      rt[(size_t)t * hs + 2 * i + 1] = fci[t * (hs / 2) + i];
    }
  if ((rc = alloc((void **)&rope, rt.size() * 4))) return rc;
  TRY_HIP(hipMemcpyAsync(rope, rt.data(), rt.size() * 4, hipMemcpyHostToDevice, stream), "rope upload");
  // KV: the whole context, as runState's caches (model.go:379-398).
  // One buffer: per layer K, then V, then spare bytes for the one-launch
  // kernel's whole-chunk reads.
  kv.resize(L);
  {
    const size_t per = (size_t)kv_dim * seq * 4;
    if (hipMalloc(&kv_base, 2 * L * per + kTinyPad) != hipSuccess) return fail(TINYOAI_ENOMEM, "KV allocation");
    for (int64_t l = 0; l < L; l++) {
      kv[l].k = (uint8_t *)kv_base + 2 * l * per;
      kv[l].v = (uint8_t *)kv_base + (2 * l + 1) * per;
      kv[l].cap = (int)seq;
      kv[l].half = 0;
    }
  }
  max_splits = (int)(seq / 64 + 1);
  if ((rc = alloc((void **)&x, dim * 4)) || (rc = alloc((void **)&qbuf, dim * 4)) ||
      (rc = alloc((void **)&abuf, dim * 4)) || (rc = alloc((void **)&hbuf, hidden * 4)) ||
      (rc = alloc((void **)&params, 4096)) ||
      (rc = alloc((void **)&partials, (size_t)c.n_heads * partial_region(max_splits, hs) * 4)) ||
      (rc = alloc((void **)&counters, (size_t)c.n_heads * 4)) ||
      (rc = alloc((void **)&head_out, (size_t)vocab * 4)) || (rc = ensure_logits(1)))
    return rc;
  TRY_HIP(hipMemsetAsync(counters, 0, (size_t)c.n_heads * 4, stream), "counter init");
  TRY_HIP(hipEventCreateWithFlags(&params_copied, hipEventDisableTiming), "hipEventCreate");
  TRY_HIP(hipHostMalloc(&h_pinned, 4096, hipHostMallocDefault), "hipHostMalloc");
  TRY_HIP(hipStreamSynchronize(stream), "model upload");
  grid_in = grid_for((dim + 2 * kv_dim) / 2, 256);
  grid_mlp = grid_for(hidden, 256);
  grid_out = grid_for(dim, 256);
  grid_head = grid_for((vocab + 1) / 2, 256);
  // The one-launch kernel reads unpadded fp32 rows and a cache of seq_len
  // positions per kv head.
  tiny_ok = tiny_llama_supported(c.dim, c.hidden_dim, c.n_heads, c.n_kv_heads, c.n_layers, c.vocab_size, c.seq_len) &&
            embed.desc.vstride == dim * 4;
  for (int64_t l = 0; l < L && tiny_ok; l++) {
    const DevMatrix *m = &mats[l * 4];
    tiny_ok = m[0].desc.vstride == dim * 4 && m[1].desc.vstride == dim * 4 && m[2].desc.vstride == dim * 4 &&
              m[3].desc.vstride == hidden * 4 && kv[l].cap == seq;
  }
  if (tiny_ok) {  // the packed copy of every layer's matrices
    if ((rc = alloc((void **)&tiny_w, (size_t)L * kTinyLayerBytes + kTinyPad))) return rc;
    TRY_HIP(hipMemsetAsync(tiny_w + L * kTinyLayerBytes, 0, kTinyPad, stream), "packed weights");
    const int64_t off[4] = {kTinyQkvOff, kTinyWoOff, kTinyW13Off, kTinyW2Off};
    for (int64_t l = 0; l < L; l++)
      for (int k = 0; k < 4; k++) {
        const MatDesc &d = mats[l * 4 + k].desc;
        TRY_HIP(hipMemcpyAsync(tiny_w + l * kTinyLayerBytes + off[k], d.vals, (size_t)d.rows * d.vstride,
                               hipMemcpyDeviceToDevice, stream),
                "packed weights");
      }
    TRY_HIP(hipStreamSynchronize(stream), "packed weights");
  }
  tiny = tiny_ok;
  return TINYOAI_OK;
}

int LlamaModel::ensure_logits(int rows) {
  if (rows <= logits_rows) return TINYOAI_OK;
  float *p = nullptr;
  int rc = alloc((void **)&p, (size_t)rows * cfg.vocab_size * 4);
  if (rc) return rc;
  if (logits_dev) {
    hipStreamSynchronize(stream);
    buffers.erase(std::find(buffers.begin(), buffers.end(), (void *)logits_dev));
    hipFree(logits_dev);
  }
  logits_dev = p;
  logits_rows = rows;
  return TINYOAI_OK;
}

// One token; token and position come from `params`, the logits go to
// `logits` (device, null: none).
int LlamaModel::enqueue_step(int steps, int splits, float *logits) {
  const int *pos = params + 1;
  const float *rope_row = reinterpret_cast<const float *>(params + 16);
  for (int l = 0; l < cfg.n_layers; l++) {
    TRY_HIP(launch_decode_in(att_layers[l], att, kv[l], x, l == 0 ? &embed.desc : nullptr, params, rope_row, pos, qbuf,
                             hbuf, grid_in, 256, stream),
            "attention projections");
    TRY_HIP(launch_attention(att, kv[l], qbuf, pos, 1, 0, partials, counters, abuf, stream, steps, splits),
            "attention");
    TRY_HIP(launch_decode_out(att_layers[l].wout, cfg.dim, 0, abuf, nullptr, x, grid_out, 256, stream), "wo");
    TRY_HIP(launch_decode_in(mlp_layers[l], mlp, kv[l], x, nullptr, params, rope_row, pos, qbuf, hbuf, grid_mlp, 256,
                             stream),
            "w1/w3");
    TRY_HIP(launch_decode_out(mlp_layers[l].wout, cfg.hidden_dim, 0, hbuf, nullptr, x, grid_out, 256, stream), "w2");
  }
  if (logits)
    TRY_HIP(launch_ln_matvec(embed.desc, rms_final, nullptr, 1e-5, 1, x, logits, grid_head, 256, stream),
            "classifier");
  return TINYOAI_OK;
}

// transformer(token, pos) (model.go:407-481) from a HIP graph keyed by the
// attention launch shape and the logits row.
int LlamaModel::step(int token, int pos, float *logits) {
  int *hp = (int *)h_pinned;
  TRY_HIP(hipEventSynchronize(params_copied), "parameter slot");
  hp[0] = token;
  hp[1] = pos;
  memcpy(hp + 16, rope_host.data() + (size_t)pos * att.rot, (size_t)att.rot * 4);  // the token's rotary row
  TRY_HIP(hipMemcpyAsync(params, hp, (size_t)(16 + att.rot) * 4, hipMemcpyHostToDevice, stream), "parameters");
  TRY_HIP(hipEventRecord(params_copied, stream), "parameter event");
  const int steps = attention_steps(pos, att.heads), splits = attention_splits(pos, steps);
  const int64_t key = ((int64_t)steps << 40) | ((int64_t)splits << 8) | (logits ? 1 : 0);
  auto it = graphs.find(key);
  if (it == graphs.end()) {
    hipGraph_t g = nullptr;
    TRY_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "graph capture");
    int rc = enqueue_step(steps, splits, logits);
    hipError_t e = hipStreamEndCapture(stream, &g);
    if (rc) {
      if (g) hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "graph capture");
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "graph instantiate");
    it = graphs.emplace(key, exec).first;
  }
  TRY_HIP(hipGraphLaunch(it->second, stream), "graph launch");
  return TINYOAI_OK;
}

// Row j of the logits returned by a forward; the graphs write the head's
// output to head_out, which is copied to its row.
static float *row_of(float *base, int j, int vocab) { return base + (size_t)j * vocab; }

// nativeLlamaMLX.Forward (mlx_llama_native.go:119-175): replace the suffix
// after prefix with tokens; all rows of logits or the last one.
int LlamaModel::forward(int prefix, const int32_t *tokens, int n, bool all_logits, float *logits) {
  if (prefix < 0 || prefix > offset || n <= 0 || !tokens || prefix + n > cfg.seq_len)
    return fail(TINYOAI_EINVAL, "invalid Llama prefix or context length");
  if (!logits) return fail(TINYOAI_EINVAL, "logits output is required");
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= cfg.vocab_size) return fail(TINYOAI_EINVAL, "invalid token %d", tokens[i]);
  offset = prefix;
  if (tiny) {
    const int rc = forward_tiny(prefix, tokens, n, all_logits, logits);
    if (rc) {
      hipStreamSynchronize(stream);
      offset = 0;  // native errors reset KV (mlx_llama_native.go:170-172)
      return rc;
    }
    offset = prefix + n;
    return TINYOAI_OK;
  }
  const int rows = all_logits ? n : 1;
  int rc = ensure_logits(rows);
  for (int j = 0; j < n && !rc; j++) {
    const bool want = all_logits || j == n - 1;
    rc = step(tokens[j], prefix + j, want ? head_out : nullptr);
    if (!rc && want) {
      const hipError_t e = hipMemcpyAsync(row_of(logits_dev, all_logits ? j : 0, cfg.vocab_size), head_out,
                                          (size_t)cfg.vocab_size * 4, hipMemcpyDeviceToDevice, stream);
      if (e != hipSuccess) rc = hip_fail(e, "logits row");
    }
  }
  if (!rc) {
    hipError_t e = hipMemcpyAsync(logits, logits_dev, (size_t)rows * cfg.vocab_size * 4, hipMemcpyDeviceToHost,
                                  stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) rc = hip_fail(e, "logits");
  }
  if (rc) {
    hipStreamSynchronize(stream);
    offset = 0;  // native errors reset KV (mlx_llama_native.go:170-172)
    return rc;
  }
  offset = prefix + n;
  return TINYOAI_OK;
}

constexpr int kTinySpinMs = 200;  // host wait for the completion word before waiting on the stream

// forward for the stories260K shape: one launch per kTinyMaxTokens tokens
// (every token of the call in one workgroup, in order), the logits rows
// written by the kernel into mapped pinned host memory.
int LlamaModel::forward_tiny(int prefix, const int32_t *tokens, int n, bool all_logits, float *logits) {
  const int rows = all_logits ? n : 1, vocab = cfg.vocab_size;
  if (!done_host) {
    void *h = nullptr;
    hipError_t e = hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent);
    if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipHostMalloc: %s", hipGetErrorString(e));
    done_host = (unsigned *)h;
    *done_host = 0;
    e = hipHostGetDevicePointer((void **)&done_dev, h, 0);
    if (e != hipSuccess) return hip_fail(e, "mapped completion word");
  }
  if (rows > out_rows) {
    if (out_host) {
      TRY_HIP(hipStreamSynchronize(stream), "logits rows");
      hipHostFree(out_host);
      out_host = out_dev = nullptr;
      out_rows = 0;
    }
    void *h = nullptr;
    hipError_t e = hipHostMalloc(&h, (size_t)rows * vocab * 4, hipHostMallocMapped | hipHostMallocCoherent);
    if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipHostMalloc: %s", hipGetErrorString(e));
    out_host = (float *)h;
    e = hipHostGetDevicePointer((void **)&out_dev, h, 0);
    if (e != hipSuccess) return hip_fail(e, "mapped logits rows");
    out_rows = rows;
  }
  TinyLlamaArgs a{};
  a.w = tiny_w;
  a.kv = (float *)kv_base;
  a.emb = embed.desc.vals;
  a.rms_att = att_layers[0].ln_w;
  a.rms_ffn = mlp_layers[0].ln_w;
  a.rms_final = rms_final;
  a.rope = rope;
  a.att_scale = att.att_scale;
  a.layers = cfg.n_layers;
  a.vocab = vocab;
  a.cap = cfg.seq_len;
  for (int c0 = 0; c0 < n; c0 += kTinyMaxTokens) {
    const int cnt = std::min(kTinyMaxTokens, n - c0);
    a.prefix = prefix + c0;
    a.n = cnt;
    a.all = all_logits;
    a.last = !all_logits && c0 + cnt == n;
    a.out = out_dev + (all_logits ? (size_t)c0 * vocab : 0);
    const bool final = c0 + cnt == n;
    a.done = final ? done_dev : nullptr;
    a.seq = ++done_seq;
    std::memcpy(a.tokens, tokens + c0, (size_t)cnt * 4);
    TRY_HIP(launch_tiny_llama(a, stream), "token launch");
  }
  // The last launch sets the completion word after its rows: the rows are
  // read as soon as it appears (the stream's own completion comes later).
  // Past the time limit, or if the word never comes, the stream is waited
  // for, which also reports a failed launch.
  const auto t0 = std::chrono::steady_clock::now();
  bool seen = false;
  for (int spin = 0; !seen; spin++) {
    seen = __atomic_load_n(done_host, __ATOMIC_ACQUIRE) == done_seq;
    if (!seen && (spin & 1023) == 1023 &&
        std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(kTinySpinMs))
      break;
  }
  if (!seen) TRY_HIP(hipStreamSynchronize(stream), "logits");
  if (!seen && __atomic_load_n(done_host, __ATOMIC_ACQUIRE) != done_seq)
    return fail(TINYOAI_EDEVICE, "the token launch ended without its completion word");
  std::memcpy(logits, out_host, (size_t)rows * vocab * 4);
  return TINYOAI_OK;
}

}  // namespace tinyoai

using namespace tinyoai;

extern "C" {

int tinyoai_llama_load(const tinyoai_llama_config *config, const float *weights, uint64_t n_floats,
                       tinyoai_model **out) {
  if (!config || !weights || !out) return fail(TINYOAI_EINVAL, "invalid load arguments");
  *out = nullptr;
  auto h = std::make_unique<tinyoai_model>();
  h->llama = std::make_unique<LlamaModel>();
  int rc = h->llama->init(*config, weights, n_floats);
  if (rc) return rc;
  *out = h.release();
  return TINYOAI_OK;
}

int tinyoai_llama_forward(tinyoai_model *m, int32_t prefix, const int32_t *tokens, int32_t n, int32_t all_logits,
                          float *logits) {
  if (!m || !m->llama) return fail(TINYOAI_EINVAL, "not a Llama handle");
  return m->llama->forward(prefix, tokens, n, all_logits != 0, logits);
}

int tinyoai_llama_reset(tinyoai_model *m) {
  if (!m || !m->llama) return fail(TINYOAI_EINVAL, "not a Llama handle");
  hipStreamSynchronize(m->llama->stream);
  m->llama->offset = 0;
  return TINYOAI_OK;
}

int tinyoai_llama_set_launch(tinyoai_model *m, int32_t stage, int32_t value) {
  if (!m || !m->llama) return fail(TINYOAI_EINVAL, "not a Llama handle");
  LlamaModel &l = *m->llama;
  if (stage != 0) return fail(TINYOAI_EINVAL, "unknown Llama launch stage %d", stage);
  if (value && !l.tiny_ok) return fail(TINYOAI_EINVAL, "the one-launch kernel does not fit this model's shape");
  hipStreamSynchronize(l.stream);
  l.tiny = value != 0;
  return TINYOAI_OK;
}

int tinyoai_llama_close(tinyoai_model *m) {
  if (!m) return TINYOAI_OK;
  if (m->llama) hipStreamSynchronize(m->llama->stream);
  delete m;
  return TINYOAI_OK;
}

}  // extern "C"
