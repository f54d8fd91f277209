// C ABI of the gfx950 backend: weight upload, the StableLM forwarder and the
// single-matrix entry points. The forward orchestration follows
// StableLM.forward (stablelm.go:332-387) for one token and StableLM.prefill
// (prefill.go:33-115) for longer suffixes, with the resident-prefix
// semantics of nativeMLX.forward (mlx_native.go:324-495).
#include "tinyoai_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.h"
#include "model.h"

LaunchTiming &launch_timing() {
  thread_local LaunchTiming t;
  return t;
}

namespace tinyoai {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(TINYOAI_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

// ---------------------------------------------------------------- matrices
int64_t gguf_bytes(int32_t dtype, int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  switch (dtype) {
    case FMT_F32: return n * 4;
    case FMT_F16: case FMT_BF16: return n * 2;
    case FMT_Q8_0: return cols % 32 ? -1 : n / 32 * 34;
    case FMT_Q5_1: return cols % 32 ? -1 : n / 32 * 24;
    case FMT_Q4_K: return cols % 256 ? -1 : n / 256 * 144;
    case FMT_Q5_K: return cols % 256 ? -1 : n / 256 * 176;
    case FMT_Q6_K: return cols % 256 ? -1 : n / 256 * 210;
  }
  return -1;
}

// 5/6-bit GGUF blocks -> the chunk planes of formats.h for one row: per
// chunk of 32 values the 4-bit low parts (byte b: values b and b + 16),
// the high bits, and each block's header bytes. Follows the bit layout of
// decodeKBlock (quant_k.go:31-86); Q4_K is laid out as Q5_K without qh.
static void kquant_repack_row(int fmt, const uint8_t *raw, int64_t cols, uint8_t *vals, uint8_t *meta,
                              uint8_t *hbits) {
  const int64_t chunks = cols / 32;
  for (int64_t c = 0; c < chunks; c++) {
    int q[32];
    if (fmt == FMT_Q5_1) {
      const uint8_t *b = raw + c * 24;
      uint32_t high;
      memcpy(&high, b + 4, 4);
      for (int i = 0; i < 32; i++) q[i] = ((b[8 + i % 16] >> (i / 16 * 4)) & 15) | ((high >> i) & 1) << 4;
      memcpy(meta + c * 4, b, 4);
    } else if (fmt == FMT_Q6_K) {
      const uint8_t *b = raw + (c / 8) * 210;
      for (int t = 0; t < 32; t++) {
        const int i = (int)(c % 8) * 32 + t;
        const int low = (b[(i / 128) * 64 + i % 64] >> ((i % 128) / 64 * 4)) & 15;
        const int high = (b[128 + (i / 128) * 32 + i % 32] >> ((i % 128) / 32 * 2)) & 3;
        q[t] = low | high << 4;
      }
      if (c % 8 == 0) {
        memset(meta + (c / 8) * 32, 0, 32);
        memcpy(meta + (c / 8) * 32, b + 192, 16);
        memcpy(meta + (c / 8) * 32 + 16, b + 208, 2);
      }
    } else {  // Q4_K / Q5_K
      const bool q5 = fmt == FMT_Q5_K;
      const uint8_t *b = raw + (c / 8) * (q5 ? 176 : 144);
      const int g = (int)(c % 8);
      for (int j = 0; j < 32; j++) {
        const int low = (b[(q5 ? 48 : 16) + (g / 2) * 32 + j] >> (g % 2 * 4)) & 15;
        const int high = q5 ? (b[16 + j] >> g) & 1 : 0;
        q[j] = low | high << 4;
      }
      if (g == 0) memcpy(meta + (c / 8) * 16, b, 16);
    }
    for (int i = 0; i < 16; i++) vals[c * 16 + i] = (uint8_t)((q[i] & 15) | (q[i + 16] & 15) << 4);
    if (fmt == FMT_Q5_1 || fmt == FMT_Q5_K) {
      uint32_t h = 0;
      for (int i = 0; i < 32; i++) h |= (uint32_t)((q[i] >> 4) & 1) << i;
      memcpy(hbits + c * 4, &h, 4);
    } else if (fmt == FMT_Q6_K) {
      uint64_t h = 0;
      for (int i = 0; i < 32; i++) h |= (uint64_t)((q[i] >> 4) & 3) << (2 * i);
      memcpy(hbits + c * 8, &h, 8);
    }
  }
}

DevMatrix::~DevMatrix() {
  if (mem) hipFree(mem);
}

static int64_t value_width(int32_t dtype) { return dtype == FMT_F32 ? 4 : (dtype == FMT_Q8_0 ? 1 : 2); }

int DevMatrix::create(int32_t dtype, int64_t rows, int64_t cols, hipStream_t st) {
  if (rows <= 0 || cols <= 0 || rows > INT32_MAX || cols > INT32_MAX)
    return fail(TINYOAI_EINVAL, "invalid matrix shape [%lld, %lld]", (long long)rows, (long long)cols);
  if (dtype != FMT_F32 && dtype != FMT_F16 && dtype != FMT_BF16 && dtype != FMT_Q8_0 && !is_kquant(dtype))
    return fail(TINYOAI_EINVAL, "unsupported tensor type %d", dtype);
  if (gguf_bytes(dtype, 1, cols) < 0)
    return fail(TINYOAI_EINVAL, "rows of type %d must hold whole quant blocks (%lld values)", dtype, (long long)cols);
  MatDesc m{};
  m.fmt = dtype;
  m.rows = (int32_t)rows;
  m.cols = (int32_t)cols;
  const int64_t chunks = is_kquant(dtype) ? cols / 32 : (cols * value_width(dtype) + 15) / 16;
  m.vstride = chunks * 16;
  m.chunks = (int32_t)chunks;
  m.mstride = meta_offset(dtype, chunks);
  m.hstride = hbits_offset(dtype, chunks);
  auto round256 = [](size_t v) { return (v + 255) / 256 * 256; };
  const size_t vbytes = round256((size_t)(m.vstride * rows)), mbytes = round256((size_t)(m.mstride * rows));
  const size_t hbytes = round256((size_t)(m.hstride * rows));
  const size_t total = vbytes + mbytes + hbytes + 256;
  hipError_t e = hipMalloc(&mem, total);
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipMalloc(%zu): %s", total, hipGetErrorString(e));
  bytes = total;
  e = hipMemsetAsync(mem, 0, total, st);  // row padding reads as zeros
  if (e != hipSuccess) return hip_fail(e, "weight init");
  m.vals = (const uint8_t *)mem;
  m.meta = (const uint8_t *)mem + vbytes;
  m.hbits = (const uint8_t *)mem + vbytes + mbytes;
  desc = m;
  return TINYOAI_OK;
}

int DevMatrix::place(int32_t dtype, int64_t rows, int64_t cols, const void *data, uint64_t nbytes, const RowMap &map,
                     int64_t col0, hipStream_t st) {
  const MatDesc &m = desc;
  if (!mem || dtype != m.fmt) return fail(TINYOAI_EINVAL, "tensor type %d does not match its matrix (%d)", dtype, m.fmt);
  const int64_t want = gguf_bytes(dtype, rows, cols);
  if (want < 0 || rows <= 0) return fail(TINYOAI_EINVAL, "invalid tensor shape [%lld, %lld]", (long long)rows, (long long)cols);
  if ((int64_t)nbytes != want)
    return fail(TINYOAI_EINVAL, "tensor [%lld, %lld] of type %d needs %lld bytes, got %llu", (long long)rows,
                (long long)cols, dtype, (long long)want, (unsigned long long)nbytes);
  // Every destination row and byte must fall inside the matrix.
  int64_t last_row;
  switch (map.kind) {
    case ROWMAP_HEADS:
      if (map.hd <= 0 || rows % map.hd || map.rot < 0 || map.rot % 2 || map.rot > map.hd)
        return fail(TINYOAI_EINVAL, "invalid head row map");
      last_row = map.offset + rows - 1;
      break;
    case ROWMAP_INTERLEAVE: last_row = map.offset + 2 * (rows - 1) + map.phase; break;
    default: last_row = map.offset + rows - 1;
  }
  const int64_t blk = dtype == FMT_Q8_0 || dtype == FMT_Q5_1 ? 32 : (is_kquant(dtype) ? 256 : 1);
  const int64_t used = is_kquant(dtype) ? (col0 + cols) / 32 * 16 : (col0 + cols) * value_width(dtype);
  if (map.offset < 0 || last_row >= m.rows || col0 < 0 || col0 % blk || used > m.vstride ||
      (dtype == FMT_Q8_0 && (col0 + cols) / 32 * 2 > m.mstride))
    return fail(TINYOAI_EINVAL, "tensor [%lld, %lld] does not fit its place in a [%d, %d] matrix", (long long)rows,
                (long long)cols, m.rows, m.cols);
  const int64_t width = value_width(dtype);
  hipError_t e;
  if (is_kquant(dtype)) {
    // Repack on the host into the tensor's own planes, then place each
    // plane's rows on the device.
    const int64_t chunks = cols / 32, c0 = col0 / 32;
    const int64_t vb = chunks * 16, mb = meta_offset(dtype, chunks), hb = hbits_offset(dtype, chunks);
    const int64_t raw_row = gguf_bytes(dtype, 1, cols);
    std::vector<uint8_t> host((size_t)(rows * (vb + mb + hb)));
    uint8_t *hv = host.data(), *hm = hv + rows * vb, *hh = hm + rows * mb;
    for (int64_t r = 0; r < rows; r++)
      kquant_repack_row(dtype, (const uint8_t *)data + r * raw_row, cols, hv + r * vb, hm + r * mb, hh + r * hb);
    void *dev = nullptr;
    e = hipMalloc(&dev, host.size());
    if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipMalloc(%zu): %s", host.size(), hipGetErrorString(e));
    const uint8_t *dv = (const uint8_t *)dev, *dm = dv + rows * vb, *dh = dm + rows * mb;
    e = hipMemcpyAsync(dev, host.data(), host.size(), hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
      e = launch_place_bytes(dv, rows, vb, (uint8_t *)m.vals, m.vstride, c0 * 16, map, st);
    if (e == hipSuccess && mb)
      e = launch_place_bytes(dm, rows, mb, (uint8_t *)m.meta, m.mstride, meta_offset(dtype, c0), map, st);
    if (e == hipSuccess && hb)
      e = launch_place_bytes(dh, rows, hb, (uint8_t *)m.hbits, m.hstride, hbits_offset(dtype, c0), map, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    hipFree(dev);
    return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "weight repack");
  }
  if (dtype != FMT_Q8_0 && map.kind == ROWMAP_IDENTITY && col0 == 0 && m.vstride == cols * width) {
    e = hipMemcpyAsync((uint8_t *)mem + map.offset * m.vstride, data, nbytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "weight upload");
  }
  void *raw = nullptr;
  e = hipMalloc(&raw, nbytes);
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipMalloc(%llu): %s", (unsigned long long)nbytes, hipGetErrorString(e));
  e = hipMemcpyAsync(raw, data, nbytes, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = launch_repack(dtype, (const uint8_t *)raw, rows, cols, m, map, col0, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  hipFree(raw);
  return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "weight repack");
}

int DevMatrix::upload(int32_t dtype, int64_t rows, int64_t cols, const void *data, uint64_t nbytes, hipStream_t st) {
  const int64_t want = gguf_bytes(dtype, rows, cols);
  if (want >= 0 && (int64_t)nbytes != want)
    return fail(TINYOAI_EINVAL, "tensor [%lld, %lld] of type %d needs %lld bytes, got %llu", (long long)rows,
                (long long)cols, dtype, (long long)want, (unsigned long long)nbytes);
  int rc = create(dtype, rows, cols, st);
  return rc ? rc : place(dtype, rows, cols, data, nbytes, RowMap{ROWMAP_IDENTITY, 0, 0, 0, 0}, 0, st);
}

MatDesc column_view(const MatDesc &m, int64_t col0, int64_t cols) {
  MatDesc v = m;
  if (is_kquant(m.fmt)) {
    const RowPtr r = row_ptr(m, 0, col0 / 32);
    v.vals = r.v;
    v.meta = r.m;
    v.hbits = r.h;
    v.chunks = (int32_t)(cols / 32);
  } else {
    const int64_t width = value_width(m.fmt);
    v.vals = m.vals + col0 * width;
    v.meta = m.fmt == FMT_Q8_0 ? m.meta + col0 / 32 * 2 : m.meta;
    v.chunks = (int32_t)((cols * width + 15) / 16);
  }
  v.cols = (int32_t)cols;
  return v;
}

// ---------------------------------------------------------------- profiling
Profiler::~Profiler() {
  for (hipEvent_t e : pool) hipEventDestroy(e);
}

hipEvent_t Profiler::next() {
  if (used == pool.size()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    pool.push_back(e);
  }
  return pool[used++];
}

// begin records event i on the stream and offers events i + 1, i + 2 to
// the launch; end records event i + 3 and keeps the dispatch's pair when
// the launch took it.
void Profiler::begin(int stage, hipStream_t st) {
  if (!on) return;
  const size_t i = used;
  hipEvent_t e0 = next(), e1 = next(), e2 = next();
  if (!e0 || !e1 || !e2) return;
  hipEventRecord(e0, st);
  marks.push_back(Mark{stage, i, i});
  launch_timing() = LaunchTiming{e1, e2, false};
}

void Profiler::end(hipStream_t st) {
  if (!on || marks.empty()) return;
  LaunchTiming &lt = launch_timing();
  Mark &m = marks.back();
  const size_t i = m.a;
  if (lt.used) {
    m.a = i + 1;
    m.b = i + 2;
  } else {
    hipEvent_t e3 = next();
    if (e3) hipEventRecord(e3, st);
    m.b = used - 1;
  }
  lt = LaunchTiming{};
}

// Called after the stream has synchronized.
void Profiler::resolve() {
  for (auto &m : marks) {
    float t = 0;
    if (m.b > m.a && m.b < used && hipEventElapsedTime(&t, pool[m.a], pool[m.b]) == hipSuccess) {
      ms[m.stage] += t;
      count[m.stage]++;
    }
  }
  marks.clear();
  used = 0;
}

void Profiler::clear() {
  for (int i = 0; i < ST_COUNT; i++) { ms[i] = 0; count[i] = 0; }
}

// ---------------------------------------------------------------- StableLM
StableModel::~StableModel() {
  free_kv();
  for (void *p : buffers) hipFree(p);
  if (h_pinned) hipHostFree(h_pinned);
  if (h_io) hipHostFree(h_io);
  if (score_mem) hipFree(score_mem);
  if (params_copied) hipEventDestroy(params_copied);
  if (stream) hipStreamDestroy(stream);
}

int StableModel::alloc(void **p, size_t bytes) {
  hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 256));
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  buffers.push_back(*p);
  return TINYOAI_OK;
}

// Graphs bake in the KV pointers, so they go with the buffers.
void StableModel::free_kv() {
  drop_graphs();
  for (auto &l : kv) {
    if (l.k) hipFree(l.k);
    if (l.v) hipFree(l.v);
  }
  kv.clear();
  cap = 0;
  offset = 0;
}

// RoPE table with stableRotate's arithmetic (stablelm.go:311-318): float32
// frequency and angle, float64 sincos rounded to float32.
static std::vector<float> rope_table(int max_pos, int rot, double theta) {
  std::vector<float> t((size_t)max_pos * (rot / 2) * 2);
  for (int i = 0; i < rot / 2; i++) {
    const float expo = (float)(2 * i) / (float)rot;
    const float power = (float)std::pow((double)(float)theta, (double)expo);
    const float inv = 1.0f / power;
    for (int p = 0; p < max_pos; p++) {
      const float angle = (float)p * inv;
      t[((size_t)p * (rot / 2) + i) * 2] = (float)std::cos((double)angle);
      t[((size_t)p * (rot / 2) + i) * 2 + 1] = (float)std::sin((double)angle);
    }
  }
  return t;
}

int StableModel::init(const tinyoai_stablelm_config &c, const tinyoai_tensor *tensors, int n) {
  cfg = c;
  if (c.hidden_size <= 0 || c.intermediate_size <= 0 || c.num_hidden_layers <= 0 || c.num_attention_heads <= 0 ||
      c.num_key_value_heads <= 0 || c.vocab_size <= 0 || c.max_position_embeddings <= 0 ||
      c.hidden_size % c.num_attention_heads || c.num_attention_heads % c.num_key_value_heads)
    return fail(TINYOAI_EINVAL, "invalid StableLM dimensions");
  const int hd = c.hidden_size / c.num_attention_heads;
  const double rotary = hd * c.partial_rotary_factor;
  if (!(c.layer_norm_eps > 0) || !(c.rope_theta > 0) || !(c.partial_rotary_factor > 0) ||
      c.partial_rotary_factor > 1 || rotary != std::trunc(rotary) || (int)rotary % 2 || rotary < 2)
    return fail(TINYOAI_EINVAL, "invalid LayerNorm or partial RoPE settings");
  if (hd % 2 || (hd != 8 && hd != 16 && hd != 32 && hd != 64 && hd != 80 && hd != 96 && hd != 128))
    return fail(TINYOAI_EINVAL, "head width %d is not supported by the attention kernels", hd);
  dims = StableDims{c.hidden_size, hd, (int)rotary, c.num_attention_heads, c.num_key_value_heads,
                    c.intermediate_size, c.vocab_size, c.layer_norm_eps, (float)std::sqrt((double)hd),
                    /*norm=*/0, /*rope_adjacent=*/0, /*silu=*/0, c.hidden_size, hd * c.num_key_value_heads};
  hipError_t e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");

  std::map<std::string, const tinyoai_tensor *> by_name;
  for (int i = 0; i < n; i++) {
    if (!tensors[i].name) return fail(TINYOAI_EINVAL, "tensor %d has no name", i);
    if (!by_name.emplace(tensors[i].name, &tensors[i]).second)
      return fail(TINYOAI_EINVAL, "duplicate tensor %s", tensors[i].name);
  }
  const int d = c.hidden_size, I = c.intermediate_size, kvw = hd * c.num_key_value_heads;
  auto load = [&](const std::string &name, int64_t rows, int64_t cols, DevMatrix &dst) -> int {
    auto it = by_name.find(name);
    if (it == by_name.end()) return fail(TINYOAI_EINVAL, "missing tensor %s", name.c_str());
    const tinyoai_tensor *t = it->second;
    if (t->rows != rows || t->cols != cols)
      return fail(TINYOAI_EINVAL, "tensor %s: shape [%lld %lld], want [%lld %lld]", name.c_str(), (long long)t->rows,
                  (long long)t->cols, (long long)rows, (long long)cols);
    int rc = dst.upload(t->dtype, rows, cols, t->data, t->nbytes, stream);
    if (rc) g_error = "tensor " + name + ": " + g_error;
    return rc;
  };
  // Norm vectors are kept as fp32 (weight.at(i) of any dtype, stablelm.go:303).
  auto load_vec = [&](const std::string &name, const float **dst) -> int {
    DevMatrix tmp;
    int rc = load(name, 1, d, tmp);
    if (rc) return rc;
    float *out;
    if ((rc = alloc((void **)&out, (size_t)d * 4))) return rc;
    hipError_t e2 = launch_read_values(tmp.desc, 0, d, out, stream);
    if (e2 == hipSuccess) e2 = hipStreamSynchronize(stream);
    if (e2 != hipSuccess) return hip_fail(e2, "norm upload");
    *dst = out;
    return TINYOAI_OK;
  };
  int rc;
  if ((rc = load("model.embed_tokens.weight", c.vocab_size, d, embed))) return rc;
  if ((rc = load("lm_head.weight", c.vocab_size, d, head))) return rc;
  if ((rc = load_vec("model.norm.weight", &norm_w))) return rc;
  if ((rc = load_vec("model.norm.bias", &norm_b))) return rc;
  mats.resize((size_t)c.num_hidden_layers * 4);
  layers.resize(c.num_hidden_layers);
  win_rows = d + 2 * kvw + 2 * I;
  auto find = [&](const std::string &name, int64_t rows, int64_t cols, const tinyoai_tensor **t) -> int {
    auto it = by_name.find(name);
    if (it == by_name.end()) return fail(TINYOAI_EINVAL, "missing tensor %s", name.c_str());
    *t = it->second;
    if ((*t)->rows != rows || (*t)->cols != cols)
      return fail(TINYOAI_EINVAL, "tensor %s: shape [%lld %lld], want [%lld %lld]", name.c_str(),
                  (long long)(*t)->rows, (long long)(*t)->cols, (long long)rows, (long long)cols);
    return TINYOAI_OK;
  };
  auto place = [&](DevMatrix &dst, const std::string &name, const tinyoai_tensor *t, const RowMap &map,
                   int64_t col0) -> int {
    int rc2 = dst.place(t->dtype, t->rows, t->cols, t->data, t->nbytes, map, col0, stream);
    if (rc2) g_error = "tensor " + name + ": " + g_error;
    return rc2;
  };
  for (int l = 0; l < c.num_hidden_layers; l++) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    static const char *names[7] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                   "self_attn.o_proj.weight", "mlp.gate_proj.weight",    "mlp.up_proj.weight",
                                   "mlp.down_proj.weight"};
    const int64_t shape[7][2] = {{d, d}, {kvw, d}, {kvw, d}, {d, d}, {I, d}, {I, d}, {d, I}};
    const tinyoai_tensor *t[7];
    for (int i = 0; i < 7; i++)
      if ((rc = find(p + names[i], shape[i][0], shape[i][1], &t[i]))) return rc;
    const int32_t fin = t[0]->dtype, fmlp = t[4]->dtype, fout = t[3]->dtype, fdown = t[6]->dtype;
    if (t[1]->dtype != fin || t[2]->dtype != fin || t[5]->dtype != fmlp)
      return fail(TINYOAI_EINVAL, "layer %d: q/k/v must share one storage format, and gate/up another", l);
    DevMatrix &win = mats[(size_t)l * 4], &wout = mats[(size_t)l * 4 + 1];
    DevMatrix &win2 = mats[(size_t)l * 4 + 2], &wout2 = mats[(size_t)l * 4 + 3];
    // win: [q | k | v | gate/up interleaved], rotary pairs adjacent in q and
    // k; the gate/up pairs in a section of their own when their format differs.
    const bool split_in = fmlp != fin, split_out = fdown != fout;
    if ((rc = win.create(fin, split_in ? d + 2 * kvw : win_rows, d, stream))) return rc;
    DevMatrix &mlp = split_in ? win2 : win;
    const int64_t mlp0 = split_in ? 0 : d + 2 * kvw;
    if (split_in && (rc = win2.create(fmlp, 2 * I, d, stream))) return rc;
    if ((rc = place(win, p + names[0], t[0], RowMap{ROWMAP_HEADS, 0, hd, dims.rot, 0}, 0)) ||
        (rc = place(win, p + names[1], t[1], RowMap{ROWMAP_HEADS, d, hd, dims.rot, 0}, 0)) ||
        (rc = place(win, p + names[2], t[2], RowMap{ROWMAP_IDENTITY, d + kvw, 0, 0, 0}, 0)) ||
        (rc = place(mlp, p + names[4], t[4], RowMap{ROWMAP_INTERLEAVE, mlp0, 0, 0, 0}, 0)) ||
        (rc = place(mlp, p + names[5], t[5], RowMap{ROWMAP_INTERLEAVE, mlp0, 0, 0, 1}, 0)))
      return rc;
    // wout: [o | down] per output row, down starting on a chunk boundary;
    // o and down as matrices of their own when their formats differ.
    const int64_t vpc = values_per_chunk(fout), down0 = split_out ? 0 : (d + vpc - 1) / vpc * vpc;
    if ((rc = wout.create(fout, d, split_out ? d : down0 + I, stream))) return rc;
    DevMatrix &down = split_out ? wout2 : wout;
    if (split_out && (rc = wout2.create(fdown, d, I, stream))) return rc;
    if ((rc = place(wout, p + names[3], t[3], RowMap{ROWMAP_IDENTITY, 0, 0, 0, 0}, 0)) ||
        (rc = place(down, p + names[6], t[6], RowMap{ROWMAP_IDENTITY, 0, 0, 0, 0}, down0)))
      return rc;
    LayerDev &L = layers[l];
    L.win = win.desc;
    L.wout = wout.desc;
    L.win2 = split_in ? win2.desc : MatDesc{};
    L.wout2 = split_out ? wout2.desc : MatDesc{};
    mixed_layers |= split_in || split_out;
    if ((rc = load_vec(p + "input_layernorm.weight", &L.ln_w))) return rc;
    if ((rc = load_vec(p + "input_layernorm.bias", &L.ln_b))) return rc;
  }
  // Device workspaces.
  const int maxp = c.max_position_embeddings;
  rope_host = rope_table(maxp, dims.rot, c.rope_theta);
  const std::vector<float> &rt = rope_host;
  if ((rc = alloc((void **)&rope, rt.size() * 4))) return rc;
  e = hipMemcpyAsync(rope, rt.data(), rt.size() * 4, hipMemcpyHostToDevice, stream);
  if (e != hipSuccess) return hip_fail(e, "rope upload");
  if (16 + dims.rot > 1024) return fail(TINYOAI_EINVAL, "rotary width %d too large", dims.rot);
  // Prefill chunk: the matrix-core GEMMs and the flash attention fill the
  // device better with more rows (2048 rows: ~480 against ~390 TFLOP/s per
  // projection at 512); the vector-unit attention fallback, whose split
  // partials grow with the chunk, keeps 512.
  chunk = std::min(flash_prefill_supported(hd) ? 2048 : 512, maxp);
  const size_t w_att = (size_t)dims.heads * hd;
  if ((rc = alloc((void **)&x, (size_t)d * 4)) || (rc = alloc((void **)&qbuf, w_att * 4)) ||
      (rc = alloc((void **)&mbuf, (size_t)I * 4)) || (rc = alloc((void **)&abuf, w_att * 4)) ||
      (rc = alloc((void **)&logits_dev, (size_t)c.vocab_size * 4 + 256)) ||
      (rc = alloc((void **)&params, (size_t)(16 + std::max(chunk, dims.rot) + 2 * chunk) * 4)) ||
      (rc = alloc((void **)&trace_dev, (size_t)c.num_hidden_layers * d * 4)) ||
      (rc = alloc((void **)&trace_att, (size_t)c.num_hidden_layers * w_att * 4)) ||
      (rc = alloc((void **)&trace_gate, (size_t)c.num_hidden_layers * I * 4)) ||
      (rc = alloc((void **)&fuse_ctr, fuse_bytes())))
    return rc;
  e = hipMemsetAsync(fuse_ctr, 0, fuse_bytes(), stream);
  if (e != hipSuccess) return hip_fail(e, "decode counters");
  max_splits = maxp / 64 + 1;
  const size_t att_queries = flash_prefill_supported(hd) ? 1 : chunk;  // split-K attention queries at once
  if ((rc = alloc((void **)&counters, att_queries * dims.heads * 4))) return rc;
  e = hipMemsetAsync(counters, 0, att_queries * dims.heads * 4, stream);
  if (e != hipSuccess) return hip_fail(e, "counter init");
  if ((rc = alloc((void **)&partials, att_queries * dims.heads * partial_region(max_splits, hd) * 4))) return rc;
  const size_t B = chunk, wide = std::max(d, I);
  if ((rc = alloc((void **)&X, B * d * 4)) || (rc = alloc((void **)&H, B * d * 4)) ||
      (rc = alloc((void **)&Y, B * win_rows * 4)) || (rc = alloc((void **)&Q, B * w_att * 4)) ||
      (rc = alloc((void **)&M, B * I * 4)) || (rc = alloc((void **)&A, B * w_att * 4)) ||
      (rc = alloc((void **)&P, kPrefillSplits * B * d * 4)) || (rc = alloc((void **)&D, kPrefillSplits * B * d * 4)) ||
      (rc = alloc((void **)&XH, 2 * B * wide * 2)) || (rc = alloc((void **)&MH, 2 * B * I * 2)))
    return rc;
  // One allocation per operand: the hi plane, then the lo plane.
  XL = XH + B * wide;
  ML = MH + B * I;
  // The error word after the logits: set by a decode step whose bounded
  // in-kernel wait timed out.
  perr = (unsigned *)(logits_dev + c.vocab_size);
  e = hipMemsetAsync(perr, 0, 4, stream);
  if (e != hipSuccess) return hip_fail(e, "decode error word");
  e = hipEventCreateWithFlags(&params_copied, hipEventDisableTiming);
  if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
  e = hipHostMalloc(&h_pinned,
                    (size_t)c.vocab_size * 4 + 4096 + (size_t)(std::max(chunk, dims.rot) + 2 * chunk) * 4 + 64,
                    hipHostMallocDefault);
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipHostMalloc: %s", hipGetErrorString(e));
  e = hipHostMalloc(&h_io, (size_t)(io_words_logits() + 16 + dims.rot) * 4 + 256, hipHostMallocMapped);
  if (e == hipSuccess) e = hipHostGetDevicePointer(&d_io, h_io, 0);
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "mapped host memory: %s", hipGetErrorString(e));
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "model upload");
  const int cus = device_cu_count();
  // Row-streaming matvecs (measured on MI355X at the 3B shapes): two
  // 256-thread blocks per CU for the layer products, one 512-thread block
  // per CU for the classifier.
  grid_in = cus * 2;
  threads_in = 256;
  grid_out = cus * 2;
  threads_out = 256;
  grid_head = cus;
  threads_head = 512;
  return TINYOAI_OK;
}

// After a decode forward has synchronized: a set error word means an
// in-kernel dependency wait timed out, so the arrival counters are rebuilt
// from zero.
int StableModel::check_wait_error(int rc) {
  unsigned word = 0;
  if (hipMemcpy(&word, perr, 4, hipMemcpyDeviceToHost) != hipSuccess || word == 0) return rc;
  hipMemset(perr, 0, 4);
  reset_fused();
  return rc ? rc : fail(TINYOAI_EDEVICE, "decode step did not complete: a dependency wait timed out");
}

// Whether a decode step with this attention shape runs some layer's
// attention inside its decode_in launch.
bool StableModel::decode_fused(int steps) const {
  if (!fuse_attention) return false;
  for (const LayerDev &w : layers)
    if (decode_in_att_supported(w, dims, threads_in, steps)) return true;
  return false;
}

// The fused launches' counters from zero (after a failed step or a change
// of the decode_in launch shape, which changes the counters' step); the
// split-K arrival counters too, which a failed step may have left set.
void StableModel::reset_fused() {
  hipStreamSynchronize(stream);
  hipMemset(fuse_ctr, 0, fuse_bytes());
  hipMemset(counters, 0, (size_t)dims.heads * 4);
  fuse_epoch = 0;
}

// Grows KV to `needed` positions: power-of-two capacity capped at the
// context (stableContext.resize, prefix_cache.go:14-43), never below the
// LimitCache reservation; valid positions are copied head by head (growKV,
// kv_cache.go:101-109).
int StableModel::ensure_kv(int needed) {
  if (needed <= cap) return TINYOAI_OK;
  int want = 1;
  while (want < needed) want *= 2;
  want = std::max(want, reserve);
  want = std::min(want, cfg.max_position_embeddings);
  const size_t esz = kv_half ? 2 : 4;
  const size_t per_head = (size_t)dims.hd * esz;
  std::vector<KVDev> grown(cfg.num_hidden_layers);
  for (auto &l : grown) {
    const size_t bytes = (size_t)dims.kv_heads * want * per_head;
    hipError_t e = hipMalloc(&l.k, bytes);
    if (e == hipSuccess) e = hipMalloc(&l.v, bytes);
    if (e != hipSuccess) {
      for (auto &g : grown) { if (g.k) hipFree(g.k); if (g.v) hipFree(g.v); }
      return fail(TINYOAI_ENOMEM, "KV allocation of %d positions: %s", want, hipGetErrorString(e));
    }
    l.cap = want;
    l.half = kv_half;
  }
  for (int l = 0; l < (int)kv.size() && offset > 0; l++)
    for (int h = 0; h < dims.kv_heads; h++) {
      const size_t src = (size_t)h * cap * per_head, dst = (size_t)h * want * per_head;
      hipMemcpyAsync((char *)grown[l].k + dst, (char *)kv[l].k + src, offset * per_head, hipMemcpyDeviceToDevice, stream);
      hipMemcpyAsync((char *)grown[l].v + dst, (char *)kv[l].v + src, offset * per_head, hipMemcpyDeviceToDevice, stream);
    }
  hipError_t e = hipStreamSynchronize(stream);
  const int keep = offset;
  free_kv();
  kv = grown;
  cap = want;
  offset = keep;
  return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "KV growth");
}

#define TRY_HIP(expr, what)                 \
  do {                                      \
    hipError_t e_ = (expr);                 \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

// A kernel launch attributed to a profiling stage.
#define STAGE(stage, expr, what)       \
  do {                                 \
    prof.begin(stage, stream);         \
    TRY_HIP(expr, what);               \
    prof.end(stream);                  \
  } while (0)

// Copies head[0..nh), then from int 16 on the ids or the float row, and
// the n (position, slot) pairs of `rows` into the device parameter block
// (see rows_dev) through the pinned slot, first waiting for the slot's
// previous copy.
int StableModel::upload_params(const int *head_vals, int nh, const int32_t *ids, int n, const float *row, int nrow,
                               const int *rows) {
  int *hp = (int *)((char *)h_pinned + (size_t)cfg.vocab_size * 4 + 64);  // after the logits and error word
  if (params_copied) TRY_HIP(hipEventSynchronize(params_copied), "parameter slot");
  for (int i = 0; i < nh; i++) hp[i] = head_vals[i];
  if (n) memcpy(hp + 16, ids, (size_t)n * 4);
  if (nrow) memcpy(hp + 16, row, (size_t)nrow * 4);
  int count = n ? 16 + n : (nrow ? 16 + nrow : nh);
  if (rows) {
    const int off = 16 + std::max(chunk, dims.rot);
    memcpy(hp + off, rows, (size_t)n * 8);
    count = off + 2 * n;
  }
  TRY_HIP(hipMemcpyAsync(params, hp, (size_t)count * 4, hipMemcpyHostToDevice, stream), "parameters");
  TRY_HIP(hipEventRecord(params_copied, stream), "parameter event");
  return TINYOAI_OK;
}

// The kernels of one decode token; token and position come from `params`.
// The attention launch shape (steps, splits) is fixed by the caller so the
// sequence can be captured once per shape.
int StableModel::enqueue_decode(int steps, int splits, bool want_logits) {
  const int io_params = io_words_logits();
  TRY_HIP(launch_copy_words((const uint32_t *)d_io + io_params, params, 16 + dims.rot, stream), "parameters");
  for (int l = 0; l < cfg.num_hidden_layers; l++) {
    const LayerDev &w = layers[l];
    const float *rope_row = reinterpret_cast<const float *>(params + 16);
    const MatDesc *emb = l == 0 ? &embed.desc : nullptr;
    if (fuse_attention && decode_in_att_supported(w, dims, threads_in, steps)) {
      // q/k/v rows, then the attention on extra blocks while gate/up stream
      STAGE(ST_DECODE_IN,
            launch_decode_in_att(w, dims, kv[l], x, emb, params, rope_row, params + 1, qbuf, mbuf, grid_in, steps,
                                 splits, partials, counters, abuf, fuse_ctr + (size_t)l * 32 * fuse_lines(),
                                 params + 2, perr,
                                 stream),
            "decode_in + attention");
    } else {
      STAGE(ST_DECODE_IN,
            launch_decode_in(w, dims, kv[l], x, emb, params, rope_row, params + 1, qbuf, mbuf, grid_in, threads_in,
                             stream),
            "decode_in");
      if (w.win2.rows) {  // the gate/up section in a format of its own: every row pair is a SiLU-gate pair
        LayerDev wm = w;
        wm.win = w.win2;
        StableDims dm = dims;
        dm.win_q = dm.win_kv = 0;
        STAGE(ST_DECODE_IN,
              launch_decode_in(wm, dm, kv[l], x, nullptr, params, rope_row, params + 1, qbuf, mbuf, grid_in,
                               threads_in, stream),
              "decode_in");
      }
      STAGE(ST_ATTENTION,
            launch_attention(dims, kv[l], qbuf, params + 1, 1, 0, partials, counters, abuf, stream, steps, splits),
            "attention");
    }
    if (w.wout2.rows) {  // o and down in formats of their own: x = (x + o*a) + down*m in two products
      STAGE(ST_DECODE_OUT, launch_decode_out(w.wout, dims.d, 0, abuf, nullptr, x, grid_out, threads_out, stream),
            "decode_out");
      STAGE(ST_DECODE_OUT, launch_decode_out(w.wout2, dims.inter, 0, mbuf, nullptr, x, grid_out, threads_out, stream),
            "decode_out");
    } else {
      STAGE(ST_DECODE_OUT,
            launch_decode_out(w.wout, dims.d, dims.inter, abuf, mbuf, x, grid_out, threads_out, stream),
            "decode_out");
    }
    if (tracing) {
      const int hq = dims.heads * dims.hd;
      TRY_HIP(launch_copy_row(x, trace_dev + (size_t)l * dims.d, dims.d, stream), "trace");
      TRY_HIP(launch_copy_row(abuf, trace_att + (size_t)l * hq, hq, stream), "trace");
      TRY_HIP(launch_copy_row(mbuf, trace_gate + (size_t)l * dims.inter, dims.inter, stream), "trace");
    }
  }
  if (want_logits) {
    STAGE(ST_LM_HEAD, launch_ln_matvec(head.desc, norm_w, norm_b, dims.eps, 0, x, logits_dev, grid_head, threads_head, stream),
          "lm_head");
    // the logits and the error word after them
    TRY_HIP(launch_copy_words(logits_dev, d_io, cfg.vocab_size + 1, stream), "logits");
  }
  return TINYOAI_OK;
}

void StableModel::drop_graphs() {
  for (auto &g : graphs) hipGraphExecDestroy(g.second);
  graphs.clear();
}

// One token at `pos` (StableLM.forward, stablelm.go:332-387). Replays a HIP
// graph of the whole layer stack keyed by the attention launch shape;
// profiling runs launch the kernels directly so each can be timed.
int StableModel::decode_step(int token, int pos, bool want_logits) {
  const int vals[3] = {token, pos, fuse_epoch};
  logits_mapped = false;
  // The parameter block goes to host-mapped memory, which the step's first
  // kernel reads (the previous step has completed: every forward ends
  // with a synchronisation).
  int *hp = (int *)h_io + io_words_logits();
  for (int i = 0; i < 3; i++) hp[i] = vals[i];
  memcpy(hp + 16, rope_host.data() + (size_t)pos * dims.rot, (size_t)dims.rot * 4);
  logits_mapped = want_logits;
  const int steps = att_steps > 0 ? att_steps : decode_attention_steps(pos, dims.heads, dims.hd);
  const int splits = attention_splits(pos, steps);
  if (decode_fused(steps)) fuse_epoch++;  // the value the step's launches read is the one written above
  if (prof.on || !use_graphs) return enqueue_decode(steps, splits, want_logits);
  const int64_t key = ((int64_t)steps << 40) | ((int64_t)splits << 8) | (want_logits ? 2 : 0) | (tracing ? 1 : 0);
  auto it = graphs.find(key);
  if (it == graphs.end()) {
    hipGraph_t g = nullptr;
    TRY_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "graph capture");
    int rc = enqueue_decode(steps, splits, want_logits);
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

// y[n][ldy] = x[n][ldx] * W^T: on the matrix cores when the format allows
// (activations split into bf16 hi/lo planes first), else the vector-unit
// GEMM. Without rowstream every output row depends only on its own input
// row, whatever the chunk size (a prefix reused from the cache gives the
// same results).
int StableModel::project(const MatDesc &w, const float *x, int ldx, int n, float *y, int ldy, int *splits,
                         bool rowstream, int max_splits, bool *staged) {
  if (splits) *splits = 1;
  const bool reuse = staged && *staged;
  if (staged) *staged = false;
  if (gemm_mfma_supported(w)) {
    const bool two = gemm_planes(w, bf16_acts) == 2;
    // K-split partial products (summed by the caller) where the output
    // tiles alone would leave most of the device idle.
    const int ks = splits ? gemm_splits(w, n, std::max(1, std::min(max_splits, (int)kPrefillSplits))) : 1;
    if (splits) *splits = ks;
    STAGE(ST_PREFILL_GEMM, launch_split_bf16(x, ldx, w.cols, n, XH, two ? XL : nullptr, stream), "bf16 split");
    STAGE(ST_PREFILL_GEMM, launch_gemm_mfma(w, XH, two ? XL : nullptr, n, y, ldy, stream, ks), "projection");
  } else if (rowstream && kq_rows_supported(w, n) && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % 4 == 0 &&
             kq_rows_stage_bytes(w.cols, n) <= (size_t)chunk * std::max(dims.d, dims.inter) * 2) {
    // A few branch rows with a 5/6-bit matrix: every quant read once for
    // all rows, on the matrix cores (X staged in the XH workspace); K-split
    // partials where the caller sums.
    const int ks = splits ? kq_rows_splits(w, max_splits) : 1;
    if (splits) *splits = ks;
    STAGE(ST_PREFILL_GEMM, launch_kq_rows(w, x, ldx, n, y, ldy, ks, XH, stream, reuse), "projection");
    if (staged) *staged = true;
  } else if (rowstream && n <= kRowStreamMax) {
    // A few branch rows: one row-streaming matvec per row. The vector-unit
    // GEMM costs about as much for 16 rows as for 64 (677 us for a 16-row
    // K-quant product at the 3B shapes); the row kernels stream the matrix
    // per row, from the last-level cache after the first row.
    for (int j = 0; j < n; j++)
      STAGE(ST_PREFILL_GEMM,
            launch_ln_matvec(w, nullptr, nullptr, 0.0, 0, x + (size_t)j * ldx, y + (size_t)j * ldy, grid_out,
                             threads_out, stream),
            "projection");
  } else if (kq_rows_supported(w, 32) && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % 4 == 0 &&
             kq_rows_stage_bytes(w.cols, 32) <= (size_t)chunk * std::max(dims.d, dims.inter) * 2) {
    // Prefill rows (and branch appends of more than 32 rows) with a 5/6-bit
    // matrix: the few-row matrix-core product over slices of 32 rows (each
    // slice re-reads the matrix, mostly from the last-level cache), its K
    // splits in the caller's layout; as many slices per launch as the
    // staging workspace holds (each staged once, the launch's blocks
    // covering every slice at once). The 4096-token prefix of the 3B
    // K-quant branch workload prefills in 0.23 s against 0.84 s on the
    // vector-unit GEMM and 0.63 s with one launch per slice.
    const int ks = splits ? kq_rows_splits(w, max_splits) : 1;
    if (splits) *splits = ks;
    const size_t cap = (size_t)chunk * std::max(dims.d, dims.inter) * 2;
    const int per = std::max<int>(1, (int)(cap / kq_rows_stage_bytes(w.cols, 32))) * 32;
    for (int j0 = 0; j0 < n; j0 += per)
      STAGE(ST_PREFILL_GEMM,
            launch_kq_rows(w, x + (size_t)j0 * ldx, ldx, std::min(per, n - j0), y + (size_t)j0 * ldy, ldy, ks, XH,
                           stream, false, (int64_t)n * ldy),
            "projection");
  } else {
    if (ldx != w.cols || ldy != w.rows) return fail(TINYOAI_EINVAL, "vector-unit GEMM needs dense operands");
    STAGE(ST_PREFILL_GEMM, launch_gemm(w, x, n, y, stream), "projection");
  }
  return TINYOAI_OK;
}


// The wide-tile shape (rows per block 128 * mf, columns 32 * nf) for an
// n-row product with N outputs: the fewest rounds of 256 blocks weighted
// by the tile area, the 64-row-per-wave tiles counted at their measured
// advantage (2048 x 21504 x 2560 with two planes: 472 us at 256 x 224
// against 551 at 128 x 256).
static void wide_shape(int n, int N, int *mf, int *nf) {
  double best = 1e30;
  for (int f = 2; f >= 1; f--)
    for (int c = 7; c <= 8; c++) {
      const int64_t tiles = (int64_t)((n + 128 * f - 1) / (128 * f)) * ((N + 32 * c - 1) / (32 * c));
      const double cost = (double)((tiles + 255) / 256) * (128 * f) * (32 * c) / (f == 2 ? 1.0 : 0.85);
      if (cost < best) {
        best = cost;
        *mf = f;
        *nf = c;
      }
    }
}

// The same for a Q8_0 product on the wide tiles, 128 * mf rows x 32 * nf
// columns (nf 8 or 6), the 256-row tiles counted at their measured
// advantage (about 1.25x the work per K step of the 128-row ones): the 3B
// 512-row in-projection takes 256 x 192 tiles (224 blocks, one round).
static void wide_q8_shape(int n, int N, int *mf, int *nf) {
  double best = 1e30;
  for (int f = 2; f >= 1; f--)
    for (int c = 8; c >= 6; c -= 2) {
      const int64_t tiles = (int64_t)((n + 128 * f - 1) / (128 * f)) * ((N + 32 * c - 1) / (32 * c));
      const double cost = (double)((tiles + 255) / 256) * (128 * f) * (32 * c) / (f == 2 ? 1.0 : 0.8);
      if (cost < best) {
        best = cost;
        *mf = f;
        *nf = c;
      }
    }
}

// K splits of the o and down products of an n-row chunk on 256 x 256
// tiles, launched together: about one block per CU in all, shared in
// proportion to the K lengths (2048 rows at the 3B shapes: 1 + 2, 225 us
// against 258 for 2 + 6 and 326 for 1 + 1), each split at least four K
// steps.
static void wide_out_splits(int n, int d, int64_t ko, int64_t kd, int max_splits, int *so, int *sd, int bm = 256) {
  const int tiles = ((n + bm - 1) / bm) * ((d + 255) / 256);
  const int total = std::max(2, (256 + tiles / 2) / tiles);
  int o = std::max<int>(1, (int)std::lround((double)total * ko / (ko + kd)));
  int m = std::max(1, total - o);
  *so = std::max(1, std::min({o, max_splits, (int)(ko / 32 / 4)}));
  *sd = std::max(1, std::min({m, max_splits, (int)(kd / 32 / 4)}));
}

int StableModel::project_planes(const MatDesc &w, const uint16_t *xh, const uint16_t *xl, int n, float *y, int ldy,
                                int *splits) {
  if (use_wide && w.fmt == FMT_BF16) {
    int mf, nf;
    wide_shape(n, w.rows, &mf, &nf);
    const int64_t tiles = (int64_t)((n + 128 * mf - 1) / (128 * mf)) * ((w.rows + 32 * nf - 1) / (32 * nf));
    int ks = 1;
    if (splits) ks = (int)std::max<int64_t>(1, std::min<int64_t>({256 / std::max<int64_t>(1, tiles), kPrefillSplits, w.cols / 128}));
    if (splits) *splits = ks;
    const WideGemm g{w, xh, xl, w.cols, y, ldy, ks, (int64_t)n * ldy};
    STAGE(ST_PREFILL_GEMM, launch_gemm_wide(&g, 1, n, mf, nf, stream), "projection");
    return TINYOAI_OK;
  }
  const int ks = splits ? gemm_splits(w, n, kPrefillSplits) : 1;
  if (splits) *splits = ks;
  STAGE(ST_PREFILL_GEMM, launch_gemm_mfma(w, xh, xl, n, y, ldy, stream, ks), "projection");
  return TINYOAI_OK;
}

// Whether layer l's prefill takes the wide-tile BF16 path: fused BF16
// win and wout, operands in bf16 planes from their producers.
bool StableModel::wide_layer(int l) const {
  const LayerDev &w = layers[l];
  const bool bf16 = w.win.fmt == FMT_BF16 && w.wout.fmt == FMT_BF16;
  // Q8_0: the down section of wout starts on an even quant block (d % 64)
  const bool q8 = q8_wide && w.win.fmt == FMT_Q8_0 && w.wout.fmt == FMT_Q8_0 && wide_q8_ok(w.win) &&
                  wide_q8_ok(w.wout) && dims.d % 64 == 0;
  return use_wide && (bf16 || q8) && !w.win2.rows && !w.wout2.rows &&
         flash_prefill_supported(dims.hd) && dims.heads * dims.hd == dims.d && w.win.cols % 32 == 0 &&
         dims.inter % 32 == 0;
}

// n tokens at positions start.. (StableLM.prefill, prefill.go:33-115): per
// layer LayerNorm, one product with win and its fused epilogue, causal
// attention over the cache, the o and down products over the two column
// ranges of wout, and the parallel residual.
int StableModel::prefill_chunk(const int32_t *ids, int n, int start, bool want_logits) {
  const int vals[1] = {start};
  if (int rc = upload_params(vals, 1, ids, n)) return rc;
  const int *d_pos0 = params, *d_ids = params + 16;
  const int d = dims.d, I = dims.inter;
  STAGE(ST_EMBED, launch_embed(embed.desc, d_ids, n, X, stream), "embed");
  // Where layer l's LayerNorm output goes: bf16 planes XH, XL for a
  // matrix-core in-projection, else fp32 H.
  auto ln_out = [&](int l, float *&out, uint16_t *&oh, uint16_t *&ol) {
    const LayerDev &w = layers[l];
    const bool planes = wide_layer(l) || (!w.win2.rows && gemm_mfma_supported(w.win));
    out = planes ? nullptr : H;
    oh = planes ? XH : nullptr;
    ol = planes ? XL : nullptr;
  };
  // The residual of layer l and the LayerNorm of layer l + 1 in one launch
  // (LayerNorm models); normed: layer l's LayerNorm is already formed.
  auto residual = [&](int l, int sp, int sd) -> int {
    if (l + 1 < cfg.num_hidden_layers && dims.norm == 0) {
      float *out;
      uint16_t *oh, *ol;
      ln_out(l + 1, out, oh, ol);
      const LayerDev &nw = layers[l + 1];
      STAGE(ST_PREFILL_ELEMENTWISE,
            launch_residual_norm_rows(X, P, sp, D, sd, n, d, nw.ln_w, nw.ln_b, dims.eps, out, oh, ol, stream),
            "residual + layer_norm");
      return TINYOAI_OK;
    }
    STAGE(ST_PREFILL_ELEMENTWISE, launch_residual(X, P, sp, D, sd, (int64_t)n * d, stream), "residual");
    return TINYOAI_OK;
  };
  for (int l = 0; l < cfg.num_hidden_layers; l++) {
    const LayerDev &w = layers[l];
    const bool split_in = w.win2.rows > 0, split_out = w.wout2.rows > 0;
    const int64_t vpc = values_per_chunk(w.wout.fmt), down0 = (d + vpc - 1) / vpc * vpc;
    const MatDesc wo = split_out ? w.wout : column_view(w.wout, 0, d);
    const bool normed = l > 0 && dims.norm == 0;  // formed with the previous layer's residual
    const MatDesc wd = split_out ? w.wout2 : column_view(w.wout, down0, I);
    int rc;
    // Inputs of matrix-core projections leave their producers as bf16
    // planes (no separate split pass); the fp32 copies are kept where
    // another format or the trace needs them. LayerNorm -> XH, XL -> win;
    // its epilogue (fused into the product when both win and down run on
    // the matrix cores) -> MH, ML -> down; attention -> XH, XL -> o.
    const bool pin = !split_in && gemm_mfma_supported(w.win), pd = gemm_mfma_supported(wd);
    const bool flash = flash_prefill_supported(dims.hd), po = flash && gemm_mfma_supported(wo);
    if (wide_layer(l)) {
      // BF16 layers on wide tiles: LayerNorm -> planes; win, then its
      // epilogue (q, K/V, SiLU-gate planes); attention -> planes; the o and
      // down products as one launch of K splits; the parallel residual sums
      // them in order.
      const uint16_t *lo = lo_plane(w.win);
      if (!normed)
        STAGE(ST_PREFILL_NORM, launch_layer_norm_rows(X, w.ln_w, w.ln_b, dims.eps, n, d, nullptr, stream, XH, XL),
              "layer_norm");
      const bool q8 = w.win.fmt == FMT_Q8_0;
      int mf, nf;
      if (q8) wide_q8_shape(n, w.win.rows, &mf, &nf);
      else wide_shape(n, w.win.rows, &mf, &nf);
      if (q8 && n < 256 && 2 * n <= chunk) {
        // Below 256 rows the Q8_0 in-projection runs on the 128 x 256 tiles
        // as two K halves that the epilogue sums (more blocks than the wide
        // tiles give a short chunk).
        STAGE(ST_PREFILL_GEMM, launch_gemm_mfma(w.win, XH, lo, n, Y, win_rows, stream, 2), "projection");
        STAGE(ST_PREFILL_EPILOGUE,
              launch_in_epilogue(dims, kv[l], Y, win_rows, rope, d_pos0, n, Q, tracing ? M : nullptr, stream, MH, ML,
                                 nullptr, 2),
              "in_epilogue");
      } else if (wide_epi) {
        const InEpilogue e{dims, kv[l], rope, d_pos0, Q, tracing ? M : nullptr, MH, ML, 0};
        STAGE(ST_PREFILL_GEMM, launch_gemm_wide_in_epilogue(w.win, XH, lo, d, n, e, mf, nf, stream),
              "projection + epilogue");
      } else {
        const WideGemm g{w.win, XH, lo, d, Y, win_rows, 1, 0};
        STAGE(ST_PREFILL_GEMM, launch_gemm_wide(&g, 1, n, mf, nf, stream), "projection");
        STAGE(ST_PREFILL_EPILOGUE,
              launch_in_epilogue(dims, kv[l], Y, win_rows, rope, d_pos0, n, Q, tracing ? M : nullptr, stream, MH, ML),
              "in_epilogue");
      }
      STAGE(ST_PREFILL_ATTENTION,
            launch_flash_prefill(dims, kv[l], Q, d_pos0, n, tracing ? A : nullptr, stream, XH, XL, nullptr, 0, 0, 0,
                                 nullptr, 0, flash_ksplit ? Y : nullptr, (int64_t)chunk * win_rows, start + n - 1),
            "attention");
      int so, sd;
      const int omf = q8 && n < 256 ? 1 : 2;  // Q8_0 below 256 rows: 128-row tiles
      wide_out_splits(n, d, d, I, kPrefillSplits, &so, &sd, 128 * omf);
      const WideGemm prods[2] = {{wd, MH, lo ? ML : nullptr, I, D, d, sd, (int64_t)n * d},
                                 {wo, XH, lo ? XL : nullptr, d, P, d, so, (int64_t)n * d}};
      STAGE(ST_PREFILL_GEMM, launch_gemm_wide(prods, 2, n, omf, 8, stream), "projection");
      if ((rc = residual(l, so, sd))) return rc;
    } else {
      if (!normed)
        STAGE(ST_PREFILL_NORM,
              launch_layer_norm_rows(X, w.ln_w, w.ln_b, dims.eps, n, d, pin ? nullptr : H, stream, pin ? XH : nullptr,
                                     pin ? XL : nullptr),
              "layer_norm");
      float *m32 = pd && !tracing ? nullptr : M;
      if (split_in) {
        // [q | k | v] and the gate/up pairs in formats of their own: two
        // products from the fp32 LayerNorm output, then the epilogue of each
        // section (q/k/v rows only, then gate/up pairs only).
        StableDims da = dims, dm = dims;
        da.inter = 0;
        dm.win_q = dm.win_kv = 0;
        const int ra = w.win.rows, rm = w.win2.rows;
        float *Ya = Y, *Ym = Y + (size_t)n * ra;
        if ((rc = project(w.win, H, d, n, Ya, ra)) || (rc = project(w.win2, H, d, n, Ym, rm))) return rc;
        STAGE(ST_PREFILL_EPILOGUE,
              launch_in_epilogue(da, kv[l], Ya, ra, rope, d_pos0, n, Q, M, stream, nullptr, nullptr), "in_epilogue");
        STAGE(ST_PREFILL_EPILOGUE,
              launch_in_epilogue(dm, kv[l], Ym, rm, rope, d_pos0, n, Q, m32, stream, pd ? MH : nullptr,
                                 pd ? ML : nullptr),
              "in_epilogue");
      } else if (pin && pd && w.win.fmt == FMT_Q8_0 && n <= 1024 && 2 * n <= chunk) {
        // Up to 1024 rows the Q8_0 in-projection runs as two K halves (twice
        // the blocks: 672 against 336 over 256 CUs at 512 rows) that the
        // epilogue sums: the 3B 512-token prefill takes 11.8 ms against
        // 12.7 with the epilogue fused into one product (three halves: 13.1).
        STAGE(ST_PREFILL_GEMM, launch_gemm_mfma(w.win, XH, lo_plane(w.win), n, Y, win_rows, stream, 2),
              "projection");
        STAGE(ST_PREFILL_EPILOGUE,
              launch_in_epilogue(dims, kv[l], Y, win_rows, rope, d_pos0, n, Q, m32, stream, MH, ML, nullptr, 2),
              "in_epilogue");
      } else if (pin && pd) {
        const InEpilogue e{dims, kv[l], rope, d_pos0, Q, m32, MH, ML, 0};
        STAGE(ST_PREFILL_GEMM, launch_gemm_in_epilogue(w.win, XH, lo_plane(w.win), n, e, stream),
              "projection + epilogue");
      } else {
        if ((rc = pin ? project_planes(w.win, XH, lo_plane(w.win), n, Y, win_rows)
                      : project(w.win, H, d, n, Y, win_rows)))
          return rc;
        STAGE(ST_PREFILL_EPILOGUE,
              launch_in_epilogue(dims, kv[l], Y, win_rows, rope, d_pos0, n, Q, m32, stream, pd ? MH : nullptr,
                                 pd ? ML : nullptr),
              "in_epilogue");
      }
      int sp = 1, sd = 1;
      if ((rc = pd ? project_planes(wd, MH, gemm_planes(wd, bf16_acts) == 2 ? ML : nullptr, n, D, d, &sd) : project(wd, M, I, n, D, d, &sd)))
        return rc;
      if (flash)
        STAGE(ST_PREFILL_ATTENTION,
              launch_flash_prefill(dims, kv[l], Q, d_pos0, n, po && !tracing ? nullptr : A, stream, po ? XH : nullptr,
                                   po ? XL : nullptr, nullptr, 0, 0, 0, nullptr, 0, flash_ksplit ? Y : nullptr,
                                   (int64_t)chunk * win_rows,
                                   start + n - 1),
              "attention");
      else
        STAGE(ST_PREFILL_ATTENTION,
              launch_attention(dims, kv[l], Q, d_pos0, n, start + n - 1, partials, counters, A, stream), "attention");
      if ((rc = po ? project_planes(wo, XH, lo_plane(wo), n, P, d, &sp) : project(wo, A, d, n, P, d, &sp)))
        return rc;
      if ((rc = residual(l, sp, sd))) return rc;
    }
    if (tracing) {
      TRY_HIP(launch_copy_row(X + (size_t)(n - 1) * d, trace_dev + (size_t)l * d, d, stream), "trace");
      TRY_HIP(launch_copy_row(A + (size_t)(n - 1) * d, trace_att + (size_t)l * d, d, stream), "trace");
      TRY_HIP(launch_copy_row(M + (size_t)(n - 1) * I, trace_gate + (size_t)l * I, I, stream), "trace");
    }
  }
  if (scoring.targets)
    if (int rc = score_rows(n)) return rc;
  if (want_logits) {
    TRY_HIP(launch_copy_row(X + (size_t)(n - 1) * d, x, d, stream), "last row");
    STAGE(ST_LM_HEAD, launch_ln_matvec(head.desc, norm_w, norm_b, dims.eps, 0, x, logits_dev, grid_head, threads_head, stream),
          "lm_head");
  }
  return TINYOAI_OK;
}

int StableModel::busy_with_branches() const {
  return open_branches > 0 ? fail(TINYOAI_EINVAL, "%d branch session(s) borrow this model's prefix: close them first",
                                  open_branches)
                           : TINYOAI_OK;
}

void Branches::drop_graphs() {
  for (auto &g : graphs) hipGraphExecDestroy(g.second);
  graphs.clear();
}

void Branches::free_kv() {
  for (auto &l : kv) {
    if (l.k) hipFree(l.k);
    if (l.v) hipFree(l.v);
  }
  kv.clear();
  scap = 0;
}

// Every row of the chunk through the final LayerNorm and the classifier,
// in batches that fit the product buffer Y, then its log probabilities.
int StableModel::score_rows(int n) {
  const int d = dims.d, V = cfg.vocab_size;
  TRY_HIP(launch_layer_norm_rows(X, norm_w, norm_b, dims.eps, n, d, H, stream), "final norm");
  const int per = (int)std::max<int64_t>(1, (int64_t)chunk * win_rows / V);
  for (int r0 = 0; r0 < n; r0 += per) {
    const int nr = std::min(per, n - r0);
    if (int rc = project(head.desc, H + (size_t)r0 * d, d, nr, Y, V)) return rc;
    const int row = scoring.row + r0;
    const size_t c = (size_t)scoring.count;
    TRY_HIP(launch_logprobs(Y, V, nr, V, scoring.targets + row, scoring.count, scoring.chosen + row,
                            scoring.top_ids + row * c, scoring.top_lp + row * c, scoring.scratch, stream),
            "log probabilities");
  }
  scoring.row += n;
  return TINYOAI_OK;
}

Branches::~Branches() {
  if (m && m->stream) hipStreamSynchronize(m->stream);
  drop_graphs();
  free_kv();
  if (partials) hipFree(partials);
  if (counters) hipFree(counters);
  if (last) hipFree(last);
  if (segs) hipFree(segs);
  if (logits_host) hipHostFree(logits_host);
  if (m) m->open_branches--;
}

int Branches::grow(int need) {
  if (need <= scap) return TINYOAI_OK;
  int want = 16;
  while (want < need) want *= 2;
  want = std::min(want, max_len);
  if (want < need) return fail(TINYOAI_EINVAL, "branch suffix of %d positions exceeds its limit %d", need, max_len);
  const StableDims &s = m->dims;
  const size_t esz = m->kv_half ? 2 : 4, row = (size_t)s.hd * esz;
  const size_t bytes = (size_t)s.kv_heads * count * want * row;
  std::vector<KVDev> grown(m->cfg.num_hidden_layers);
  for (auto &l : grown) {
    hipError_t e = hipMalloc(&l.k, bytes);
    if (e == hipSuccess) e = hipMalloc(&l.v, bytes);
    if (e != hipSuccess) {
      for (auto &g : grown) { if (g.k) hipFree(g.k); if (g.v) hipFree(g.v); }
      return fail(TINYOAI_ENOMEM, "branch KV of %d positions: %s", want, hipGetErrorString(e));
    }
    l.cap = count * want;
    l.half = m->kv_half;
  }
  // Existing entries: rows of scap * hd values (one per kv head and branch)
  // move to rows of want * hd.
  if (scap > 0) {
    for (size_t l = 0; l < kv.size(); l++)
      for (int which = 0; which < 2; which++) {
        hipError_t e = hipMemcpy2DAsync(which ? grown[l].v : grown[l].k, want * row, which ? kv[l].v : kv[l].k,
                                        scap * row, scap * row, (size_t)s.kv_heads * count, hipMemcpyDeviceToDevice,
                                        m->stream);
        if (e != hipSuccess) {
          hipStreamSynchronize(m->stream);
          for (auto &g : grown) { hipFree(g.k); hipFree(g.v); }
          return hip_fail(e, "branch KV growth");
        }
      }
  }
  hipError_t e = hipStreamSynchronize(m->stream);
  drop_graphs();  // they name the old caches
  free_kv();
  kv = grown;
  scap = want;
  return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "branch KV growth");
}

int Branches::ensure_partials(int nq, int splits) {
  const size_t need = (size_t)nq * m->dims.heads * partial_region(splits, m->dims.hd);
  const size_t words = (size_t)nq * m->dims.heads;
  if (need > partial_floats) {
    hipStreamSynchronize(m->stream);
    drop_graphs();
    if (partials) hipFree(partials);
    partials = nullptr;
    partial_floats = 0;
    hipError_t e = hipMalloc(&partials, need * 4);
    if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "branch attention scratch (%zu floats): %s", need, hipGetErrorString(e));
    partial_floats = need;
  }
  if (words > counter_words) {
    hipStreamSynchronize(m->stream);
    drop_graphs();
    if (counters) hipFree(counters);
    counters = nullptr;
    counter_words = 0;
    hipError_t e = hipMalloc(&counters, words * 4);
    if (e == hipSuccess) e = hipMemsetAsync(counters, 0, words * 4, m->stream);
    if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "branch attention counters: %s", hipGetErrorString(e));
    counter_words = words;
  }
  return TINYOAI_OK;
}

// Branch rows (nativeBranches.Forward, mlx_branches.go:120-182, extended to
// several rows per branch): the rows go through the prefill products; each
// row's K and V land in its branch's suffix slots; attention reads the
// shared prefix and the row's own branch suffix under one softmax
// (branchAttention, mlx_branches.go:98-114). A branch's run of rows is
// causal within itself, like a prefill chunk.
int StableModel::branch_rows(Branches &b, const int32_t *ids, const int32_t *br, int n, float *logits) {
  const int d = dims.d, I = dims.inter, V = cfg.vocab_size, pfx = b.prefix;
  std::vector<int> add(b.count, 0), rows((size_t)2 * n);
  int need = 0, run = 0;  // suffix positions needed; most rows of one branch in this call
  for (int i = 0; i < n; i++) {
    need = std::max(need, b.len[br[i]] + ++add[br[i]]);
    run = std::max(run, add[br[i]]);
  }
  if (int rc = b.grow(need)) return rc;
  for (int i = 0, k = 0; i < n; i++) {
    const int j = br[i], s = b.len[j] + (k = (i > 0 && br[i - 1] == j) ? k + 1 : 0);
    rows[2 * i] = pfx + s;
    rows[2 * i + 1] = j * b.scap + s;
  }
  const bool flash = flash_prefill_supported(dims.hd);
  // Rows per chunk: the prefill workspaces hold `chunk`; one row per branch
  // (count <= chunk, checked at opening) runs as one chunk on the split-K
  // attention; longer runs take the matrix-core attention per branch, or
  // the split-K one in chunks whose partials stay within 64 MB.
  int per = chunk;
  if (run > 1 && !flash) {
    const size_t region = (size_t)dims.heads * partial_region(attention_splits(pfx + need, 1), dims.hd) * 4;
    per = (int)std::min<size_t>(per, std::max<size_t>(1, ((size_t)64 << 20) / region));
  }
  const int hq = dims.heads * dims.hd;
  // Final LayerNorm of every branch's newest row, then the classifier.
  auto enqueue_head = [&]() -> int {
    TRY_HIP(launch_layer_norm_rows(b.last, norm_w, norm_b, dims.eps, b.count, d, H, stream), "final norm");
    return project(head.desc, H, d, b.count, Y, V, nullptr, true);
  };
  const bool lockstep = use_graphs && !prof.on && n == b.count && run == 1 && n <= per;
  for (int r0 = 0; r0 < n; r0 += per) {
    const int nc = std::min(per, n - r0);
    const int32_t *cid = ids + r0;
    const int *crow = rows.data() + 2 * r0;
    if (int rc = upload_params(nullptr, 0, cid, nc, nullptr, 0, crow)) return rc;
    const int *d_ids = params + 16, *d_rows = rows_dev();
    // runs of one branch within the chunk: [seg[k], seg[k + 1])
    std::vector<int> seg{0};
    for (int i = 1; i < nc; i++)
      if (br[r0 + i] != br[r0 + i - 1]) seg.push_back(i);
    seg.push_back(nc);
    int max_pos = 0;
    for (int i = 0; i < nc; i++) max_pos = std::max(max_pos, crow[2 * i]);
    const bool use_flash = flash && run > 1;
    // The chunk's runs for the flash attention: one launch covers them all.
    int longest = 0;
    if (use_flash) {
      if (!b.segs) {  // at most one run per row of a chunk
        hipError_t e = hipMalloc(&b.segs, (size_t)chunk * 3 * sizeof(int));
        if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "branch run table: %s", hipGetErrorString(e));
      }
      // the previous chunk's table may still be in flight from the host copy
      if (!b.segs_host.empty()) TRY_HIP(hipStreamSynchronize(stream), "branch run table");
      b.segs_host.assign((seg.size() - 1) * 3, 0);
      for (size_t k = 0; k + 1 < seg.size(); k++) {
        const int a0 = seg[k], cnt = seg[k + 1] - seg[k];
        b.segs_host[3 * k] = a0;
        b.segs_host[3 * k + 1] = cnt;
        b.segs_host[3 * k + 2] = br[r0 + a0] * b.scap;
        longest = std::max(longest, cnt);
      }
      TRY_HIP(hipMemcpyAsync(b.segs, b.segs_host.data(), b.segs_host.size() * sizeof(int), hipMemcpyHostToDevice,
                             stream),
              "branch run table");
    }
    int max_splits = 0;
    if (!use_flash) {
      max_splits = branch_attention_records(dims, pfx, max_pos, nc);
      if (int rc = b.ensure_partials(nc, max_splits)) return rc;
    }
    // The chunk's kernels: embedding, the layers, each branch's newest row.
    auto enqueue_chunk = [&]() -> int {
      TRY_HIP(launch_embed(embed.desc, d_ids, nc, X, stream), "embed");
      for (int l = 0; l < cfg.num_hidden_layers; l++) {
        const LayerDev &w = layers[l];
        const bool split_in = w.win2.rows > 0, split_out = w.wout2.rows > 0;
        const int64_t vpc = values_per_chunk(w.wout.fmt), down0 = (d + vpc - 1) / vpc * vpc;
        const MatDesc wo = split_out ? w.wout : column_view(w.wout, 0, d);
        const MatDesc wd = split_out ? w.wout2 : column_view(w.wout, down0, I);
        int rc;
        // Y holds chunk * win_rows floats: with few rows, K-split partials of
        // the in-products fit within it (half each when the two groups are
        // separate matrices); P and D hold kPrefillSplits * chunk * d.
        const size_t ycap = (size_t)chunk * win_rows;
        const bool few = nc <= 32;
        // When the in-products run on the few-row kernel, the LayerNorm is
        // formed in their shared staging of X (no LayerNorm launch); the
        // conditions are those under which project() takes that kernel.
        const bool norm_in_stage = few && dims.norm == 0 && w.ln_b && d % 256 == 0 && kq_rows_supported(w.win, nc) &&
                                   (!split_in || kq_rows_supported(w.win2, nc)) &&
                                   kq_rows_stage_bytes(d, nc) <= (size_t)chunk * std::max(dims.d, dims.inter) * 2;
        bool staged = false;  // XH holds this layer's staged LayerNorm output
        if (norm_in_stage) {
          TRY_HIP(launch_kq_stage_norm(X, d, nc, d, w.ln_w, w.ln_b, dims.eps, XH, stream), "layer_norm + staging");
          staged = true;
        } else {
          TRY_HIP(launch_layer_norm_rows(X, w.ln_w, w.ln_b, dims.eps, nc, d, H, stream), "layer_norm");
        }
        const int pd_splits = (int)std::min<int64_t>(256, (int64_t)kPrefillSplits * chunk / nc);
        if (split_in) {
          StableDims da = dims, dm = dims;
          da.inter = 0;
          dm.win_q = dm.win_kv = 0;
          const int ra = w.win.rows, rm = w.win2.rows;
          float *Ya = Y, *Ym = few ? Y + ycap / 2 / 4 * 4 : Y + (size_t)nc * ra;
          int sa = 1, sm = 1;
          if (kq_pair && norm_in_stage && staged && kq_rows_pair_supported(w.win.fmt, w.win2.fmt)) {
            // both few-row in-products from the LayerNorm's staging of X in
            // one launch, with the split counts project() gives each
            sa = kq_rows_splits(w.win, (int)(ycap / 2 / ((size_t)nc * ra)));
            sm = kq_rows_splits(w.win2, (int)(ycap / 2 / ((size_t)nc * rm)));
            const KqProduct pa{w.win, XH, Ya, ra, sa, 0}, pm{w.win2, XH, Ym, rm, sm, 0};
            STAGE(ST_PREFILL_GEMM, launch_kq_rows_pair(pa, pm, nc, stream), "projection");
          } else if ((rc = project(w.win, H, d, nc, Ya, ra, few ? &sa : nullptr, true,
                                   (int)(ycap / 2 / ((size_t)nc * ra)), &staged)) ||
                     (rc = project(w.win2, H, d, nc, Ym, rm, few ? &sm : nullptr, true,
                                   (int)(ycap / 2 / ((size_t)nc * rm)), &staged))) {
            // H staged by the first product (or with the LayerNorm) serves the second
            return rc;
          }
          if (kq_pair) {  // both epilogues in one launch
            TRY_HIP(launch_in_epilogue_pair(da, Ya, ra, sa, dm, Ym, rm, sm, b.kv[l], rope, d_rows, nc, Q, M, stream),
                    "in_epilogue");
          } else {
            TRY_HIP(launch_in_epilogue(da, b.kv[l], Ya, ra, rope, nullptr, nc, Q, M, stream, nullptr, nullptr, d_rows,
                                       sa),
                    "in_epilogue");
            TRY_HIP(launch_in_epilogue(dm, b.kv[l], Ym, rm, rope, nullptr, nc, Q, M, stream, nullptr, nullptr, d_rows,
                                       sm),
                    "in_epilogue");
          }
        } else {
          int sy = 1;
          if ((rc = project(w.win, H, d, nc, Y, win_rows, few ? &sy : nullptr, true,
                            (int)(ycap / ((size_t)nc * win_rows)), &staged)))
            return rc;
          TRY_HIP(launch_in_epilogue(dims, b.kv[l], Y, win_rows, rope, nullptr, nc, Q, M, stream, nullptr, nullptr,
                                     d_rows, sy),
                  "in_epilogue");
        }
        int sp = 1, sd = 1;
        // Few rows with two K-quant output-side matrices: the attention
        // output and m staged together after the attention, and the o and
        // down products as one launch (the conditions under which project()
        // takes the few-row kernel for each; the two staged inputs side by
        // side in XH).
        const size_t cap = (size_t)chunk * std::max(dims.d, dims.inter) * 2;
        const size_t st_a = (kq_rows_stage_bytes(d, nc) + 255) / 256 * 256;
        const bool out_pair = kq_pair && few && kq_rows_pair_supported(wo.fmt, wd.fmt) && kq_rows_supported(wo, nc) &&
                              kq_rows_supported(wd, nc) && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
                              (reinterpret_cast<uintptr_t>(M) & 15) == 0 && d % 4 == 0 && I % 4 == 0 &&
                              st_a + kq_rows_stage_bytes(I, nc) <= cap;
        if (!out_pair && (rc = project(wd, M, I, nc, D, d, &sd, true, pd_splits))) return rc;
        if (use_flash) {
          TRY_HIP(launch_flash_prefill(dims, kv[l], Q, d_rows, longest, A, stream, nullptr, nullptr, &b.kv[l], pfx, 0, 0,
                                       b.segs, (int)seg.size() - 1),
                  "branch attention");
        } else {
          TRY_HIP(launch_branch_attention(dims, kv[l], b.kv[l], pfx, Q, d_rows, nc, max_pos, b.partials, b.counters,
                                          A, max_splits, stream),
                  "branch attention");
        }
        if (out_pair) {
          uint8_t *sa = reinterpret_cast<uint8_t *>(XH), *sm = sa + st_a;
          sp = kq_rows_splits(wo, pd_splits);
          sd = kq_rows_splits(wd, pd_splits);
          STAGE(ST_PREFILL_GEMM, launch_kq_stage_pair(A, d, d, sa, M, I, I, sm, nc, stream), "staging");
          const KqProduct po{wo, sa, P, d, sp, 0}, pm{wd, sm, D, d, sd, 0};
          STAGE(ST_PREFILL_GEMM, launch_kq_rows_pair(po, pm, nc, stream), "projection");
        } else if ((rc = project(wo, A, d, nc, P, d, &sp, true, pd_splits))) {
          return rc;
        }
        TRY_HIP(launch_residual(X, P, sp, D, sd, (int64_t)nc * d, stream), "residual");
      }
      // each branch's newest row of this chunk
      for (size_t k = 0; k + 1 < seg.size(); k++) {
        const int last_row = seg[k + 1] - 1, j = br[r0 + last_row];
        TRY_HIP(launch_copy_row(X + (size_t)last_row * d, b.last + (size_t)j * d, d, stream), "branch row");
      }
      return TINYOAI_OK;
    };
    if (lockstep) {
      // One row per branch in one chunk: the step's kernels, with the final
      // LayerNorm and the classifier, replay from a graph keyed by the
      // attention's launch shape (the model's buffers, the branch caches
      // and their scratch stay in place while the graph lives; the caches'
      // growth and larger scratch drop the graphs).
      const int64_t key = ((int64_t)branch_attention_shape(dims, pfx, max_pos, nc) << 24) ^
                          ((int64_t)max_splits << 8) ^ (int64_t)launch_gen;
      auto it = b.graphs.find(key);
      if (it == b.graphs.end()) {
        hipGraph_t g = nullptr;
        TRY_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "graph capture");
        int rc = enqueue_chunk();
        if (!rc) rc = enqueue_head();
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
        it = b.graphs.emplace(key, exec).first;
      }
      TRY_HIP(hipGraphLaunch(it->second, stream), "graph launch");
    } else if (int rc = enqueue_chunk()) {
      return rc;
    }
  }
  if (!lockstep)
    if (int rc = enqueue_head()) return rc;
  // The logits reach the caller through the session's pinned buffer: one
  // DMA and one host copy (a copy straight into pageable memory goes
  // through the runtime's staging buffer in pieces, each waited for).
  const size_t lbytes = (size_t)b.count * V * 4;
  if (b.logits_bytes < lbytes) {
    TRY_HIP(hipStreamSynchronize(stream), "branch step");
    if (b.logits_host) hipHostFree(b.logits_host);
    b.logits_host = nullptr;
    b.logits_bytes = 0;
    if (hipHostMalloc((void **)&b.logits_host, lbytes, hipHostMallocDefault) != hipSuccess)
      return fail(TINYOAI_ENOMEM, "pinned logits buffer");
    b.logits_bytes = lbytes;
  }
  TRY_HIP(hipMemcpyAsync(b.logits_host, Y, lbytes, hipMemcpyDeviceToHost, stream), "logits");
  TRY_HIP(hipStreamSynchronize(stream), "branch step");
  memcpy(logits, b.logits_host, lbytes);
  for (int j = 0; j < b.count; j++) b.len[j] += add[j];
  return TINYOAI_OK;
}

// ForwardWithLogprobs (mlx.go:53-57; mlx_native.go:300-311): the forward
// of `tokens` through the prefill path (every row's logits are needed),
// scoring row i against targets[i]; results copied to the caller's arrays.
int StableModel::forward_logprobs(int prefix, const int32_t *tokens, const int32_t *targets, int n, int count,
                                  float *logits, double *chosen, int32_t *top_ids, double *top_lp) {
  if (int rc = busy_with_branches()) return rc;
  const int V = cfg.vocab_size;
  if (!tokens || !targets || !logits || !chosen || !top_ids || !top_lp || n <= 0 || count < 1 || count > V)
    return fail(TINYOAI_EINVAL, "invalid probability request");
  for (int i = 0; i < n; i++)
    if (targets[i] < 0 || targets[i] >= V) return fail(TINYOAI_EINVAL, "invalid probability target %d", targets[i]);
  if (prefix < 0 || prefix > offset || prefix + n > cfg.max_position_embeddings)
    return fail(TINYOAI_EINVAL, "invalid cached prefix or context length (prefix %d, offset %d, n %d)", prefix,
                offset, n);
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= V) return fail(TINYOAI_EINVAL, "invalid token %d", tokens[i]);
  // device scratch: targets, chosen, top ids, top log probabilities, the
  // ranking scratch (its first word the NaN error word)
  auto r256 = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t bt = r256((size_t)n * 4), bc = r256((size_t)n * 8), bi = r256((size_t)n * count * 4),
               bl = r256((size_t)n * count * 8), bs = r256(logprob_scratch_bytes(count));
  if (bt + bc + bi + bl + bs > score_bytes) {
    hipStreamSynchronize(stream);
    if (score_mem) hipFree(score_mem);
    score_mem = nullptr;
    score_bytes = 0;
    hipError_t e = hipMalloc(&score_mem, bt + bc + bi + bl + bs);
    if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "probability scratch: %s", hipGetErrorString(e));
    score_bytes = bt + bc + bi + bl + bs;
  }
  char *base = (char *)score_mem;
  int *d_targets = (int *)base;
  void *rank = base + bt + bc + bi + bl;
  TRY_HIP(hipMemcpyAsync(d_targets, targets, (size_t)n * 4, hipMemcpyHostToDevice, stream), "targets");
  TRY_HIP(hipMemsetAsync(rank, 0, 4, stream), "probability error word");
  scoring = Scoring{d_targets, count, 0, (double *)(base + bt), (double *)(base + bt + bc + bi),
                    (int *)(base + bt + bc), rank};
  offset = prefix;
  int rc = ensure_kv(prefix + n);
  for (int done = 0; done < n && !rc;) {
    const int m = std::min(chunk, n - done);
    rc = prefill_chunk(tokens + done, m, prefix + done, done + m == n);
    done += m;
  }
  const Scoring sc = scoring;
  scoring = Scoring{};
  if (!rc) {
    hipError_t e = hipMemcpyAsync(h_pinned, logits_dev, (size_t)V * 4, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipMemcpyAsync(chosen, sc.chosen, (size_t)n * 8, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipMemcpyAsync(top_ids, sc.top_ids, (size_t)n * count * 4, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipMemcpyAsync(top_lp, sc.top_lp, (size_t)n * count * 8, hipMemcpyDeviceToHost, stream);
    int bad = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&bad, sc.scratch, 4, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) rc = hip_fail(e, "log probabilities");
    else if (bad) rc = fail(TINYOAI_EINVAL, "the logits of position %d hold NaN", prefix + bad - 1);
    else memcpy(logits, h_pinned, (size_t)V * 4);
  }
  if (rc) {
    std::string msg = g_error;
    hipStreamSynchronize(stream);
    prof.marks.clear();
    prof.used = 0;
    free_kv();
    g_error = msg;
    return rc;
  }
  prof.resolve();
  offset = prefix + n;
  return TINYOAI_OK;
}

int StableModel::forward(int prefix, const int32_t *tokens, int n, bool want_logits, float *logits) {
  if (int rc = busy_with_branches()) return rc;
  if (prefix < 0 || prefix > offset || n <= 0 || !tokens || prefix + n > cfg.max_position_embeddings)
    return fail(TINYOAI_EINVAL, "invalid cached prefix or context length (prefix %d, offset %d, n %d)", prefix,
                offset, n);
  if (want_logits && !logits) return fail(TINYOAI_EINVAL, "logits output is required");
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= cfg.vocab_size) return fail(TINYOAI_EINVAL, "invalid token %d", tokens[i]);
  offset = prefix;
  int rc = ensure_kv(prefix + n);
  if (rc) return rc;
  for (int done = 0; done < n && !rc;) {
    const int m = std::min(chunk, n - done);
    const bool last = done + m == n;
    if (m == 1)
      rc = decode_step(tokens[done], prefix + done, last && want_logits);
    else
      rc = prefill_chunk(tokens + done, m, prefix + done, last && want_logits);
    done += m;
  }
  // The word after the logits is the error word of the decode kernels'
  // bounded waits: it comes back with the logits, which a decode step's
  // graph has already copied to h_io (otherwise they come through h_pinned).
  const bool mapped = logits_mapped && n == 1;
  float *src = (float *)(mapped ? h_io : h_pinned);
  unsigned *err_host = (unsigned *)src + cfg.vocab_size;
  if (!rc && want_logits) {
    hipError_t e = mapped ? hipSuccess
                          : hipMemcpyAsync(h_pinned, logits_dev, (size_t)cfg.vocab_size * 4 + 4,
                                           hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) rc = hip_fail(e, "logits");
    else if (*err_host) rc = check_wait_error(rc);
    else memcpy(logits, src, (size_t)cfg.vocab_size * 4);
  } else if (!rc) {
    hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) rc = hip_fail(e, "forward");
    else if (n == 1) rc = check_wait_error(rc);
  }
  if (rc) {
    std::string msg = g_error;
    hipStreamSynchronize(stream);
    prof.marks.clear();
    prof.used = 0;
    free_kv();
    g_error = msg;
    return rc;
  }
  prof.resolve();
  offset = prefix + n;
  return TINYOAI_OK;
}

}  // namespace tinyoai

using namespace tinyoai;

struct tinyoai_weight {
  DevMatrix m;
  int device = 0;  // the device the weight lives on
  hipStream_t stream = nullptr;
  uint16_t *planes = nullptr;  // bf16 hi/lo planes of the last batched product's input
  size_t planes_bytes = 0;
  ~tinyoai_weight() {
    if (planes) hipFree(planes);
    if (stream) hipStreamDestroy(stream);
  }
};

extern "C" {

const char *tinyoai_last_error(void) { return g_error.c_str(); }

int tinyoai_stablelm_load(const tinyoai_stablelm_config *config, const tinyoai_tensor *tensors, int32_t n_tensors,
                          tinyoai_model **out) {
  if (!config || !tensors || !out || n_tensors <= 0) return fail(TINYOAI_EINVAL, "invalid load arguments");
  *out = nullptr;
  auto h = std::make_unique<tinyoai_model>();
  h->stable = std::make_unique<StableModel>();
  int rc = h->stable->init(*config, tensors, n_tensors);
  if (rc) return rc;
  *out = h.release();
  return TINYOAI_OK;
}

int tinyoai_stablelm_forward(tinyoai_model *m, int32_t prefix, const int32_t *tokens, int32_t n, int32_t want_logits,
                             float *logits) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  return m->stable->forward(prefix, tokens, n, want_logits != 0, logits);
}

int tinyoai_stablelm_forward_logprobs(tinyoai_model *m, int32_t prefix, const int32_t *tokens,
                                      const int32_t *targets, int32_t n, int32_t count, float *logits,
                                      double *chosen, int32_t *top_ids, double *top_logprobs) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  return m->stable->forward_logprobs(prefix, tokens, targets, n, count, logits, chosen, top_ids, top_logprobs);
}

int tinyoai_summarize_logits(const float *logits, int32_t rows, int32_t vocab, const int32_t *targets, int32_t count,
                             double *chosen, int32_t *top_ids, double *top_logprobs) {
  if (!logits || !targets || !chosen || !top_ids || !top_logprobs || rows < 1 || vocab < 1 || count < 1 ||
      count > vocab)
    return fail(TINYOAI_EINVAL, "invalid probability request");
  for (int i = 0; i < rows; i++)
    if (targets[i] < 0 || targets[i] >= vocab) return fail(TINYOAI_EINVAL, "invalid probability target %d", targets[i]);
  const size_t nl = (size_t)rows * vocab * 4, nt = (size_t)rows * 4, nc = (size_t)rows * 8;
  const size_t ni = (size_t)rows * count * 4, np = (size_t)rows * count * 8, ns = logprob_scratch_bytes(count);
  auto r256 = [](size_t b) { return (b + 255) / 256 * 256; };
  char *mem = nullptr;
  hipError_t e = hipMalloc(&mem, r256(nl) + r256(nt) + r256(nc) + r256(ni) + r256(np) + r256(ns));
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipMalloc: %s", hipGetErrorString(e));
  float *dl = (float *)mem;
  int *dt = (int *)(mem + r256(nl));
  double *dc = (double *)((char *)dt + r256(nt));
  int *di = (int *)((char *)dc + r256(nc));
  double *dp = (double *)((char *)di + r256(ni));
  void *ds = (char *)dp + r256(np);
  int bad = 0;
  e = hipMemcpy(dl, logits, nl, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dt, targets, nt, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(ds, 0, 4);
  if (e == hipSuccess) e = launch_logprobs(dl, vocab, rows, vocab, dt, count, dc, di, dp, ds, nullptr);
  if (e == hipSuccess) e = hipMemcpy(chosen, dc, nc, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(top_ids, di, ni, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(top_logprobs, dp, np, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(&bad, ds, 4, hipMemcpyDeviceToHost);
  hipFree(mem);
  if (e != hipSuccess) return hip_fail(e, "log probabilities");
  if (bad) return fail(TINYOAI_EINVAL, "logits row %d holds NaN", bad - 1);
  return TINYOAI_OK;
}

int tinyoai_stablelm_set_kv_bits(tinyoai_model *m, int32_t bits, int32_t *cleared) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  if (bits != 16 && bits != 32)
    return fail(TINYOAI_EINVAL, "KV bits must be 16 (fp16) or 32 (fp32); affine 8-bit KV is not supported");
  StableModel &s = *m->stable;
  if (int rc = s.busy_with_branches()) return rc;
  const int half = bits == 16;
  int c = 0;
  if (half != s.kv_half) {
    hipStreamSynchronize(s.stream);
    s.free_kv();
    s.kv_half = half;
    c = 1;
  }
  if (cleared) *cleared = c;
  return TINYOAI_OK;
}

int tinyoai_stablelm_limit_cache(tinyoai_model *m, int32_t limit, int32_t *cleared) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  StableModel &s = *m->stable;
  if (int rc = s.busy_with_branches()) return rc;
  if (limit <= 0 || limit > s.cfg.max_position_embeddings) return fail(TINYOAI_EINVAL, "invalid cache limit %d", limit);
  int c = 0;
  s.reserve = limit;
  if (s.cap > limit) {
    hipStreamSynchronize(s.stream);
    s.free_kv();
    c = 1;
  }
  if (cleared) *cleared = c;
  return TINYOAI_OK;
}

int tinyoai_stablelm_reset(tinyoai_model *m) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  if (int rc = m->stable->busy_with_branches()) return rc;
  hipStreamSynchronize(m->stable->stream);
  m->stable->free_kv();
  return TINYOAI_OK;
}

int tinyoai_stablelm_offset(const tinyoai_model *m) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  return m->stable->offset;
}

int tinyoai_stablelm_close(tinyoai_model *m) {
  if (!m) return TINYOAI_OK;
  if (m->stable) {
    if (int rc = m->stable->busy_with_branches()) return rc;
    hipStreamSynchronize(m->stable->stream);
  }
  delete m;
  return TINYOAI_OK;
}

}  // extern "C"

struct tinyoai_branches {
  std::unique_ptr<tinyoai::Branches> b;
};

extern "C" {

int tinyoai_stablelm_branches_open(tinyoai_model *m, int32_t prefix, int32_t count, int32_t max_len,
                                   tinyoai_branches **out) {
  if (!m || !m->stable || !out) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  *out = nullptr;
  StableModel &s = *m->stable;
  const int hd = s.dims.hd, room = s.cfg.max_position_embeddings - prefix;
  if (prefix < 0 || prefix > s.offset || count < 1 || max_len < 0 || count > s.chunk ||
      (int64_t)count * s.cfg.vocab_size > (int64_t)s.chunk * s.win_rows || room < 1)
    return fail(TINYOAI_EINVAL, "invalid branch prefix or batch size (prefix %d, offset %d, count %d)", prefix,
                s.offset, count);
  if (hd != 8 && hd != 64 && hd != 80 && hd != 128) return fail(TINYOAI_EINVAL, "branch attention: head width %d", hd);
  if (int rc = s.ensure_kv(std::max(prefix, 1))) return rc;
  auto h = std::make_unique<tinyoai_branches>();
  h->b = std::make_unique<Branches>();
  Branches &b = *h->b;
  b.m = &s;
  s.open_branches++;
  b.prefix = prefix;
  b.count = count;
  b.max_len = max_len > 0 ? std::min(max_len, room) : room;
  b.len.assign(count, 0);
  hipError_t e = hipMalloc(&b.last, (size_t)count * s.dims.d * 4);
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "branch rows: %s", hipGetErrorString(e));
  *out = h.release();
  return TINYOAI_OK;
}

// Validates and runs `n` rows; a native failure closes the branches'
// storage, as nativeBranches.Forward closes its caches on an evaluation
// error (mlx_branches.go:172-175).
static int branches_run(tinyoai_branches *h, const int32_t *tokens, const int32_t *br, int n, float *logits) {
  Branches &b = *h->b;
  StableModel &s = *b.m;
  std::vector<int> add(b.count, 0);
  for (int i = 0; i < n; i++) {
    if (tokens[i] < 0 || tokens[i] >= s.cfg.vocab_size) return fail(TINYOAI_EINVAL, "invalid branch token %d", tokens[i]);
    const int j = br[i];
    if (++add[j] + b.len[j] > b.max_len)
      return fail(TINYOAI_EINVAL, "branch %d: suffix of %d tokens exceeds the context (%d positions after prefix %d)",
                  j, add[j] + b.len[j], b.max_len, b.prefix);
  }
  const int rc = s.branch_rows(b, tokens, br, n, logits);
  if (rc) h->b.reset();
  return rc;
}

int tinyoai_stablelm_branches_forward(tinyoai_branches *h, const int32_t *tokens, int32_t count, float *logits) {
  if (!h || !h->b) return fail(TINYOAI_EINVAL, "branches are closed");
  Branches &b = *h->b;
  if (!tokens || !logits || count != b.count) return fail(TINYOAI_EINVAL, "invalid branch batch or context length");
  std::vector<int32_t> br(count);
  for (int j = 0; j < count; j++) br[j] = j;
  return branches_run(h, tokens, br.data(), count, logits);
}

int tinyoai_stablelm_branches_append(tinyoai_branches *h, const int32_t *tokens, const int32_t *lengths,
                                     int32_t count, float *logits) {
  if (!h || !h->b) return fail(TINYOAI_EINVAL, "branches are closed");
  Branches &b = *h->b;
  if (!tokens || !lengths || !logits || count != b.count) return fail(TINYOAI_EINVAL, "invalid branch batch");
  std::vector<int32_t> br;
  for (int j = 0; j < count; j++) {
    if (lengths[j] < 1 || lengths[j] > b.max_len) return fail(TINYOAI_EINVAL, "branch %d: invalid length %d", j, lengths[j]);
    br.insert(br.end(), lengths[j], j);
  }
  return branches_run(h, tokens, br.data(), (int)br.size(), logits);
}

int tinyoai_stablelm_branches_length(const tinyoai_branches *h, int32_t branch) {
  if (!h || !h->b) return fail(TINYOAI_EINVAL, "branches are closed");
  if (branch < 0 || branch >= h->b->count) return fail(TINYOAI_EINVAL, "invalid branch %d", branch);
  return h->b->len[branch];
}

int tinyoai_stablelm_branches_close(tinyoai_branches *h) {
  delete h;
  return TINYOAI_OK;
}

int tinyoai_stablelm_read_kv(tinyoai_model *m, int32_t layer, int32_t kv_head, int32_t n, float *keys, float *values) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  StableModel &s = *m->stable;
  if (layer < 0 || layer >= s.cfg.num_hidden_layers || kv_head < 0 || kv_head >= s.dims.kv_heads || n < 0 ||
      n > s.offset || !keys || !values)
    return fail(TINYOAI_EINVAL, "invalid KV read");
  const int hd = s.dims.hd;
  std::vector<uint8_t> buf((size_t)n * hd * 4);
  for (int which = 0; which < 2; which++) {
    const KVDev &k = s.kv[layer];
    const size_t esz = k.half ? 2 : 4;
    const char *src = (const char *)(which ? k.v : k.k) + (size_t)kv_head * k.cap * hd * esz;
    hipError_t e = hipMemcpy(buf.data(), src, (size_t)n * hd * esz, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "KV read");
    float *dst = which ? values : keys;
    for (size_t i = 0; i < (size_t)n * hd; i++) {
      if (k.half) {
        uint16_t h;
        memcpy(&h, buf.data() + i * 2, 2);
        dst[i] = (float)*reinterpret_cast<const _Float16 *>(&h);
      } else {
        memcpy(&dst[i], buf.data() + i * 4, 4);
      }
    }
  }
  return TINYOAI_OK;
}

// cachePayload (cache_file.go:188-216): per layer, per kv head, K then V,
// positions [0, n) of head_dim values in the KV format (capacity padding
// left out). The device cache is [kv_heads][cap][hd] per layer, so each of
// K and V of a layer is one strided copy.
static int kv_payload(StableModel &s, int32_t n, int32_t half, void *payload, uint64_t nbytes, bool save) {
  if (n < 0 || n > s.cfg.max_position_embeddings || (half != 0) != (s.kv_half != 0) || (n > 0 && !payload))
    return fail(TINYOAI_EINVAL, "invalid KV payload request (n %d, float16 %d, model float16 %d)", n, half, s.kv_half);
  const size_t esz = s.kv_half ? 2 : 4, row = (size_t)n * s.dims.hd * esz;
  const uint64_t want = (uint64_t)s.cfg.num_hidden_layers * s.dims.kv_heads * 2 * row;
  if (nbytes != want) return fail(TINYOAI_EINVAL, "KV payload of %d positions is %llu bytes, got %llu", n,
                                  (unsigned long long)want, (unsigned long long)nbytes);
  if (save && n > s.offset) return fail(TINYOAI_EINVAL, "only %d positions are resident", s.offset);
  if (!save) {
    if (int rc = s.busy_with_branches()) return rc;
    if (n == 0) {
      s.offset = 0;
      return TINYOAI_OK;
    }
    if (int rc = s.ensure_kv(n)) return rc;
  }
  if (n == 0) return TINYOAI_OK;
  hipStreamSynchronize(s.stream);
  for (int l = 0; l < s.cfg.num_hidden_layers; l++)
    for (int kind = 0; kind < 2; kind++) {
      const size_t pitch = (size_t)s.kv[l].cap * s.dims.hd * esz;  // one head's positions on the device
      char *dev = (char *)(kind ? s.kv[l].v : s.kv[l].k);
      char *host = (char *)payload + ((size_t)l * s.dims.kv_heads * 2 + kind) * row;
      hipError_t e = save ? hipMemcpy2D(host, 2 * row, dev, pitch, row, s.dims.kv_heads, hipMemcpyDeviceToHost)
                          : hipMemcpy2D(dev, pitch, host, 2 * row, row, s.dims.kv_heads, hipMemcpyHostToDevice);
      if (e != hipSuccess) {
        if (!save) s.free_kv();
        return hip_fail(e, save ? "KV save" : "KV load");
      }
    }
  if (!save) s.offset = n;
  return TINYOAI_OK;
}

int tinyoai_stablelm_kv_save(tinyoai_model *m, int32_t n, int32_t half, void *payload, uint64_t nbytes) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  return kv_payload(*m->stable, n, half, payload, nbytes, true);
}

int tinyoai_stablelm_kv_load(tinyoai_model *m, int32_t n, int32_t half, const void *payload, uint64_t nbytes) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  return kv_payload(*m->stable, n, half, const_cast<void *>(payload), nbytes, false);
}

int tinyoai_stablelm_trace(tinyoai_model *m, int32_t enable) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  m->stable->tracing = enable != 0;
  return TINYOAI_OK;
}

int tinyoai_stablelm_trace_read(tinyoai_model *m, float *residual) {
  if (!m || !m->stable || !residual) return fail(TINYOAI_EINVAL, "invalid trace read");
  StableModel &s = *m->stable;
  hipError_t e = hipStreamSynchronize(s.stream);
  if (e == hipSuccess)
    e = hipMemcpy(residual, s.trace_dev, (size_t)s.cfg.num_hidden_layers * s.dims.d * 4, hipMemcpyDeviceToHost);
  return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "trace read");
}

int tinyoai_stablelm_trace_read_stages(tinyoai_model *m, float *attention, float *gate) {
  if (!m || !m->stable || !attention || !gate) return fail(TINYOAI_EINVAL, "invalid trace read");
  StableModel &s = *m->stable;
  const size_t L = s.cfg.num_hidden_layers;
  hipError_t e = hipStreamSynchronize(s.stream);
  if (e == hipSuccess)
    e = hipMemcpy(attention, s.trace_att, L * s.dims.heads * s.dims.hd * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(gate, s.trace_gate, L * s.dims.inter * 4, hipMemcpyDeviceToHost);
  return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "trace read");
}


int tinyoai_stablelm_set_launch(tinyoai_model *m, int32_t stage, int32_t grid, int32_t threads) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  StableModel &s = *m->stable;
  s.launch_gen++;  // an open branch session's step graphs are not replayed after this
  if (stage == 7) {  // BF16-weight prefill products on wide tiles (1, the default) or 128 x 256 tiles (0)
    s.use_wide = grid != 0;
    return TINYOAI_OK;
  }
  if (stage == 10) {  // Q8_0 prefill products on wide tiles (1, the default) or 128 x 256 tiles (0)
    s.q8_wide = grid != 0;
    return TINYOAI_OK;
  }
  if (stage == 11) {  // a branch step's launch pairs (1, the default) or each launch of its own (0)
    s.kq_pair = grid != 0;
    return TINYOAI_OK;
  }
  if (stage == 8) {  // wide-tile in-projection with its epilogue fused (1) or a kernel of its own (0, the default)
    s.wide_epi = grid != 0;
    return TINYOAI_OK;
  }
  if (stage == 5) {  // BF16-weight prefill products with bf16 activations (1) or two planes (0, the default)
    s.bf16_acts = grid != 0;
    return TINYOAI_OK;
  }
  if (stage == 9) {  // prefill attention split over keys where query tiles leave CUs idle (1, the default) or not (0)
    s.flash_ksplit = grid != 0;
    return TINYOAI_OK;
  }
  if (stage == 4) {  // decode attention inside the decode_in launch (1, the default) or after it (0)
    s.fuse_attention = grid != 0;
    s.reset_fused();
    s.drop_graphs();
    return TINYOAI_OK;
  }
  if (stage == 3) {  // decode attention: grid = positions per block / 64 (0 = by position)
    if (grid != 0 && grid != 1 && grid != 2 && grid != 4 && grid != 8 && grid != 16)
      return fail(TINYOAI_EINVAL, "attention steps %d", grid);
    s.att_steps = grid;
    s.drop_graphs();
    return TINYOAI_OK;
  }
  if (grid <= 0 || grid > (1 << 20) || (threads != 256 && threads != 512))
    return fail(TINYOAI_EINVAL, "launch shape %d x %d", grid, threads);
  switch (stage) {
    case 0: s.grid_in = grid; s.threads_in = threads; s.reset_fused(); break;
    case 1: s.grid_out = grid; s.threads_out = threads; break;
    case 2: s.grid_head = grid; s.threads_head = threads; break;
    default: return fail(TINYOAI_EINVAL, "launch stage %d", stage);
  }
  s.drop_graphs();
  return TINYOAI_OK;
}

int tinyoai_stablelm_profile(tinyoai_model *m, int32_t enable) {
  if (!m || !m->stable) return fail(TINYOAI_EINVAL, "not a StableLM handle");
  m->stable->prof.on = enable != 0;
  m->stable->prof.clear();
  return TINYOAI_OK;
}


int tinyoai_stablelm_profile_read(tinyoai_model *m, double *ms, int64_t *counts, int32_t n_stages) {
  if (!m || !m->stable || !ms || !counts || n_stages < ST_COUNT) return fail(TINYOAI_EINVAL, "invalid profile read");
  for (int i = 0; i < ST_COUNT; i++) {
    ms[i] = m->stable->prof.ms[i];
    counts[i] = m->stable->prof.count[i];
  }
  return ST_COUNT;
}

int tinyoai_weight_upload(int32_t dtype, int64_t rows, int64_t cols, const void *data, uint64_t nbytes,
                          tinyoai_weight **out) {
  if (!out || !data) return fail(TINYOAI_EINVAL, "invalid weight upload arguments");
  *out = nullptr;
  auto w = std::make_unique<tinyoai_weight>();
  hipError_t e = hipGetDevice(&w->device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  e = hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");
  int rc = w->m.upload(dtype, rows, cols, data, nbytes, w->stream);
  if (rc) return rc;
  e = hipStreamSynchronize(w->stream);
  if (e != hipSuccess) return hip_fail(e, "weight upload");
  *out = w.release();
  return TINYOAI_OK;
}

int tinyoai_weight_read_values(tinyoai_weight *w, int64_t offset, int64_t n, float *out) {
  if (!w || !out || offset < 0 || n < 0 || offset + n > (int64_t)w->m.desc.rows * w->m.desc.cols)
    return fail(TINYOAI_EINVAL, "invalid readValues span");
  if (n == 0) return TINYOAI_OK;
  float *dev;
  hipError_t e = hipMalloc(&dev, (size_t)n * 4);
  if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipMalloc: %s", hipGetErrorString(e));
  e = launch_read_values(w->m.desc, offset, n, dev, w->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out, dev, (size_t)n * 4, hipMemcpyDeviceToHost, w->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
  hipFree(dev);
  return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "readValues");
}

}  // extern "C"

// Bytes of operand scratch a product of n rows needs: bf16 planes of the
// matrix-core GEMM, the staged X of the few-row 5/6-bit product, or none
// (one row: the row-streaming matvec; other formats: the vector-unit GEMM).
// K splits of a matrix-core product (the output tiles alone leave most of
// the CUs idle below a few hundred rows: 27 tiles for 128 x 6912), their
// partials within kProductPartialBytes. A rule of the shape alone, so the
// allocating and the no-allocation entry points sum alike.
constexpr size_t kProductPartialBytes = (size_t)32 << 20;
static int product_splits(const MatDesc &m, int n) {
  if (n == 1 || !gemm_mfma_supported(m)) return 1;
  int ks = gemm_splits(m, n, StableModel::kPrefillSplits);
  while (ks > 1 && (size_t)ks * n * m.rows * 4 > kProductPartialBytes) ks--;
  return ks;
}
static size_t product_planes_bytes(const MatDesc &m, int n) {
  return ((size_t)n * m.cols * 2 * gemm_planes(m) + 255) / 256 * 256;
}

static size_t product_scratch(const MatDesc &m, const float *x_dev, int n) {
  if (n == 1) return 0;
  if (gemm_mfma_supported(m)) {
    const int ks = product_splits(m, n);
    return product_planes_bytes(m, n) + (ks > 1 ? (size_t)ks * n * m.rows * 4 : 0);
  }
  if (kq_rows_supported(m, n) && (reinterpret_cast<uintptr_t>(x_dev) & 15) == 0 && m.cols % 4 == 0)
    return kq_rows_stage_bytes(m.cols, n);
  return 0;
}

// out = x * W^T with `scratch` of product_scratch bytes.
static hipError_t product_launch(const MatDesc &m, const float *x_dev, int n, float *out_dev, void *scratch,
                                 hipStream_t st) {
  // One row: the row-streaming matvec, two blocks per CU (6912 x 2560 Q8_0:
  // 7.2 us against 9.4 with four and 8.1 with one).
  if (n == 1) return launch_ln_matvec(m, nullptr, nullptr, 0.0, 0, x_dev, out_dev, device_cu_count() * 2, 256, st);
  if (gemm_mfma_supported(m)) {
    uint16_t *hi = (uint16_t *)scratch, *lo = gemm_planes(m) == 2 ? hi + (size_t)n * m.cols : nullptr;
    const int ks = product_splits(m, n);
    float *part = reinterpret_cast<float *>((char *)scratch + product_planes_bytes(m, n));
    hipError_t e = launch_split_bf16(x_dev, m.cols, m.cols, n, hi, lo, st);
    if (e == hipSuccess) e = launch_gemm_mfma(m, hi, lo, n, ks > 1 ? part : out_dev, m.rows, st, ks);
    if (e == hipSuccess && ks > 1) e = launch_sum_splits(out_dev, part, ks, (int64_t)n * m.rows, st);
    return e;
  }
  if (product_scratch(m, x_dev, n)) return launch_kq_rows(m, x_dev, m.cols, n, out_dev, m.rows, 1, scratch, st);
  return launch_gemm(m, x_dev, n, out_dev, st);
}

extern "C" {

int tinyoai_weight_mul_device(tinyoai_weight *w, const float *x_dev, int32_t n, float *out_dev, void *stream) {
  if (!w || !x_dev || !out_dev || n <= 0) return fail(TINYOAI_EINVAL, "invalid product arguments");
  hipStream_t st = stream ? (hipStream_t)stream : w->stream;
  const MatDesc &m = w->m.desc;
  // The operand scratch grows on demand (the stream is drained before an
  // old buffer is released).
  const size_t need = product_scratch(m, x_dev, n);
  if (need > w->planes_bytes) {
    if (w->planes) {
      hipStreamSynchronize(st);
      hipFree(w->planes);
      w->planes = nullptr;
      w->planes_bytes = 0;
    }
    hipError_t e = hipMalloc(&w->planes, need);
    if (e != hipSuccess) return fail(TINYOAI_ENOMEM, "hipMalloc(%zu): %s", need, hipGetErrorString(e));
    w->planes_bytes = need;
  }
  const hipError_t e = product_launch(m, x_dev, n, out_dev, w->planes, st);
  return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "product launch");
}

}  // extern "C"

// ---------------------------------------------------------------- no-allocation product
// The operand planes of tinyoai_weight_mul_device_noalloc: a file-scope
// device array, one copy on each GPU the library runs on, held until the
// process ends. In host code `scratch` names a host-side stand-in; the
// device address of each GPU's copy comes from hipGetSymbolAddress (once
// per device, with that device current) and only that address is used.
constexpr size_t kScratchValues = (size_t)4 << 20;  // activation values per call (n * cols)
// bf16 hi and lo planes (16 MiB), then the K-split partials (32 MiB)
static __device__ __align__(256) uint16_t scratch[2 * kScratchValues + kProductPartialBytes / 2];

namespace {
constexpr int kMaxDevices = 64;
// Per device: the array's address, the library stream that calls with a
// null stream share, and an event that orders every call's use of the
// array after the previous call's (whatever streams they came on).
struct ScratchDev {
  void *ptr = nullptr;
  hipStream_t stream = nullptr;
  hipEvent_t done = nullptr;
};
std::mutex g_scratch_mu;
ScratchDev g_scratch_dev[kMaxDevices];

// The current device's set-up, made on the first call on that device
// (the caller holds g_scratch_mu).
int scratch_device(ScratchDev **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(TINYOAI_EINVAL, "device %d out of range", dev);
  ScratchDev &d = g_scratch_dev[dev];
  if (!d.ptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if ((e = hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking)) != hipSuccess)
      return hip_fail(e, "no-allocation stream");
    if ((e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming)) != hipSuccess)
      return hip_fail(e, "no-allocation event");
    d.ptr = p;
  }
  *out = &d;
  return TINYOAI_OK;
}
}  // namespace

extern "C" {

int tinyoai_weight_mul_device_noalloc(tinyoai_weight *w, const float *x_dev, int32_t n, float *out_dev, void *stream) {
  if (!w || !x_dev || !out_dev || n <= 0) return fail(TINYOAI_EINVAL, "invalid product arguments");
  const MatDesc &m = w->m.desc;
  if ((size_t)n * m.cols > kScratchValues)
    return fail(TINYOAI_EINVAL, "product of %d x %d activation values exceeds the no-allocation limit of %zu", n, m.cols,
                kScratchValues);
  if (product_scratch(m, x_dev, n) > sizeof(scratch))
    return fail(TINYOAI_EINVAL, "product of %d x %d needs more than the no-allocation limit of %zu bytes", n, m.cols,
                sizeof(scratch));
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev != w->device) return fail(TINYOAI_EINVAL, "the weight lives on device %d, not the current %d", w->device, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchDev *d = nullptr;
  if (int rc = scratch_device(&d)) return rc;
  // A null stream means the library's own stream for this device, so
  // such calls run one after another; a caller's stream waits for the
  // previous call (on any stream) to finish with the array first. Under
  // stream capture the captured graph orders the calls instead.
  hipStream_t st = stream ? (hipStream_t)stream : d->stream;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if ((e = hipStreamIsCapturing(st, &cap)) != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  const bool order = cap == hipStreamCaptureStatusNone;
  if (order && (e = hipStreamWaitEvent(st, d->done, 0)) != hipSuccess) return hip_fail(e, "no-allocation ordering");
  e = product_launch(m, x_dev, n, out_dev, product_scratch(m, x_dev, n) ? d->ptr : nullptr, st);
  if (e == hipSuccess && order) e = hipEventRecord(d->done, st);
  return e == hipSuccess ? TINYOAI_OK : hip_fail(e, "product launch");
}

int tinyoai_weight_mul(tinyoai_weight *w, const float *x, int32_t n, float *out) {
  if (!w || !x || !out || n <= 0) return fail(TINYOAI_EINVAL, "invalid product arguments");
  const MatDesc &m = w->m.desc;
  float *dx = nullptr, *dout = nullptr;
  hipError_t e = hipMalloc(&dx, (size_t)n * m.cols * 4);
  if (e == hipSuccess) e = hipMalloc(&dout, (size_t)n * m.rows * 4);
  if (e != hipSuccess) {
    hipFree(dx);
    return fail(TINYOAI_ENOMEM, "hipMalloc: %s", hipGetErrorString(e));
  }
  e = hipMemcpyAsync(dx, x, (size_t)n * m.cols * 4, hipMemcpyHostToDevice, w->stream);
  int rc = e == hipSuccess ? tinyoai_weight_mul_device(w, dx, n, dout, w->stream) : hip_fail(e, "product input");
  if (!rc) {
    e = hipMemcpyAsync(out, dout, (size_t)n * m.rows * 4, hipMemcpyDeviceToHost, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    if (e != hipSuccess) rc = hip_fail(e, "product output");
  }
  hipStreamSynchronize(w->stream);
  hipFree(dx);
  hipFree(dout);
  return rc;
}

int tinyoai_weight_free(tinyoai_weight *w) {
  if (w) {
    hipStreamSynchronize(w->stream);
    delete w;
  }
  return TINYOAI_OK;
}

}  // extern "C"
