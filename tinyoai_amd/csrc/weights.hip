// Weight upload kernels: regroup GGUF-encoded bytes into the plane layout of
// formats.h (optionally placing rows into a fused matrix under a row map
// and column offset), and the bit-exact dequantizer readValues
// (matmul.go:12-50).
#include "kernels.h"

namespace {

// Destination row of source row r under a RowMap (kernels.h).
__device__ __forceinline__ int64_t map_row(const RowMap &m, int64_t r) {
  switch (m.kind) {
    case ROWMAP_HEADS: {  // rotary pairs (j, j + rot/2) adjacent within each head
      const int64_t head = r / m.hd, j = r % m.hd;
      const int rh = m.rot / 2;
      int64_t p;
      if (j < rh) p = 2 * j;
      else if (j < m.rot) p = 2 * (j - rh) + 1;
      else p = j;
      return m.offset + head * m.hd + p;
    }
    case ROWMAP_INTERLEAVE: return m.offset + 2 * r + m.phase;
    default: return m.offset + r;
  }
}

// Q8_0 block {fp16 d, int8 q[32]} (34 B) -> vals int8, meta fp16, at the
// mapped row and the column offset col0 (a multiple of 32).
__global__ void repack_q8_0_kernel(const uint8_t *raw, int64_t rows, int64_t nb, MatDesc dst, RowMap map,
                                   int64_t col0) {
  uint8_t *vals = const_cast<uint8_t *>(dst.vals);
  uint8_t *meta = const_cast<uint8_t *>(dst.meta);
  const int64_t total = rows * nb;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = map_row(map, i / nb), b = i % nb;
    const uint8_t *src = raw + i * 34;
    uint8_t *qd = vals + row * dst.vstride + col0 + b * 32;
    for (int k = 0; k < 32; k++) qd[k] = src[2 + k];
    meta[row * dst.mstride + (col0 / 32 + b) * 2] = src[0];
    meta[row * dst.mstride + (col0 / 32 + b) * 2 + 1] = src[1];
  }
}

// Row-major values (row_bytes per source row) placed at byte offset col0b
// of the mapped destination row; the padding of each destination row past
// the last segment is cleared by the host beforehand.
__global__ void repack_plain_kernel(const uint8_t *raw, int64_t rows, int64_t row_bytes, MatDesc dst, RowMap map,
                                    int64_t col0b) {
  uint8_t *vals = const_cast<uint8_t *>(dst.vals);
  const int64_t total = rows * row_bytes;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / row_bytes, c = i % row_bytes;
    vals[map_row(map, r) * dst.vstride + col0b + c] = raw[i];
  }
}

__global__ void read_values_kernel(MatDesc m, int64_t offset, int64_t n, float *out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = offset + i;
    out[i] = mat_value(m, e / m.cols, e % m.cols);
  }
}

}  // namespace

hipError_t launch_repack(int fmt, const uint8_t *raw, int64_t rows, int64_t cols, const MatDesc &dst,
                         const RowMap &map, int64_t col0, hipStream_t st) {
  if (fmt == FMT_Q8_0) {
    hipLaunchKernelGGL(repack_q8_0_kernel, dim3(4096), dim3(256), 0, st, raw, rows, cols / 32, dst, map, col0);
  } else {
    const int64_t width = fmt == FMT_F32 ? 4 : 2;
    hipLaunchKernelGGL(repack_plain_kernel, dim3(4096), dim3(256), 0, st, raw, rows, cols * width, dst, map,
                       col0 * width);
  }
  return hipGetLastError();
}

hipError_t launch_place_bytes(const uint8_t *src, int64_t rows, int64_t row_bytes, uint8_t *dst, int64_t dst_stride,
                              int64_t col0b, const RowMap &map, hipStream_t st) {
  MatDesc d{};
  d.vals = dst;
  d.vstride = dst_stride;
  hipLaunchKernelGGL(repack_plain_kernel, dim3(4096), dim3(256), 0, st, src, rows, row_bytes, d, map, col0b);
  return hipGetLastError();
}

hipError_t launch_read_values(const MatDesc &m, int64_t offset, int64_t n, float *out, hipStream_t st) {
  hipLaunchKernelGGL(read_values_kernel, dim3(1024), dim3(256), 0, st, m, offset, n, out);
  return hipGetLastError();
}
