// Weight upload kernels: regroup GGUF-encoded bytes into the plane layout of
// formats.h, and the bit-exact dequantizer readValues (matmul.go:12-50).
#include "kernels.h"

namespace {

// Q8_0 block {fp16 d, int8 q[32]} (34 B) -> vals int8 [rows][cols], meta fp16 [rows][cols/32].
__global__ void repack_q8_0_kernel(const uint8_t *raw, int64_t rows, int64_t nb, MatDesc dst) {
  uint8_t *vals = const_cast<uint8_t *>(dst.vals);
  uint8_t *meta = const_cast<uint8_t *>(dst.meta);
  const int64_t total = rows * nb;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / nb, b = i % nb;
    const uint8_t *src = raw + i * 34;
    uint8_t *qd = vals + row * dst.vstride + b * 32;
    for (int k = 0; k < 32; k++) qd[k] = src[2 + k];
    meta[row * dst.mstride + b * 2] = src[0];
    meta[row * dst.mstride + b * 2 + 1] = src[1];
  }
}

// Row-major values of `width` bytes each into rows padded to dst.vstride.
__global__ void repack_pad_kernel(const uint8_t *raw, int64_t rows, int64_t row_bytes, MatDesc dst) {
  uint8_t *vals = const_cast<uint8_t *>(dst.vals);
  const int64_t total = rows * dst.vstride;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / dst.vstride, c = i % dst.vstride;
    vals[i] = c < row_bytes ? raw[row * row_bytes + c] : 0;
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
                         hipStream_t st) {
  if (fmt == FMT_Q8_0) {
    hipLaunchKernelGGL(repack_q8_0_kernel, dim3(4096), dim3(256), 0, st, raw, rows, cols / 32, dst);
  } else {
    const int64_t width = fmt == FMT_F32 ? 4 : 2;
    hipLaunchKernelGGL(repack_pad_kernel, dim3(4096), dim3(256), 0, st, raw, rows, cols * width, dst);
  }
  return hipGetLastError();
}

hipError_t launch_read_values(const MatDesc &m, int64_t offset, int64_t n, float *out, hipStream_t st) {
  hipLaunchKernelGGL(read_values_kernel, dim3(1024), dim3(256), 0, st, m, offset, n, out);
  return hipGetLastError();
}
