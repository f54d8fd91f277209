"""The no-allocation product (tinyoai_weight_mul_device_noalloc) against the
allocating one (tinyoai_weight_mul_device) through the C ABI.

The two run the same kernels; only where the activations' bf16 operand
planes live differs (the library's per-GPU array instead of a buffer grown
with hipMalloc), so the outputs must be bit-identical. Each weight takes
calls in a row with shrinking inputs (the array keeps the previous call's
planes), and an input beyond the array's limit is refused before any work.

Device buffers come from the HIP runtime the library itself is linked
against (torch bundles another one, which cannot initialise the device
once this one has in the same process).
"""
import ctypes as C

import numpy as np
import pytest

from tinyoai_amd import weights as W

pytestmark = pytest.mark.gpu


class DeviceBuffers:
    """hipMalloc'd buffers of the library's own HIP runtime."""

    def __init__(self):
        from tinyoai_amd import hip
        hip.lib()  # loads libamdhip64 as the library's dependency
        self.rt = C.CDLL("libamdhip64.so.7")
        self.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.rt.hipFree.argtypes = [C.c_void_p]
        self.rt.hipDeviceSynchronize.argtypes = []
        self.ptrs = []

    def alloc(self, nbytes):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), nbytes) == 0
        self.ptrs.append(p.value)
        return p.value

    def upload(self, a: np.ndarray):
        p = self.alloc(a.nbytes)
        assert self.rt.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0  # host to device
        return p

    def download(self, p, shape):
        out = np.empty(shape, np.float32)
        assert self.rt.hipDeviceSynchronize() == 0
        assert self.rt.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0  # device to host
        return out

    def close(self):
        for p in self.ptrs:
            self.rt.hipFree(p)
        self.ptrs = []


@pytest.mark.parametrize("dtype,rows,cols", [(W.Q8_0, 1000, 2560), (W.BF16, 512, 1024), (W.Q4_K, 300, 512)])
def test_no_alloc_product_matches_allocating_entry_point(dtype, rows, cols):
    from tinyoai_amd import hip
    rng = np.random.default_rng(rows + cols)
    if dtype == W.Q8_0:
        t = W.synthetic_q8_0(rows, cols, rng)
    elif dtype == W.BF16:
        t = W.synthetic_bf16(rows, cols, rng)
    else:
        t = W.synthetic_kquant(dtype, rows, cols, rng)
    buf = DeviceBuffers()
    w = hip.Weight(t)
    try:
        for n in (96, 17, 1):
            x = buf.upload(rng.standard_normal((n, cols)).astype(np.float32))
            y1 = buf.upload(np.zeros((n, rows), np.float32))
            y2 = buf.upload(np.full((n, rows), np.nan, np.float32))
            w.mul_device(x, n, y1)
            w.mul_device_noalloc(x, n, y2)
            a, b = buf.download(y1, (n, rows)), buf.download(y2, (n, rows))
            assert np.array_equal(a, b), (dtype, n)
            assert np.all(np.isfinite(b))
        limit = (4 << 20) // cols
        with pytest.raises(hip.TinyoaiError, match="no-allocation limit"):
            w.mul_device_noalloc(x, limit + 1, y1)
    finally:
        w.close()
        buf.close()


def test_no_alloc_calls_on_two_weights_are_ordered():
    """Calls with a null stream on two weights, back to back, each on a
    weight whose own stream would let them overlap: both results equal the
    allocating entry point's (the library runs such calls one after
    another on its own stream, so the second does not overwrite the
    first's operand planes or partials while that one still reads them)."""
    from tinyoai_amd import hip
    rng = np.random.default_rng(77)
    t1, t2 = W.synthetic_q8_0(2048, 2560, rng), W.synthetic_bf16(1536, 2560, rng)
    buf = DeviceBuffers()
    w1, w2 = hip.Weight(t1), hip.Weight(t2)
    try:
        n = 128
        x1 = buf.upload(rng.standard_normal((n, 2560)).astype(np.float32))
        x2 = buf.upload(rng.standard_normal((n, 2560)).astype(np.float32))
        r1, r2 = buf.upload(np.zeros((n, 2048), np.float32)), buf.upload(np.zeros((n, 1536), np.float32))
        w1.mul_device(x1, n, r1)
        w2.mul_device(x2, n, r2)
        want1, want2 = buf.download(r1, (n, 2048)), buf.download(r2, (n, 1536))
        for _ in range(3):
            y1 = buf.upload(np.full((n, 2048), np.nan, np.float32))
            y2 = buf.upload(np.full((n, 1536), np.nan, np.float32))
            w1.mul_device_noalloc(x1, n, y1)
            w2.mul_device_noalloc(x2, n, y2)
            assert np.array_equal(buf.download(y1, (n, 2048)), want1)
            assert np.array_equal(buf.download(y2, (n, 1536)), want2)
    finally:
        w1.close()
        w2.close()
        buf.close()

