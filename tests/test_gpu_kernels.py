"""Kernel-level parity on the GPU: bit-exact dequantization and matvec /
batched products against the CPU oracle (float64 accumulation).

Mirrors TestKQuantReference's decode checks (quant_k_test.go:14-62),
TestBatchedProjection (prefill_test.go:183-212) and TestMatvecLengths
(dot_test.go:214-260) at the isolated Q8_0 kernel shape 6912 x 2560.
"""
import numpy as np
import pytest

from tinyoai_amd import weights as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from tinyoai_amd import hip as H
    H.lib()
    return H


def _q8_edge(rows, cols, seed):
    rng = np.random.default_rng(seed)
    nb = rows * cols // 32
    d = rng.integers(0, 0x7C00, nb).astype(np.uint16)
    d[:8] = [0, 1, 0x3FF, 0x8001, 0x8000, 0x3C00, 0xBC00, 0x2400]
    d[8:64] |= 0x8000
    qs = rng.integers(-128, 128, (nb, 32)).astype(np.int8)
    return W.Tensor(W.Q8_0, rows, cols, W.encode_q8_0(d, qs))


def _tensor(dtype, rows, cols, seed):
    rng = np.random.default_rng(seed)
    if dtype == W.Q8_0:
        return W.synthetic_q8_0(rows, cols, rng)
    if dtype == W.BF16:
        return W.synthetic_bf16(rows, cols, rng)
    if dtype == W.F16:
        v = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
        return W.Tensor(W.F16, rows, cols, W.f32_to_f16_bits(v).view(np.uint8))
    return W.synthetic_f32(rows, cols, rng)


@pytest.mark.parametrize("dtype,cols", [(W.Q8_0, 1024), (W.BF16, 255), (W.F32, 33), (W.F16, 40)])
def test_read_values_bit_exact(hip, oracle, dtype, cols):
    t = _q8_edge(16, cols, 3) if dtype == W.Q8_0 else _tensor(dtype, 16, cols, 3)
    if dtype == W.F16:  # include subnormal, signed zero and non-finite patterns
        bits = t.data.view(np.uint16).copy()
        bits[:6] = [0x0001, 0x8000, 0x7C00, 0xFC00, 0x03FF, 0x7E01]
        t = W.Tensor(W.F16, 16, cols, bits.view(np.uint8))
    g = hip.Weight(t)
    n = t.rows * t.cols
    got = g.read_values(0, n)
    want = oracle.read_values(oracle.weight(t.dtype, t.rows, t.cols, t.data), 0, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(g.read_values(37, 100), want[37:137])


@pytest.mark.parametrize("dtype", [W.Q8_0, W.BF16, W.F32, W.F16])
@pytest.mark.parametrize("cols", [32, 256, 2560, 7552])
def test_matvec_against_float64(hip, oracle, dtype, cols):
    """mulScratch on the GPU vs mulRowsScalar (dot.go:14-70): fp32
    accumulation within 2e-5 * max(1, sum |x w|)."""
    rows = 37
    t = _tensor(dtype, rows, cols, cols)
    g = hip.Weight(t)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(cols).astype(np.float32)
    got = g.mul(x)[0]
    w = oracle.weight(t.dtype, rows, cols, t.data)
    want = oracle.mul(w, x)
    dense = oracle.read_values(w, 0, rows * cols).reshape(rows, cols).astype(np.float64)
    mag = np.abs(dense) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(got - want) <= 2e-5 * np.maximum(1, mag))


@pytest.mark.parametrize("n", [2, 7, 64, 65, 128])
def test_batched_projection(hip, oracle, n):
    """TestBatchedProjection tolerance 2e-4 * max(1, |y|)."""
    for dtype in (W.Q8_0, W.BF16, W.F32):
        t = _tensor(dtype, 7, 2816, 621)
        g = hip.Weight(t)
        x = np.sin(np.arange(n * 2816) * 0.13).astype(np.float32).reshape(n, 2816)
        got = g.mul(x)
        want = x.astype(np.float64) @ oracle.read_values(oracle.weight(t.dtype, 7, 2816, t.data), 0, 7 * 2816
                                                         ).reshape(7, 2816).astype(np.float64).T
        assert np.all(np.abs(got - want) <= 2e-4 * np.maximum(1, np.abs(want))), dtype


@pytest.mark.parametrize("m", [1, 128])
def test_isolated_q8_0_kernel_shape(hip, oracle, m):
    """The isolated Q8_0 kernel workload: W 6912 x 2560 (int8 uniform
    [-127, 127], d = |N(0, 0.02)| / 127), x ~ N(0, 1), M = 1 and M = 128,
    against the float64 dequant-dot of the oracle."""
    rng = np.random.default_rng(2024)
    t = W.synthetic_q8_0(6912, 2560, rng)
    x = rng.standard_normal((m, 2560)).astype(np.float32)
    g = hip.Weight(t)
    got = g.mul(x)
    w = oracle.weight(t.dtype, 6912, 2560, t.data)
    oracle.set_threads(8)
    want = np.stack([oracle.mul(w, x[i]) for i in range(m)])
    dense = oracle.read_values(w, 0, 6912 * 2560).reshape(6912, 2560).astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(dense).T
    assert np.all(np.abs(got - want) <= 2e-5 * np.maximum(1, mag))


# ---------------------------------------------------------------- 5/6-bit formats
KQ_GOLDEN = {"Q5_K": W.Q5_K, "Q6_K": W.Q6_K, "Q5_1": W.Q5_1}


def _kq_golden(name):
    import os
    base = os.path.join(os.path.dirname(__file__), "golden", name.lower())
    return np.fromfile(base + ".bin", np.uint8), np.fromfile(base + "-f32.bin", np.float32)


@pytest.mark.parametrize("name", sorted(KQ_GOLDEN))
def test_kquant_golden_on_device(hip, name):
    """TestKQuantReference (quant_k_test.go:14-62) on the device: readValues of
    the reference's golden blocks bit for bit, partial spans included."""
    raw, want = _kq_golden(name)
    g = hip.Weight(W.Tensor(KQ_GOLDEN[name], 4, 2048, raw))
    got = g.read_values(0, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for start, n in [(0, 1), (255, 3), (257, 511), (1000, 777)]:
        assert np.array_equal(g.read_values(start, n), want[start:start + n])


@pytest.mark.parametrize("dtype", [W.Q4_K, W.Q5_K, W.Q6_K])
def test_kquant_synthetic_decode(hip, oracle, dtype):
    """Seeded super-blocks (random bits, scales and mins): device readValues
    equals the oracle's decodeKBlock bit for bit (Q4_K through its Q5_K
    embedding, pinned by the golden vectors)."""
    rng = np.random.default_rng(dtype)
    t = W.synthetic_kquant(dtype, 12, 1536, rng)
    want = oracle.read_values(oracle.weight(dtype, 12, 1536, t.data), 0, 12 * 1536)
    got = hip.Weight(t).read_values(0, 12 * 1536)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q5_1_tail_row(hip, oracle):
    """A 7552-wide Q5_1 row (quant_k_test.go:75-87): decode and the one-row
    product against float64."""
    raw, want = _kq_golden("Q5_1")
    t = W.Tensor(W.Q5_1, 1, 7552, raw[: 7552 // 32 * 24])
    g = hip.Weight(t)
    assert np.array_equal(g.read_values(0, 7552), want[:7552])
    x = np.sin(np.arange(7552) * 0.19).astype(np.float32)
    exp = float(x.astype(np.float64) @ want[:7552].astype(np.float64))
    assert abs(float(g.mul(x)[0, 0]) - exp) <= 2e-4 * max(1, abs(exp))


@pytest.mark.parametrize("dtype", [W.Q5_1, W.Q4_K, W.Q5_K, W.Q6_K])
@pytest.mark.parametrize("n,rows,cols", [(1, 37, 2560), (7, 37, 2560), (128, 37, 2560), (2, 300, 6912),
                                         (16, 129, 2560), (17, 300, 1024), (32, 300, 6912)])
def test_kquant_products(hip, oracle, dtype, n, rows, cols):
    """mulScratch (n = 1) and mulBatch (n > 1) of 5/6-bit matrices against
    float64 of the decoded values: 2e-5 * sum |x w| for the single row,
    2e-4 * max(1, |y|) batched (the reference's tolerances). 2 to 32 rows
    take the few-row matrix-core product (row counts past its 128-row
    blocks, K ranges of several staging windows)."""
    rng = np.random.default_rng(100 + n)
    if dtype == W.Q5_1:
        raw, _ = _kq_golden("Q5_1")
        reps = -(-rows * cols // 32 * 24 // raw.size)
        t = W.Tensor(dtype, rows, cols, np.tile(raw, reps)[: rows * cols // 32 * 24].copy())
    else:
        t = W.synthetic_kquant(dtype, rows, cols, rng)
    g = hip.Weight(t)
    dense = oracle.read_values(oracle.weight(dtype, rows, cols, t.data), 0, rows * cols).reshape(rows, cols)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    got = g.mul(x)
    exp = x.astype(np.float64) @ dense.astype(np.float64).T
    if n == 1:
        mag = np.abs(x.astype(np.float64)) @ np.abs(dense.astype(np.float64)).T
        assert np.all(np.abs(got - exp) <= 2e-5 * np.maximum(1, mag))
    else:
        assert np.all(np.abs(got - exp) <= 2e-4 * np.maximum(1, np.abs(exp)))
