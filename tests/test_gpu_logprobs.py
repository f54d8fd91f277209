"""Log probabilities on the device against the mathematics.

Mirrors summarizeLogits (logprobs.go:60-95) and ForwardWithLogprobs
(mlx.go:53-57; mlx_native.go:300-311): every row normalised over the whole
vocabulary in float64, the target's log probability, and the `count` best
ids in descending order with ties to the lower id. The checker is scipy's
log_softmax (a library routine) and numpy's lexicographic sort, not a
restatement of the Go loop.
"""
import numpy as np
import pytest
from scipy.special import log_softmax

from tinyoai_amd import weights as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from tinyoai_amd import hip as H
    H.lib()
    return H


def expected(logits, targets, count):
    v = logits.astype(np.float64)
    lp = log_softmax(v, axis=-1)
    order = np.stack([np.lexsort((np.arange(v.shape[1]), -v[r]))[:count] for r in range(v.shape[0])])
    return lp[np.arange(v.shape[0]), targets], order, np.take_along_axis(lp, order, axis=1)


@pytest.mark.parametrize("vocab,count", [(65536, 20), (342, 342), (5000, 1024), (7, 1), (5000, 1025),
                                         (65536, 2000), (65536, 65536)])
def test_summarize_random_rows(hip, vocab, count):
    """Random logits (N(0, 4)): chosen and top values within 1e-12 of
    log_softmax (float64 arithmetic on both sides), ids identical; the
    probabilities of a full-vocabulary top list sum to 1. Counts above 1024
    rank their candidates in global scratch (a bitonic sort) instead of
    LDS, up to the whole 65536-entry vocabulary."""
    rng = np.random.default_rng(vocab + count)
    rows = 6
    x = (rng.standard_normal((rows, vocab)) * 4).astype(np.float32)
    t = rng.integers(0, vocab, rows)
    chosen, ids, lp = hip.summarize_logits(x, t, count)
    wc, wi, wl = expected(x, t, count)
    assert np.max(np.abs(chosen - wc)) <= 1e-12 * max(1.0, np.max(np.abs(wc)))
    assert np.array_equal(ids, wi)
    assert np.max(np.abs(lp - wl)) <= 1e-12 * max(1.0, np.max(np.abs(wl)))
    if count == vocab:
        assert np.allclose(np.exp(lp).sum(axis=1), 1.0, atol=1e-12)


def test_summarize_ties_go_to_the_lower_id(hip):
    """Equal logits (quantised rows with many ties, a row of one value, and
    ties straddling the count boundary): ties ordered by ascending id, as
    summarizeLogits keeps them."""
    rng = np.random.default_rng(3)
    x = np.round(rng.standard_normal((4, 3000)) * 2).astype(np.float32)
    x[1] = 0.5
    x[2, :] = -1.0
    x[2, [5, 77, 2999, 1000, 3]] = 2.0  # five tied maxima; count 3 takes ids 3, 5, 77
    t = np.array([0, 10, 2999, 17])
    chosen, ids, lp = hip.summarize_logits(x, t, 3)
    _, wi, wl = expected(x, t, 3)
    assert np.array_equal(ids, wi)
    assert list(ids[1]) == [0, 1, 2] and list(ids[2]) == [3, 5, 77]
    assert np.max(np.abs(lp - wl)) <= 1e-12
    assert abs(chosen[1] - (-np.log(3000.0))) <= 1e-12


@pytest.mark.parametrize("count", [3, 1500])
def test_summarize_signed_zeros_tie(hip, count):
    """-0 and +0 compare equal in summarizeLogits (v > x and v == x), so
    they tie and the lower id goes first even when the +0 entries come
    later and the count boundary falls among them; in both rankings (LDS
    up to 1024 candidates, global scratch beyond)."""
    x = np.full((2, 4000), -3.0, np.float32)
    x[0, [10, 20, 30]] = np.float32(-0.0)
    x[0, [5, 15, 25]] = np.float32(0.0)
    x[1, :2000] = np.float32(-0.0)
    x[1, 2000:] = np.float32(0.0)
    _, ids, _ = hip.summarize_logits(x, np.array([0, 0]), count)
    assert list(ids[0][:3]) == [5, 10, 15]
    assert list(ids[1][: min(count, 2000)]) == list(range(min(count, 2000)))


def test_summarize_refuses_nan_rows(hip):
    """A row holding NaN: the reference's float64 max turns every value
    NaN; the library refuses the request with an error that names the row
    (the other rows' results are not returned either)."""
    x = np.zeros((3, 100), np.float32)
    x[2, 40] = np.nan
    with pytest.raises(hip.TinyoaiError, match="row 2 holds NaN"):
        hip.summarize_logits(x, np.array([0, 1, 2]), 5)
    with pytest.raises(hip.TinyoaiError, match="row 2 holds NaN"):
        hip.summarize_logits(np.tile(x, (1, 30)), np.array([0, 1, 2]), 1100)


def test_forward_with_logprobs_reference_model(hip, oracle, tiny_stablelm):
    """ForwardWithLogprobs on the reference's tiny StableLM: every position of
    a 9-token suffix after a 3-token prefix scored against its target; the
    oracle's per-position logits through log_softmax agree within 1e-4,
    ids identical, the last row's logits within 3e-5; the resident offset
    advances as a forward's does."""
    config, tensors = tiny_stablelm
    ids = [2, 40, 41, 7, 300, 12, 99, 5, 5, 5, 17, 201]
    targets = ids[4:] + [3]
    ref = oracle.StableLM(config, tensors, capacity=32)
    rows = [ref.forward(tok, i) for i, tok in enumerate(ids)]
    f = hip.StableLMForwarder(config, tensors)
    f.forward(0, ids[:3], want_logits=False)
    logits, chosen, top, lp = f.forward_with_logprobs(3, ids[3:], targets, 8)
    assert f.offset == len(ids)
    want = np.stack(rows[3:])
    wc, wi, wl = expected(want, np.array(targets), 8)
    assert np.max(np.abs(chosen - wc)) <= 1e-4
    assert np.max(np.abs(lp - wl)) <= 1e-4
    assert np.array_equal(top, wi)
    assert np.max(np.abs(logits - rows[-1])) <= 3e-5
    with pytest.raises(hip.TinyoaiError):
        f.forward_with_logprobs(f.offset, [1, 2], [1], 4)  # targets do not align
    with pytest.raises(hip.TinyoaiError):
        f.forward_with_logprobs(f.offset, [1], [config["vocab_size"]], 4)
    f.close()


def test_forward_with_logprobs_3b_shapes(hip, oracle):
    """StableLM-3B layer shapes (two layers, Q8_0, vocab 65536): a 40-token
    prompt scored in one call (one decode-sized call after it too), against
    the oracle's logits per position: log probabilities within 1e-3 of the
    logits' range, top-20 ids identical."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=256))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=7)
    rng = np.random.default_rng(19)
    ids = rng.integers(0, 65536, 41).astype(np.int32)
    targets = np.concatenate([ids[1:40], [int(ids[0])]])
    oracle.set_threads(8)
    ref = oracle.StableLM(config, tensors, capacity=64)
    rows = np.stack([ref.forward(int(t), i) for i, t in enumerate(ids[:40])])
    f = hip.StableLMForwarder(config, tensors)
    logits, chosen, top, lp = f.forward_with_logprobs(0, ids[:40], targets, 20)
    wc, wi, wl = expected(rows, targets, 20)
    span = float(np.max(np.ptp(rows, axis=1)))
    assert np.max(np.abs(chosen - wc)) <= 1e-3 * span
    assert np.max(np.abs(lp - wl)) <= 1e-3 * span
    assert np.array_equal(top, wi)
    want40 = ref.forward(int(ids[40]), 40)
    logits, chosen, top, lp = f.forward_with_logprobs(40, ids[40:41], ids[:1], 20)
    wc, wi, wl = expected(want40[None], ids[:1], 20)
    assert abs(chosen[0] - wc[0]) <= 1e-3 * float(np.ptp(want40))
    assert np.array_equal(top, wi)
    f.close()
