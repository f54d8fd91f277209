"""The legacy Llama forwarder on the GPU against the oracle's
Model.transformer restatement (model.go:407-481).

Mirrors TestLlamaMLXForwardParity (mlx_llama_native_test.go:51-134): the
prompt in 64-token chunks with every logit row, then greedy tokens one at a
time; every row within KL 1e-6 of the CPU engine's distribution, the same
argmax, finite values. The reference prompt is BPE text; no tokenizer runs
here, so the prompt is BOS followed by seeded ids in [3, 512).
"""
import os

import numpy as np
import pytest

from tinyoai_amd import weights as W

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def stories():
    return W.read_llama2c(os.path.join(GOLDEN, "stories260K.bin"))


def _kl(want, got):
    p = np.exp(want.astype(np.float64) - want.max())
    p /= p.sum()
    q = np.exp(got.astype(np.float64) - got.max())
    q /= q.sum()
    return float(np.sum(p * (np.log(p) - np.log(q))))


def _check(want, got, tie=0.0):
    """KL within 1e-6 and the same argmax (or, with tie > 0, an argmax
    whose CPU logit is within tie of the CPU maximum: seeded N(0, 0.02)
    weights give flat logits with near ties)."""
    assert np.all(np.isfinite(got))
    a, b = int(np.argmax(want)), int(np.argmax(got))
    assert a == b or want[a] - want[b] <= tie, (a, b, want[a] - want[b])
    assert _kl(want, got) <= 1e-6


@pytest.mark.parametrize("single", [1, 0], ids=["one_launch", "per_layer"])
@pytest.mark.parametrize("prompt,generated", [(128, 256), (480, 32)])
def test_forward_parity(oracle, stories, prompt, generated, single):
    from tinyoai_amd import hip
    c, w = stories
    ref = oracle.Llama(c, w)
    f = hip.LlamaForwarder(c, w)
    f.set_launch("single_launch", single)
    rng = np.random.default_rng(prompt)
    ids = np.concatenate([[1], rng.integers(3, 512, prompt - 1)]).astype(np.int32)
    want = None
    for pos in range(0, prompt, 64):
        end = min(pos + 64, prompt)
        got = f.forward(pos, ids[pos:end], all_logits=True)
        assert got.shape == (end - pos, c["vocab_size"])
        for i in range(pos, end):
            want = ref.transformer(int(ids[i]), i)
            _check(want, got[i - pos])
    for i in range(generated):
        tok = int(np.argmax(want))
        got = f.forward(prompt + i, [tok])
        want = ref.transformer(tok, prompt + i)
        _check(want, got)
    f.close()
    ref.close()


def test_one_launch_long_call(oracle, stories):
    """One forward of 300 tokens (two launches of the one-launch kernel:
    256 tokens, then 44) with every row, then greedy tokens: the same bar
    as above against the CPU engine."""
    from tinyoai_amd import hip
    c, w = stories
    ref = oracle.Llama(c, w)
    f = hip.LlamaForwarder(c, w)
    rng = np.random.default_rng(300)
    ids = np.concatenate([[1], rng.integers(3, 512, 299)]).astype(np.int32)
    got = f.forward(0, ids, all_logits=True)
    assert got.shape == (300, c["vocab_size"])
    want = None
    for i in range(300):
        want = ref.transformer(int(ids[i]), i)
        _check(want, got[i])
    for i in range(8):
        tok = int(np.argmax(want))
        got = f.forward(300 + i, [tok])
        want = ref.transformer(tok, 300 + i)
        _check(want, got)
    f.close()
    ref.close()


def test_one_launch_matches_per_layer_kernels(stories):
    """The one-launch kernel and the per-layer kernels on the same calls:
    logits within 1e-4 of their range (the sums' order differs) and the
    same argmax, for a 64-token prompt and 64 greedy steps."""
    from tinyoai_amd import hip
    c, w = stories
    fs = [hip.LlamaForwarder(c, w) for _ in range(2)]
    fs[1].set_launch("single_launch", 0)
    rng = np.random.default_rng(64)
    ids = np.concatenate([[1], rng.integers(3, 512, 63)]).astype(np.int32)
    a, b = (f.forward(0, ids, all_logits=True) for f in fs)
    for i in range(64):
        assert np.max(np.abs(a[i] - b[i])) <= 1e-4 * float(np.ptp(b[i])), i
        assert int(np.argmax(a[i])) == int(np.argmax(b[i])), i
    tok = int(np.argmax(a[-1]))
    for i in range(64):
        a, b = (f.forward(64 + i, [tok]) for f in fs)
        assert np.max(np.abs(a - b)) <= 1e-4 * float(np.ptp(b)), i
        assert int(np.argmax(a)) == int(np.argmax(b)), i
        tok = int(np.argmax(b))
    for f in fs:
        f.close()


@pytest.mark.parametrize("layers,vocab,seq", [(1, 300, 100), (8, 512, 77), (3, 97, 512)])
def test_one_launch_edge_shapes(oracle, layers, vocab, seq):
    """Seeded models of the stories260K widths at the one-launch kernel's
    edges: one layer (its next token reads the position the same launch
    just stored), eight layers, vocabularies below 512 (classifier rows
    past the vocabulary), contexts shorter than 512 (K/V streams reaching
    into the buffer's padding). Prompt in one call with every row, then
    greedy steps to the end of the context; the CPU engine's bar and the
    per-layer kernels' logits within 1e-4 of their range."""
    from tinyoai_amd import hip
    c = dict(dim=64, hidden_dim=172, n_layers=layers, n_heads=8, n_kv_heads=4, vocab_size=vocab, seq_len=seq)
    w = W.synthetic_llama(c, seed=layers * 1000 + vocab)
    ref = oracle.Llama(c, w)
    f, g = hip.LlamaForwarder(c, w), hip.LlamaForwarder(c, w)
    g.set_launch("single_launch", 0)
    rng = np.random.default_rng(seq)
    prompt = min(40, seq - 1)
    ids = rng.integers(0, vocab, prompt).astype(np.int32)
    got, per_layer = f.forward(0, ids, all_logits=True), g.forward(0, ids, all_logits=True)
    want = None
    for i in range(prompt):
        want = ref.transformer(int(ids[i]), i)
        _check(want, got[i], tie=1e-5 * float(np.ptp(want)))
        assert np.max(np.abs(got[i] - per_layer[i])) <= 1e-4 * float(np.ptp(per_layer[i])), i
    for pos in range(prompt, seq):
        tok = int(np.argmax(want))
        a, b = f.forward(pos, [tok]), g.forward(pos, [tok])
        want = ref.transformer(tok, pos)
        _check(want, a, tie=1e-5 * float(np.ptp(want)))
        assert np.max(np.abs(a - b)) <= 1e-4 * float(np.ptp(b)), pos
    for x in (f, g, ref):
        x.close()


def test_grouped_query_shapes(oracle):
    """A seeded llama2.c model with wider heads and 4:1 grouped KV: per-step
    logits within 1e-3 of their range (fp32 path) and the same greedy ids."""
    from tinyoai_amd import hip
    c = dict(dim=256, hidden_dim=688, n_layers=3, n_heads=8, n_kv_heads=2, vocab_size=1000, seq_len=160)
    w = W.synthetic_llama(c, seed=9)
    ref = oracle.Llama(c, w)
    f = hip.LlamaForwarder(c, w)
    with pytest.raises(hip.TinyoaiError):
        f.set_launch("single_launch", 1)  # not the stories260K shape
    tok = 1
    for pos in range(100):
        got = f.forward(pos, [tok])
        want = ref.transformer(tok, pos)
        assert np.max(np.abs(got - want)) <= 1e-3 * float(np.ptp(want)), pos
        assert int(np.argmax(got)) == int(np.argmax(want)), pos
        tok = int(np.argmax(want))
    f.close()
    ref.close()


def test_prefix_rewind_and_errors(stories):
    """Forward replaces the suffix after prefix (rewind allowed); invalid
    prefixes, tokens and lengths are rejected and reset the cache."""
    from tinyoai_amd import hip
    c, w = stories
    f = hip.LlamaForwarder(c, w)
    ids = np.array([1, 50, 60, 70, 80, 90], np.int32)
    full = f.forward(0, ids, all_logits=True)
    again = f.forward(3, ids[3:], all_logits=True)  # rewind to 3 and redo
    assert np.array_equal(again, full[3:])
    last = f.forward(0, ids)
    assert np.array_equal(last, full[-1])
    for bad in [lambda: f.forward(7, [5]),           # prefix beyond the cache
                lambda: f.forward(0, [512]),         # token outside the vocabulary
                lambda: f.forward(0, [-1]),
                lambda: f.forward(0, np.zeros(c["seq_len"] + 1, np.int32))]:
        with pytest.raises(hip.TinyoaiError):
            bad()
    f.reset()
    with pytest.raises(hip.TinyoaiError):
        f.forward(1, [5])  # nothing resident after reset
    assert np.array_equal(f.forward(0, ids, all_logits=True), full)
    f.close()
