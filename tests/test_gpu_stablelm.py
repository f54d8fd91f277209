"""End-to-end StableLM parity of the HIP forwarder against the reference's
fixtures and the CPU oracle.

Mirrors TestStableLMReference (stablelm_test.go:50-82), TestBatchedPrefill
(prefill_test.go:217-277), TestHalfKVPrefixReuse (kv_cache_test.go:45-80)
and the forwarder semantics of nativeMLX.Forward (mlx_native.go:292-495).
"""
import json
import os

import numpy as np
import pytest

from tinyoai_amd import weights as W

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
HELLO_ABC = [2, 340, 328, 331]  # see test_oracle.HELLO_ABC


@pytest.fixture(scope="module")
def hip():
    from tinyoai_amd import hip as H
    H.lib()
    return H


@pytest.fixture(scope="module")
def expected():
    with open(os.path.join(GOLDEN, "stablelm", "expected.json")) as f:
        return json.load(f)


def greedy(fwd, ids, max_tokens, eos):
    """MLX.generate's greedy path over the forwarder (mlx.go:342-468)."""
    logits = fwd.forward(0, ids, True)
    out, resident = [], len(ids)
    for n in range(max_tokens):
        tok = int(np.argmax(logits))
        out.append(tok)
        if tok == eos:
            break
        if n + 1 < max_tokens:
            logits = fwd.forward(resident, [tok], True)
            resident += 1
    return out


def test_reference_logits_sequential(hip, tiny_stablelm, expected):
    """Seven one-token forwards against Transformers fp32 within 3e-5."""
    config, tensors = tiny_stablelm
    f = hip.StableLMForwarder(config, tensors)
    for pos, tok in enumerate(expected["input_ids"]):
        got = f.forward(pos, [tok])
        assert np.max(np.abs(got - np.array(expected["logits"][pos], np.float32))) <= 3e-5, pos
    assert f.offset == len(expected["input_ids"])


def test_reference_logits_batched(hip, tiny_stablelm, expected):
    """One batched prefill forward; last-row logits within 3e-5."""
    config, tensors = tiny_stablelm
    f = hip.StableLMForwarder(config, tensors)
    ids = expected["input_ids"]
    got = f.forward(0, ids)
    assert np.max(np.abs(got - np.array(expected["logits"][-1], np.float32))) <= 3e-5


@pytest.mark.parametrize("kv_bits", [32, 16])
def test_reference_greedy(hip, tiny_stablelm, expected, kv_bits):
    config, tensors = tiny_stablelm
    f = hip.StableLMForwarder(config, tensors)
    f.set_kv_bits(kv_bits)
    assert greedy(f, HELLO_ABC, 8, config["eos_token_id"]) == expected["generation"]["ids"]


@pytest.mark.parametrize("n", [2, 17, 63, 64, 65, 129, 257])
def test_batched_prefill_against_oracle(hip, oracle, tiny_stablelm, n):
    """TestBatchedPrefill: a 7-token prefix, then a batched suffix; logits and
    KV against the oracle's sequential forwards within 3e-5, then one decode."""
    config, tensors = tiny_stablelm
    config = dict(config, max_position_embeddings=384)
    ids = [32 + (i * 13) % 250 for i in range(n + 7)]
    seq = oracle.StableLM(config, tensors, capacity=384)
    for i, tok in enumerate(ids):
        want = seq.forward(tok, i)
    f = hip.StableLMForwarder(config, tensors)
    f.forward(0, ids[:7], False)
    got = f.forward(7, ids[7:])
    assert np.max(np.abs(got - want)) <= 3e-5
    for layer in range(config["num_hidden_layers"]):
        k1, v1 = seq.read_kv(layer, 0, len(ids))
        k2, v2 = f.read_kv(layer, 0, len(ids))
        assert np.max(np.abs(k1 - k2)) <= 3e-5 and np.max(np.abs(v1 - v2)) <= 3e-5
    assert np.max(np.abs(seq.forward(123, len(ids)) - f.forward(len(ids), [123]))) <= 3e-5


def test_prefix_rewind_and_errors(hip, tiny_stablelm):
    """Forward replaces the suffix after `prefix` (rewind allowed); invalid
    requests fail, and a failed forward leaves no resident prefix."""
    config, tensors = tiny_stablelm
    f = hip.StableLMForwarder(config, tensors)
    ids = [5, 9, 13, 17, 21, 25]
    full = f.forward(0, ids)
    f.forward(0, [5, 9, 100, 101])
    assert f.offset == 4
    rewound = f.forward(2, ids[2:])
    assert np.max(np.abs(rewound - full)) <= 1e-6
    with pytest.raises(hip.TinyoaiError):
        f.forward(f.offset + 1, [1])  # prefix beyond the resident tokens
    with pytest.raises(hip.TinyoaiError):
        f.forward(0, [config["vocab_size"]])
    with pytest.raises(hip.TinyoaiError):
        f.forward(0, list(range(config["max_position_embeddings"] + 1)))
    assert f.offset == 6  # validation failures happen before any work
    assert f.set_kv_bits(16) is True and f.offset == 0
    assert f.set_kv_bits(16) is False
    # LimitCache (mlx_native.go:231-244): cleared only when the retained
    # capacity exceeds the limit, which also becomes the capacity reserved
    # at the next allocation. The precision change released the KV, so
    # nothing is retained; six tokens then take the reserved 32 positions.
    assert f.limit_cache(32) is False
    f.forward(0, ids)
    assert f.offset == 6
    assert f.limit_cache(32) is False and f.offset == 6
    assert f.limit_cache(16) is True and f.offset == 0


def test_half_kv_prefix_reuse(hip, tiny_stablelm):
    """TestHalfKVPrefixReuse: warm, extended and replaced prompts on an fp16
    KV cache match cold forwards."""
    config, tensors = tiny_stablelm
    config = dict(config, max_position_embeddings=384)
    warm = hip.StableLMForwarder(config, tensors)
    warm.set_kv_bits(16)
    resident = []
    for prompt in ([2, 40, 41], [2, 40, 41], [2, 40, 41] + [7] * 140, [2, 40, 41] + [7] * 155, [2, 99]):
        prefix = 0
        while prefix < min(len(resident), len(prompt) - 1) and resident[prefix] == prompt[prefix]:
            prefix += 1  # reusablePrefix (generation_policy.go:26-32)
        got = warm.forward(prefix, prompt[prefix:])
        resident = list(prompt)
        cold = hip.StableLMForwarder(config, tensors)
        cold.set_kv_bits(16)
        want = cold.forward(0, prompt)
        assert np.max(np.abs(got - want)) <= 1e-5
        cold.close()


def test_three_b_shapes_two_layers(hip, oracle):
    """StableLM-3B layer shapes (hidden 2560, 32 x 80 heads, 25% rotary,
    MLP 6912, vocab 65536, Q8_0) cut to two layers: per-layer residuals and
    logits against the oracle within 1e-3 relative to their range, and greedy
    agreement over 24 tokens after a 64-token prompt."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=256))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=7)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, 65536, 64).astype(np.int32)
    oracle.set_threads(8)
    ref = oracle.StableLM(config, tensors, capacity=256)
    ref.trace(True)
    f = hip.StableLMForwarder(config, tensors)
    f.trace(True)
    want = ref.prefill(prompt, 0)
    got = f.forward(0, prompt)
    span = float(want.max() - want.min())
    assert np.max(np.abs(got - want)) <= 1e-3 * span
    rt, gt = ref.trace_data(), f.trace_read()
    for layer in range(2):
        assert np.max(np.abs(rt[layer] - gt[layer])) <= 1e-3 * float(np.ptp(rt[layer]))
    toks_ref, toks_gpu = [], []
    lr, lg = want, got
    for step in range(24):
        tr, tg = int(np.argmax(lr)), int(np.argmax(lg))
        toks_ref.append(tr)
        toks_gpu.append(tg)
        if tr != tg:
            break
        lr = ref.forward(tr, 64 + step)
        lg = f.forward(64 + step, [tg])
        assert np.max(np.abs(lg - lr)) <= 1e-3 * float(np.ptp(lr))
    assert toks_gpu == toks_ref


@pytest.mark.parametrize("kv_bits", [32, 16])
def test_decode_attention_shapes_agree(hip, kv_bits):
    """Every decode attention shape (64, 128 and 256 positions per 4-wave
    block; 512 and 1024 per 16-wave block) against the shape chosen from the
    position, at the 3B head layout: 40 decode tokens from position 1000
    cross the 1024-position block boundary (one split, then two). Logits and
    per-layer residuals within 2e-5 of their range (only the order of the
    softmax sums differs), identical greedy tokens."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=3, max_position_embeddings=2048))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=9)
    prompt = np.random.default_rng(13).integers(0, 65536, 1000).astype(np.int32)
    shapes = [0, 1, 4, 8, 16]
    fwds = {}
    for steps in shapes:
        f = hip.StableLMForwarder(config, tensors)
        f.set_kv_bits(kv_bits)
        f.set_launch("attention", steps, 0)
        f.trace(True)
        fwds[steps] = f
    logits = {k: f.forward(0, prompt) for k, f in fwds.items()}
    for step in range(40):
        tok = int(np.argmax(logits[0]))
        for k in shapes[1:]:
            assert int(np.argmax(logits[k])) == tok, (k, step)
        logits = {k: f.forward(1000 + step, [tok]) for k, f in fwds.items()}
        span = float(np.ptp(logits[0]))
        tr = fwds[0].trace_read()
        for k in shapes[1:]:
            assert np.max(np.abs(logits[k] - logits[0])) <= 2e-5 * span, (k, step)
            assert np.max(np.abs(fwds[k].trace_read() - tr)) <= 2e-5 * float(np.ptp(tr)), (k, step)
    with pytest.raises(RuntimeError):
        fwds[0].set_launch("attention", 3, 0)
    for f in fwds.values():
        f.close()


@pytest.mark.parametrize("start", [1790, 4990])
def test_decode_attention_shape_by_position(hip, start):
    """The decode step's attention shape chosen by position (fused two
    steps up to 1800 positions, four steps as a launch of its own up to
    5000, 1024 positions per 16-wave block beyond) against the fused shape
    forced at every position (launch stage 3 = 2), fp32 KV: 20 decode
    tokens across each switch give logits and per-layer residuals within
    2e-5 of their range (only the order of the softmax sums differs) and the
    same greedy ids."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=8192))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=17)
    prompt = np.random.default_rng(19).integers(0, 65536, start).astype(np.int32)
    auto, ref = hip.StableLMForwarder(config, tensors), hip.StableLMForwarder(config, tensors)
    del tensors
    ref.set_launch("attention", 2, 0)
    for f in (auto, ref):
        f.trace(True)
    la, lr = auto.forward(0, prompt), ref.forward(0, prompt)
    for step in range(20):
        tok = int(np.argmax(lr))
        assert int(np.argmax(la)) == tok, step
        la, lr = auto.forward(start + step, [tok]), ref.forward(start + step, [tok])
        assert np.max(np.abs(la - lr)) <= 2e-5 * float(np.ptp(lr)), step
        tr = ref.trace_read()
        assert np.max(np.abs(auto.trace_read() - tr)) <= 2e-5 * float(np.ptp(tr)), step
    auto.close()
    ref.close()


@pytest.mark.parametrize("dtype,kv_bits", [(W.Q8_0, 32), (W.Q8_0, 16), (W.BF16, 32)])
def test_fused_decode_attention_matches_separate_launch(hip, dtype, kv_bits):
    """The decode attention on extra blocks of the decode_in launch (the
    default) against the attention as a launch of its own (launch stage 4
    off), same weights, prompt and KV: 40 decode tokens crossing several
    attention splits give bit-identical logits, per-layer residuals and KV
    (the same arithmetic in both)."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=3, max_position_embeddings=512))
    tensors = W.synthetic_stablelm(config, dtype, seed=3)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, 65536, 37).astype(np.int32)
    fused = hip.StableLMForwarder(config, tensors)
    ref = hip.StableLMForwarder(config, tensors)
    for f in (fused, ref):
        f.set_kv_bits(kv_bits)
        f.trace(True)
    ref.set_launch("fused_attention", 0, 0)
    lf, lr = fused.forward(0, prompt), ref.forward(0, prompt)
    assert np.array_equal(lf, lr)
    for step in range(40):
        tok = int(np.argmax(lr))
        lf = fused.forward(37 + step, [tok])
        lr = ref.forward(37 + step, [tok])
        assert np.array_equal(lf, lr), step
        assert np.array_equal(fused.trace_read(), ref.trace_read()), step
    for layer in range(3):
        k1, v1 = fused.read_kv(layer, 5, 77)
        k2, v2 = ref.read_kv(layer, 5, 77)
        assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    fused.close()
    ref.close()


@pytest.mark.parametrize("fmt,kv_bits", [(W.Q8_0, 32), (W.BF16, 16)])
def test_key_split_prefill_matches_one_block_per_tile(hip, fmt, kv_bits):
    """A 1600-token prompt submitted in 512-token calls and a 64-token tail
    (as MLX.generate chunks a prompt, mlx.go:346-354): every call, its last
    position past 256, splits its attention over key ranges (the default)
    and combines the ranges' records; against one block per query
    tile (launch stage 9 off) the logits of every call, the last token's
    per-layer residuals and the fp32 KV agree within 1e-5 of their range
    (the same products summed in another order), with the same greedy ids.
    With an fp16 cache a last-bit difference in one layer's attention may
    flip the fp16 rounding of the next layer's K/V: an entry within one
    fp16 step of its largest value, logits and residuals within 1e-4."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=2048))
    tensors = W.synthetic_stablelm(config, fmt, seed=61)
    prompt = np.random.default_rng(67).integers(0, 65536, 1600).astype(np.int32)
    split, whole = hip.StableLMForwarder(config, tensors), hip.StableLMForwarder(config, tensors)
    whole.set_launch("flash_key_split", 0, 0)
    for f in (split, whole):
        f.set_kv_bits(kv_bits)
        f.trace(True)
    tol = 1e-5 if kv_bits == 32 else 1e-4
    for a, b in ((0, 512), (512, 1024), (1024, 1536), (1536, 1600)):
        ls, lw = split.forward(a, prompt[a:b]), whole.forward(a, prompt[a:b])
        assert np.max(np.abs(ls - lw)) <= tol * float(np.ptp(lw)), a
        assert int(np.argmax(ls)) == int(np.argmax(lw)), a
    ts, tw = split.trace_read(), whole.trace_read()
    for layer in range(2):
        assert np.max(np.abs(ts[layer] - tw[layer])) <= tol * float(np.ptp(tw[layer])), layer
        k1, v1 = split.read_kv(layer, 0, 1600)
        k2, v2 = whole.read_kv(layer, 0, 1600)
        for got, want in ((k1, k2), (v1, v2)):
            tol = 1e-5 * float(np.ptp(want)) if kv_bits == 32 else float(np.max(np.abs(want))) * 2.0 ** -10
            assert np.max(np.abs(got - want)) <= tol, layer
    split.close()
    whole.close()


def test_wide_bf16_prefill_matches_large_tiles(hip):
    """The BF16 prefill on wide tiles (the default: the in-projection, its
    epilogue kernel, the o and down products as one launch of K splits)
    against the 128 x 256 tiles with the epilogue fused and a separate down
    product (launch stage 7 off): the same fp32 products summed in another
    order, so a 2100-token prefill (a full 2048-token chunk and a partial
    one) gives logits, per-layer residuals and (fp32) KV within 1e-5 of their
    range, and the same greedy ids over 8 decode tokens. The wide-tile
    in-projection with its epilogue in the product's launch (stage 8 on)
    gives bit-identical results to the default."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=4096))
    tensors = W.synthetic_stablelm(config, W.BF16, seed=21)
    prompt = np.random.default_rng(23).integers(0, 65536, 2100).astype(np.int32)
    wide = hip.StableLMForwarder(config, tensors)
    fused = hip.StableLMForwarder(config, tensors)
    ref = hip.StableLMForwarder(config, tensors)
    del tensors
    ref.set_launch("wide", 0, 0)
    fused.set_launch("wide_epilogue", 1, 0)
    for f in (wide, fused, ref):
        f.trace(True)
    lw, lf, lr = wide.forward(0, prompt), fused.forward(0, prompt), ref.forward(0, prompt)
    assert np.array_equal(lw, lf)
    span = float(np.ptp(lr))
    assert np.max(np.abs(lw - lr)) <= 1e-5 * span
    tr = ref.trace_read()
    assert np.max(np.abs(wide.trace_read() - tr)) <= 1e-5 * float(np.ptp(tr))
    assert np.array_equal(wide.trace_read(), fused.trace_read())
    for layer in range(2):
        for head in (0, 19):
            kw, kr = wide.read_kv(layer, head, 2100), ref.read_kv(layer, head, 2100)
            for a, b in zip(kw, kr):
                assert np.max(np.abs(a - b)) <= 1e-5 * float(np.ptp(b)), (layer, head)
            for a, b in zip(kw, fused.read_kv(layer, head, 2100)):
                assert np.array_equal(a, b), (layer, head)
    for step in range(8):
        tok = int(np.argmax(lr))
        assert int(np.argmax(lw)) == tok, step
        lw, lr = wide.forward(2100 + step, [tok]), ref.forward(2100 + step, [tok])
    for f in (wide, fused, ref):
        f.close()


def test_wide_q8_0_prefill_matches_large_tiles(hip):
    """The Q8_0 prefill on wide tiles (the default: the in-projection of a
    chunk of 256 rows or more and the o and down products, as one launch of
    K splits, on the Q8_0 ring kernel; shorter chunks take their
    in-projection on the 128 x 256 tiles in two K halves) against the
    128 x 256 tiles throughout (launch stage 10 off): the same exact quants
    and fp32 products summed in another order. A 2400-token call (chunks of
    2048 rows on 256 x 256 tiles and 352 rows on 256 x 192) and a 52-token
    continuation give logits, per-layer residuals and (fp32) KV within 1e-5
    of their range, and the same greedy ids over 8 decode tokens. The wide
    in-projection with its epilogue in the product's launch (stage 8 on)
    gives bit-identical results to the default."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=4096))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=31)
    prompt = np.random.default_rng(33).integers(0, 65536, 2452).astype(np.int32)
    wide = hip.StableLMForwarder(config, tensors)
    fused = hip.StableLMForwarder(config, tensors)
    ref = hip.StableLMForwarder(config, tensors)
    del tensors
    ref.set_launch("q8_wide", 0, 0)
    fused.set_launch("wide_epilogue", 1, 0)
    for f in (wide, fused, ref):
        f.trace(True)
    for start, end in ((0, 2400), (2400, 2452)):
        part = prompt[start:end]
        lw, lf, lr = wide.forward(start, part), fused.forward(start, part), ref.forward(start, part)
        assert np.array_equal(lw, lf), start
        assert np.max(np.abs(lw - lr)) <= 1e-5 * float(np.ptp(lr)), start
        tr = ref.trace_read()
        assert np.max(np.abs(wide.trace_read() - tr)) <= 1e-5 * float(np.ptp(tr)), start
        assert np.array_equal(wide.trace_read(), fused.trace_read()), start
    for layer in range(2):
        for head in (0, 19):
            kw, kr = wide.read_kv(layer, head, 2452), ref.read_kv(layer, head, 2452)
            for a, b in zip(kw, kr):
                assert np.max(np.abs(a - b)) <= 1e-5 * float(np.ptp(b)), (layer, head)
            for a, b in zip(kw, fused.read_kv(layer, head, 2452)):
                assert np.array_equal(a, b), (layer, head)
    for step in range(8):
        tok = int(np.argmax(lr))
        assert int(np.argmax(lw)) == tok, step
        lw, lr = wide.forward(2452 + step, [tok]), ref.forward(2452 + step, [tok])
    for f in (wide, fused, ref):
        f.close()


def test_f32_weights_against_oracle(hip, oracle):
    """F32 weights at the 3B layer shapes (a wout row spans 8 column slices
    of five chunks per lane: 512-thread blocks). Prefill and 12 decode
    logits against the oracle within 1e-3 of their range, identical greedy
    ids."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, vocab_size=4096,
                                             max_position_embeddings=256))
    tensors = W.synthetic_stablelm(config, W.F32, seed=17)
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, 4096, 30).astype(np.int32)
    oracle.set_threads(8)
    ref = oracle.StableLM(config, tensors, capacity=256)
    f = hip.StableLMForwarder(config, tensors)
    want = ref.prefill(prompt, 0)
    got = f.forward(0, prompt)
    assert np.max(np.abs(got - want)) <= 1e-3 * float(np.ptp(want))
    for step in range(12):
        tr, tg = int(np.argmax(want)), int(np.argmax(got))
        assert tr == tg, step
        want = ref.forward(tr, 30 + step)
        got = f.forward(30 + step, [tg])
        assert np.max(np.abs(got - want)) <= 1e-3 * float(np.ptp(want)), step
    f.close()


@pytest.mark.parametrize("dtype", [W.Q4_K, W.Q6_K])
def test_kquant_layers_against_oracle(hip, oracle, dtype):
    """StableLM-3B layer shapes (two layers) with every matrix in one 5/6-bit
    format and fp16 KV: prefill and decode logits against the oracle within
    1e-3 of their range, identical greedy ids."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=256))
    tensors = W.synthetic_stablelm(config, dtype, seed=21)
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, 65536, 40).astype(np.int32)
    oracle.set_threads(8)
    ref = oracle.StableLM(config, tensors, half_kv=True, capacity=256)
    f = hip.StableLMForwarder(config, tensors)
    f.set_kv_bits(16)
    want = ref.prefill(prompt, 0)
    got = f.forward(0, prompt)
    assert np.max(np.abs(got - want)) <= 1e-3 * float(np.ptp(want))
    for step in range(8):
        tr, tg = int(np.argmax(want)), int(np.argmax(got))
        assert tr == tg, step
        want = ref.forward(tr, 40 + step)
        got = f.forward(40 + step, [tg])
        assert np.max(np.abs(got - want)) <= 1e-3 * float(np.ptp(want)), step
    f.close()


@pytest.mark.parametrize("mlp,attn", [(W.Q4_K, W.Q6_K), (W.Q8_0, W.Q6_K), (W.Q6_K, W.BF16)])
def test_mixed_format_layers_against_oracle(hip, oracle, mlp, attn):
    """Layers whose attention matrices (q, k, v, o) and MLP matrices (gate,
    up, down) come in different formats, as GGUF K-quant mixes store them
    (Q6_K attention with Q4_K MLP is the mix of the K-quant workload): each
    keeps its sections as matrices of their own. StableLM-3B layer shapes,
    two layers, fp16 KV, a 300-token prompt (prefill in one chunk) and 8
    decode tokens: logits within 1e-3 of their range of the oracle's (2e-2
    where a section is BF16: north_star's bound for the bf16 paths, which
    the two-plane products meet by far), identical greedy ids."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=512))
    tensors = W.synthetic_stablelm(config, mlp, seed=23, attn_dtype=attn, head_dtype=attn)
    prompt = np.random.default_rng(29).integers(0, 65536, 300).astype(np.int32)
    oracle.set_threads(8)
    ref = oracle.StableLM(config, tensors, half_kv=True, capacity=512)
    f = hip.StableLMForwarder(config, tensors)
    f.set_kv_bits(16)
    tol = 2e-2 if W.BF16 in (mlp, attn) else 1e-3
    want = ref.prefill(prompt, 0)
    got = f.forward(0, prompt)
    assert np.max(np.abs(got - want)) <= tol * float(np.ptp(want))
    for step in range(8):
        tr, tg = int(np.argmax(want)), int(np.argmax(got))
        assert tr == tg, step
        want = ref.forward(tr, 300 + step)
        got = f.forward(300 + step, [tg])
        assert np.max(np.abs(got - want)) <= tol * float(np.ptp(want)), step
    f.close()


@pytest.mark.parametrize("kv_bits", [32, 16])
def test_prefill_after_prefix_against_oracle(hip, oracle, kv_bits):
    """Matrix-core prefill attention at a nonzero start: a 100-token prefix,
    then a 300-token suffix (several 64-position tiles, a partial query
    tile) on StableLM-3B layer shapes, against the oracle's batched prefill:
    logits and per-layer residuals within 1e-3 of their range."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=512))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=17)
    rng = np.random.default_rng(8)
    ids = rng.integers(0, 65536, 400).astype(np.int32)
    oracle.set_threads(8)
    ref = oracle.StableLM(config, tensors, half_kv=kv_bits == 16, capacity=512)
    ref.trace(True)
    f = hip.StableLMForwarder(config, tensors)
    f.set_kv_bits(kv_bits)
    f.trace(True)
    ref.prefill(ids[:100], 0)
    f.forward(0, ids[:100], want_logits=False)
    want = ref.prefill(ids[100:], 100)
    got = f.forward(100, ids[100:])
    assert np.max(np.abs(got - want)) <= 1e-3 * float(np.ptp(want))
    rt, gt = ref.trace_data(), f.trace_read()
    for layer in range(2):
        assert np.max(np.abs(rt[layer] - gt[layer])) <= 1e-3 * float(np.ptp(rt[layer]))
    f.close()
