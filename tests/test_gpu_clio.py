"""Parity at Clio's layer shapes, the reference's own model (attention
fixture dot_test.go:17-19, model widths dot_test.go:132-134; "Running
Clio", README.md): hidden 2816, 22 heads x 128 with 22 kv heads
(multi-head), 25% partial rotary (32 of 128 dims, as rope.json pins),
MLP 7552, vocab 65536, cut to two layers. Head width 128 runs the
128-wide instances of every attention kernel: the decode attention fused
into the decode_in launch (up to 1800 positions) and the separate 4-step
launch beyond, the matrix-core prefill, and the branch passes (the shared
prefix on the matrix cores, each branch's suffix split-K).

Tolerances are north_star's: 1e-3 of the range for fp32-KV paths, 2e-2
where the KV cache is fp16. The GPU is fed the oracle's greedy tokens, so
every step compares the same positions; the argmax must agree at each.
"""
import os
import sys

import numpy as np
import pytest

from tinyoai_amd import weights as W

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_gpu_branches import branch_case  # noqa: E402

pytestmark = pytest.mark.gpu

CLIO_2L = dict(W.STABLELM_3B, hidden_size=2816, intermediate_size=7552, num_attention_heads=22,
               num_key_value_heads=22, num_hidden_layers=2, max_position_embeddings=8192)


@pytest.fixture(scope="module")
def hip():
    from tinyoai_amd import hip as H
    H.lib()
    return H


@pytest.mark.parametrize("fmt,kv_bits,prompt_len,steps", [(W.Q8_0, 32, 300, 12), (W.BF16, 16, 2100, 8)])
def test_clio_prefill_and_decode(hip, oracle, fmt, kv_bits, prompt_len, steps):
    """Q8_0 weights with fp32 KV (a 300-token prompt: one prefill chunk,
    decode attention fused into the decode_in launch) and BF16 weights with
    fp16 KV (2100 tokens: a full 2048-token chunk and a partial one on the
    wide-tile products, decode attention beyond 1800 positions as a launch
    of its own): per-layer residuals of the last prompt token, the prompt's
    logits and each decode step's logits against the oracle, identical
    greedy ids."""
    config = W.validate_stablelm_config(dict(CLIO_2L))
    assert config["hidden_size"] // config["num_attention_heads"] == 128
    tensors = W.synthetic_stablelm(config, fmt, seed=51)
    prompt = np.random.default_rng(53).integers(0, 65536, prompt_len).astype(np.int32)
    tol = 1e-3 if kv_bits == 32 else 2e-2
    oracle.set_threads(16)
    ref = oracle.StableLM(config, tensors, half_kv=kv_bits == 16, capacity=prompt_len + steps + 1)
    ref.trace(True)
    f = hip.StableLMForwarder(config, tensors)
    del tensors
    f.set_kv_bits(kv_bits)
    f.trace(True)
    want = ref.prefill(prompt, 0)
    got = f.forward(0, prompt)
    rt, gt = ref.trace_data(), f.trace_read()
    for layer in range(2):
        assert np.max(np.abs(rt[layer] - gt[layer])) <= tol * float(np.ptp(rt[layer])), layer
    for step in range(steps):
        span = float(np.ptp(want))
        assert np.max(np.abs(got - want)) <= tol * span, step
        tok = int(np.argmax(want))
        assert int(np.argmax(got)) == tok, step
        want = ref.forward(tok, prompt_len + step)
        got = f.forward(prompt_len + step, [tok])
    f.close()
    ref.close()


@pytest.mark.parametrize("fmt,kv_bits", [(W.Q8_0, 16), (W.BF16, 32)])
def test_clio_branches(hip, oracle, fmt, kv_bits):
    """Five branches at Clio's shapes borrowing a 300-token prefix, with
    ragged private suffixes (1-64 tokens, one append), then three lockstep
    tokens, against the oracle's replay of each branch (the shared prefix
    on the 128-wide matrix-core pass, each suffix on the 128-wide split-K
    attention)."""
    config = W.validate_stablelm_config(dict(CLIO_2L, max_position_embeddings=512))
    tensors = W.synthetic_stablelm(config, fmt, seed=57)
    rng = np.random.default_rng(59)
    prompt = list(rng.integers(0, 65536, 300))
    suffixes = [list(rng.integers(0, 65536, n)) for n in (1, 64, 13, 40, 7)]
    oracle.set_threads(16)
    branch_case(hip, oracle, config, tensors, prompt, 300, suffixes, 3, kv_bits, True)
