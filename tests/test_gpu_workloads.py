"""Parity of the HIP forwarder with the oracle at the three StableLM-3B-shape
workloads, one test each (a failure in one does not hide the others):

  Q8_0 decode       32 layers, GGUF Q8_0, fp32 KV, a 512-token prompt and
                    256 greedy tokens (stablelm.go:332-387, prefill.go:33-115);
  BF16 long context BF16, fp16 KV, an 8129-token prefill through the
                    2048-token chunks, then greedy tokens: 2 layers at full
                    layer shapes with 16 tokens, and all 32 layers with 64
                    tokens (to position 8192);
  K-quant branches  Q6_K attention and classifier, Q4_K MLP, fp16 KV: 16
                    branches on a 4096-token prefix, private suffixes of
                    1-256 tokens, then lockstep tokens (mlx_branches.go:98-182):
                    2 layers with 8 tokens, and all 32 layers with 64.

The oracle needs minutes for these, so its results are committed fixtures
(tests/golden/make_workload_fixtures.py writes them from the same seeds);
the weights and prompts are rebuilt here from those seeds. A logits vector
is compared through its summary: the values at a fixed sample of 253 ids
and the 16 largest entries, against the oracle's range (max - min).
Tolerances are north_star's: 1e-3 of the range for fp32 paths, 2e-2 where
the KV cache is fp16. Greedy ids must be identical; the GPU is fed the
oracle's tokens (teacher forcing), so every step is compared at the same
positions even if an id ever differed.
"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_workload_fixtures as F  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from tinyoai_amd import hip as H
    H.lib()
    return H


def load(name):
    path = F.fixture_path(name)
    if not os.path.exists(path):
        pytest.fail(f"fixture {path} is missing: run tests/golden/make_workload_fixtures.py {name}")
    with np.load(path) as z:
        return {k: z[k] for k in z.files}


def check_logits(got, fx, idx, tol, tag):
    """got: the GPU's logits; fx: fixture arrays; idx: the summary's index."""
    span = float(fx["logits_hi"][idx] - fx["logits_lo"][idx])
    sample = fx["logits_sample"][idx]
    err = float(np.max(np.abs(got[F.LOGIT_SAMPLE] - sample)))
    top_i, top_v = fx["logits_top_idx"][idx], fx["logits_top_val"][idx]
    err = max(err, float(np.max(np.abs(got[top_i] - top_v))))
    assert err <= tol * span, (tag, err / span)
    assert int(np.argmax(got)) == int(top_i[0]), (tag, int(np.argmax(got)), int(top_i[0]))
    return err / span


def test_q8_0_decode_workload(hip):
    """32 layers, 512 + 256 tokens: all 256 logits vectors within 1e-3 of
    their range, the per-layer residual of the last prompt token within 1e-3
    of each layer's range, and the GPU's own greedy stream (no teacher
    forcing) identical to the oracle's."""
    fx = load("q8_0_decode")
    p = F.Q8_DECODE
    config, tensors, prompt = F.q8_0_inputs(p)
    f = hip.StableLMForwarder(config, tensors)
    del tensors
    f.trace(True)
    toks = fx["tokens"]
    logits = f.forward(0, prompt)
    trace = f.trace_read()
    for layer in range(p["layers"]):
        want = fx["trace_prompt"][layer]
        assert np.max(np.abs(trace[layer] - want)) <= 1e-3 * float(np.ptp(want)), layer
    f.trace(False)
    worst = 0.0
    for n in range(p["generate"]):
        worst = max(worst, check_logits(logits, fx, n, 1e-3, f"step {n}"))
        if n + 1 < p["generate"]:
            logits = f.forward(p["prompt"] + n, [int(toks[n])])
    # free-running greedy stream
    logits = f.forward(0, prompt)
    mine = []
    for n in range(p["generate"]):
        mine.append(int(np.argmax(logits)))
        if n + 1 < p["generate"]:
            logits = f.forward(p["prompt"] + n, [mine[-1]])
    assert mine == [int(t) for t in toks]
    f.close()
    print(f"q8_0 decode: worst logits error {worst:.2e} of the range")


@pytest.mark.parametrize("name", ["bf16_long", "bf16_long_full"])
def test_bf16_long_context_workload(hip, name):
    """BF16 weights, fp16 KV, an 8129-token prefill (2048-token chunks, the
    last one partial), then greedy tokens: 2 layers at full shapes with 16
    tokens, and the whole workload (32 layers, 64 tokens, to position 8192).
    Logits within 2e-2 of their range, the last prompt token's and the last
    decode token's per-layer residuals within 2e-2 of each layer's range,
    identical greedy ids at every step."""
    fx = load(name)
    p = F.BF16_LONG_FULL if name.endswith("_full") else F.BF16_LONG
    config, tensors, prompt = F.bf16_inputs(p)
    f = hip.StableLMForwarder(config, tensors)
    del tensors
    f.set_kv_bits(16)
    f.trace(True)
    toks = fx["tokens"]
    logits = f.forward(0, prompt)
    for layer, row in enumerate(f.trace_read()):
        want = fx["trace_prompt"][layer]
        assert np.max(np.abs(row - want)) <= 2e-2 * float(np.ptp(want)), layer
    worst = 0.0
    for n in range(p["generate"]):
        assert int(np.argmax(logits)) == int(toks[n]), n
        worst = max(worst, check_logits(logits, fx, n, 2e-2, f"step {n}"))
        if n + 1 < p["generate"]:
            logits = f.forward(p["prompt"] + n, [int(toks[n])])
    for layer, row in enumerate(f.trace_read()):
        want = fx["trace_last"][layer]
        assert np.max(np.abs(row - want)) <= 2e-2 * float(np.ptp(want)), layer
    f.close()
    print(f"{name}: worst logits error {worst:.2e} of the range")


@pytest.mark.parametrize("name", ["kquant_branches", "kquant_branches_full"])
def test_kquant_branches_workload(hip, name):
    """K-quant mix, fp16 KV: a 4096-token prefix, 16 branches given private
    suffixes of 1-256 tokens in one append, then lockstep steps at ragged
    positions: 2 layers at full shapes with 7 steps, and the whole workload
    (32 layers, 63 steps). Every branch's logits within 2e-2 of their range,
    identical greedy ids."""
    fx = load(name)
    p = F.KQ_BRANCHES_FULL if name.endswith("_full") else F.KQ_BRANCHES
    config, tensors, prefix, lengths, suffixes = F.branch_inputs(p)
    assert np.array_equal(lengths, fx["lengths"])
    f = hip.StableLMForwarder(config, tensors)
    del tensors
    f.set_kv_bits(16)
    f.forward(0, prefix, want_logits=False)
    br = f.new_branches(p["prefix"], p["branches"])
    toks = fx["tokens"]
    rows = br.append(suffixes)
    worst = 0.0
    for s in range(p["steps"]):
        for j in range(p["branches"]):
            sub = {k: v[j] for k, v in fx.items() if k.startswith("logits_")}
            assert int(np.argmax(rows[j])) == int(toks[j, s]), (j, s)
            worst = max(worst, check_logits(rows[j], sub, s, 2e-2, f"branch {j} step {s}"))
        if s + 1 < p["steps"]:
            rows = br.forward(toks[:, s])
    for j in range(p["branches"]):
        assert br.length(j) == lengths[j] + p["steps"] - 1
    br.close()
    f.close()
    print(f"{name}: worst logits error {worst:.2e} of the range")
