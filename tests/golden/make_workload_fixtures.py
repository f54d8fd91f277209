#!/usr/bin/env python3
"""Writes the oracle's results at the three StableLM-3B-shape workloads as
golden fixtures for the GPU parity tests (tests/test_gpu_workloads.py).

The oracle (oracle/, a C restatement of tinyoai's Go scalar engine) needs
minutes for these runs, longer than a GPU test may take, so its results are
computed once here and committed. Every input is regenerated from seeds by
tinyoai_amd.weights (numpy's default generator), so the GPU test rebuilds the
same weights and prompts without storing them.

    python tests/golden/make_workload_fixtures.py q8_0_decode   # 32 layers, 512 + 256
    python tests/golden/make_workload_fixtures.py bf16_long     # 2 layers, 8129 + 16, fp16 KV
    python tests/golden/make_workload_fixtures.py kquant_branches  # 2 layers, 16 ragged branches
    python tests/golden/make_workload_fixtures.py bf16_long_full   # 32 layers, 8129 + 64, fp16 KV
    python tests/golden/make_workload_fixtures.py kquant_branches_full  # 32 layers, 16 x 64 steps

The two-layer versions run in minutes; the full-depth ones take hours of CPU
time (ORACLE_THREADS sets the thread count) and carry the whole trajectory:
every decode token of the long-context workload and every lockstep token of
the branch workload.

A logits vector is kept as a summary: its minimum and maximum, its 16
largest entries (index and value) and its values at LOGIT_SAMPLE, a fixed
set of 253 indices.
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import pyoracle  # noqa: E402
from tinyoai_amd import weights as W  # noqa: E402

VOCAB = 65536
LOGIT_SAMPLE = np.sort(np.random.default_rng(99).choice(VOCAB, 253, replace=False)).astype(np.int64)

# The workloads (BASELINE configs 3-5 at the shapes the tests run).
Q8_DECODE = dict(layers=32, max_pos=1024, weights_seed=1234, prompt_seed=1235, prompt=512, generate=256)
BF16_LONG = dict(layers=2, max_pos=8192, weights_seed=41, prompt_seed=43, prompt=8129, generate=16)
KQ_BRANCHES = dict(layers=2, max_pos=8192, weights_seed=31, prompt_seed=37, prefix=4096, branches=16,
                   min_suffix=1, max_suffix=256, steps=8)
# Full depth: the same weights seeds and prompts with all 32 layers and the
# workloads' own token counts. The branch suffixes go through the oracle's
# batched prefill (prefill.go:33-115), as the forwarder's append submits them.
BF16_LONG_FULL = dict(BF16_LONG, layers=32, generate=64)
KQ_BRANCHES_FULL = dict(KQ_BRANCHES, layers=32, steps=64, suffix_prefill=True)


def summarize(logits: np.ndarray) -> dict:
    top = np.argsort(-logits.astype(np.float64), kind="stable")[:16]
    return {"lo": float(logits.min()), "hi": float(logits.max()), "top_idx": top.astype(np.int64),
            "top_val": logits[top].astype(np.float32), "sample": logits[LOGIT_SAMPLE].astype(np.float32)}


def stack(summaries: list[dict]) -> dict:
    return {k: np.array([s[k] for s in summaries]) for k in summaries[0]}


def q8_0_config(p: dict) -> dict:
    return W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=p["layers"],
                                           max_position_embeddings=p["max_pos"]))


def q8_0_inputs(p: dict):
    config = q8_0_config(p)
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=p["weights_seed"])
    prompt = np.random.default_rng(p["prompt_seed"]).integers(0, VOCAB, p["prompt"]).astype(np.int32)
    return config, tensors, prompt


def bf16_inputs(p: dict):
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=p["layers"],
                                             max_position_embeddings=p["max_pos"]))
    tensors = W.synthetic_stablelm(config, W.BF16, seed=p["weights_seed"])
    prompt = np.random.default_rng(p["prompt_seed"]).integers(0, VOCAB, p["prompt"]).astype(np.int32)
    return config, tensors, prompt


def branch_inputs(p: dict):
    """Prefix ids, and per branch a private suffix of ragged length."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=p["layers"],
                                             max_position_embeddings=p["max_pos"]))
    tensors = W.synthetic_stablelm(config, W.Q4_K, seed=p["weights_seed"], attn_dtype=W.Q6_K, head_dtype=W.Q6_K)
    rng = np.random.default_rng(p["prompt_seed"])
    prefix = rng.integers(0, VOCAB, p["prefix"]).astype(np.int32)
    lengths = rng.integers(p["min_suffix"], p["max_suffix"] + 1, p["branches"]).astype(np.int32)
    suffixes = [rng.integers(0, VOCAB, n).astype(np.int32) for n in lengths]
    return config, tensors, prefix, lengths, suffixes


def make_q8_0_decode(path: str) -> None:
    """Greedy decoding as MLX.generate drives the forwarder (mlx.go:342-468):
    the prompt's logits give the first token, then one forward per token."""
    p = Q8_DECODE
    config, tensors, prompt = q8_0_inputs(p)
    m = pyoracle.StableLM(config, tensors, capacity=p["max_pos"])
    m.trace(True)
    t0 = time.time()
    logits = m.prefill(prompt, 0)
    trace_prompt = m.trace_data()
    print(f"prefill {time.time() - t0:.1f}s", flush=True)
    toks, sums = [], []
    for n in range(p["generate"]):
        sums.append(summarize(logits))
        toks.append(int(np.argmax(logits)))
        if n + 1 < p["generate"]:
            logits = m.forward(toks[-1], p["prompt"] + n)
        if n % 32 == 0:
            print(f"token {n} ({time.time() - t0:.0f}s)", flush=True)
    np.savez_compressed(path, tokens=np.array(toks, np.int32), trace_prompt=trace_prompt.astype(np.float32),
                        **{f"logits_{k}": v for k, v in stack(sums).items()})


def make_bf16_long(path: str, p: dict = BF16_LONG) -> None:
    config, tensors, prompt = bf16_inputs(p)
    m = pyoracle.StableLM(config, tensors, half_kv=True, capacity=p["max_pos"])
    m.trace(True)
    t0 = time.time()
    logits = m.prefill(prompt, 0)
    trace_prompt = m.trace_data()
    print(f"prefill {time.time() - t0:.1f}s", flush=True)
    toks, sums = [], []
    for n in range(p["generate"]):
        sums.append(summarize(logits))
        toks.append(int(np.argmax(logits)))
        if n + 1 < p["generate"]:
            logits = m.forward(toks[-1], p["prompt"] + n)
        if n % 16 == 0:
            print(f"token {n} ({time.time() - t0:.0f}s)", flush=True)
    trace_last = m.trace_data()
    np.savez_compressed(path, tokens=np.array(toks, np.int32), trace_prompt=trace_prompt.astype(np.float32),
                        trace_last=trace_last.astype(np.float32),
                        **{f"logits_{k}": v for k, v in stack(sums).items()})


def make_kquant_branches(path: str, p: dict = KQ_BRANCHES) -> None:
    """One oracle prefilled with the shared prefix; each branch is replayed
    on it in turn (forward at position P + s rewrites only positions >= P,
    and attention at position t reads [0, t]), as nativeBranches evaluates a
    branch against the borrowed prefix (mlx_branches.go:98-182)."""
    config, tensors, prefix, lengths, suffixes = branch_inputs(p)
    P = p["prefix"]
    m = pyoracle.StableLM(config, tensors, half_kv=True, capacity=p["max_pos"])
    t0 = time.time()
    m.prefill(prefix, 0)
    print(f"prefill {time.time() - t0:.1f}s", flush=True)
    toks = np.zeros((p["branches"], p["steps"]), np.int32)
    sums = []
    for j, suf in enumerate(suffixes):
        if p.get("suffix_prefill"):
            logits = m.prefill(suf, P)
        else:
            for i, tok in enumerate(suf):
                logits = m.forward(int(tok), P + i, i + 1 == len(suf))
        row = []
        for s in range(p["steps"]):
            row.append(summarize(logits))
            toks[j, s] = int(np.argmax(logits))
            if s + 1 < p["steps"]:
                logits = m.forward(int(toks[j, s]), P + len(suf) + s)
        sums.append(row)
        print(f"branch {j} (suffix {len(suf)}) {time.time() - t0:.0f}s", flush=True)
    flat = stack([s for row in sums for s in row])
    np.savez_compressed(path, tokens=toks, lengths=lengths,
                        **{f"logits_{k}": v.reshape(p["branches"], p["steps"], *v.shape[1:])
                           for k, v in flat.items()})


MAKERS = {"q8_0_decode": make_q8_0_decode, "bf16_long": make_bf16_long, "kquant_branches": make_kquant_branches,
          "bf16_long_full": lambda path: make_bf16_long(path, BF16_LONG_FULL),
          "kquant_branches_full": lambda path: make_kquant_branches(path, KQ_BRANCHES_FULL)}


def fixture_path(name: str) -> str:
    return os.path.join(HERE, f"workload_{name}.npz")


if __name__ == "__main__":
    pyoracle.set_threads(int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 8)))
    for name in sys.argv[1:] or list(MAKERS):
        print(f"== {name}", flush=True)
        MAKERS[name](fixture_path(name))
