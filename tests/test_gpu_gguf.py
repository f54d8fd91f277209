"""GGUF-loaded forwarders on the device (TestGGUFRoundTrip,
gguf_test.go:143-174): the tiny fixture converted to GGUF gives logits
bit-identical to the safetensors load, and a StableLM-3B-width Q8_0 layer
written through GGUF's reversed dimensions gives the same logits as its
tensors handed over directly."""
import json
import os

import numpy as np
import pytest
from gguf_fixture import I32, stablelm_gguf

from tinyoai_amd import gguf
from tinyoai_amd import weights as W

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "stablelm")


@pytest.fixture(scope="module")
def hip():
    from tinyoai_amd import hip as H
    H.lib()
    return H


def test_tiny_fixture_logits_identical(hip, tiny_stablelm, tmp_path):
    config, tensors = tiny_stablelm
    pieces = gguf.tokenizer_pieces(os.path.join(GOLDEN, "tokenizer.json"), config["vocab_size"])

    def pad(meta, _):
        meta["tokenizer.ggml.tokens"][1][341] = "[PAD341]"
        meta["tokenizer.ggml.token_type"] = (("arr", I32), [0] * 341 + [5])
    path = stablelm_gguf(str(tmp_path), config, tensors, pieces, os.path.join(GOLDEN, "tokenizer.json"), pad)
    c, ts = gguf.load_stablelm_gguf(path)
    ids = json.load(open(os.path.join(GOLDEN, "expected.json")))["input_ids"]
    a = hip.StableLMForwarder(config, tensors)
    b = hip.StableLMForwarder(c, ts)
    want, got = a.forward(0, ids), b.forward(0, ids)
    assert np.array_equal(want, got)
    assert np.array_equal(a.forward(len(ids), [5]), b.forward(len(ids), [5]))
    a.close()
    b.close()


def test_q8_0_layer_through_gguf(hip, tmp_path):
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=1, vocab_size=4096,
                                             max_position_embeddings=512))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=11)
    path = stablelm_gguf(str(tmp_path), config, tensors, [f"p{i}" for i in range(4096)])
    c, ts = gguf.load_stablelm_gguf(path)
    ids = np.random.default_rng(12).integers(0, 4096, 40)
    a = hip.StableLMForwarder(config, tensors)
    b = hip.StableLMForwarder(c, ts)
    assert np.array_equal(a.forward(0, ids), b.forward(0, ids))
    assert np.array_equal(a.forward(40, [7]), b.forward(40, [7]))
    a.close()
    b.close()
