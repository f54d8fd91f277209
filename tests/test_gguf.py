"""GGUF v3 loading without a GPU: TestGGUFRoundTrip's conversion of the tiny
safetensors fixture (gguf_test.go:143-174) and every TestGGUFRejects case
(gguf_test.go:179-247), on files written by an independent writer."""
import os
import struct

import numpy as np
import pytest
from gguf_fixture import I32, STR, U32, stablelm_gguf, write_gguf

from tinyoai_amd import gguf
from tinyoai_amd import weights as W

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "stablelm")
TOKENIZER = os.path.join(GOLDEN, "tokenizer.json")


@pytest.fixture(scope="module")
def pieces(tiny_stablelm):
    return gguf.tokenizer_pieces(TOKENIZER, tiny_stablelm[0]["vocab_size"])


def padded(meta, _):
    """The round trip's edit: the unused id 341 becomes "[PAD341]" with
    token type 5."""
    meta["tokenizer.ggml.tokens"][1][341] = "[PAD341]"
    types = [0] * 342
    types[341] = 5
    meta["tokenizer.ggml.token_type"] = (("arr", I32), types)


def fixture(tmp_path, tiny_stablelm, pieces, edit=None):
    config, tensors = tiny_stablelm

    def both(meta, ts):
        padded(meta, ts)
        if edit:
            edit(meta, ts)
    return stablelm_gguf(str(tmp_path), config, tensors, pieces, TOKENIZER, both)


def test_round_trip_config_and_bytes(tmp_path, tiny_stablelm, pieces):
    """Same configuration (rope_scaling null and absent both mean none) and
    the same tensor bytes under the same names as the safetensors load."""
    config, tensors = tiny_stablelm
    c, ts = gguf.load_stablelm_gguf(fixture(tmp_path, tiny_stablelm, pieces))
    want = {k: v for k, v in config.items() if k != "rope_scaling"}
    for k, v in want.items():
        if k in c:
            assert c[k] == v, k
    for k in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
              "num_key_value_heads", "max_position_embeddings", "layer_norm_eps", "rope_theta",
              "partial_rotary_factor", "bos_token_id", "eos_token_id"):
        assert c[k] == config[k], k
    assert set(ts) == set(tensors)
    for n, t in tensors.items():
        g = ts[n]
        assert (g.dtype, g.rows, g.cols) == (t.dtype, t.rows, t.cols) and np.array_equal(g.data, t.data), n


def _set(key, kind, value):
    def edit(meta, _):
        meta[key] = (kind, value)
    return edit


def _tensor(name, **change):
    def edit(_, ts):
        if not change:
            del ts[name]
            return
        dtype, shape, data = ts[name]
        ts[name] = (change.get("dtype", dtype), change.get("shape", shape), data)
    return edit


def _token(meta, _):
    meta["tokenizer.ggml.tokens"][1][30] = "wrong"


@pytest.mark.parametrize("edit,message", [
    (_set("general.architecture", STR, "llama"), "StableLM"),
    (_set("stablelm.attention.layer_norm_epsilon", "f64", float("nan")), "LayerNorm"),
    (_set("stablelm.rope.freq_base", "f64", float("inf")), "RoPE"),
    (_set("general.alignment", U32, 3), "alignment"),
    (_token, "vocabulary mismatch"),
    (_tensor("output.weight"), "tensor count"),
    (_tensor("output.weight", shape=[16, 342]), "shape"),
    (_tensor("output.weight", dtype="Q4_K"), "unsupported type"),
    (_tensor("output.weight", dtype="Q8_0"), "divisible by 32"),
], ids=["architecture", "nan", "infinite", "alignment", "vocabulary", "missing", "shape", "unsupported",
        "q8-alignment"])
def test_rejects(tmp_path, tiny_stablelm, pieces, edit, message):
    with pytest.raises(ValueError, match=message):
        gguf.load_stablelm_gguf(fixture(tmp_path, tiny_stablelm, pieces, edit))


def test_rejects_truncated_and_overlapping(tmp_path, tiny_stablelm, pieces):
    path = fixture(tmp_path, tiny_stablelm, pieces)
    data = bytearray(open(path, "rb").read())
    open(path, "wb").write(data[:-100])
    with pytest.raises(ValueError):
        gguf.load_stablelm_gguf(path)
    name = b"blk.0.attn_norm.bias"
    at = data.index(name) + len(name)
    (rank,) = struct.unpack_from("<I", data, at)
    at += 4 + 8 * rank + 4
    struct.pack_into("<Q", data, at, 0)
    open(path, "wb").write(data)
    with pytest.raises(ValueError, match="overlapping"):
        gguf.load_stablelm_gguf(path)


def test_header_limits(tmp_path):
    """Magic and version, tensor counts, ranks, zero dimensions, booleans,
    nested arrays and a header that ends early."""
    p = str(tmp_path / "x.gguf")

    def expect(blob, message):
        open(p, "wb").write(blob)
        with pytest.raises(ValueError, match=message):
            gguf.read_gguf(p)
    expect(b"GGUF", "GGUF v3")
    expect(struct.pack("<IIQQ", 0x46554747, 2, 1, 0), "GGUF v3")
    expect(struct.pack("<IIQQ", 0x46554747, 3, 0, 0), "counts")
    expect(struct.pack("<IIQQ", 0x46554747, 3, 10001, 0), "counts")
    name = struct.pack("<Q", 1) + b"t"
    expect(struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + name + struct.pack("<I", 5), "rank")
    expect(struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + name + struct.pack("<IQ", 1, 0), "dimensions")
    expect(struct.pack("<IIQQ", 0x46554747, 3, 1, 1) + name + struct.pack("<IB", 7, 2), "boolean")
    expect(struct.pack("<IIQQ", 0x46554747, 3, 1, 1) + name + struct.pack("<IIQ", 9, 9, 0), "array")
    expect(struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + name + struct.pack("<I", 1), "GGUF header")


def test_dimension_order_and_q4_k_extension(tmp_path):
    """A [4, 256] Q4_K matrix and a [3, 64] F32 one: dimensions come back
    row-major, offsets absolute and aligned, bytes where the writer put
    them; Q4_K is refused unless asked for."""
    p = str(tmp_path / "q.gguf")
    rng = np.random.default_rng(0)
    q = rng.integers(0, 256, 4 * 144, dtype=np.uint8)
    f = rng.standard_normal(3 * 64).astype(np.float32)
    write_gguf(p, {"general.alignment": (U32, 32)}, {"a.weight": ("Q4_K", [4, 256], q.tobytes()),
                                                     "b.weight": ("F32", [3, 64], f.tobytes())})
    with pytest.raises(ValueError, match="unsupported type 12"):
        gguf.read_gguf(p)
    meta, ts = gguf.read_gguf(p, q4_k=True)
    assert ts["a.weight"].shape == [4, 256] and ts["a.weight"].dtype == "Q4_K" and ts["a.weight"].size == 576
    assert ts["b.weight"].shape == [3, 64] and ts["b.weight"].size == 768
    raw = open(p, "rb").read()
    for name, want in (("a.weight", q.tobytes()), ("b.weight", f.tobytes())):
        t = ts[name]
        assert t.offset % 32 == 0 and raw[t.offset:t.offset + t.size] == want
    assert isinstance(meta["general.alignment"], gguf.U64)


def test_integer_metadata_must_be_unsigned(tmp_path, tiny_stablelm, pieces):
    """A signed 32-bit block count is not a GGUF integer to the reference
    (its integer() accepts only the unsigned kinds)."""
    with pytest.raises(ValueError, match="invalid GGUF integer stablelm.block_count"):
        gguf.load_stablelm_gguf(fixture(tmp_path, tiny_stablelm, pieces, _set("stablelm.block_count", I32, 2)))


def test_synthetic_q8_0_model_round_trip(tmp_path):
    """StableLM-3B widths (one layer, Q8_0 matrices, BF16 head): every
    tensor's bytes come back unchanged through the reversed dimensions."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=1, vocab_size=1024))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=3, head_dtype=W.BF16)
    pieces = [f"p{i}" for i in range(1024)]
    path = stablelm_gguf(str(tmp_path), config, tensors, pieces)
    c, ts = gguf.load_stablelm_gguf(path)
    assert c["partial_rotary_factor"] == config["partial_rotary_factor"]
    for n, t in tensors.items():
        assert ts[n].dtype == t.dtype and (ts[n].rows, ts[n].cols) == (t.rows, t.cols)
        assert np.array_equal(ts[n].data, t.data), n
