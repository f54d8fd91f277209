"""The TNYKV001 container (cache_file.go) without a GPU.

The payload side is a stand-in forwarder that keeps KV bytes in host memory;
what is checked here is the container the host keeps: encoding/json's
formatting of the config and header, the model identity's sensitivity, and
every damaged or incompatible file TestCacheFile (cache_file_test.go:19-121)
feeds LoadCache, each rejected with the resident state unchanged.
"""
import json
import os
import struct

import numpy as np
import pytest

from tinyoai_amd import kv_cache as K
from tinyoai_amd import weights as W


class HostForwarder:
    """Resident KV in host memory with the forwarder's payload methods."""

    def __init__(self, config, half=False, seed=0):
        self.config = config
        self.kv_half = half
        self.offset = 0
        self.rng = np.random.default_rng(seed)
        self.kv = b""

    def fill(self, n):
        self.kv = self.rng.integers(0, 256, K.payload_bytes(self.config, n, self.kv_half), dtype=np.uint8).tobytes()
        self.offset = n

    def kv_save(self, n, half):
        assert half == self.kv_half and n <= self.offset
        per = K.payload_bytes(self.config, 1, half) // (2 * self.config["num_hidden_layers"]
                                                        * self.config["num_key_value_heads"])
        rows = np.frombuffer(self.kv, np.uint8).reshape(-1, self.offset * per)
        return rows[:, :n * per].tobytes()

    def kv_load(self, n, half, payload):
        assert half == self.kv_half and len(payload) == K.payload_bytes(self.config, n, half)
        self.kv, self.offset = bytes(payload), n


def test_go_float_matches_encoding_json():
    """encoding/json's float64 output: shortest round-trip digits, positional
    inside [1e-6, 1e21), exponent form with the exponent's leading zeros
    dropped outside (json.Marshal(1e-7) is "1e-7")."""
    cases = {1e-05: "0.00001", 10000.0: "10000", 0.25: "0.25", 0.1: "0.1", 1e-06: "0.000001",
             1e-07: "1e-7", 1e21: "1e+21", 1e20: "100000000000000000000", 123456789.0: "123456789",
             -2.5e-9: "-2.5e-9", 1.5e300: "1.5e+300", 5e-324: "5e-324", 0.0: "0", 1e6: "1000000"}
    for x, want in cases.items():
        assert K.go_float(x) == want, x
        assert float(K.go_float(x)) == x
    with pytest.raises(ValueError):
        K.go_float(float("nan"))


def test_config_json_of_reference_fixture(tiny_stablelm):
    """json.Marshal of the tiny fixture's validated StableLMConfig: struct
    field order, the float fields as Go prints them, unknown keys dropped,
    rope_scaling null kept (a RawMessage holds the literal), no
    rope_parameters (nil pointer, omitempty)."""
    config, _ = tiny_stablelm
    want = ('{"model_type":"stablelm","vocab_size":342,"hidden_size":16,"intermediate_size":40,'
            '"num_hidden_layers":2,"num_attention_heads":2,"num_key_value_heads":1,"hidden_act":"silu",'
            '"max_position_embeddings":64,"layer_norm_eps":0.00001,"rope_theta":10000,'
            '"partial_rotary_factor":0.5,"use_parallel_residual":true,"use_qkv_bias":false,'
            '"qk_layernorm":false,"tie_word_embeddings":false,"bos_token_id":2,"eos_token_id":3,'
            '"rope_scaling":null}')
    assert K.go_config_json(config).decode() == want
    nested = dict(config, rope_parameters={"rope_type": "default", "rope_theta": 1e6, "partial_rotary_factor": 0.25})
    del nested["rope_scaling"]
    got = K.go_config_json(W.validate_stablelm_config(nested)).decode()
    assert '"rope_theta":1000000,' in got and got.endswith(
        '"rope_parameters":{"rope_type":"default","rope_theta":1000000,"partial_rotary_factor":0.25}}')


def test_model_identity_binds_config_and_bytes(tiny_stablelm):
    """Stable for equal inputs; changed by one weight bit (the test's
    `q.data[0] ^= 1`) and by a config field; a weight whose element count
    does not fit its Go shape is refused."""
    config, tensors = tiny_stablelm
    a = K.model_identity(config, tensors)
    assert len(a) == 32 and a == K.model_identity(dict(config), dict(tensors))
    flipped = dict(tensors)
    q = tensors["model.layers.0.self_attn.q_proj.weight"]
    data = q.data.copy()
    data[0] ^= 1
    flipped["model.layers.0.self_attn.q_proj.weight"] = W.Tensor(q.dtype, q.rows, q.cols, data)
    assert K.model_identity(config, flipped) != a
    assert K.model_identity(dict(config, max_position_embeddings=384), tensors) != a
    retyped = dict(tensors)
    n = tensors["model.norm.weight"]
    retyped["model.norm.weight"] = W.Tensor(W.F16, n.rows, n.cols * 2, n.data)  # 2d values where [d] is declared
    with pytest.raises(ValueError):
        K.model_identity(config, retyped)


@pytest.mark.parametrize("half", [False, True])
def test_container_round_trip_and_damaged_files(tmp_path, tiny_stablelm, half):
    """SaveCache then LoadCache restores tokens and payload; the file is
    mode 0600 with the exact size; truncated, extended, bit-flipped,
    foreign-model and other-precision files are refused and leave the
    resident state as it was."""
    config, tensors = tiny_stablelm
    config = dict(config, max_position_embeddings=384)
    ident = K.model_identity(config, tensors)
    src = HostForwarder(config, half, seed=1)
    src.fill(96)
    tokens = [int(t) for t in np.random.default_rng(2).integers(0, 342, 64)]
    path = str(tmp_path / "prefix.kv")
    K.save_cache(src, path, tokens, ident)
    assert os.stat(path).st_mode & 0o777 == 0o600
    raw = open(path, "rb").read()
    (n,) = struct.unpack("<I", raw[8:12])
    header = json.loads(raw[12:12 + n])
    assert raw[:8] == b"TNYKV001" and header == {"model_sha256": list(ident), "float16": half, "tokens": tokens}
    assert len(raw) == 12 + n + K.payload_bytes(config, 64, half) + 32
    dst = HostForwarder(config, half, seed=3)
    dst.fill(10)
    assert K.load_cache(dst, path, ident) == tokens
    assert dst.offset == 64 and dst.kv == src.kv_save(64, half)
    before = (dst.kv, dst.offset)
    corrupt = bytearray(raw)
    corrupt[12 + n + 10] ^= 1
    for data in (raw[:10], raw[:-1], raw + b"\0", bytes(corrupt)):
        open(path, "wb").write(data)
        with pytest.raises((ValueError, EOFError)):
            K.load_cache(dst, path, ident)
        assert (dst.kv, dst.offset) == before
    open(path, "wb").write(raw)
    with pytest.raises(ValueError, match="does not match checkpoint"):
        K.load_cache(dst, path, bytes(32))
    other = HostForwarder(config, not half)
    with pytest.raises(ValueError, match="precision"):
        K.load_cache(other, path, ident)
    small = HostForwarder(dict(config, max_position_embeddings=32), half)
    with pytest.raises(ValueError, match="exceeds model context"):
        K.load_cache(small, path, ident)


def test_empty_prefix_and_header_checks(tmp_path, tiny_stablelm):
    """No tokens: header with "tokens":null, no payload, and loading it
    empties the resident prefix. Wrong magic, oversized header length and
    out-of-range token ids are refused."""
    config, tensors = tiny_stablelm
    ident = K.model_identity(config, tensors)
    path = str(tmp_path / "empty.kv")
    src = HostForwarder(config)
    K.save_cache(src, path, [], ident)
    raw = open(path, "rb").read()
    (n,) = struct.unpack("<I", raw[8:12])
    assert b'"tokens":null' in raw[12:12 + n] and len(raw) == 12 + n + 32
    dst = HostForwarder(config)
    dst.fill(5)
    assert K.load_cache(dst, path, ident) == [] and dst.offset == 0
    for data in (b"TNYKV002" + raw[8:], raw[:8] + struct.pack("<I", (1 << 20) + 1) + raw[12:]):
        open(path, "wb").write(data)
        with pytest.raises(ValueError):
            K.load_cache(dst, path, ident)
    header = K.encode_header(ident, False, [1, 342])
    body = b"TNYKV001" + struct.pack("<I", len(header)) + header
    open(path, "wb").write(body + bytes(K.payload_bytes(config, 2, False)) + bytes(32))
    with pytest.raises(ValueError, match="invalid KV cache token 342"):
        K.load_cache(dst, path, ident)
