"""KV snapshots on the device: SaveCache / LoadCache (cache_file.go:49-216)
through tinyoai_stablelm_kv_save / _kv_load.

The payload bytes are checked against the resident cache read back per
layer and kv head (bit-exact) and against the oracle's KV (fp32 within 3e-5,
fp16 within one half-precision step); a restored forwarder continues with
logits bit-identical to the forwarder that wrote the file, and within 3e-5
of the oracle that never stopped; damaged and foreign files leave a
forwarder's resident prefix working as before (TestCacheFile,
cache_file_test.go:19-121).
"""
import numpy as np
import pytest

from tinyoai_amd import kv_cache as K
from tinyoai_amd import weights as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from tinyoai_amd import hip as H
    H.lib()
    return H


def payload_view(config, payload, n, half):
    """[layer][kv head][K/V][position][head_dim] as float32."""
    hd = config["hidden_size"] // config["num_attention_heads"]
    a = np.frombuffer(payload, np.float16 if half else np.float32)
    return a.reshape(config["num_hidden_layers"], config["num_key_value_heads"], 2, n, hd).astype(np.float32)


@pytest.mark.parametrize("half", [False, True])
def test_snapshot_round_trip_tiny(hip, oracle, tiny_stablelm, tmp_path, half):
    config, tensors = tiny_stablelm
    config = dict(config, max_position_embeddings=384)
    ident = K.model_identity(config, tensors)
    ids = [2] + [32 + (i * 17) % 300 for i in range(140)]
    p = 100
    ref = oracle.StableLM(config, tensors, half_kv=half, capacity=384)
    for i, t in enumerate(ids[:p]):
        ref.forward(t, i)
    f = hip.StableLMForwarder(config, tensors)
    if half:
        f.set_kv_bits(16)
    f.forward(0, ids[:p], False)
    path = str(tmp_path / "prefix.kv")
    K.save_cache(f, path, ids[:p], ident)
    raw = open(path, "rb").read()
    n = int.from_bytes(raw[8:12], "little")
    kv = payload_view(config, raw[12 + n:-32], p, half)
    step = 1e-3 if half else 0.0
    for layer in range(config["num_hidden_layers"]):
        k, v = f.read_kv(layer, 0, p)
        assert np.array_equal(kv[layer, 0, 0], k) and np.array_equal(kv[layer, 0, 1], v)
        k, v = ref.read_kv(layer, 0, p)
        tol = np.maximum(3e-5, step * np.abs(k))
        assert np.all(np.abs(kv[layer, 0, 0] - k) <= tol)
        tol = np.maximum(3e-5, step * np.abs(v))
        assert np.all(np.abs(kv[layer, 0, 1] - v) <= tol)

    g = hip.StableLMForwarder(config, tensors)
    if half:
        g.set_kv_bits(16)
    g.forward(0, ids[:5], False)
    assert K.load_cache(g, path, ident) == ids[:p]
    assert g.offset == p
    suffix = ids[p:]
    want = f.forward(p, suffix)
    got = g.forward(p, suffix)
    assert np.array_equal(got, want)
    for i, t in enumerate(suffix):
        last = ref.forward(t, p + i)
    assert np.max(np.abs(got - last)) <= 3e-5

    # damaged and foreign files are refused; g's prefix stays usable
    corrupt = bytearray(raw)
    corrupt[12 + n + 10] ^= 1
    for data in (raw[:10], raw[:-1], raw + b"\0", bytes(corrupt)):
        open(path, "wb").write(data)
        with pytest.raises((ValueError, EOFError)):
            K.load_cache(g, path, ident)
    open(path, "wb").write(raw)
    flipped = dict(tensors)
    q = tensors["model.layers.0.self_attn.q_proj.weight"]
    data = q.data.copy()
    data[0] ^= 1
    flipped["model.layers.0.self_attn.q_proj.weight"] = W.Tensor(q.dtype, q.rows, q.cols, data)
    with pytest.raises(ValueError, match="checkpoint"):
        K.load_cache(g, path, K.model_identity(config, flipped))
    other = hip.StableLMForwarder(config, tensors)
    other.set_kv_bits(32 if half else 16)
    with pytest.raises(ValueError, match="precision"):
        K.load_cache(other, path, ident)
    with pytest.raises(hip.TinyoaiError):
        other.kv_load(p, half, raw[12 + n:-32])  # the library refuses a payload of the other format too
    other.close()
    assert g.offset == len(ids)
    assert np.array_equal(g.forward(p, suffix), want)
    with pytest.raises(hip.TinyoaiError):
        g.kv_save(len(ids) + 1, half)  # beyond the resident prefix
    f.close()
    g.close()


def test_snapshot_3b_shapes_payload_round_trip(hip, tmp_path):
    """StableLM-3B layer shapes (two layers, Q8_0, 32 kv heads of 80): 1500
    positions in fp16 saved, loaded into a fresh forwarder and saved again
    give the same bytes; the next token's logits agree bit for bit."""
    config = W.validate_stablelm_config(dict(W.STABLELM_3B, num_hidden_layers=2, max_position_embeddings=2048))
    tensors = W.synthetic_stablelm(config, W.Q8_0, seed=5)
    ident = K.model_identity(config, tensors)
    ids = np.random.default_rng(6).integers(0, config["vocab_size"], 1501).tolist()
    f = hip.StableLMForwarder(config, tensors)
    f.set_kv_bits(16)
    f.forward(0, ids[:1500], False)
    path = str(tmp_path / "big.kv")
    K.save_cache(f, path, ids[:1500], ident)
    g = hip.StableLMForwarder(config, tensors)
    g.set_kv_bits(16)
    assert K.load_cache(g, path, ident) == ids[:1500]
    assert g.kv_save(1500, True) == f.kv_save(1500, True)
    assert np.array_equal(g.forward(1500, ids[1500:]), f.forward(1500, ids[1500:]))
    f.close()
    g.close()
