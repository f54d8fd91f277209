"""KV snapshots: SaveCache / LoadCache (cache_file.go:49-186) over the HIP forwarder.

The container is the reference's TNYKV001 file, byte for byte:

    "TNYKV001" | uint32 LE header length n (<= 1 MiB) | n bytes of JSON
    {"model_sha256":[32 ints],"float16":bool,"tokens":[ids] or null}
    | payload (only when tokens is non-empty) | SHA-256 of all preceding bytes

The payload is cachePayload's order (cache_file.go:188-216): for each layer,
each kv head, K then V, positions [0, len(tokens)) of head_dim values as
little-endian float32 or raw float16 bits. The library moves that payload
between the file's bytes and the resident device cache
(tinyoai_stablelm_kv_save / _kv_load); this module keeps the container, the
model identity and the checks, as the Go host does.

The model identity (modelIdentity, cache_file.go:26-47) is SHA-256 over the
json.Marshal bytes of the validated StableLMConfig, then for each weight in
load order (embed, head, final norm weight and bias, then per layer: norm
weight and bias, q, k, v, o, gate, up, down) json.Marshal of {Type, Shape}
followed by the tensor's bytes in file encoding. ``go_config_json`` and
``go_float`` reproduce encoding/json's output for the values that occur
there.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
import tempfile

import numpy as np

from . import weights as W

MAGIC = b"TNYKV001"
MAX_HEADER = 1 << 20

# StableLMConfig's fields in declaration order with their Go kinds
# (stablelm.go:18-77); rope_parameters and rope_scaling are omitempty.
_CONFIG_FIELDS = (
    ("model_type", str), ("vocab_size", int), ("hidden_size", int), ("intermediate_size", int),
    ("num_hidden_layers", int), ("num_attention_heads", int), ("num_key_value_heads", int),
    ("hidden_act", str), ("max_position_embeddings", int), ("layer_norm_eps", float),
    ("rope_theta", float), ("partial_rotary_factor", float), ("use_parallel_residual", bool),
    ("use_qkv_bias", bool), ("qk_layernorm", bool), ("tie_word_embeddings", bool),
    ("bos_token_id", int), ("eos_token_id", int),
)
_ROPE_FIELDS = (("rope_type", str), ("rope_theta", float), ("partial_rotary_factor", float))


def go_float(x: float) -> str:
    """encoding/json's float64 encoding: the shortest decimal that reads back
    as x, positional for 1e-6 <= |x| < 1e21, otherwise exponent form with
    at least one exponent digit ("1e-7", "1e+21")."""
    x = float(x)
    if x != x or x in (float("inf"), float("-inf")):
        raise ValueError("json: unsupported value")
    if x == 0:
        return "-0" if np.signbit(x) else "0"
    if 1e-6 <= abs(x) < 1e21:
        return np.format_float_positional(x, unique=True, trim="-")
    s = np.format_float_scientific(x, unique=True, trim="-", exp_digits=1)
    m, e = s.split("e")
    return m + "e" + ("-" if e[0] == "-" else "+") + e[1:].lstrip("0").rjust(1, "0")


def _go_str(s: str) -> str:
    # encoding/json writes UTF-8 with <, >, & and U+2028/U+2029 escaped as
    # \\uXXXX; json.dumps(ensure_ascii=False) agrees on everything else
    # that can occur in a config string.
    out = json.dumps(s, ensure_ascii=False)
    for a, b in (("<", "\\u003c"), (">", "\\u003e"), ("&", "\\u0026"), ("\u2028", "\\u2028"), ("\u2029", "\\u2029")):
        out = out.replace(a, b)
    return out


def _go_value(v, kind) -> str:
    if kind is str:
        return _go_str(str(v))
    if kind is bool:
        return "true" if v else "false"
    if kind is int:
        if isinstance(v, float) and v != int(v):
            raise ValueError(f"json: cannot unmarshal number {v} into an int field")
        return str(int(v))
    return go_float(v)


def go_config_json(config: dict) -> bytes:
    """json.Marshal of the validated StableLMConfig (stablelm.go:18-77)."""
    parts = [f'"{k}":{_go_value(config.get(k, kind()), kind)}' for k, kind in _CONFIG_FIELDS]
    rp = config.get("rope_parameters")
    if rp is not None:
        inner = ",".join(f'"{k}":{_go_value(rp.get(k, kind()), kind)}' for k, kind in _ROPE_FIELDS)
        parts.append(f'"rope_parameters":{{{inner}}}')
    if "rope_scaling" in config:  # a RawMessage keeps JSON null as the 4 bytes "null"
        if config["rope_scaling"] is not None:
            raise ValueError("RoPE scaling is not supported")
        parts.append('"rope_scaling":null')
    return ("{" + ",".join(parts) + "}").encode()


def identity_tensors(config: dict, tensors: dict):
    """(name, Go shape) in modelIdentity's order (cache_file.go:33-36)."""
    d, h = config["hidden_size"], config["intermediate_size"]
    kv = d // config["num_attention_heads"] * config["num_key_value_heads"]
    v = config["vocab_size"]
    out = [("model.embed_tokens.weight", [v, d]), ("lm_head.weight", [v, d]),
           ("model.norm.weight", [d]), ("model.norm.bias", [d])]
    for i in range(config["num_hidden_layers"]):
        p = f"model.layers.{i}."
        out += [(p + "input_layernorm.weight", [d]), (p + "input_layernorm.bias", [d]),
                (p + "self_attn.q_proj.weight", [d, d]), (p + "self_attn.k_proj.weight", [kv, d]),
                (p + "self_attn.v_proj.weight", [kv, d]), (p + "self_attn.o_proj.weight", [d, d]),
                (p + "mlp.gate_proj.weight", [h, d]), (p + "mlp.up_proj.weight", [h, d]),
                (p + "mlp.down_proj.weight", [d, h])]
    for name, shape in out:
        t = tensors[name]
        if t.rows * t.cols != int(np.prod(shape)):
            raise ValueError(f"tensor {name}: shape [{t.rows},{t.cols}], want {shape}")
    return out


def model_identity(config: dict, tensors: dict) -> bytes:
    """modelIdentity (cache_file.go:26-47): 32 bytes binding a snapshot to
    the configuration and the exact weight bytes."""
    c = W.validate_stablelm_config(config)
    h = hashlib.sha256(go_config_json(c))
    for name, shape in identity_tensors(c, tensors):
        t = tensors[name]
        h.update(('{"Type":%s,"Shape":[%s]}' % (_go_str(W.DTYPE_NAMES[t.dtype]), ",".join(map(str, shape)))).encode())
        h.update(memoryview(t.data))
    return h.digest()


def payload_bytes(config: dict, tokens: int, half: bool) -> int:
    hd = config["hidden_size"] // config["num_attention_heads"]
    return config["num_hidden_layers"] * 2 * config["num_key_value_heads"] * hd * tokens * (2 if half else 4)


def encode_header(identity: bytes, half: bool, tokens) -> bytes:
    """json.Marshal(cacheHeader) (cache_file.go:18-22): [32]byte is a JSON
    array of numbers, a nil token slice is null."""
    toks = "null" if len(tokens) == 0 else "[" + ",".join(str(int(t)) for t in tokens) + "]"
    ident = "[" + ",".join(str(b) for b in identity) + "]"
    return f'{{"model_sha256":{ident},"float16":{"true" if half else "false"},"tokens":{toks}}}'.encode()


def save_cache(fwd, path: str, tokens, identity: bytes) -> None:
    """SaveCache (cache_file.go:52-101): the first len(tokens) resident
    positions of `fwd` with their token ids, written to a temporary file in
    the destination directory (mode 0600), synced and renamed over `path`."""
    tokens = [int(t) for t in tokens]
    half = fwd.kv_half
    header = encode_header(identity, half, tokens)
    digest = hashlib.sha256()
    d = os.path.dirname(os.path.abspath(path))
    fd, tmp = tempfile.mkstemp(prefix=".tinyoai-kv-", dir=d)  # created 0600
    try:
        with os.fdopen(fd, "wb") as f:
            for chunk in (MAGIC + struct.pack("<I", len(header)), header,
                          fwd.kv_save(len(tokens), half) if tokens else b""):
                digest.update(chunk)
                f.write(chunk)
            f.write(digest.digest())
            f.flush()
            os.fsync(f.fileno())
        os.rename(tmp, path)
    finally:
        if os.path.exists(tmp):
            os.remove(tmp)


def load_cache(fwd, path: str, identity: bytes) -> list[int]:
    """LoadCache (cache_file.go:103-186): verifies the whole file (format,
    header bounds, token ids, model identity, KV precision, exact size,
    checksum) before replacing the resident cache; any error leaves it as it
    was. Returns the restored token ids; the forwarder's offset becomes
    their count."""
    c = fwd.config
    with open(path, "rb") as f:
        prefix = f.read(len(MAGIC) + 4)
        if len(prefix) < len(MAGIC) + 4:
            raise EOFError("unexpected EOF")
        if prefix[:len(MAGIC)] != MAGIC:
            raise ValueError("unsupported KV cache format")
        (n,) = struct.unpack("<I", prefix[len(MAGIC):])
        if n > MAX_HEADER:
            raise ValueError("KV cache header too large")
        data = f.read(n)
        if len(data) < n:
            raise EOFError("unexpected EOF")
        header = json.loads(data)
        if not isinstance(header, dict):
            raise ValueError("json: cannot unmarshal KV cache header")
        tokens = header.get("tokens") or []
        if not isinstance(tokens, list) or any(isinstance(t, bool) or not isinstance(t, int) for t in tokens):
            raise ValueError("json: cannot unmarshal KV cache tokens")
        if len(tokens) > c["max_position_embeddings"]:
            raise ValueError("KV cache exceeds model context")
        for t in tokens:
            if not 0 <= t < c["vocab_size"]:
                raise ValueError(f"invalid KV cache token {t}")
        model = header.get("model_sha256")
        if (not isinstance(model, list) or any(isinstance(b, bool) or not isinstance(b, int) or not 0 <= b < 256
                                               for b in model)):
            raise ValueError("json: cannot unmarshal model_sha256")
        if bytes(model[:32]).ljust(32, b"\0") != identity:
            raise ValueError("KV cache model does not match checkpoint")
        half = bool(header.get("float16", False))
        if half != fwd.kv_half:
            raise ValueError("KV cache precision does not match model options")
        size = os.fstat(f.fileno()).st_size
        want = len(prefix) + n + payload_bytes(c, len(tokens), half) + 32
        if size != want:
            raise ValueError(f"KV cache size {size}, expected {want}")
        payload = f.read(payload_bytes(c, len(tokens), half))
        checksum = f.read(32)
    if hashlib.sha256(prefix + data + payload).digest() != checksum:
        raise ValueError("KV cache checksum mismatch")
    fwd.kv_load(len(tokens), half, payload)
    return tokens
