"""Host-side weight containers, checkpoint readers and synthetic workloads.

A ``Tensor`` keeps a tensor in its on-disk encoding (raw little-endian bytes,
a GGUF type code and a row-major [rows, cols] shape), as the reference's
``weightTensor`` does (safetensors.go:193-197). The HIP library receives
exactly these bytes and repacks them for HBM itself.
"""
from __future__ import annotations

import json
import math
import os
import struct
from dataclasses import dataclass

import numpy as np

# GGUF tensor type codes (gguf.go:183-214); Q4_K (12) is the public GGML code.
F32, F16, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 7, 8, 12, 13, 14, 30
DTYPE_NAMES = {F32: "F32", F16: "F16", Q5_1: "Q5_1", Q8_0: "Q8_0", Q4_K: "Q4_K",
               Q5_K: "Q5_K", Q6_K: "Q6_K", BF16: "BF16"}
NAME_DTYPES = {v: k for k, v in DTYPE_NAMES.items()}
# (values per block, bytes per block)
BLOCKS = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q5_1: (32, 24),
          Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}


def nbytes(dtype: int, rows: int, cols: int) -> int:
    per, size = BLOCKS[dtype]
    if (rows * cols) % per:
        raise ValueError(f"{DTYPE_NAMES[dtype]} needs a multiple of {per} values")
    return rows * cols // per * size


@dataclass
class Tensor:
    dtype: int
    rows: int
    cols: int
    data: np.ndarray  # uint8, raw bytes in on-disk encoding

    def __post_init__(self):
        self.data = np.ascontiguousarray(self.data).view(np.uint8).reshape(-1)
        if self.data.size != nbytes(self.dtype, self.rows, self.cols):
            raise ValueError(f"{DTYPE_NAMES[self.dtype]} [{self.rows},{self.cols}] expects "
                             f"{nbytes(self.dtype, self.rows, self.cols)} bytes, got {self.data.size}")


# ---------------------------------------------------------------- safetensors
def _read_safetensors(path: str) -> dict:
    """Minimal safetensors reader with the reference's header checks
    (safetensors.go:34-109): bounded header, known dtypes, exact byte counts,
    no gaps or overlaps, no trailing data."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        (length,) = struct.unpack("<Q", f.read(8))
        if length == 0 or length > 16 << 20 or length > size - 8:
            raise ValueError(f"invalid safetensors header length {length}")
        header = json.loads(f.read(length))
        payload = np.frombuffer(f.read(), np.uint8)
    width = {"F32": 4, "BF16": 2, "F16": 2}
    out, ranges = {}, []
    for name, info in header.items():
        if name == "__metadata__":
            continue
        if info["dtype"] not in width:
            raise ValueError(f"tensor {name}: unsupported dtype {info['dtype']}")
        a, b = info["data_offsets"]
        n = width[info["dtype"]]
        for d in info["shape"]:
            n *= d
        if n != b - a or b > payload.size:
            raise ValueError(f"tensor {name}: shape does not match byte count")
        ranges.append((a, b))
        shape = info["shape"]
        rows, cols = (shape[0], shape[1]) if len(shape) == 2 else (1, shape[0])
        out[name] = Tensor(NAME_DTYPES[info["dtype"]], rows, cols, payload[a:b].copy())
    end = 0
    for a, b in sorted(ranges):
        if a != end:
            raise ValueError("safetensors data contains gaps or overlapping tensors")
        end = b
    if end != payload.size:
        raise ValueError("safetensors has trailing data")
    return out


def load_safetensors_dir(path: str) -> tuple[dict, dict]:
    """Reads config.json plus single-file or indexed safetensors
    (stablelm.go:136-161, safetensors.go:130-185)."""
    with open(os.path.join(path, "config.json")) as f:
        config = json.load(f)
    index = os.path.join(path, "model.safetensors.index.json")
    tensors = {}
    if os.path.exists(index):
        with open(index) as f:
            weight_map = json.load(f)["weight_map"]
        for shard in sorted(set(weight_map.values())):
            if os.path.basename(shard) != shard:
                raise ValueError(f"invalid shard filename {shard!r}")
            for name, t in _read_safetensors(os.path.join(path, shard)).items():
                if name in tensors:
                    raise ValueError(f"duplicate tensor {name}")
                if weight_map.get(name) != shard:
                    raise ValueError(f"index disagrees with shard for {name}")
                tensors[name] = t
        missing = set(weight_map) - set(tensors)
        if missing:
            raise ValueError(f"index tensor {sorted(missing)[0]} missing from shard")
    else:
        tensors = _read_safetensors(os.path.join(path, "model.safetensors"))
    return config, tensors


# ---------------------------------------------------------------- encoders
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """IEEE round-to-nearest-even float16 bits (numpy's cast is RNE)."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def encode_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bytes by round-to-nearest-even of the high half
    (finite values: the sum below stays within 32 bits)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32)
    r = (b >> 16) & np.uint32(1)
    r += np.uint32(0x7FFF)
    r += b
    r >>= 16
    return r.astype(np.uint16).view(np.uint8)


def encode_q8_0(scales: np.ndarray, qs: np.ndarray) -> np.ndarray:
    """Packs GGUF Q8_0 blocks {fp16 d, int8 q[32]} = 34 B (dot.go:31-40)."""
    nb = scales.size
    out = np.empty((nb, 34), np.uint8)
    out[:, :2] = np.asarray(scales, np.uint16).reshape(nb, 1).view(np.uint8)
    out[:, 2:] = np.asarray(qs, np.int8).reshape(nb, 32).view(np.uint8)
    return out.reshape(-1)


def synthetic_q8_0(rows: int, cols: int, rng: np.random.Generator, std: float = 0.02) -> Tensor:
    """int8 uniform in [-127, 127] with fp16 d = RNE(|N(0, std)| / 127)."""
    nb = rows * cols // 32
    qs = rng.integers(-127, 128, size=(nb, 32), dtype=np.int16).astype(np.int8)
    d = f32_to_f16_bits((np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(std)) / np.float32(127))
    return Tensor(Q8_0, rows, cols, encode_q8_0(d, qs))


def synthetic_bf16(rows: int, cols: int, rng: np.random.Generator, std: float = 0.02) -> Tensor:
    return Tensor(BF16, rows, cols, encode_bf16(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(std)))


def synthetic_f32(rows: int, cols: int, rng: np.random.Generator, std: float = 0.02, mean: float = 0.0) -> Tensor:
    v = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(std) + np.float32(mean)
    return Tensor(F32, rows, cols, v.astype(np.float32).view(np.uint8))


def synthetic_kquant(dtype: int, rows: int, cols: int, rng: np.random.Generator, std: float = 0.02) -> Tensor:
    """Random K-quant super-blocks with seeded fp16 scales/mins sized so that
    weights are O(std): random quant bits, 6-bit scales/mins in [0, 63]."""
    nb = rows * cols // 256
    size = BLOCKS[dtype][1]
    b = rng.integers(0, 256, size=(nb, size), dtype=np.int32).astype(np.uint8)
    if dtype == Q6_K:
        d = f32_to_f16_bits(np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(std / (32 * 32)))
        b[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
        b[:, 208:210] = d.reshape(nb, 1).view(np.uint8)
    else:  # Q4_K, Q5_K: d, dmin, 12-byte scales
        top = 16 if dtype == Q4_K else 32
        d = f32_to_f16_bits(np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(std / (32 * top)))
        dmin = f32_to_f16_bits(np.abs(rng.standard_normal(nb, dtype=np.float32)) * np.float32(std / (32 * 2)))
        b[:, 0:2] = d.reshape(nb, 1).view(np.uint8)
        b[:, 2:4] = dmin.reshape(nb, 1).view(np.uint8)
    return Tensor(dtype, rows, cols, b.reshape(-1))


def synthetic_stablelm(config: dict, dtype: int, seed: int, attn_dtype: int | None = None,
                       head_dtype: int | None = None) -> dict:
    """Seeded StableLM weights: matrices in ``dtype`` (attention matrices in
    ``attn_dtype`` when given), F32 LayerNorm w = 1 + N(0, 0.1), b = N(0, 0.1).
    Quantized scales follow |N(0, 0.02)| / 127 (Q8_0) or the K-quant recipe."""
    rng = np.random.default_rng(seed)
    d, h, L, V = config["hidden_size"], config["intermediate_size"], config["num_hidden_layers"], config["vocab_size"]
    kv = d // config["num_attention_heads"] * config["num_key_value_heads"]

    def mat(rows, cols, dt):
        if dt == Q8_0:
            return synthetic_q8_0(rows, cols, rng)
        if dt == BF16:
            return synthetic_bf16(rows, cols, rng)
        if dt == F32:
            return synthetic_f32(rows, cols, rng)
        if dt == F16:
            return Tensor(F16, rows, cols, f32_to_f16_bits(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)).view(np.uint8))
        return synthetic_kquant(dt, rows, cols, rng)

    def norm(mean):
        return synthetic_f32(1, d, rng, std=0.1, mean=mean)

    attn = dtype if attn_dtype is None else attn_dtype
    head = dtype if head_dtype is None else head_dtype
    t = {"model.embed_tokens.weight": mat(V, d, dtype), "lm_head.weight": mat(V, d, head),
         "model.norm.weight": norm(1.0), "model.norm.bias": norm(0.0)}
    for i in range(L):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = norm(1.0)
        t[p + "input_layernorm.bias"] = norm(0.0)
        t[p + "self_attn.q_proj.weight"] = mat(d, d, attn)
        t[p + "self_attn.k_proj.weight"] = mat(kv, d, attn)
        t[p + "self_attn.v_proj.weight"] = mat(kv, d, attn)
        t[p + "self_attn.o_proj.weight"] = mat(d, d, attn)
        t[p + "mlp.gate_proj.weight"] = mat(h, d, dtype)
        t[p + "mlp.up_proj.weight"] = mat(h, d, dtype)
        t[p + "mlp.down_proj.weight"] = mat(d, h, dtype)
    return t


# StableLM-3B-4E1T-like shapes used by the decode/prefill workloads.
STABLELM_3B = dict(model_type="stablelm", vocab_size=65536, hidden_size=2560, intermediate_size=6912,
                   num_hidden_layers=32, num_attention_heads=32, num_key_value_heads=32,
                   max_position_embeddings=8192, layer_norm_eps=1e-5, rope_theta=10000.0,
                   partial_rotary_factor=0.25, bos_token_id=0, eos_token_id=0,
                   use_parallel_residual=True, use_qkv_bias=False, qk_layernorm=False,
                   tie_word_embeddings=False, hidden_act="silu")


def validate_stablelm_config(c: dict) -> dict:
    """StableLMConfig.validate (stablelm.go:85-111), returning a normalized copy."""
    c = dict(c)
    if (c.get("model_type") != "stablelm" or not c.get("use_parallel_residual", False)
            or c.get("use_qkv_bias", False) or c.get("qk_layernorm", False)
            or c.get("tie_word_embeddings", False) or c.get("hidden_act", "silu") != "silu"):
        raise ValueError("unsupported StableLM variant: require parallel residuals, no QKV bias/QK norm, "
                         "untied embeddings, and silu")
    for k in ("hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
              "num_key_value_heads", "vocab_size", "max_position_embeddings"):
        if c.get(k, 0) <= 0:
            raise ValueError("invalid StableLM dimensions")
    if c["hidden_size"] % c["num_attention_heads"] or c["num_attention_heads"] % c["num_key_value_heads"]:
        raise ValueError("invalid StableLM dimensions")
    rp = c.get("rope_parameters")
    if rp is not None:
        if rp.get("rope_type") != "default":
            raise ValueError(f"unsupported RoPE type {rp.get('rope_type')!r}")
        c["rope_theta"], c["partial_rotary_factor"] = rp["rope_theta"], rp["partial_rotary_factor"]
    if c.get("rope_scaling") is not None:
        raise ValueError("RoPE scaling is not supported")
    c.setdefault("layer_norm_eps", 1e-5)
    c.setdefault("rope_theta", 10000.0)
    c.setdefault("partial_rotary_factor", 0.25)
    rot = c["hidden_size"] // c["num_attention_heads"] * c["partial_rotary_factor"]
    if (not c["layer_norm_eps"] > 0 or math.isinf(c["layer_norm_eps"]) or not c["rope_theta"] > 0
            or math.isinf(c["rope_theta"]) or not 0 < c["partial_rotary_factor"] <= 1
            or rot != int(rot) or int(rot) % 2 or rot < 2):
        raise ValueError("invalid LayerNorm or partial RoPE settings")
    for k in ("bos_token_id", "eos_token_id"):
        if not 0 <= c.get(k, 0) < c["vocab_size"]:
            raise ValueError("invalid BOS/EOS token IDs")
    return c


# ---------------------------------------------------------------- llama2.c
LLAMA_HEADER = ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len")


def read_llama2c(path: str) -> tuple[dict, np.ndarray]:
    """llama2.c checkpoint: 7 int32 header + float32 payload (model.go:90-166)."""
    raw = np.fromfile(path, np.uint8)
    header = raw[:28].view(np.int32)
    c = dict(zip(LLAMA_HEADER, (int(v) for v in header)))
    if (c["dim"] <= 0 or c["hidden_dim"] <= 0 or c["n_layers"] <= 0 or c["n_heads"] <= 0
            or c["n_kv_heads"] <= 0 or c["n_heads"] % c["n_kv_heads"] or c["vocab_size"] < 2
            or c["seq_len"] <= 0 or c["dim"] % c["n_heads"] or (c["dim"] // c["n_heads"]) % 2):
        raise ValueError(f"invalid config header: {c}")
    weights = raw[28:].view(np.float32)
    if weights.size != llama_payload_floats(c):
        raise ValueError("checkpoint size does not match its header layout")
    return c, weights


def llama_payload_floats(c: dict) -> int:
    dim, hid, L, V, S = c["dim"], c["hidden_dim"], c["n_layers"], c["vocab_size"], c["seq_len"]
    hs = dim // c["n_heads"]
    kv = hs * c["n_kv_heads"]
    return V * dim + L * dim + L * dim * dim + 2 * L * dim * kv + L * dim * dim + L * dim + 3 * L * hid * dim + dim + S * hs


def synthetic_llama(c: dict, seed: int) -> np.ndarray:
    """Seeded N(0, 0.02) llama2.c payload with RMSNorm weights 1 and the
    checkpoint's RoPE tables cos/sin(pos * 10000^(-2i/hs))."""
    rng = np.random.default_rng(seed)
    n = llama_payload_floats(c)
    w = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    dim, hid, L, V, S = c["dim"], c["hidden_dim"], c["n_layers"], c["vocab_size"], c["seq_len"]
    hs = dim // c["n_heads"]
    kv = hs * c["n_kv_heads"]
    off = V * dim
    w[off:off + L * dim] = 1.0
    off += L * dim + L * dim * dim + 2 * L * dim * kv + L * dim * dim
    w[off:off + L * dim] = 1.0
    off += L * dim + 3 * L * hid * dim
    w[off:off + dim] = 1.0
    off += dim
    freqs = 1.0 / (10000.0 ** (np.arange(0, hs, 2, dtype=np.float64) / hs))
    ang = np.arange(S, dtype=np.float64)[:, None] * freqs[None, :]
    w[off:off + S * hs // 2] = np.cos(ang).astype(np.float32).reshape(-1)
    w[off + S * hs // 2:] = np.sin(ang).astype(np.float32).reshape(-1)
    return w
