"""An independent GGUF v3 writer for the tests (the layout ggufFixture
writes, gguf_test.go:19-138): sorted metadata keys, tensors sorted by name
with their dimensions written contiguous-first, data at 32-byte aligned
offsets after a header padded to 32 bytes."""
import json
import os
import shutil
import struct

import numpy as np

from tinyoai_amd import weights as W

# metadata value kinds: (GGUF type code, struct format)
U32, I32, F64, BOOL, STR = "u32", "i32", "f64", "bool", "str"
_CODES = {"F32": 0, "F16": 1, "BF16": 30, "Q8_0": 8, "Q5_K": 13, "Q6_K": 14, "Q5_1": 7, "Q4_K": 12}
HF_TO_GGUF = [("model.embed_tokens", "token_embd"), ("lm_head", "output"), ("model.norm", "output_norm"),
              ("model.layers.", "blk."), ("input_layernorm", "attn_norm"), ("self_attn.q_proj", "attn_q"),
              ("self_attn.k_proj", "attn_k"), ("self_attn.v_proj", "attn_v"), ("self_attn.o_proj", "attn_output"),
              ("mlp.gate_proj", "ffn_gate"), ("mlp.up_proj", "ffn_up"), ("mlp.down_proj", "ffn_down")]


def to_gguf_name(name):
    for a, b in HF_TO_GGUF:
        name = name.replace(a, b)
    return name


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind, v):
    if kind == STR:
        return struct.pack("<I", 8) + _str(v)
    if kind == U32:
        return struct.pack("<II", 4, v)
    if kind == I32:
        return struct.pack("<Ii", 5, v)
    if kind == F64:
        return struct.pack("<Id", 12, v)
    if kind == BOOL:
        return struct.pack("<IB", 7, int(v))
    if kind == ("arr", STR):
        return struct.pack("<IIQ", 9, 8, len(v)) + b"".join(_str(s) for s in v)
    if kind == ("arr", I32):
        return struct.pack("<IIQ", 9, 5, len(v)) + np.asarray(v, "<i4").tobytes()
    raise ValueError(kind)


def write_gguf(path, meta, tensors):
    """meta: {key: (kind, value)}; tensors: {gguf name: (dtype name, shape
    row-major, bytes)}."""
    head = bytearray(struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(meta)))
    for key in sorted(meta):
        kind, v = meta[key]
        head += _str(key) + _value(kind, v)
    body = bytearray()
    for name in sorted(tensors):
        dtype, shape, data = tensors[name]
        head += _str(name) + struct.pack("<I", len(shape))
        for d in reversed(shape):
            head += struct.pack("<Q", d)
        head += struct.pack("<IQ", _CODES.get(dtype, 99), len(body))
        body += bytes(data)
        body += bytes(-len(body) % 32)
    head += bytes(-len(head) % 32)
    with open(path, "wb") as f:
        f.write(head + body)


def go_shape(name, t):
    """The reference's declared shape: [d] for the norm vectors."""
    return [t.cols] if "norm" in name else [t.rows, t.cols]


def stablelm_gguf(directory, config, tensors, pieces, tokenizer=None, edit=None):
    """The tiny-fixture layout of ggufFixture: StableLM metadata from
    `config`, the vocabulary `pieces`, every tensor under its GGUF name;
    `edit(meta, tensors)` alters either before writing. The tokenizer.json
    beside the file is copied from `tokenizer`, or written from `pieces`."""
    c = config
    hd = c["hidden_size"] // c["num_attention_heads"]
    meta = {
        "general.architecture": (STR, "stablelm"), "stablelm.embedding_length": (U32, c["hidden_size"]),
        "stablelm.feed_forward_length": (U32, c["intermediate_size"]),
        "stablelm.block_count": (U32, c["num_hidden_layers"]),
        "stablelm.attention.head_count": (U32, c["num_attention_heads"]),
        "stablelm.attention.head_count_kv": (U32, c["num_key_value_heads"]),
        "stablelm.context_length": (U32, c["max_position_embeddings"]),
        "stablelm.rope.dimension_count": (U32, int(hd * c["partial_rotary_factor"])),
        "stablelm.use_parallel_residual": (BOOL, True),
        "stablelm.attention.layer_norm_epsilon": (F64, c["layer_norm_eps"]),
        "tokenizer.ggml.bos_token_id": (U32, c["bos_token_id"]),
        "tokenizer.ggml.eos_token_id": (U32, c["eos_token_id"]),
        "tokenizer.ggml.tokens": (("arr", STR), list(pieces)),
    }
    if c["rope_theta"] != 10000:
        meta["stablelm.rope.freq_base"] = (F64, c["rope_theta"])
    ts = {to_gguf_name(n): (W.DTYPE_NAMES[t.dtype], go_shape(n, t), t.data.tobytes()) for n, t in tensors.items()}
    if edit:
        edit(meta, ts)
    os.makedirs(directory, exist_ok=True)
    if tokenizer:
        shutil.copy(tokenizer, os.path.join(directory, "tokenizer.json"))
    else:
        with open(os.path.join(directory, "tokenizer.json"), "w") as f:
            json.dump({"model": {"vocab": {p: i for i, p in enumerate(pieces) if p}}}, f)
    path = os.path.join(directory, "model.gguf")
    write_gguf(path, meta, ts)
    return path
