"""GGUF v3 StableLM checkpoints for the HIP forwarder (gguf.go:133-357).

``read_gguf`` parses and validates the container without loading weights:
little-endian v3 header, bounded counts and strings, metadata values
normalised to unsigned / signed 64-bit integers, floats, booleans, strings
and one level of arrays, tensor infos with GGUF's contiguous-first
dimensions reversed to row-major, type codes with their block-size rules,
and then alignment, bounds and overlap of every tensor. ``load_stablelm_gguf``
maps the metadata onto StableLMConfig, checks the vocabulary against the
tokenizer.json that must sit beside the file, and returns the tensors under
their Hugging Face names in file encoding, ready for
``hip.StableLMForwarder``. Error messages are the reference's.

Q4_K (type 12) is rejected like the reference does, unless ``q4_k=True``:
the HIP library implements Q4_K matrices as an extension.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import weights as W

MAGIC = 0x46554747
MAX_INT = (1 << 63) - 1


class U64(int):
    """A metadata integer read from an unsigned GGUF type (Go's uint64)."""


class I64(int):
    """A metadata integer read from a signed GGUF type (Go's int64)."""


@dataclass
class GGUFTensor:
    shape: list
    dtype: str
    offset: int  # absolute file position once read_gguf returns
    size: int


class _HeaderError(Exception):
    """A failed read inside the header (ggufReader.err), reported as
    "GGUF header: ..." once the header loops stop (gguf.go:219-221)."""


class _Reader:
    """Sequential little-endian reads over the first 64 MiB of the file
    (gguf.go:143-144)."""

    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n):
        if n > len(self.buf) - self.pos:
            raise _HeaderError("unexpected EOF")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def unpack(self, fmt):
        return struct.unpack("<" + fmt, self.take(struct.calcsize(fmt)))[0]

    def u32(self):
        return self.unpack("I")

    def u64(self):
        return self.unpack("Q")

    def str(self):
        n = self.u64()
        if n > 16 << 20:
            raise _HeaderError("GGUF string too large")
        return bytes(self.take(n)).decode("utf-8", "surrogateescape")

    def value(self, kind):
        """ggufReader.value (gguf.go:64-131)."""
        scalars = {0: ("B", U64), 1: ("b", I64), 2: ("H", U64), 3: ("h", I64), 4: ("I", U64), 5: ("i", I64),
                   10: ("Q", U64), 11: ("q", I64), 6: ("f", float), 12: ("d", float)}
        if kind in scalars:
            fmt, cast = scalars[kind]
            return cast(self.unpack(fmt))
        if kind == 7:
            v = self.unpack("B")
            if v > 1:
                raise _HeaderError("invalid GGUF boolean")
            return v == 1
        if kind == 8:
            return self.str()
        if kind == 9:
            inner, n = self.u32(), self.u64()
            if inner == 9 or n > 1 << 20:
                raise _HeaderError("unsupported GGUF array")
            return [self.value(inner) for _ in range(n)]
        raise _HeaderError(f"unsupported GGUF metadata type {kind}")


# type code -> (name, values per block, bytes per block, row multiple)
_TYPES = {0: ("F32", 1, 4, 0), 1: ("F16", 1, 2, 0), 30: ("BF16", 1, 2, 0), 8: ("Q8_0", 32, 34, 32),
          7: ("Q5_1", 32, 24, 32), 13: ("Q5_K", 256, 176, 256), 14: ("Q6_K", 256, 210, 256)}
_Q4_K = (12, ("Q4_K", 256, 144, 256))


def read_gguf(path: str, q4_k: bool = False):
    """readGGUF (gguf.go:133-248): (metadata, {name: GGUFTensor})."""
    size = os.path.getsize(path)
    types = dict(_TYPES)
    if q4_k:
        types[_Q4_K[0]] = _Q4_K[1]
    with open(path, "rb") as f:
        buf = f.read(min(size, 64 << 20))
    r = _Reader(memoryview(buf))

    def first(read):  # a failed read yields zero, as ggufReader's does
        try:
            return read()
        except _HeaderError:
            return 0

    if first(r.u32) != MAGIC or first(r.u32) != 3:
        raise ValueError("expected little-endian GGUF v3")
    n_tensors, n_meta = first(r.u64), first(r.u64)
    try:
        if n_tensors == 0 or n_tensors > 10000 or n_meta > 65536:
            raise ValueError("invalid GGUF counts")
        meta = {}
        for _ in range(n_meta):
            key = r.str()
            if key in meta:
                raise ValueError(f"duplicate GGUF key {key!r}")
            meta[key] = r.value(r.u32())
        tensors = {}
        for _ in range(n_tensors):
            name, rank = r.str(), r.u32()
            if rank == 0 or rank > 4:
                raise ValueError("invalid GGUF tensor rank")
            shape, n = [0] * rank, 1
            for j in range(rank):
                d = r.u64()
                if d == 0 or d > (MAX_INT // n) // 4:
                    raise ValueError("invalid GGUF tensor dimensions")
                n *= d
                shape[rank - 1 - j] = d  # GGUF stores the contiguous dimension first
            kind = r.u32()
            if kind not in types:
                raise ValueError(f"GGUF tensor {name}: unsupported type {kind}")
            dtype, per, nbytes, multiple = types[kind]
            if multiple and (rank != 2 or shape[1] % multiple):
                raise ValueError(f"{dtype} rows must be divisible by {multiple}" if per == 32
                                 else f"K-quant rows must be divisible by {multiple}")
            offset = r.u64()
            if offset > MAX_INT:
                raise ValueError("GGUF tensor too large")
            if name in tensors:
                raise ValueError(f"duplicate GGUF tensor {name!r}")
            tensors[name] = GGUFTensor(shape, dtype, offset, n // per * nbytes)
    except _HeaderError as e:
        raise ValueError(f"GGUF header: {e}") from None
    align = meta.get("general.alignment", U64(32))
    if not isinstance(align, U64):
        align = 0
    if align == 0 or align > 4096 or align & (align - 1):
        raise ValueError("invalid GGUF alignment")
    start = (r.pos + align - 1) & -align
    for name, t in tensors.items():
        if t.offset % align or start > size or t.offset > size - start or t.size > size - start - t.offset:
            raise ValueError(f"GGUF tensor {name} outside file or misaligned")
        t.offset += start
    ranges = sorted(tensors.values(), key=lambda t: t.offset)
    for a, b in zip(ranges, ranges[1:]):
        if b.offset < a.offset + a.size:
            raise ValueError("overlapping GGUF tensors")
    return meta, tensors


# ggufNames (gguf.go:250-255): Hugging Face name pieces -> GGUF name pieces
_NAME_PIECES = (("model.embed_tokens", "token_embd"), ("lm_head", "output"), ("model.norm", "output_norm"),
                ("model.layers.", "blk."), ("input_layernorm", "attn_norm"), ("self_attn.q_proj", "attn_q"),
                ("self_attn.k_proj", "attn_k"), ("self_attn.v_proj", "attn_v"), ("self_attn.o_proj", "attn_output"),
                ("mlp.gate_proj", "ffn_gate"), ("mlp.up_proj", "ffn_up"),
                ("mlp.down_proj", "ffn_down"))


def gguf_name(name: str) -> str:
    """strings.Replacer semantics for these pieces: scan left to right, at
    each position replace the first piece (in table order) that matches."""
    out, i = [], 0
    while i < len(name):
        for old, new in _NAME_PIECES:
            if name.startswith(old, i):
                out.append(new)
                i += len(old)
                break
        else:
            out.append(name[i])
            i += 1
    return "".join(out)


def tokenizer_pieces(path: str, vocab_size: int) -> list[str]:
    """The id -> piece table of a tokenizer.json's model.vocab (the
    vocabulary part of tokenizer.Parse, tokenizer/nerdstash.go:112-123);
    ids without a piece are empty strings."""
    with open(path, "rb") as f:
        vocab = json.load(f)["model"]["vocab"]
    pieces = [""] * vocab_size
    for piece, i in vocab.items():
        if not isinstance(i, int) or not 0 <= i < vocab_size or pieces[i] or piece == "":
            raise ValueError(f"invalid vocabulary entry {piece!r}: {i}")
        pieces[i] = piece
    return pieces


def load_stablelm_gguf(path: str, q4_k: bool = False):
    """loadStableGGUF (gguf.go:257-357): (validated config, {HF name: Tensor})."""
    meta, tensors = read_gguf(path, q4_k)
    if meta.get("general.architecture") != "stablelm" or meta.get("general.type", "model") != "model":
        raise ValueError("GGUF must contain a StableLM model")
    errors = []

    def integer(key):
        v = meta.get(key)
        if not isinstance(v, U64) or v > MAX_INT:
            errors.append(f"missing or invalid GGUF integer {key}")
            return 0
        return int(v)

    c = {"model_type": "stablelm", "hidden_act": "silu", "rope_theta": 10000.0,
         "hidden_size": integer("stablelm.embedding_length"),
         "intermediate_size": integer("stablelm.feed_forward_length"),
         "num_hidden_layers": integer("stablelm.block_count"),
         "num_attention_heads": integer("stablelm.attention.head_count"),
         "num_key_value_heads": integer("stablelm.attention.head_count_kv"),
         "max_position_embeddings": integer("stablelm.context_length"),
         "bos_token_id": integer("tokenizer.ggml.bos_token_id"),
         "eos_token_id": integer("tokenizer.ggml.eos_token_id"),
         "use_qkv_bias": False, "qk_layernorm": False, "tie_word_embeddings": False}
    v = meta.get("stablelm.use_parallel_residual")
    c["use_parallel_residual"] = v if isinstance(v, bool) else False
    v = meta.get("stablelm.attention.layer_norm_epsilon")
    c["layer_norm_eps"] = v if isinstance(v, float) else 0.0
    if "stablelm.rope.freq_base" in meta:
        v = meta["stablelm.rope.freq_base"]
        if not isinstance(v, float):
            raise ValueError("invalid GGUF RoPE frequency base")
        c["rope_theta"] = v
    c["partial_rotary_factor"] = 0.0
    if c["hidden_size"] > 0 and c["num_attention_heads"] > 0:
        c["partial_rotary_factor"] = (float(integer("stablelm.rope.dimension_count"))
                                      * float(c["num_attention_heads"]) / float(c["hidden_size"]))
    vocab = meta.get("tokenizer.ggml.tokens")
    if not isinstance(vocab, list):
        raise ValueError("GGUF missing vocabulary")
    c["vocab_size"] = len(vocab)
    if errors:
        raise ValueError(errors[-1])
    c = W.validate_stablelm_config(c)
    layers = c["num_hidden_layers"]
    if len(tensors) < 4 or (len(tensors) - 4) % 9 or (len(tensors) - 4) // 9 != layers:
        raise ValueError(f"unexpected GGUF tensor count for {layers} StableLM layers")
    if "stablelm.rope.scaling.type" in meta and meta["stablelm.rope.scaling.type"] != "none":
        raise ValueError("GGUF RoPE scaling is not supported")
    for name in tensors:
        if ("attn_q_norm" in name or "attn_k_norm" in name or "ffn_norm" in name
                or (name.endswith(".bias") and "norm" not in name)):
            raise ValueError(f"unsupported StableLM tensor {name}")
    try:
        pieces = tokenizer_pieces(os.path.join(os.path.dirname(path), "tokenizer.json"), c["vocab_size"])
    except (OSError, ValueError, KeyError) as e:
        raise ValueError(f"GGUF requires the original tokenizer.json beside it: {e}") from None
    types = meta.get("tokenizer.ggml.token_type")
    types = types if isinstance(types, list) else []
    for i, piece in enumerate(vocab):
        ok = isinstance(piece, str)
        if (ok and pieces[i] == "" and piece == f"[PAD{i}]" and len(types) == len(vocab)
                and isinstance(types[i], (U64, I64)) and types[i] == 5):
            continue  # GGUF pads an unused output row that has no tokenizer entry
        if not ok or (piece != pieces[i] and piece.replace(" ", "▁") != pieces[i]):
            raise ValueError(f"GGUF/tokenizer vocabulary mismatch at {i}")
    out = {}
    d, h = c["hidden_size"], c["intermediate_size"]
    kv = d // c["num_attention_heads"] * c["num_key_value_heads"]
    want = {"model.embed_tokens.weight": [c["vocab_size"], d], "lm_head.weight": [c["vocab_size"], d],
            "model.norm.weight": [d], "model.norm.bias": [d]}
    for i in range(layers):
        p = f"model.layers.{i}."
        want.update({p + "input_layernorm.weight": [d], p + "input_layernorm.bias": [d],
                     p + "self_attn.q_proj.weight": [d, d], p + "self_attn.k_proj.weight": [kv, d],
                     p + "self_attn.v_proj.weight": [kv, d], p + "self_attn.o_proj.weight": [d, d],
                     p + "mlp.gate_proj.weight": [h, d], p + "mlp.up_proj.weight": [h, d],
                     p + "mlp.down_proj.weight": [d, h]})
    with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        for name, shape in want.items():
            t = tensors.get(gguf_name(name))
            if t is None:
                raise ValueError(f"missing GGUF tensor {name}")
            if len(shape) != len(t.shape):
                raise ValueError(f"GGUF tensor {name} has wrong rank")
            if shape != t.shape:
                go = lambda v: "[" + " ".join(map(str, v)) + "]"  # noqa: E731 (Go's %v of []int)
                raise ValueError(f"GGUF tensor {name}: shape {go(t.shape)}, want {go(shape)}")
            rows, cols = (shape[0], shape[1]) if len(shape) == 2 else (1, shape[0])
            data = np.frombuffer(mm, np.uint8, t.size, t.offset).copy()
            out[name] = W.Tensor(W.NAME_DTYPES[t.dtype], rows, cols, data)
    return c, out
