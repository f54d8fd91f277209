"""ctypes binding of libtinyoai_hip.so (include/tinyoai_hip.h).

The library must have been built (``python -m tinyoai_amd.build`` or
``__graft_entry__.build()``); there is no CPU fallback: a missing or
unloadable library raises immediately.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import weights as W

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtinyoai_hip.so")

EXPORTS = [
    "tinyoai_last_error", "tinyoai_stablelm_load", "tinyoai_stablelm_forward", "tinyoai_stablelm_forward_logprobs",
    "tinyoai_stablelm_set_kv_bits", "tinyoai_summarize_logits",
    "tinyoai_stablelm_limit_cache", "tinyoai_stablelm_reset", "tinyoai_stablelm_offset", "tinyoai_stablelm_close",
    "tinyoai_stablelm_read_kv", "tinyoai_stablelm_kv_save", "tinyoai_stablelm_kv_load",
    "tinyoai_stablelm_trace", "tinyoai_stablelm_trace_read",
    "tinyoai_stablelm_trace_read_stages",
    "tinyoai_stablelm_set_launch", "tinyoai_stablelm_branches_open", "tinyoai_stablelm_branches_forward",
    "tinyoai_stablelm_branches_append", "tinyoai_stablelm_branches_length", "tinyoai_stablelm_branches_close",
    "tinyoai_stablelm_profile", "tinyoai_stablelm_profile_read", "tinyoai_llama_load",
    "tinyoai_llama_forward", "tinyoai_llama_reset", "tinyoai_llama_close", "tinyoai_llama_set_launch",
    "tinyoai_weight_upload",
    "tinyoai_weight_read_values", "tinyoai_weight_mul", "tinyoai_weight_mul_device",
    "tinyoai_weight_mul_device_noalloc", "tinyoai_weight_free",
]


class TinyoaiError(RuntimeError):
    pass


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int32), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p), ("nbytes", C.c_uint64)]


class StableLMConfig(C.Structure):
    _fields_ = [("vocab_size", C.c_int32), ("hidden_size", C.c_int32), ("intermediate_size", C.c_int32),
                ("num_hidden_layers", C.c_int32), ("num_attention_heads", C.c_int32),
                ("num_key_value_heads", C.c_int32), ("max_position_embeddings", C.c_int32),
                ("bos_token_id", C.c_int32), ("eos_token_id", C.c_int32), ("layer_norm_eps", C.c_double),
                ("rope_theta", C.c_double), ("partial_rotary_factor", C.c_double)]


class LlamaConfig(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden_dim", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32),
                ("n_kv_heads", C.c_int32), ("vocab_size", C.c_int32), ("seq_len", C.c_int32)]


_lib = None


def lib():
    """Loads the HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TinyoaiError(f"{LIB_PATH} is missing: build it with `python -m tinyoai_amd.build`")
        L = C.CDLL(LIB_PATH)
        P, fp, ip = C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_int32)
        L.tinyoai_last_error.restype = C.c_char_p
        L.tinyoai_stablelm_load.argtypes = [C.POINTER(StableLMConfig), C.POINTER(Tensor), C.c_int32, C.POINTER(P)]
        L.tinyoai_stablelm_forward.argtypes = [P, C.c_int32, ip, C.c_int32, C.c_int32, fp]
        dp = C.POINTER(C.c_double)
        L.tinyoai_stablelm_forward_logprobs.argtypes = [P, C.c_int32, ip, ip, C.c_int32, C.c_int32, fp, dp, ip, dp]
        L.tinyoai_stablelm_set_kv_bits.argtypes = [P, C.c_int32, ip]
        L.tinyoai_summarize_logits.argtypes = [fp, C.c_int32, C.c_int32, ip, C.c_int32, dp, ip, dp]
        L.tinyoai_stablelm_limit_cache.argtypes = [P, C.c_int32, ip]
        L.tinyoai_stablelm_reset.argtypes = [P]
        L.tinyoai_stablelm_offset.argtypes = [P]
        L.tinyoai_stablelm_close.argtypes = [P]
        L.tinyoai_stablelm_read_kv.argtypes = [P, C.c_int32, C.c_int32, C.c_int32, fp, fp]
        L.tinyoai_stablelm_kv_save.argtypes = [P, C.c_int32, C.c_int32, P, C.c_uint64]
        L.tinyoai_stablelm_kv_load.argtypes = [P, C.c_int32, C.c_int32, P, C.c_uint64]
        L.tinyoai_stablelm_trace.argtypes = [P, C.c_int32]
        L.tinyoai_stablelm_trace_read.argtypes = [P, fp]
        L.tinyoai_stablelm_trace_read_stages.argtypes = [P, fp, fp]
        L.tinyoai_stablelm_set_launch.argtypes = [P, C.c_int32, C.c_int32, C.c_int32]
        L.tinyoai_stablelm_branches_open.argtypes = [P, C.c_int32, C.c_int32, C.c_int32, C.POINTER(P)]
        L.tinyoai_stablelm_branches_forward.argtypes = [P, ip, C.c_int32, fp]
        L.tinyoai_stablelm_branches_append.argtypes = [P, ip, ip, C.c_int32, fp]
        L.tinyoai_stablelm_branches_length.argtypes = [P, C.c_int32]
        L.tinyoai_stablelm_branches_close.argtypes = [P]
        L.tinyoai_stablelm_profile.argtypes = [P, C.c_int32]
        L.tinyoai_stablelm_profile_read.argtypes = [P, C.POINTER(C.c_double), C.POINTER(C.c_int64), C.c_int32]
        L.tinyoai_llama_load.argtypes = [C.POINTER(LlamaConfig), fp, C.c_uint64, C.POINTER(P)]
        L.tinyoai_llama_forward.argtypes = [P, C.c_int32, ip, C.c_int32, C.c_int32, fp]
        L.tinyoai_llama_reset.argtypes = [P]
        L.tinyoai_llama_close.argtypes = [P]
        L.tinyoai_llama_set_launch.argtypes = [P, C.c_int32, C.c_int32]
        L.tinyoai_weight_upload.argtypes = [C.c_int32, C.c_int64, C.c_int64, P, C.c_uint64, C.POINTER(P)]
        L.tinyoai_weight_read_values.argtypes = [P, C.c_int64, C.c_int64, fp]
        L.tinyoai_weight_mul.argtypes = [P, fp, C.c_int32, fp]
        L.tinyoai_weight_mul_device.argtypes = [P, P, C.c_int32, P, P]
        L.tinyoai_weight_mul_device_noalloc.argtypes = [P, P, C.c_int32, P, P]
        L.tinyoai_weight_free.argtypes = [P]
        _lib = L
    return _lib


def check(rc: int) -> int:
    if rc < 0:
        raise TinyoaiError(lib().tinyoai_last_error().decode(errors="replace"))
    return rc


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _ip(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def summarize_logits(logits: np.ndarray, targets, count: int):
    """summarizeLogits (logprobs.go:60-95) on the device for rows of logits
    [rows][vocab]: (chosen [rows], top ids [rows][count], top log
    probabilities [rows][count])."""
    x = np.ascontiguousarray(np.atleast_2d(logits), np.float32)
    tg = np.ascontiguousarray(targets, np.int32)
    rows, vocab = x.shape
    chosen = np.empty(rows, np.float64)
    ids = np.empty((rows, count), np.int32)
    lp = np.empty((rows, count), np.float64)
    dp = C.POINTER(C.c_double)
    check(lib().tinyoai_summarize_logits(_fp(x), rows, vocab, _ip(tg), count, chosen.ctypes.data_as(dp), _ip(ids),
                                         lp.ctypes.data_as(dp)))
    return chosen, ids, lp


class Weight:
    """One weight matrix in HBM (weightTensor, safetensors.go:193-280)."""

    def __init__(self, t: W.Tensor):
        self.rows, self.cols, self.dtype = t.rows, t.cols, t.dtype
        h = C.c_void_p()
        check(lib().tinyoai_weight_upload(t.dtype, t.rows, t.cols, t.data.ctypes.data, t.data.size, C.byref(h)))
        self.h = h

    def read_values(self, offset: int, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        check(lib().tinyoai_weight_read_values(self.h, offset, n, _fp(out)))
        return out

    def mul(self, x: np.ndarray) -> np.ndarray:
        """x [n, cols] -> [n, rows] (mulScratch for n == 1, mulBatch otherwise)."""
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        out = np.empty((x.shape[0], self.rows), np.float32)
        check(lib().tinyoai_weight_mul(self.h, _fp(x), x.shape[0], _fp(out)))
        return out

    def mul_device(self, x_ptr: int, n: int, out_ptr: int, stream: int = 0) -> None:
        check(lib().tinyoai_weight_mul_device(self.h, x_ptr, n, out_ptr, stream or None))

    def mul_device_noalloc(self, x_ptr: int, n: int, out_ptr: int, stream: int = 0) -> None:
        """mul_device without any allocation (operand planes in the
        library's per-GPU array; n * cols <= 4,194,304)."""
        check(lib().tinyoai_weight_mul_device_noalloc(self.h, x_ptr, n, out_ptr, stream or None))

    def close(self):
        if self.h:
            lib().tinyoai_weight_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


STABLELM_TENSORS = ("model.embed_tokens.weight", "lm_head.weight", "model.norm.weight", "model.norm.bias")
LAYER_TENSORS = ("input_layernorm.weight", "input_layernorm.bias", "self_attn.q_proj.weight",
                 "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                 "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")


class Branches:
    """nativeBranches (mlx_branches.go:14-182) over the C ABI: forward() takes
    one token per branch (branch j at position prefix + length(j)) and
    returns the logits rows [count][vocab]; append() gives each branch a
    private suffix of its own length. The session borrows its forwarder's
    prefix, so it keeps the forwarder alive; close it before the forwarder."""

    def __init__(self, fwd, prefix: int, count: int, max_len: int = 0):
        self.h = C.c_void_p()
        self.fwd = fwd
        self.count = count
        self.vocab = fwd.config["vocab_size"]
        check(lib().tinyoai_stablelm_branches_open(fwd.h, prefix, count, max_len, C.byref(self.h)))
        self._logits = np.empty((count, self.vocab), np.float32)

    def _out(self, out):
        """The caller's float32 [count][vocab] C-contiguous array, or None."""
        if out is None:
            return None
        if out.dtype != np.float32 or out.shape != (self.count, self.vocab) or not out.flags.c_contiguous:
            raise ValueError(f"out must be a C-contiguous float32 array of shape {(self.count, self.vocab)}")
        return out

    def forward(self, tokens, out=None) -> np.ndarray:
        """One token per branch; returns the logits rows [count][vocab], in a
        new array or, with `out`, written into it (no copy)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        dst = self._out(out)
        buf = self._logits if dst is None else dst
        check(lib().tinyoai_stablelm_branches_forward(self.h, _ip(toks), toks.size, _fp(buf)))
        return buf.copy() if dst is None else dst

    def append(self, suffixes, out=None) -> np.ndarray:
        """Appends suffixes[j] (a nonempty id sequence) to branch j; returns
        each branch's last-row logits [count][vocab] (into `out` as forward
        does)."""
        lengths = np.array([len(x) for x in suffixes], np.int32)
        toks = np.ascontiguousarray(np.concatenate([np.asarray(x, np.int32) for x in suffixes]), np.int32)
        dst = self._out(out)
        buf = self._logits if dst is None else dst
        check(lib().tinyoai_stablelm_branches_append(self.h, _ip(toks), _ip(lengths), lengths.size, _fp(buf)))
        return buf.copy() if dst is None else dst

    def length(self, branch: int) -> int:
        return check(lib().tinyoai_stablelm_branches_length(self.h, branch))

    def close(self):
        if self.h:
            lib().tinyoai_stablelm_branches_close(self.h)
            self.h = None
        self.fwd = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class StableLMForwarder:
    """The HIP StableLM forwarder: the mlxForwarder contract (mlx.go:45-51)
    plus SetKVBits / LimitCache (mlx_kv.go:78-91, mlx_native.go:231-244)."""

    def __init__(self, config: dict, tensors: dict):
        c = W.validate_stablelm_config(config)
        self.config = c
        self.vocab = c["vocab_size"]
        cfg = StableLMConfig(c["vocab_size"], c["hidden_size"], c["intermediate_size"], c["num_hidden_layers"],
                             c["num_attention_heads"], c["num_key_value_heads"], c["max_position_embeddings"],
                             c.get("bos_token_id", 0), c.get("eos_token_id", 0), c["layer_norm_eps"],
                             c["rope_theta"], c["partial_rotary_factor"])
        names = list(STABLELM_TENSORS) + [f"model.layers.{i}.{n}" for i in range(c["num_hidden_layers"])
                                          for n in LAYER_TENSORS]
        arr = (Tensor * len(names))()
        keep = []
        for i, n in enumerate(names):
            t = tensors[n]
            b = n.encode()
            keep.append(b)
            arr[i] = Tensor(b, t.dtype, t.rows, t.cols, t.data.ctypes.data, t.data.size)
        h = C.c_void_p()
        check(lib().tinyoai_stablelm_load(C.byref(cfg), arr, len(names), C.byref(h)))
        self.h = h
        self.kv_half = False
        self._logits = np.empty(self.vocab, np.float32)

    def forward(self, prefix: int, tokens, want_logits: bool = True) -> np.ndarray | None:
        toks = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.vocab, np.float32) if want_logits else self._logits  # the caller's own copy
        check(lib().tinyoai_stablelm_forward(self.h, prefix, _ip(toks), toks.size, int(want_logits), _fp(out)))
        return out if want_logits else None

    def forward_with_logprobs(self, prefix: int, tokens, targets, count: int):
        """ForwardWithLogprobs (mlx.go:53-57): the forward of `tokens` after
        `prefix`, scoring position i against targets[i]. Returns (last
        logits [vocab], chosen [n] float64, top ids [n][count], top log
        probabilities [n][count] float64)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        tg = np.ascontiguousarray(targets, np.int32)
        n = toks.size
        if tg.size != n:  # the C entry point takes one count for both (mlx_native.go:303-305)
            raise TinyoaiError("invalid probability request: targets do not align with tokens")
        logits = np.empty(self.vocab, np.float32)
        chosen = np.empty(n, np.float64)
        ids = np.empty((n, count), np.int32)
        lp = np.empty((n, count), np.float64)
        dp = C.POINTER(C.c_double)
        check(lib().tinyoai_stablelm_forward_logprobs(self.h, prefix, _ip(toks), _ip(tg), n, count, _fp(logits),
                                                      chosen.ctypes.data_as(dp), _ip(ids), lp.ctypes.data_as(dp)))
        return logits, chosen, ids, lp

    def new_branches(self, prefix: int, count: int, max_len: int = 0) -> "Branches":
        """NewBranches (mlx_branches.go:25-33): `count` suffixes borrowing
        the resident prefix [0, prefix), each at most `max_len` tokens long
        (0: up to the context). Close them before this forwarder."""
        return Branches(self, prefix, count, max_len)

    def set_kv_bits(self, bits: int) -> bool:
        cleared = C.c_int32()
        check(lib().tinyoai_stablelm_set_kv_bits(self.h, bits, C.byref(cleared)))
        self.kv_half = bits == 16
        return bool(cleared.value)

    def limit_cache(self, limit: int) -> bool:
        cleared = C.c_int32()
        check(lib().tinyoai_stablelm_limit_cache(self.h, limit, C.byref(cleared)))
        return bool(cleared.value)

    def reset(self) -> None:
        check(lib().tinyoai_stablelm_reset(self.h))

    @property
    def offset(self) -> int:
        return check(lib().tinyoai_stablelm_offset(self.h))

    def read_kv(self, layer: int, kv_head: int, n: int):
        hd = self.config["hidden_size"] // self.config["num_attention_heads"]
        k = np.empty(n * hd, np.float32)
        v = np.empty(n * hd, np.float32)
        check(lib().tinyoai_stablelm_read_kv(self.h, layer, kv_head, n, _fp(k), _fp(v)))
        return k.reshape(n, hd), v.reshape(n, hd)

    def kv_payload_bytes(self, n: int, half: bool) -> int:
        c = self.config
        hd = c["hidden_size"] // c["num_attention_heads"]
        return c["num_hidden_layers"] * c["num_key_value_heads"] * 2 * n * hd * (2 if half else 4)

    def kv_save(self, n: int, half: bool) -> bytes:
        """The cachePayload bytes of resident positions [0, n)."""
        buf = np.empty(self.kv_payload_bytes(n, half), np.uint8)
        check(lib().tinyoai_stablelm_kv_save(self.h, n, int(half), buf.ctypes.data, buf.size))
        return buf.tobytes()

    def kv_load(self, n: int, half: bool, payload: bytes) -> None:
        """Replaces the resident cache with a cachePayload of n positions."""
        buf = np.frombuffer(payload, np.uint8)
        check(lib().tinyoai_stablelm_kv_load(self.h, n, int(half), buf.ctypes.data, buf.size))

    def trace(self, enable: bool = True) -> None:
        check(lib().tinyoai_stablelm_trace(self.h, int(enable)))

    def trace_read(self) -> np.ndarray:
        c = self.config
        out = np.empty((c["num_hidden_layers"], c["hidden_size"]), np.float32)
        check(lib().tinyoai_stablelm_trace_read(self.h, _fp(out)))
        return out

    def trace_read_stages(self) -> tuple[np.ndarray, np.ndarray]:
        """Per-layer attention outputs [layers][heads * head_dim] and
        SiLU-gate outputs [layers][intermediate] of the traced token."""
        c = self.config
        L = c["num_hidden_layers"]
        att = np.empty((L, c["hidden_size"]), np.float32)
        gate = np.empty((L, c["intermediate_size"]), np.float32)
        check(lib().tinyoai_stablelm_trace_read_stages(self.h, _fp(att), _fp(gate)))
        return att, gate

    STAGES = ("embedding", "decode_in", "attention", "decode_out", "lm_head", "prefill_layer_norm",
              "prefill_projections", "prefill_epilogue", "prefill_attention", "prefill_elementwise")

    LAUNCH_STAGES = {"decode_in": 0, "decode_out": 1, "lm_head": 2, "attention": 3, "fused_attention": 4,
                     "bf16_activations": 5, "wide": 7, "wide_epilogue": 8, "flash_key_split": 9, "q8_wide": 10,
                     "kq_pair": 11}

    def set_launch(self, stage: str, grid: int, threads: int) -> None:
        """Launch shape (blocks, threads per block) of a decode matrix
        kernel (results do not depend on it), or a switch (stages
        "fused_attention", "bf16_activations", "wide", "wide_epilogue",
        "flash_key_split", "q8_wide" and "kq_pair": grid nonzero = on)."""
        check(lib().tinyoai_stablelm_set_launch(self.h, self.LAUNCH_STAGES[stage], int(grid), int(threads)))

    def profile(self, enable: bool = True) -> None:
        check(lib().tinyoai_stablelm_profile(self.h, int(enable)))

    def profile_read(self) -> dict:
        n = len(self.STAGES)
        ms = (C.c_double * n)()
        counts = (C.c_int64 * n)()
        check(lib().tinyoai_stablelm_profile_read(self.h, ms, counts, n))
        return {s: (ms[i], counts[i]) for i, s in enumerate(self.STAGES)}

    def close(self) -> None:
        if self.h:
            lib().tinyoai_stablelm_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LlamaForwarder:
    """The legacy Llama forwarder (llamaMLXForwarder, mlx_llama.go:27-35)
    over a llama2.c checkpoint payload in readWeights order."""

    def __init__(self, config: dict, weights: np.ndarray):
        c = config
        self.config = c
        cfg = LlamaConfig(c["dim"], c["hidden_dim"], c["n_layers"], c["n_heads"], c["n_kv_heads"],
                          c["vocab_size"], c["seq_len"])
        w = np.ascontiguousarray(weights, np.float32)
        h = C.c_void_p()
        check(lib().tinyoai_llama_load(C.byref(cfg), _fp(w), w.size, C.byref(h)))
        self.h = h

    def forward(self, prefix: int, tokens, all_logits: bool = False) -> np.ndarray:
        """Forward (mlx_llama_native.go:119-175): every row [n][vocab] when
        all_logits, else the last row [vocab]."""
        ids = np.ascontiguousarray(tokens, np.int32)
        rows = ids.size if all_logits else 1
        out = np.empty((rows, self.config["vocab_size"]), np.float32)
        check(lib().tinyoai_llama_forward(self.h, prefix, _ip(ids), ids.size, int(all_logits), _fp(out)))
        return out if all_logits else out[0]

    def reset(self) -> None:
        check(lib().tinyoai_llama_reset(self.h))

    LAUNCH_STAGES = {"single_launch": 0}

    def set_launch(self, stage: str, value: int) -> None:
        """Stage "single_launch": nonzero (the default for stories260K-shaped
        models) runs every token of a forward in one launch, zero five
        kernels per layer and token."""
        check(lib().tinyoai_llama_set_launch(self.h, self.LAUNCH_STAGES[stage], int(value)))

    def close(self) -> None:
        if self.h:
            lib().tinyoai_llama_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
