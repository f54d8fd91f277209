"""ctypes view of the CPU oracle (oracle/oracle.c) -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline``
leg, as the checker or the timed CPU baseline. The product path never imports
this module. The restated reference functions are documented in oracle.c.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")

F32, F16, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 7, 8, 12, 13, 14, 30


class Weight(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p)]


class StableLMConfig(C.Structure):
    _fields_ = [("vocab_size", C.c_int32), ("hidden_size", C.c_int32),
                ("intermediate_size", C.c_int32), ("num_hidden_layers", C.c_int32),
                ("num_attention_heads", C.c_int32), ("num_key_value_heads", C.c_int32),
                ("max_position_embeddings", C.c_int32), ("bos_token_id", C.c_int32),
                ("eos_token_id", C.c_int32), ("layer_norm_eps", C.c_double),
                ("rope_theta", C.c_double), ("partial_rotary_factor", C.c_double)]


class LlamaConfig(C.Structure):
    _fields_ = [("dim", C.c_int32), ("hidden_dim", C.c_int32), ("n_layers", C.c_int32),
                ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("vocab_size", C.c_int32),
                ("seq_len", C.c_int32)]


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        fp = C.POINTER(C.c_float)
        L.or_half_float.restype = C.c_float
        L.or_half_float.argtypes = [C.c_uint16]
        L.or_float_half.restype = C.c_uint16
        L.or_float_half.argtypes = [C.c_float]
        L.or_read_values.argtypes = [C.POINTER(Weight), C.c_int64, C.c_int64, fp]
        L.or_mul.argtypes = [C.POINTER(Weight), fp, fp]
        L.or_mul_batch.argtypes = [C.POINTER(Weight), fp, C.c_int, fp]
        L.or_layer_norm.argtypes = [fp, fp, C.c_int, C.POINTER(Weight), C.POINTER(Weight), C.c_double]
        L.or_stable_rotate.argtypes = [fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double]
        L.or_softmax.argtypes = [fp, C.c_int]
        L.or_argmax.argtypes = [fp, C.c_int]
        L.or_argmax.restype = C.c_int
        L.or_set_threads.argtypes = [C.c_int]
        L.or_get_threads.restype = C.c_int
        L.or_stablelm_create.restype = C.c_void_p
        L.or_stablelm_create.argtypes = [C.POINTER(StableLMConfig), C.POINTER(Weight), C.c_int,
                                         C.c_int, C.c_int]
        L.or_stablelm_destroy.argtypes = [C.c_void_p]
        L.or_stablelm_forward.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, fp]
        L.or_stablelm_prefill.argtypes = [C.c_void_p, C.POINTER(C.c_int32), C.c_int, C.c_int, fp]
        L.or_stablelm_read_kv.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, fp, fp]
        L.or_stablelm_trace.argtypes = [C.c_void_p, C.c_int]
        L.or_stablelm_trace_data.restype = fp
        L.or_stablelm_trace_data.argtypes = [C.c_void_p]
        L.or_llama_create.restype = C.c_void_p
        L.or_llama_create.argtypes = [C.POINTER(LlamaConfig), fp, C.c_size_t]
        L.or_llama_destroy.argtypes = [C.c_void_p]
        L.or_llama_transformer.argtypes = [C.c_void_p, C.c_int, C.c_int, fp]
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def weight(dtype: int, rows: int, cols: int, data: np.ndarray) -> Weight:
    data = np.ascontiguousarray(data)
    w = Weight(dtype, rows, cols, data.ctypes.data)
    w._keep = data  # keep the buffer alive with the struct
    return w


def half_float(h: int) -> float:
    return lib().or_half_float(h)


def float_half(v: float) -> int:
    return lib().or_float_half(v)


def read_values(w: Weight, offset: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_read_values(C.byref(w), offset, n, _fp(out))
    return out


def mul(w: Weight, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(w.rows, np.float32)
    lib().or_mul(C.byref(w), _fp(x), _fp(out))
    return out


def mul_batch(w: Weight, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[0]
    out = np.empty((n, w.rows), np.float32)
    lib().or_mul_batch(C.byref(w), _fp(x), n, _fp(out))
    return out


def layer_norm(x: np.ndarray, w: Weight, b: Weight, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().or_layer_norm(_fp(out), _fp(x), x.size, C.byref(w), C.byref(b), eps)
    return out


def stable_rotate(x: np.ndarray, head: int, rotary: int, pos: int, theta: float) -> np.ndarray:
    x = np.array(x, np.float32)
    lib().or_stable_rotate(_fp(x), x.size, head, rotary, pos, theta)
    return x


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.array(x, np.float32)
    lib().or_softmax(_fp(x), x.size)
    return x


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return lib().or_argmax(_fp(x), x.size)


class StableLM:
    """The oracle StableLM engine over a dict of on-disk tensors.

    ``tensors`` maps Hugging Face names to (dtype, rows, cols, bytes) as in
    ``tinyoai_amd.weights``; ``capacity`` is the KV capacity in positions.
    """

    def __init__(self, config: dict, tensors: dict, half_kv: bool = False, capacity: int | None = None):
        c = config
        self.config = c
        self.capacity = capacity or c["max_position_embeddings"]
        cfg = StableLMConfig(c["vocab_size"], c["hidden_size"], c["intermediate_size"],
                             c["num_hidden_layers"], c["num_attention_heads"],
                             c["num_key_value_heads"], c["max_position_embeddings"],
                             c.get("bos_token_id", 0), c.get("eos_token_id", 0),
                             c.get("layer_norm_eps", 1e-5), c.get("rope_theta", 10000.0),
                             c.get("partial_rotary_factor", 0.25))
        names = ["model.embed_tokens.weight", "lm_head.weight", "model.norm.weight", "model.norm.bias"]
        for i in range(c["num_hidden_layers"]):
            p = f"model.layers.{i}."
            names += [p + "input_layernorm.weight", p + "input_layernorm.bias",
                      p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                      p + "self_attn.v_proj.weight", p + "self_attn.o_proj.weight",
                      p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", p + "mlp.down_proj.weight"]
        arr = (Weight * len(names))()
        self._keep = []
        for i, n in enumerate(names):
            t = tensors[n]
            data = np.ascontiguousarray(t.data)
            self._keep.append(data)
            arr[i] = Weight(t.dtype, t.rows, t.cols, data.ctypes.data)
        self._arr = arr
        self.h = lib().or_stablelm_create(C.byref(cfg), arr, len(names), int(half_kv), self.capacity)
        if not self.h:
            raise ValueError("oracle rejected the StableLM configuration")
        self.vocab = c["vocab_size"]

    def close(self):
        if self.h:
            lib().or_stablelm_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def forward(self, token: int, pos: int, want_logits: bool = True) -> np.ndarray:
        logits = np.zeros(self.vocab, np.float32)
        if lib().or_stablelm_forward(self.h, token, pos, int(want_logits), _fp(logits)):
            raise ValueError("oracle forward rejected its arguments")
        return logits

    def prefill(self, ids, start: int) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        logits = np.zeros(self.vocab, np.float32)
        if lib().or_stablelm_prefill(self.h, ids.ctypes.data_as(C.POINTER(C.c_int32)), ids.size,
                                     start, _fp(logits)):
            raise ValueError("oracle prefill rejected its arguments")
        return logits

    def read_kv(self, layer: int, head: int, n: int):
        hd = self.config["hidden_size"] // self.config["num_attention_heads"]
        k = np.empty(n * hd, np.float32)
        v = np.empty(n * hd, np.float32)
        lib().or_stablelm_read_kv(self.h, layer, head, n, _fp(k), _fp(v))
        return k.reshape(n, hd), v.reshape(n, hd)

    def trace(self, enable: bool = True):
        lib().or_stablelm_trace(self.h, int(enable))

    def trace_data(self) -> np.ndarray:
        c = self.config
        n = c["num_hidden_layers"] * c["hidden_size"]
        p = lib().or_stablelm_trace_data(self.h)
        return np.ctypeslib.as_array(p, shape=(n,)).copy().reshape(c["num_hidden_layers"], c["hidden_size"])


class Llama:
    """The oracle legacy-Llama engine over a llama2.c checkpoint payload."""

    def __init__(self, config: dict, weights: np.ndarray):
        c = config
        self.config = c
        cfg = LlamaConfig(c["dim"], c["hidden_dim"], c["n_layers"], c["n_heads"], c["n_kv_heads"],
                          c["vocab_size"], c["seq_len"])
        self._w = np.ascontiguousarray(weights, np.float32)
        self.h = lib().or_llama_create(C.byref(cfg), _fp(self._w), self._w.size)
        if not self.h:
            raise ValueError("oracle rejected the Llama checkpoint layout")

    def close(self):
        if self.h:
            lib().or_llama_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def transformer(self, token: int, pos: int) -> np.ndarray:
        logits = np.empty(self.config["vocab_size"], np.float32)
        if lib().or_llama_transformer(self.h, token, pos, _fp(logits)):
            raise ValueError("oracle transformer rejected its arguments")
        return logits
