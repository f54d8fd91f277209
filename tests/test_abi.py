"""The C ABI loads on a machine without a GPU and exports every entry point
that include/tinyoai_hip.h declares. No compute calls are made here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    with open(os.path.join(ROOT, "include", "tinyoai_hip.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(tinyoai_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from tinyoai_amd import hip
    assert declared_functions() == sorted(hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    from tinyoai_amd import hip
    if not os.path.exists(hip.LIB_PATH):
        pytest.fail(f"{hip.LIB_PATH} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(hip.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from tinyoai_amd import hip
    monkeypatch.setattr(hip, "_lib", None)
    monkeypatch.setattr(hip, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(hip.TinyoaiError):
        hip.lib()


def test_closed_handles_fail_cleanly():
    """Calls on absent handles return TINYOAI_EINVAL with a message and make
    no device call (nativeBranches.Forward after Close fails, Close is
    idempotent: mlx_branches.go:36-47, 136-139)."""
    from tinyoai_amd import hip
    L = hip.lib()
    toks = (ctypes.c_int32 * 2)(1, 2)
    out = (ctypes.c_float * 2)()
    assert L.tinyoai_stablelm_branches_forward(None, toks, 2, out) == -1
    assert b"closed" in L.tinyoai_last_error()
    assert L.tinyoai_stablelm_branches_append(None, toks, toks, 2, out) == -1
    assert L.tinyoai_stablelm_branches_length(None, 0) == -1
    assert L.tinyoai_stablelm_branches_close(None) == 0
    assert L.tinyoai_stablelm_close(None) == 0
    assert L.tinyoai_stablelm_forward(None, 0, toks, 2, 1, out) == -1
    cleared = ctypes.c_int32()
    assert L.tinyoai_stablelm_set_kv_bits(None, 16, ctypes.byref(cleared)) == -1
