"""The C-ABI library loads and exports exactly what include/nva.h declares (no GPU needed)."""

import ctypes
import os
import re
import subprocess

import pytest

from nanollvm_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nva.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nva_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for name in ("nva_ctx_create", "nva_kv_create", "nva_step_set", "nva_rope_forward",
                 "nva_attention_forward", "nva_rope_attention_forward"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    lib = N.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", N.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (nva_[a-z_0-9]+)", out))
    assert exported == set(declared_symbols())


def test_python_binding_covers_the_header():
    assert set(N.SIGNATURES) == set(declared_symbols())


def test_status_strings():
    lib = N.load()
    assert lib.nva_status_string(N.NVA_OK) == b"ok"
    assert lib.nva_status_string(N.NVA_E_ROPE_POS) == b"RoPE position out of range"


def test_null_arguments_are_rejected_without_a_device():
    lib = N.load()
    assert lib.nva_ctx_create(0, None) == N.NVA_E_ARG
    assert lib.nva_ctx_sync(None) == N.NVA_E_ARG
    assert lib.nva_kv_layer(None, 0, None, None, None) == N.NVA_E_ARG
    assert lib.nva_ctx_destroy(None) == N.NVA_OK
    assert lib.nva_last_error(None) == b"null context"


def test_no_device_fails_loudly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = N.load()
    h = ctypes.c_void_p()
    assert lib.nva_ctx_create(0, ctypes.byref(h)) == N.NVA_E_HIP
    assert not h.value
