"""CPU checks of the boundary: libgllm_hip.so loads and exports every entry
point include/gllm_hip.h declares, and the ctypes table matches the header.
No compute calls (there is no GPU here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gllm_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gllm_hip_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("gllm_hip_matvec", "gllm_hip_matvec_dev", "gllm_hip_argmax", "gllm_hip_weight_new",
                 "gllm_hip_kv_store", "gllm_hip_attend_group", "gllm_hip_model_decode"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from gopherllm_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libgllm_hip.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_covers_the_header():
    from gopherllm_amd import _lib
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_no_gpu_reports_unavailable_without_crashing():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from gopherllm_amd import _lib
    L = _lib.load()
    assert L.gllm_hip_available() == 0
    assert _lib.last_error()


def test_product_does_not_import_the_oracle():
    pkg = os.path.join(ROOT, "gopherllm_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.replace("oracle_", ""), f
