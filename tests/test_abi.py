"""CPU checks of the C-ABI library: it loads, exports every symbol the header
declares, and reports host-forceable errors without touching a GPU."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

import qm38

ROOT = Path(__file__).resolve().parents[1]


def header_symbols():
    text = (ROOT / "include" / "qm38.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qm_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = qm38.load()
    declared = header_symbols()
    assert declared, "no declarations parsed"
    assert sorted(declared) == sorted(qm38.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_status_strings_cover_all_codes():
    lib = qm38.load()
    for i, name in enumerate(qm38.QM_STATUS):
        assert lib.qm_status_string(i).decode() == name


def test_null_arguments_are_rejected():
    lib = qm38.load()
    assert lib.qm_runtime_create(0, None) == qm38.QM_STATUS.index("QM_ERR_NULL_POINTER")
    assert b"NULL" in lib.qm_last_error_message()
    assert lib.qm_q4_project(None, None, 0, None, 0, 0, None) == qm38.QM_STATUS.index("QM_ERR_NULL_POINTER")
    assert lib.qm_kv_length(None) == 0
    assert lib.qm_kv_page_for_token(None, 0) == -1


def test_runtime_without_device_reports_no_device():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = qm38.load()
    h = C.c_void_p()
    assert lib.qm_runtime_create(0, C.byref(h)) == qm38.QM_STATUS.index("QM_ERR_NO_DEVICE")
