"""The C-ABI library loads without a GPU and exports every symbol that
include/vokra_hip.h declares (no compute calls here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(vokra_hip_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    for must in ("vokra_hip_create", "vokra_hip_dequant_gemv_f32", "vokra_hip_gemm_q_f32"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from vokra_amd import hip
    if not os.path.exists(hip.LIB_PATH):
        pytest.fail(f"{hip.LIB_PATH} not built (run `python -m vokra_amd.build`)")
    L = ctypes.CDLL(hip.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_integration_ffi_table_binds_every_declared_symbol():
    """INTEGRATION.md's dlsym table for the reference-side crate (fields named
    without the vokra_hip_ prefix) has an entry for every declared function."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    missing = [n for n in declared_symbols() if f"pub {n[len('vokra_hip_'):]}:" not in text]
    assert not missing, f"declared but absent from the FFI table: {missing}"


def test_missing_device_is_backend_unavailable():
    """Without a GPU the probe fails loudly (BackendUnavailable), never a CPU path."""
    from vokra_amd import hip
    try:
        n = hip.probe()
    except hip.BackendUnavailable:
        return
    assert n >= 1
