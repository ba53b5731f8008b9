"""CPU-side checks of the C ABI: the library loads and exports every entry point
include/aarambh_hip.h declares (no device calls)."""
import ctypes
import os
import re

import aarambh_hip as A

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "aarambh_hip.h")).read()
    return sorted(set(re.findall(r"\b(aarh_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    L = ctypes.CDLL(A.LIB_PATH)
    syms = header_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    assert sorted(A.EXPORTED) == syms


def test_python_mirror_binds_every_symbol():
    L = A.lib()
    for s in header_symbols():
        assert getattr(L, s).argtypes is not None, s


def test_config_validation_is_host_side():
    # SpeculativeConfig rejects zero width (speculative.rs:24-29) without touching a device.
    import pytest
    with pytest.raises(A.ConfigError):
        A.SpeculativeConfig(0)
    with pytest.raises(A.ConfigError):
        A.Sampler.top_k_top_p(-1.0)
    with pytest.raises(A.ConfigError):
        A.Sampler.top_k_top_p(1.0, top_p=1.5)
