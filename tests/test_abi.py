"""The C-ABI library loads without a GPU and exports every declared symbol."""
import ctypes as C
import os
import re

import pytest

import fronk_amd as fa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fr_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = fa.lib()
    names = declared("fronk_hip.h")
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
        assert name in fa.SIGNATURES, name


def test_unit_sizes_match_oracle():
    import oracle
    for hidden in (2560, 4096):
        for fmt in range(5):
            if fmt == fa.FMT_LEGACY and hidden != 2560:
                continue
            assert fa.unit_bytes(hidden, fmt) == oracle.layout(hidden, fmt).block
    assert fa.unit_bytes(1000, fa.FMT_NATIVE) == 0


def test_calls_before_open_are_state_errors():
    lib = fa.lib()
    assert lib.fr_hip_release(0) == fa.STATE
    assert lib.fr_hip_release(20) == fa.INVALID
    assert lib.fr_hip_reserve(0, 4096, fa.FMT_Q4KT) in (fa.STATE, fa.OK)


def test_capacity_argument_checks():
    lib = fa.lib()
    n = C.c_uint(0)
    f = C.c_uint64(0)
    assert lib.fr_hip_capacity(0, 2560, fa.FMT_NATIVE, 0, None, C.byref(n)) == fa.INVALID
    assert lib.fr_hip_capacity(0, 1000, fa.FMT_NATIVE, 0, C.byref(f), C.byref(n)) == fa.INVALID
    rc, free, blocks = fa.capacity(2560, fa.FMT_NATIVE, device=99)
    assert rc == fa.UNSUPPORTED
