"""The "hip" fr_backend's contract paths that need no device: name, argument
and state checks in the reference's order (src/backend.h:52-67,
backends/user-template.c:17-51, backends/ref.c:41-60)."""
import ctypes as C

import pytest

import fronk_amd as fa
import vtable as vt

pytestmark = pytest.mark.skipif(not vt.available(), reason="oracle/_ref or libfr_hip.so not built")


def gpu_present():
    arch = C.create_string_buffer(32)
    return fa.lib().fr_hip_probe(0, arch, 32) == fa.OK


def test_name_and_table():
    b = vt.backend()
    assert b.name == b"hip"
    for f in ("probe", "load", "unload", "run", "bench", "self_test"):
        assert getattr(b, f)
    # The module form's table (src/backend.c:56-58) is the same backend.
    m = vt.Backend.in_dll(vt.library(), "fr_module_hip")
    assert m.name == b"hip"
    for f in ("probe", "load", "unload", "run", "bench", "self_test"):
        assert C.cast(getattr(m, f), C.c_void_p).value == C.cast(getattr(b, f), C.c_void_p).value


@pytest.mark.parametrize("symbol,name", [("fr_hip_q8", b"hip-q8"), ("fr_hip_q8_256", b"hip-q8-256")])
def test_q8_table_shares_the_backend(symbol, name):
    """"hip-q8" (ref-q8 arithmetic) and "hip-q8-256" (the AVX2 backend's)
    differ from "hip" only in run, bench and self_test; probe, load and
    unload are the same functions."""
    b, q = vt.backend(), vt.backend(symbol)
    assert q.name == name
    for f in ("probe", "load", "unload"):
        assert C.cast(getattr(q, f), C.c_void_p).value == C.cast(getattr(b, f), C.c_void_p).value
    for f in ("run", "bench", "self_test"):
        assert C.cast(getattr(q, f), C.c_void_p).value != C.cast(getattr(b, f), C.c_void_p).value
    out = vt.Part()
    req = vt.Req()
    req.layer, req.burst = 0, 1
    for j in range(10):
        req.expert[0][j] = j
    assert q.run(C.byref(req), C.byref(out)) == vt.STATE   # valid request, nothing loaded


def test_backend_close_without_blocks():
    """The bench's close hook (src/bench.c:265-278) succeeds, and is
    repeatable, when no block is loaded."""
    close = vt.library().fr_hip_backend_close
    close.restype = C.c_int
    assert close() == vt.OK
    assert close() == vt.OK


def test_probe():
    b = vt.backend()
    assert b.probe(None) == vt.INVALID
    buf = C.create_string_buffer(4096)
    assert b.probe(buf) == (vt.OK if gpu_present() else vt.UNSUPPORTED)


def test_load_unload_argument_checks():
    b = vt.backend()
    data = C.create_string_buffer(16)
    assert b.load(-1, data, 16) == vt.INVALID
    assert b.load(20, data, 16) == vt.INVALID
    assert b.load(0, None, 16) == vt.INVALID
    assert b.load(0, data, 16) == vt.INVALID           # neither unit length
    assert b.unload(20) == vt.INVALID
    assert b.unload(0) == vt.STATE                     # empty slot


def test_run_validation_order_and_state():
    b = vt.backend()
    out = vt.Part()
    out.layer = 77
    req = vt.Req()
    req.layer, req.burst = 3, 1
    for e in range(vt.ROUTED):
        req.expert[0][e] = e
    assert b.run(None, C.byref(out)) == vt.INVALID
    assert b.run(C.byref(req), None) == vt.INVALID
    bad = vt.Req.from_buffer_copy(req)
    bad.layer = 48
    assert b.run(C.byref(bad), C.byref(out)) == vt.INVALID
    bad = vt.Req.from_buffer_copy(req)
    bad.burst = 9
    assert b.run(C.byref(bad), C.byref(out)) == vt.INVALID
    bad = vt.Req.from_buffer_copy(req)
    bad.expert[0][3] = 2                               # duplicate id
    assert b.run(C.byref(bad), C.byref(out)) == vt.INVALID
    bad = vt.Req.from_buffer_copy(req)
    bad.expert[0][3] = 512                             # out of range
    assert b.run(C.byref(bad), C.byref(out)) == vt.INVALID
    bad = vt.Req.from_buffer_copy(req)
    bad.gate[0][2] = float("nan")
    assert b.run(C.byref(bad), C.byref(out)) == vt.NUMERIC
    bad = vt.Req.from_buffer_copy(req)
    bad.gate[0][2] = -1.0
    assert b.run(C.byref(bad), C.byref(out)) == vt.INVALID
    bad = vt.Req.from_buffer_copy(req)
    bad.x[0][100] = float("inf")
    assert b.run(C.byref(bad), C.byref(out)) == vt.NUMERIC
    assert b.run(C.byref(req), C.byref(out)) == vt.STATE   # nothing loaded
    assert out.layer == 77                                  # untouched on failure
