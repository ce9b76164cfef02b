"""The reference's own conformance harness against the "hip" backend on the
GPU: self_test runs fr_vectors_check over the committed golden corpus
(src/vectors.c:136-174, backend tolerance src/backend.c:11-13) and then
fr_native_self_test (src/native.c:66-135: bursts 1..8 against the
reference's ref backend, corrupt scales -> FR_NUMERIC with the caller's
output preserved), both compiled from the reference sources in oracle/_ref.
"""
import ctypes as C

import pytest

import vtable as vt

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not vt.available(), reason="oracle/_ref or libfr_hip.so not built")]


def test_probe_finds_gfx950():
    buf = C.create_string_buffer(4096)
    assert vt.backend().probe(buf) == vt.OK


def test_reference_self_test():
    print("hip self_test: golden corpus, then native self-test", flush=True)
    assert vt.backend().self_test(vt.GOLDEN.encode()) == vt.OK


def test_reference_self_test_q8_256():
    """The "hip-q8-256" table (the AVX2 backend's arithmetic) through the same
    harness: the legacy corpus (run as ref-q8, whose codes that backend's
    legacy path shares) and the native self-test, within the backend
    tolerance."""
    t = vt.backend("fr_hip_q8_256")
    assert t.name == b"hip-q8-256"
    print("hip-q8-256 self_test: golden corpus, then native self-test", flush=True)
    assert t.self_test(vt.GOLDEN.encode()) == vt.OK


def test_reference_self_test_q8():
    """The "hip-q8" table (ref-q8 arithmetic) through the same harness: the
    corpus within the backend tolerance, the native self-test against ref."""
    q8 = vt.backend("fr_hip_q8")
    assert q8.name == b"hip-q8"
    print("hip-q8 self_test: golden corpus, then native self-test", flush=True)
    assert q8.self_test(vt.GOLDEN.encode()) == vt.OK
