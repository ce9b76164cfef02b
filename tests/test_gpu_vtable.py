"""The reference's own conformance harness against the "hip" backend on the
GPU: self_test runs fr_vectors_check over the committed golden corpus
(src/vectors.c:136-174, backend tolerance src/backend.c:11-13) and then
fr_native_self_test (src/native.c:66-135: bursts 1..8 against the
reference's ref backend, corrupt scales -> FR_NUMERIC with the caller's
output preserved), both compiled from the reference sources in oracle/_ref.

Each test runs in a child process that never imports torch: the backend
library then runs on the system HIP runtime it links against, as the
reference node (a C program) would load it.
"""
import os
import subprocess
import sys

import pytest

import vtable as vt

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not vt.available(), reason="oracle/_ref or libfr_hip.so not built")]

TESTS = os.path.dirname(os.path.abspath(__file__))


def in_child(body, timeout=240):
    """Run `body` (Python, with ctypes as C and vtable as vt imported) in a
    child process without torch; returns its printed lines."""
    code = ("import ctypes as C, sys\n"
            f"sys.path.insert(0, {TESTS!r})\n"
            "import vtable as vt\n"
            "assert 'torch' not in sys.modules\n" + body +
            "\nassert 'torch' not in sys.modules\nprint('child ok', flush=True)\n")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "child ok" in r.stdout, r.returncode
    return r.stdout


def test_probe_finds_gfx950():
    in_child("buf = C.create_string_buffer(4096)\nassert vt.backend().probe(buf) == vt.OK")


def test_reference_self_test():
    print("hip self_test: golden corpus, then native self-test", flush=True)
    in_child("assert vt.backend().self_test(vt.GOLDEN.encode()) == vt.OK")


def test_reference_self_test_q8_256():
    """The "hip-q8-256" table (the AVX2 backend's arithmetic) through the same
    harness: the legacy corpus (run as ref-q8, whose codes that backend's
    legacy path shares) and the native self-test, within the backend
    tolerance."""
    print("hip-q8-256 self_test: golden corpus, then native self-test", flush=True)
    in_child("t = vt.backend('fr_hip_q8_256')\nassert t.name == b'hip-q8-256'\n"
             "assert t.self_test(vt.GOLDEN.encode()) == vt.OK")


def test_reference_self_test_q8():
    """The "hip-q8" table (ref-q8 arithmetic) through the same harness: the
    corpus within the backend tolerance, the native self-test against ref."""
    print("hip-q8 self_test: golden corpus, then native self-test", flush=True)
    in_child("t = vt.backend('fr_hip_q8')\nassert t.name == b'hip-q8'\n"
             "assert t.self_test(vt.GOLDEN.encode()) == vt.OK")
