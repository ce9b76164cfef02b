"""The restated oracle regenerates the reference's committed golden corpus.

The eight files under tests/golden/vectors are the reference's own fixtures
(tests/vectors/*, recipe src/vectors.c:12-135, README tests/vectors/README).
Byte-identical regeneration pins the xorshift recipe, the SHA-256 digest, the
legacy Q4_0 decoder and the whole ref run() loop (double accumulation order,
stable SiLU, narrowing) at H=2560.
"""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "vectors")
NAMES = ["zero-input", "zero-gates", "signed", "reused", "mixed", "outliers", "tiny", "all-blocks"]


def manifest():
    out = {}
    with open(os.path.join(GOLDEN, "SHA256SUMS")) as f:
        for line in f:
            digest, name = line.split()
            out[name] = digest
    return out


def build_vector(index):
    lib = oracle.lib()
    req = oracle.Req()
    mask = C.c_uint32()
    name = C.create_string_buffer(16)
    assert lib.fo_vector_request(index, C.byref(req), C.byref(mask), name) == 0
    lay = oracle.layout(2560, oracle.FMT_LEGACY)
    # np.zeros maps untouched pages lazily: only the used slices materialize.
    blocks = [np.zeros(lay.block, np.uint8) if mask.value >> b & 1 else None for b in range(20)]
    ptrs = (C.c_void_p * 20)(*[(b.ctypes.data if b is not None else None) for b in blocks])
    digest = C.create_string_buffer(65)
    assert lib.fo_vector_fill(index, ptrs, digest) == 0
    return req, mask.value, name.value.decode(), blocks, digest.value


def golden_values(path, burst):
    with open(path) as f:
        header = f.readline().split()
        vals = np.array([float.fromhex(v) for v in f.read().split()], np.float32)
    return header, vals.reshape(burst, 2560)


@pytest.mark.parametrize("index", range(8))
def test_golden_regenerates_byte_identical(index):
    req, mask, name, blocks, digest = build_vector(index)
    assert name == NAMES[index]
    rc, y = oracle.ref_run(blocks, oracle.FMT_LEGACY, False, req)
    assert rc == oracle.OK
    buf = C.create_string_buffer(4 << 20)
    n = C.c_size_t()
    rc = oracle.lib().fo_vector_format(index, C.byref(req), mask, digest, oracle.fptr(np.ascontiguousarray(y)),
                                       buf, len(buf), C.byref(n))
    assert rc == 0
    text = buf.raw[:n.value]
    path = os.path.join(GOLDEN, name + ".txt")
    with open(path, "rb") as f:
        committed = f.read()
    assert text == committed
    assert hashlib.sha256(text).hexdigest() == manifest()[name + ".txt"]


@pytest.mark.parametrize("index", range(8))
def test_ref_q8_within_backend_tolerance(index):
    """ref-q8 passes the corpus under the frozen backend tolerance
    (tests/test_vectors.c:200); inactive tokens of the corpus are zero."""
    req, mask, name, blocks, _ = build_vector(index)
    rc, y = oracle.ref_run(blocks, oracle.FMT_LEGACY, True, req)
    assert rc == oracle.OK
    _, gold = golden_values(os.path.join(GOLDEN, name + ".txt"), req.burst)
    for t in range(req.burst):
        rc, err = oracle.compare(gold[t], y[t])
        assert rc == 0 and oracle.conforms(err, oracle.BACKEND_TOLERANCE), (name, t, err)


def test_zero_output_cannot_pass():
    """A zero-output candidate fails a nonzero golden (tests/test_vectors.c:201-202)."""
    _, gold = golden_values(os.path.join(GOLDEN, "signed.txt"), 1)
    rc, err = oracle.compare(gold[0], np.zeros(2560, np.float32))
    assert rc == 0 and not oracle.conforms(err, oracle.BACKEND_TOLERANCE)


def test_sha256_known_answers():
    for msg in [b"", b"abc", b"a" * 1000, bytes(range(256)) * 3]:
        out = (C.c_uint8 * 32)()
        oracle.lib().fo_sha256(msg, len(msg), out)
        assert bytes(out) == hashlib.sha256(msg).digest()
