"""The restated oracle against the reference's own C, compiled into oracle/_ref.

oracle/_ref/libfronk_ref.so is built by `make -C oracle ref` from the
reference's unmodified sources (H fixed at 2560 by src/model.h:16). Where it is
present these tests require the restatement to be bit-identical to it on the
native fixture recipe of src/native.c:66-93, on random rows of every native
type and on random activation groups. Skipped where the library was not built.
"""
import ctypes as C

import numpy as np
import pytest

import oracle

H = 2560
ref = oracle.ref_lib()
pytestmark = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (reference sources absent)")


class FrReq(C.Structure):
    _fields_ = [("layer", C.c_uint), ("burst", C.c_uint), ("expert", (C.c_uint16 * 10) * 8),
                ("gate", (C.c_float * 11) * 8), ("x", (C.c_float * H) * 8)]


class FrPart(C.Structure):
    _fields_ = [("layer", C.c_uint), ("burst", C.c_uint), ("y", (C.c_float * H) * 8)]


RUN = C.CFUNCTYPE(C.c_int, C.POINTER(FrReq), C.POINTER(FrPart))
LOAD = C.CFUNCTYPE(C.c_int, C.c_int, C.c_void_p, C.c_size_t)
UNLOAD = C.CFUNCTYPE(C.c_int, C.c_int)


class FrBackend(C.Structure):
    _fields_ = [("name", C.c_char_p), ("probe", C.c_void_p), ("load", LOAD), ("unload", UNLOAD),
                ("run", RUN), ("bench", C.c_void_p), ("self_test", C.c_void_p)]


def backend(name):
    return FrBackend.in_dll(ref, name)


def native_fixture(lay):
    """Sparse native unit with experts 0..79 and the shared slice of layer 47,
    then 8 tokens of activations and gates (src/native.c:66-76)."""
    data = np.zeros(lay.block, np.uint8)
    seed = 7
    for e in range(81):
        eid = 512 if e == 80 else e
        off = oracle.slice_offset(lay, 47, eid)
        size = lay.shared_slice if eid == 512 else lay.slice
        seed = oracle.fill_slice(data[off:off + size], lay, eid, seed)
    gates = np.full((8, 11), 0.0625, np.float32)
    gates[:, 10] = 0.5
    x = np.zeros((8, H), np.float32)
    for t in range(8):
        for j in range(H):
            v, seed = oracle.lcg(seed)
            x[t, j] = np.float32((v % 257) - 128) / np.float32(128)
    return data, gates, x


@pytest.fixture(scope="module")
def fixture():
    lay = oracle.layout(H, oracle.FMT_NATIVE)
    return (lay,) + native_fixture(lay)


@pytest.mark.parametrize("q8", [0, 1])
def test_native_fixture_bit_identical(fixture, q8):
    lay, data, gates, x = fixture
    b = backend("fr_ref_q8" if q8 else "fr_ref")
    assert b.load(19, data.ctypes.data, lay.block) == 0
    try:
        blocks = [None] * 20
        blocks[19] = data
        for mode in range(2):
            for burst in (1, 3, 8):
                fr, fo = FrReq(), oracle.Req()
                fr.layer = fo.layer = 47
                fr.burst = fo.burst = burst
                fo.hidden = H
                for t in range(8):
                    for e in range(10):
                        fr.expert[t][e] = fo.expert[t][e] = e + (0 if mode else t * 10)
                    for e in range(11):
                        fr.gate[t][e] = fo.gate[t][e] = gates[t, e]
                np.ctypeslib.as_array(fr.x)[:] = x
                np.ctypeslib.as_array(fo.x)[:, :H] = x
                part = FrPart()
                assert b.run(C.byref(fr), C.byref(part)) == 0
                rc, y = oracle.ref_run(blocks, oracle.FMT_NATIVE, q8, fo)
                assert rc == 0
                got = np.ctypeslib.as_array(part.y)[:burst]
                assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), (mode, burst)
    finally:
        assert b.unload(19) == 0


def test_q8_activation_bit_identical():
    ref.fr_q8_activation.argtypes = [C.POINTER(C.c_float), C.POINTER(C.c_float), C.c_size_t]
    rng = np.random.default_rng(1)
    for scale in [1e-30, 1e-3, 1.0, 1e30]:
        x = (rng.standard_normal(4096) * scale).astype(np.float32)
        x[::97] = 0
        a = np.zeros_like(x)
        assert ref.fr_q8_activation(oracle.fptr(x), oracle.fptr(a), x.size) == 0
        rc, b = oracle.q8_activation(x)
        assert rc == 0 and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("typ,n", [(oracle.Q4_K, 2560), (oracle.MXFP4, 2560), (oracle.Q8_0, 2560), (oracle.MXFP4, 32)])
def test_native_dot_bit_identical(typ, n):
    ref.fr_native_dot.argtypes = [C.POINTER(C.c_uint8), C.c_uint, C.POINTER(C.c_float), C.c_uint,
                                  C.POINTER(C.c_double)]
    rng = np.random.default_rng(typ * 7 + n)
    row = rng.integers(0, 256, oracle.lib().fo_row_bytes(typ, n), dtype=np.uint8)
    bs = 144 if typ == oracle.Q4_K else 17 if typ == oracle.MXFP4 else 34
    for k in range(0, row.size, bs):      # finite scales
        if typ == oracle.MXFP4:
            row[k] = rng.integers(100, 140)
        else:
            row[k + 1] = rng.integers(0x10, 0x30)
            if typ == oracle.Q4_K:
                row[k + 3] = rng.integers(0x10, 0x30)
    x = rng.standard_normal(n).astype(np.float32)
    a = C.c_double()
    assert ref.fr_native_dot(oracle.u8ptr(row), typ, oracle.fptr(x), n, C.byref(a)) == 0
    rc, b = oracle.native_dot(row, typ, x)
    assert rc == 0 and a.value == b


def test_f16_bit_identical():
    ref.fr_f16.restype = C.c_float
    ref.fr_f16.argtypes = [C.c_uint16]
    lib = oracle.lib()
    for i in range(0, 65536, 7):
        a, b = ref.fr_f16(i), lib.fo_f16(i)
        assert (a != a and b != b) or np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)
