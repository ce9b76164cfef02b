"""The oracle's restatement of the AVX2 backend's arithmetic (oracle.q8_256_run)
pinned against that backend itself: backends/avx2.c compiled from the
reference's sources into oracle/_ref and run here, on the CPU, on native
units filled by the reference's own fixture (src/native.c:62) at its
compiled-in H = 2560. The two differ only in the order of float additions
and in numpy's float exp against libm's, so they agree far more closely than
either agrees with ref, and a dropped term (the min term, the shared
expert, h's d) or a ref-style activation would fail the bound.
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle
from fixtures import oracle_request, softmax_gates, sparse_unit

H = 2560
AVX2_TOL = (2e-4, 2e-3)   # rel. L2, normalized max


def reference():
    if not os.path.exists(oracle.REF_PATH):
        pytest.skip("oracle/_ref not built")
    ref = C.CDLL(oracle.REF_PATH, mode=C.RTLD_GLOBAL)
    ref.fr_native_fixture.argtypes = [C.c_void_p, C.c_uint, C.c_uint32]
    ref.fr_avx2_set_tuning.argtypes = [C.c_uint] * 4
    ref.fr_avx2_configure.argtypes = [C.c_uint, C.c_uint]
    return ref


class Part(C.Structure):   # fr_part (src/backend.h:26-29) at H = 2560
    _fields_ = [("layer", C.c_uint), ("burst", C.c_uint), ("y", (C.c_float * H) * 8)]


class Req(C.Structure):    # fr_req (src/backend.h:20-25) at H = 2560
    _fields_ = [("layer", C.c_uint), ("burst", C.c_uint), ("expert", (C.c_uint16 * 10) * 8),
                ("gate", (C.c_float * 11) * 8), ("x", (C.c_float * H) * 8)]


RunFn = C.CFUNCTYPE(C.c_int, C.POINTER(Req), C.POINTER(Part))


class Backend(C.Structure):   # fr_backend (src/backend.h:52-67)
    _fields_ = [("name", C.c_char_p), ("probe", C.c_void_p), ("load", C.CFUNCTYPE(C.c_int, C.c_int, C.c_void_p,
                                                                                    C.c_size_t)),
                ("unload", C.CFUNCTYPE(C.c_int, C.c_int)), ("run", RunFn), ("bench", C.c_void_p),
                ("self_test", C.c_void_p)]


def avx2_run(avx2, layer, experts, gates, x):
    q = Req()
    q.layer, q.burst = layer, x.shape[0]
    for t in range(x.shape[0]):
        for j in range(10):
            q.expert[t][j] = int(experts[t, j])
        for j in range(11):
            q.gate[t][j] = float(gates[t, j])
        C.memmove(q.x[t], np.ascontiguousarray(x[t], np.float32).ctypes.data, 4 * H)
    out = Part()
    rc = avx2.run(C.byref(q), C.byref(out))
    return rc, np.ctypeslib.as_array(out.y)[:x.shape[0]].copy()


def worst(ref, got):
    w = (0.0, 0.0)
    for t in range(ref.shape[0]):
        rc, err = oracle.compare(ref[t], got[t])
        assert rc == 0
        w = (max(w[0], err[0]), max(w[1], err[1]))
    return w


def test_q8_256_restatement_matches_the_reference_avx2_backend():
    ref = reference()
    avx2 = Backend.in_dll(ref, "fr_avx2")
    lay = oracle.layout(H, oracle.FMT_NATIVE)
    blocks, layer = (2, 9), 1
    units = [None] * 20
    for b in blocks:
        units[b] = sparse_unit(lay)
        ref.fr_native_fixture(units[b].ctypes.data, layer, 5 + 31 * b)
    ref.fr_avx2_set_tuning(len(blocks), 1, 2, 0)
    if ref.fr_avx2_configure(len(blocks), 1) != 0:
        pytest.skip("the AVX2 backend does not run on this CPU")
    for b in blocks:
        assert avx2.load(b, units[b].ctypes.data, lay.block) == 0
    try:
        rng = np.random.default_rng(2560)
        cases = []
        e1 = (np.arange(10, dtype=np.uint16) * 7 % 80).reshape(1, 10)
        g1 = np.full((1, 11), 0.0625, np.float32)
        g1[0, 10] = 0.5
        cases.append((e1, g1, np.array([((d * 37) % 257 - 128) / 128 for d in range(H)], np.float32).reshape(1, H)))
        e2 = np.stack([rng.choice(80, 10, replace=False) for _ in range(2)]).astype(np.uint16)
        g2 = np.zeros((2, 11), np.float32)
        g2[:, :10] = softmax_gates(rng, 2)
        cases.append((e2, g2, rng.standard_normal((2, H)).astype(np.float32)))
        for experts, gates, x in cases:
            req = oracle_request(layer, experts, gates, x)
            rc, y = oracle.q8_256_run(units, oracle.FMT_NATIVE, req)
            assert rc == oracle.OK
            rc, ya = avx2_run(avx2, layer, experts, gates, x)
            assert rc == 0
            rc, yr = oracle.ref_run(units, oracle.FMT_NATIVE, False, req)
            assert rc == 0
            near, far = worst(ya, y), worst(yr, ya)
            print(f"restatement vs avx2 {near}, avx2 vs ref {far}")
            assert near[0] <= AVX2_TOL[0] and near[1] <= AVX2_TOL[1], near
            assert near[0] < 0.05 * far[0], (near, far)
        # A non-finite x is the backend's FR_NUMERIC.
        bad = cases[0][2].copy()
        bad[0, 3] = np.nan
        assert oracle.q8_256_run(units, oracle.FMT_NATIVE, oracle_request(layer, e1, g1, bad))[0] == oracle.NUMERIC
    finally:
        for b in blocks:
            avx2.unload(b)
        ref.fr_avx2_close()
