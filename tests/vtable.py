"""ctypes view of the "hip" fr_backend vtable (fronk_amd/host/hip.c) as the
reference program sees it (src/backend.h:52-67), loaded next to the
reference's own compiled sources (oracle/_ref) that provide hw_probe,
fr_vectors_check, fr_native_self_test and fr_bench_execute_backend. Not
collected by pytest."""
import ctypes as C
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libfronk_ref.so")
VTABLE_LIB = os.path.join(ROOT, "fronk_amd", "libfr_hip.so")
GOLDEN = os.path.join(ROOT, "tests", "golden", "vectors")

HIDDEN, MAX_BURST, ROUTED, ACTIVE = 2560, 8, 10, 11
OK, INVALID, STATE, NUMERIC, IO, UNSUPPORTED = 0, -1, -2, -3, -4, -5


class Req(C.Structure):           # fr_req (src/backend.h:20-25) at FR_HIDDEN = 2560
    _fields_ = [("layer", C.c_uint), ("burst", C.c_uint),
                ("expert", (C.c_uint16 * ROUTED) * MAX_BURST),
                ("gate", (C.c_float * ACTIVE) * MAX_BURST),
                ("x", (C.c_float * HIDDEN) * MAX_BURST)]


class Part(C.Structure):          # fr_part (src/backend.h:26-29)
    _fields_ = [("layer", C.c_uint), ("burst", C.c_uint), ("y", (C.c_float * HIDDEN) * MAX_BURST)]


ProbeFn = C.CFUNCTYPE(C.c_int, C.c_void_p)
LoadFn = C.CFUNCTYPE(C.c_int, C.c_int, C.c_void_p, C.c_size_t)
UnloadFn = C.CFUNCTYPE(C.c_int, C.c_int)
RunFn = C.CFUNCTYPE(C.c_int, C.POINTER(Req), C.POINTER(Part))
BenchFn = C.CFUNCTYPE(C.c_int, C.c_int, C.c_void_p)
SelfTestFn = C.CFUNCTYPE(C.c_int, C.c_char_p)


class Backend(C.Structure):       # fr_backend (src/backend.h:52-67)
    _fields_ = [("name", C.c_char_p), ("probe", ProbeFn), ("load", LoadFn), ("unload", UnloadFn),
                ("run", RunFn), ("bench", BenchFn), ("self_test", SelfTestFn)]


_vt = {}
_lib = None


def available():
    return os.path.exists(REF_LIB) and os.path.exists(VTABLE_LIB)


def library():
    """libfr_hip.so; the reference library is loaded first, globally, so that
    the vtable's reference symbols resolve."""
    global _lib
    if _lib is None:
        C.CDLL(REF_LIB, mode=C.RTLD_GLOBAL)
        _lib = C.CDLL(VTABLE_LIB, mode=C.RTLD_GLOBAL)
    return _lib


def backend(symbol="fr_hip"):
    """The fr_hip vtable (or fr_hip_q8, the same backend with ref-q8
    arithmetic)."""
    if symbol not in _vt:
        _vt[symbol] = Backend.in_dll(library(), symbol)
    return _vt[symbol]
