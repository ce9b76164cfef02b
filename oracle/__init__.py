"""ctypes binding of the oracle (the checker) and of oracle/_ref.

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()`` and
by bench.py's ``cpu_baseline`` leg. The product (``fronk_amd``) never imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfronk_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libfronk_ref.so")
REFERENCE = "/root/reference"

OK, INVALID, STATE, NUMERIC, IO = 0, -1, -2, -3, -4
Q4_0, Q8_0, Q4_K, MXFP4 = 2, 8, 12, 39
FMT_LEGACY, FMT_NATIVE, FMT_Q4KT, FMT_Q8, FMT_MXFP4 = 0, 1, 2, 3, 4
LAYERS, ROUTED, SHARED, BLOCKS, MAX_BURST, MAX_HIDDEN = 48, 512, 512, 20, 8, 4096

# Frozen tolerances (src/backend.c:11-13).
REFERENCE_TOLERANCE = (1e-6, 1e-6, 0.999999999999)
BACKEND_TOLERANCE = (0.025, 0.030, 0.9998)


class Layout(C.Structure):
    _fields_ = [("hidden", C.c_uint), ("format", C.c_uint), ("gu_type", C.c_uint),
                ("down_type", C.c_uint), ("down_transposed", C.c_uint),
                ("shared_gu_type", C.c_uint), ("shared_down_type", C.c_uint),
                ("gu_row", C.c_uint64), ("down_row", C.c_uint64), ("proj", C.c_uint64),
                ("down", C.c_uint64), ("slice", C.c_uint64), ("shared_proj", C.c_uint64),
                ("shared_down", C.c_uint64), ("shared_slice", C.c_uint64),
                ("layer", C.c_uint64), ("block", C.c_uint64)]


class Req(C.Structure):
    _fields_ = [("layer", C.c_uint), ("burst", C.c_uint), ("hidden", C.c_uint),
                ("expert", (C.c_uint16 * 10) * 8), ("gate", (C.c_float * 11) * 8),
                ("x", (C.c_float * MAX_HIDDEN) * 8)]

    def experts(self):
        return np.ctypeslib.as_array(self.expert)

    def gates(self):
        return np.ctypeslib.as_array(self.gate)

    def xs(self):
        return np.ctypeslib.as_array(self.x)


def build(ref=None):
    """Compile the restatement (and oracle/_ref when the reference is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if ref is None:
        ref = os.path.isdir(REFERENCE)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        L = C.CDLL(LIB_PATH)
        P = C.POINTER
        u8p = P(C.c_uint8)
        L.fo_f16.restype = C.c_float
        L.fo_f16.argtypes = [C.c_uint16]
        L.fo_row_bytes.restype = C.c_uint64
        L.fo_row_bytes.argtypes = [C.c_uint, C.c_uint]
        L.fo_layout_get.argtypes = [C.c_uint, C.c_uint, P(Layout)]
        L.fo_slice_offset.restype = C.c_uint64
        L.fo_slice_offset.argtypes = [P(Layout), C.c_uint, C.c_uint]
        L.fo_q4_dot.argtypes = [u8p, P(C.c_float), C.c_size_t, P(C.c_double)]
        L.fo_q8_activation.argtypes = [P(C.c_float), P(C.c_float), C.c_size_t]
        L.fo_quantize8.restype = None
        L.fo_quantize8.argtypes = [P(C.c_float), C.c_uint, C.c_uint, P(C.c_int8), P(C.c_float), P(C.c_int16)]
        L.fo_native_dot.argtypes = [u8p, C.c_uint, P(C.c_float), C.c_uint, P(C.c_double)]
        L.fo_decode.restype = C.c_float
        L.fo_decode.argtypes = [u8p, C.c_uint, C.c_uint]
        L.fo_dequant_row.argtypes = [u8p, C.c_uint, C.c_uint, P(C.c_float)]
        L.fo_ref_run.argtypes = [P(C.c_void_p), C.c_uint, C.c_int, P(Req), P(C.c_float)]
        L.fo_compare.argtypes = [P(C.c_float), P(C.c_float), C.c_size_t, P(C.c_double)]
        L.fo_conforms.argtypes = [P(C.c_double), P(C.c_double)]
        L.fo_vector_request.argtypes = [C.c_uint, P(Req), P(C.c_uint32), C.c_char_p]
        L.fo_vector_fill.argtypes = [C.c_uint, P(C.c_void_p), C.c_char_p]
        L.fo_vector_format.argtypes = [C.c_uint, P(Req), C.c_uint32, C.c_char_p, P(C.c_float),
                                       C.c_char_p, C.c_size_t, P(C.c_size_t)]
        L.fo_lcg.restype = C.c_uint32
        L.fo_lcg.argtypes = [P(C.c_uint32)]
        L.fo_fill_slice.restype = None
        L.fo_fill_slice.argtypes = [u8p, P(Layout), C.c_uint, P(C.c_uint32)]
        L.fo_sha256.restype = None
        L.fo_sha256.argtypes = [C.c_void_p, C.c_size_t, u8p]
        L.fo_synth_key.restype = C.c_uint64
        L.fo_synth_key.argtypes = [C.c_uint64, C.c_uint, C.c_uint, C.c_uint]
        L.fo_synth_scale.restype = C.c_uint16
        L.fo_synth_scale.argtypes = [C.c_uint64]
        L.fo_synth_byte.restype = C.c_uint8
        L.fo_synth_byte.argtypes = [P(Layout), C.c_uint64, C.c_uint, C.c_uint64]
        L.fo_synth_slice.restype = None
        L.fo_synth_slice.argtypes = [u8p, P(Layout), C.c_uint64, C.c_uint, C.c_uint, C.c_uint]
        _lib = L
    return _lib


def ref_lib():
    """oracle/_ref/libfronk_ref.so (the reference's own C, H=2560) or None."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        _ref = C.CDLL(REF_PATH)
    return _ref


def fptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def u8ptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


def layout(hidden, fmt):
    out = Layout()
    rc = lib().fo_layout_get(hidden, fmt, C.byref(out))
    if rc:
        raise ValueError(f"no layout for hidden={hidden} format={fmt}")
    return out


def slice_offset(lay, layer, expert):
    return lib().fo_slice_offset(C.byref(lay), layer, expert)


def ref_run(blocks, fmt, q8, req):
    """Run the restated ref/ref-q8. ``blocks`` is a list of 20 numpy uint8
    arrays (or None). Returns (rc, y[burst, hidden] float32)."""
    ptrs = (C.c_void_p * BLOCKS)(*[(b.ctypes.data if b is not None else None) for b in blocks])
    y = np.zeros((MAX_BURST, req.hidden), np.float32)
    rc = lib().fo_ref_run(ptrs, fmt, int(q8), C.byref(req), fptr(y))
    return rc, y[:req.burst]


def compare(ref, act):
    out = (C.c_double * 3)()
    ref = np.ascontiguousarray(ref, np.float32)
    act = np.ascontiguousarray(act, np.float32)
    rc = lib().fo_compare(fptr(ref), fptr(act), ref.size, out)
    return rc, tuple(out)


def conforms(err, limit):
    return bool(lib().fo_conforms((C.c_double * 3)(*err), (C.c_double * 3)(*limit)))


def q8_activation(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    rc = lib().fo_q8_activation(fptr(x), fptr(out), x.size)
    return rc, out


def quantize8(x, group):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.size, np.int8)
    d = np.zeros(x.size // group, np.float32)
    s = np.zeros(x.size // 32, np.int16)
    lib().fo_quantize8(fptr(x), x.size, group, q.ctypes.data_as(C.POINTER(C.c_int8)), fptr(d),
                       s.ctypes.data_as(C.POINTER(C.c_int16)))
    return q, d, s


def q8_256_run(blocks, fmt, req):
    """The AVX2 backend's native arithmetic (backends/avx2.c:170-174, its run
    at :615-716), restated with numpy up to the order of its float additions,
    for native (Q4_K gate/up, MXFP4 down, Q8_0 shared) and all-Q8_0 units:
    - x per token into int8 codes and one d per 256 by quantize8 (:633);
    - each gate/up row's dot as the exact sum of weight x code x d, which is
      what its integer dots times one float scale per block add up to
      (Q4_K :262-319, the 6-bit scales applied in integers and the min term
      through the int16 code sums; Q8_0 rows :237-248);
    - a and u narrowed to float, h = a/(1 + e^-a)*u in float (:428), a
      non-finite h FR_NUMERIC (:433);
    - h into int8 codes and one d per 32 by quantize8 (:434);
    - the down as the exact sum of weight x h code, times h's d and the gate
      (MXFP4 :331-362 with its codes doubled into integers, Q8_0 :364-390);
    - sums over experts and blocks in fp64, narrowed once (:705-709).
    Weights come from the oracle's float decode, exact for the checker's
    data (Q4_K d and dmin of close exponents). Returns (rc, y[burst, hidden]).
    """
    H, T = req.hidden, req.burst
    lay = layout(H, fmt)
    xs = np.ctypeslib.as_array(req.x)[:T, :H]
    experts, gates = req.experts()[:T], req.gates()[:T]
    y = np.zeros((T, H), np.float64)
    for t in range(T):
        x = np.ascontiguousarray(xs[t], np.float32)
        if not np.isfinite(x).all():
            return NUMERIC, None
        q, d, _ = quantize8(x, 256)
        xq = q.astype(np.float64) * np.repeat(d.astype(np.float64), 256)
        for j in range(11):
            g = float(gates[t, j])
            if j == 10 and g == 0.0:
                continue
            eid = SHARED if j == 10 else int(experts[t, j])
            shared = eid == SHARED
            gu = lay.shared_gu_type if shared else lay.gu_type
            dn = lay.shared_down_type if shared else lay.down_type
            proj = lay.shared_proj if shared else lay.proj
            for unit in blocks:
                if unit is None:
                    continue
                off = slice_offset(lay, req.layer, eid)
                sl = unit[off:off + (lay.shared_slice if shared else lay.slice)]
                W = dequant(sl[:2 * proj], gu, 64 * H).astype(np.float64).reshape(64, H)
                a, u = np.float32(W[:32] @ xq), np.float32(W[32:] @ xq)
                with np.errstate(over="ignore", invalid="ignore"):
                    h = (a / (np.float32(1) + np.exp(-a))) * u
                if not np.isfinite(h).all():
                    return NUMERIC, None
                hq, hd, _ = quantize8(h.astype(np.float32), 32)
                Wd = dequant(sl[2 * proj:], dn, 32 * H).astype(np.float64).reshape(H, 32)
                y[t] += g * (Wd @ hq.astype(np.float64)) * float(hd[0])
    if not np.isfinite(y).all() or (np.abs(y) > np.finfo(np.float32).max).any():
        return NUMERIC, None
    return OK, y.astype(np.float32)


def native_dot(row, typ, x, n=None):
    x = np.ascontiguousarray(x, np.float32)
    out = C.c_double(123.0)
    rc = lib().fo_native_dot(u8ptr(row), typ, fptr(x), n if n is not None else x.size, C.byref(out))
    return rc, out.value


def dequant(row, typ, n):
    row = np.ascontiguousarray(row, np.uint8)
    out = np.zeros(n, np.float32)
    rc = lib().fo_dequant_row(u8ptr(row), typ, n, fptr(out))
    assert rc == OK
    return out


def fill_slice(buf, lay, expert, seed):
    """fill_slice of the native fixture recipe; returns the advanced seed."""
    s = C.c_uint32(seed)
    lib().fo_fill_slice(u8ptr(buf), C.byref(lay), expert, C.byref(s))
    return s.value


def lcg(seed):
    s = C.c_uint32(seed)
    v = lib().fo_lcg(C.byref(s))
    return v, s.value


def synth_slice(lay, seed, block, layer, expert):
    """Synthetic measurement slice (layer, expert) of ownership block `block`
    in the reference slice layout, as a new uint8 array."""
    n = lay.shared_slice if expert == 512 else lay.slice
    out = np.zeros(n, np.uint8)
    lib().fo_synth_slice(u8ptr(out), C.byref(lay), seed, block, layer, expert)
    return out


def synth_scale(h):
    return lib().fo_synth_scale(h)
