"""fronk_amd: MI355X-native expert neuron-slice backend for Fronk.

Python is test and benchmark plumbing over the C ABI of libfronk_hip.so
(include/fronk_hip.h); the compute path is HIP. Importing works without a GPU;
every call that needs the library raises if libfronk_hip.so was not built.
"""
import ctypes as C
import os

import numpy as np

from . import build as _build

OK, INVALID, STATE, NUMERIC, IO, UNSUPPORTED = 0, -1, -2, -3, -4, -5
FMT_LEGACY, FMT_NATIVE, FMT_Q4KT, FMT_Q8, FMT_MXFP4 = 0, 1, 2, 3, 4
MODE_F32, MODE_F64, MODE_Q8, MODE_Q8_256 = 0, 1, 2, 3
Q4_0, Q8_0, Q4_K, MXFP4 = 2, 8, 12, 39
MAX_BURST, MAX_HIDDEN, BLOCKS = 8, 4096, 20
ROUTE_NO_DECODE, ROUTE_NO_BURST, ROUTE_BURST = 2, 4, 8
# Plan kinds (the kernel a plan runs), plan header word 16.
KIND_LAYER, KIND_DECODE, KIND_DECODE_ROWS, KIND_DECODE_SPLIT, KIND_DECODE_BURST = 0, 1, 2, 3, 4
# fr_hip_phase_get's phases, in order.
PHASES = ("plan", "enqueue", "wait", "gpu", "overhead", "total")

LIB_PATH = _build.HIP_LIB


class Request(C.Structure):
    _fields_ = [("layer", C.c_uint), ("burst", C.c_uint), ("hidden", C.c_uint), ("mode", C.c_uint),
                ("expert", C.POINTER(C.c_uint16)), ("gate", C.POINTER(C.c_float)),
                ("x", C.POINTER(C.c_float))]


class Batch(C.Structure):
    _fields_ = [("layer", C.c_uint), ("tokens", C.c_uint), ("hidden", C.c_uint), ("mode", C.c_uint),
                ("expert", C.POINTER(C.c_uint16)), ("gate", C.POINTER(C.c_float)),
                ("x", C.POINTER(C.c_float))]


class Sample(C.Structure):
    _fields_ = [("runs", C.c_uint64), ("weight_bytes", C.c_uint64), ("hot_allocations", C.c_uint64),
                ("blocks", C.c_uint), ("unique_experts", C.c_uint), ("pairs", C.c_uint), ("grid", C.c_uint),
                ("last_kernel_ns", C.c_double)]


# Every symbol include/fronk_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "fr_hip_open": (C.c_int, [C.c_int]),
    "fr_hip_close": (C.c_int, []),
    "fr_hip_probe": (C.c_int, [C.c_int, C.c_char_p, C.c_size_t]),
    "fr_hip_upload": (C.c_int, [C.c_uint, C.c_void_p, C.c_uint64, C.c_uint, C.c_uint]),
    "fr_hip_reserve": (C.c_int, [C.c_uint, C.c_uint, C.c_uint]),
    "fr_hip_refresh": (C.c_int, [C.c_uint, C.c_void_p, C.c_uint, C.c_uint]),
    "fr_hip_synthetic": (C.c_int, [C.c_uint, C.c_uint, C.c_uint, C.c_uint, C.c_uint64]),
    "fr_hip_release": (C.c_int, [C.c_uint]),
    "fr_hip_unit_bytes": (C.c_uint64, [C.c_uint, C.c_uint]),
    "fr_hip_capacity": (C.c_int, [C.c_int, C.c_uint, C.c_uint, C.c_uint64, C.POINTER(C.c_uint64),
                                  C.POINTER(C.c_uint)]),
    "fr_hip_run": (C.c_int, [C.POINTER(Request), C.POINTER(C.c_float)]),
    "fr_hip_plan_bytes": (C.c_size_t, [C.c_uint, C.c_uint]),
    "fr_hip_plan": (C.c_int, [C.POINTER(Request), C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t),
                              C.POINTER(C.c_uint)]),
    "fr_hip_launch": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "fr_hip_last_output": (C.c_int, [C.c_void_p, C.POINTER(C.c_float), C.c_size_t, C.POINTER(C.c_uint)]),
    "fr_hip_launch_static": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "fr_hip_sample_get": (C.c_int, [C.POINTER(Sample)]),
    "fr_hip_phase_events": (C.c_int, [C.c_int]),
    "fr_hip_phase_get": (C.c_int, [C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    "fr_hip_route": (C.c_int, [C.c_uint]),
    "fr_hip_stream_probe": (C.c_int, [C.c_void_p, C.c_uint, C.c_uint, C.c_uint, C.c_void_p, C.c_void_p]),
    "fr_hip_run_batch": (C.c_int, [C.POINTER(Batch), C.POINTER(C.c_float)]),
    "fr_hip_batch_plan_bytes": (C.c_size_t, [C.c_uint, C.c_uint]),
    "fr_hip_batch_plan": (C.c_int, [C.POINTER(Batch), C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "fr_hip_batch_launch": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "fr_hip_batch_output": (C.c_int, [C.c_void_p, C.POINTER(C.c_float), C.c_size_t, C.POINTER(C.c_uint)]),
    "fr_hip_timing": (C.c_int, [C.c_uint]),
    "fr_hip_timing_read": (C.c_int, [C.POINTER(C.c_double), C.POINTER(C.c_double), C.POINTER(C.c_uint)]),
    "fr_hip_debug_dequant": (C.c_int, [C.c_uint, C.c_void_p, C.c_uint, C.POINTER(C.c_float)]),
    "fr_hip_debug_dequant_down": (C.c_int, [C.c_uint, C.c_void_p, C.c_uint, C.POINTER(C.c_float)]),
    "fr_hip_debug_quantize": (C.c_int, [C.POINTER(C.c_float), C.c_uint, C.POINTER(C.c_float)]),
    "fr_hip_debug_quantize64": (C.c_int, [C.POINTER(C.c_float), C.c_uint, C.POINTER(C.c_float)]),
    "fr_hip_debug_quantize8": (C.c_int, [C.POINTER(C.c_float), C.c_uint, C.c_uint, C.POINTER(C.c_int8),
                                         C.POINTER(C.c_float), C.POINTER(C.c_int16)]),
    "fr_hip_debug_quantize_staged": (C.c_int, [C.POINTER(C.c_float), C.c_uint, C.c_uint, C.POINTER(C.c_float),
                                               C.POINTER(C.c_double)]),
    "fr_hip_debug_partials": (C.c_int, [C.c_uint, C.c_uint, C.POINTER(C.c_float)]),
    "fr_hip_debug_read": (C.c_int, [C.c_uint, C.c_uint64, C.c_void_p, C.c_uint64]),
}

_lib = None


def lib():
    """The loaded libfronk_hip.so. Raises if it was not built: there is no
    fallback path."""
    global _lib
    if _lib is None:
        # The library runs on the HIP runtime it finds (its runpath: the
        # system ROCm), like any C consumer of the backend. A process that
        # also uses torch, which carries its own runtime of the same soname,
        # imports torch before this call, so that one runtime serves both
        # (bench.py and the test suite do).
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (hipcc, gfx950)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def fptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def check(rc, what):
    if rc != OK:
        raise RuntimeError(f"{what} failed with {rc}")


def unit_bytes(hidden, fmt):
    return lib().fr_hip_unit_bytes(hidden, fmt)


def capacity(hidden, fmt, reserve=0, device=0):
    """(rc, free HBM bytes, units of (hidden, fmt) the device holds)."""
    free, blocks = C.c_uint64(0), C.c_uint(0)
    rc = lib().fr_hip_capacity(device, hidden, fmt, reserve, C.byref(free), C.byref(blocks))
    return rc, free.value, blocks.value


def make_request(layer, experts, gates, x, mode=MODE_F32):
    """Build a Request over numpy arrays; returns (request, keepalive)."""
    experts = np.ascontiguousarray(experts, np.uint16).reshape(-1, 10)
    gates = np.ascontiguousarray(gates, np.float32).reshape(-1, 11)
    x = np.ascontiguousarray(x, np.float32)
    burst, hidden = x.shape
    req = Request(layer, burst, hidden, mode, experts.ctypes.data_as(C.POINTER(C.c_uint16)),
                  fptr(gates), fptr(x))
    return req, (experts, gates, x)


def make_batch(layer, experts, gates, x, mode=MODE_F32):
    """Build a Batch over numpy arrays; returns (batch, keepalive)."""
    experts = np.ascontiguousarray(experts, np.uint16).reshape(-1, 10)
    gates = np.ascontiguousarray(gates, np.float32).reshape(-1, 11)
    x = np.ascontiguousarray(x, np.float32)
    tokens, hidden = x.shape
    req = Batch(layer, tokens, hidden, mode, experts.ctypes.data_as(C.POINTER(C.c_uint16)), fptr(gates), fptr(x))
    return req, (experts, gates, x)


class Engine:
    """Thin owner of the process-wide device engine (one GPU)."""

    def __init__(self, device=0):
        self.device = device
        check(lib().fr_hip_open(device), "fr_hip_open")

    def close(self):
        return lib().fr_hip_close()

    def upload(self, block, unit, hidden, fmt):
        unit = np.asarray(unit)
        return lib().fr_hip_upload(block, unit.ctypes.data, unit.nbytes, hidden, fmt)

    def reserve(self, block, hidden, fmt):
        return lib().fr_hip_reserve(block, hidden, fmt)

    def load_sparse(self, block, unit, hidden, fmt, slices):
        """Reserve a zeroed device unit and copy only the (layer, expert) slices
        listed: equivalent to a full upload of a sparse unit."""
        rc = self.reserve(block, hidden, fmt)
        if rc != OK:
            return rc
        for layer, expert in slices:
            rc = self.refresh(block, unit, layer, expert)
            if rc != OK:
                return rc
        return OK

    def refresh(self, block, unit, layer, expert):
        return lib().fr_hip_refresh(block, np.asarray(unit).ctypes.data, layer, expert)

    def synthetic(self, block, hidden, fmt, layers, seed):
        return lib().fr_hip_synthetic(block, hidden, fmt, layers, seed)

    def read(self, block, offset, length):
        out = np.zeros(length, np.uint8)
        check(lib().fr_hip_debug_read(block, offset, out.ctypes.data, length), "fr_hip_debug_read")
        return out

    def release(self, block):
        return lib().fr_hip_release(block)

    def run(self, layer, experts, gates, x, mode=MODE_F32):
        req, keep = make_request(layer, experts, gates, x, mode)
        y = np.zeros((req.burst, req.hidden), np.float32)
        rc = lib().fr_hip_run(C.byref(req), fptr(y))
        return rc, y

    def plan(self, layer, experts, gates, x, mode=MODE_F32):
        req, keep = make_request(layer, experts, gates, x, mode)
        cap = lib().fr_hip_plan_bytes(req.burst, req.hidden)
        buf = np.zeros(cap, np.uint8)
        used, grid = C.c_size_t(), C.c_uint()
        rc = lib().fr_hip_plan(C.byref(req), buf.ctypes.data, cap, C.byref(used), C.byref(grid))
        check(rc, "fr_hip_plan")
        return buf[:used.value].copy(), grid.value

    def run_batch(self, layer, experts, gates, x, mode=MODE_F32):
        """fr_hip_run_batch: a prefill chunk of any number of tokens."""
        req, keep = make_batch(layer, experts, gates, x, mode)
        y = np.zeros((req.tokens, req.hidden), np.float32)
        rc = lib().fr_hip_run_batch(C.byref(req), fptr(y))
        return rc, y

    def batch_plan(self, layer, experts, gates, x, mode=MODE_F32):
        req, keep = make_batch(layer, experts, gates, x, mode)
        cap = lib().fr_hip_batch_plan_bytes(req.tokens, req.hidden)
        buf = np.zeros(cap, np.uint8)
        used = C.c_size_t()
        rc = lib().fr_hip_batch_plan(C.byref(req), buf.ctypes.data, cap, C.byref(used))
        check(rc, "fr_hip_batch_plan")
        return buf[:used.value].copy()

    def route(self, flags):
        """fr_hip_route: send requests past the decode kernels to layer_kernel
        (ROUTE_NO_DECODE) for plans built from now on; 0 restores the default."""
        check(lib().fr_hip_route(flags), "fr_hip_route")

    def sample(self):
        s = Sample()
        lib().fr_hip_sample_get(C.byref(s))
        return s

    def phase_events(self, on):
        """fr_hip_phase_events: time run()'s launches with HIP events (the
        GPU phase) from now on, or stop."""
        check(lib().fr_hip_phase_events(1 if on else 0), "fr_hip_phase_events")

    def phases(self):
        """fr_hip_phase_get: ({phase: ns} of the last run() call, calls sampled)."""
        ns = (C.c_double * len(PHASES))()
        runs = C.c_uint64()
        check(lib().fr_hip_phase_get(ns, C.byref(runs)), "fr_hip_phase_get")
        return dict(zip(PHASES, list(ns))), runs.value

    def dequant(self, typ, row, n):
        out = np.zeros(n, np.float32)
        rc = lib().fr_hip_debug_dequant(typ, np.ascontiguousarray(row, np.uint8).ctypes.data, n, fptr(out))
        return rc, out

    def dequant_down(self, fmt, down, hidden):
        out = np.zeros((hidden, 32), np.float32)
        rc = lib().fr_hip_debug_dequant_down(fmt, np.ascontiguousarray(down, np.uint8).ctypes.data, hidden,
                                             fptr(out))
        return rc, out

    def quantize(self, x, regs=False):
        """fr_q8_activation on the device: the group form, or with `regs` the
        register form of the single-token Q8 path."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        fn = lib().fr_hip_debug_quantize64 if regs else lib().fr_hip_debug_quantize
        rc = fn(fptr(x), x.size, fptr(out))
        return rc, out

    def partials(self, first, count):
        """fr_hip_debug_partials: items [first, first + count) of the last F32
        decode launch, [count][4096] in output order."""
        out = np.zeros((count, MAX_HIDDEN), np.float32)
        check(lib().fr_hip_debug_partials(first, count, fptr(out)), "fr_hip_debug_partials")
        return out

    def quantize_staged(self, x, form):
        """fr_q8_activation through the ref-q8 decode kernels' own staging
        (form 0: decode_q8_kernel, 1: decode_rows_q8_kernel, 2: their h
        quantizer on 32 values): (rc, rebuilt values, exact sub-block sums)."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        sums = np.zeros(max(x.size // 32, 1), np.float64)
        rc = lib().fr_hip_debug_quantize_staged(fptr(x), x.size, form, fptr(out),
                                                sums.ctypes.data_as(C.POINTER(C.c_double)))
        return rc, out, sums

    def quantize8(self, x, group):
        """The q8_256 quantizers on the device (the AVX2 backend's quantize8):
        (rc, codes, d per group, int16 sums per 32 or None for group 32)."""
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(x.size, np.int8)
        d = np.zeros(max(x.size // group, 1), np.float32)
        s = np.zeros(max(x.size // 32, 1), np.int16)
        rc = lib().fr_hip_debug_quantize8(fptr(x), x.size, group, q.ctypes.data_as(C.POINTER(C.c_int8)), fptr(d),
                                          s.ctypes.data_as(C.POINTER(C.c_int16)))
        return rc, q, d, (s if group == 256 else None)
