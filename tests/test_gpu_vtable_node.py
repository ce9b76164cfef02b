"""The "hip" fr_backend as a node drives it, on the GPU.

- bench: the vtable's bench hook runs the reference's own measurement
  (fr_bench_execute_backend -> fr_bench_measure_backend, src/bench.c:213-225,
  :285-443, compiled from the reference sources in oracle/_ref): 3 resident
  native blocks of fr_native_fill data, 512 warm-ups, the sampled run()
  timings per burst 1..4 in distinct and reused routing, then its cost-model
  fit (src/bench.c:163-198).
- the bench's close hook (src/bench.c:265-278) refuses while a block is loaded.
- run() from a thread other than load's, as the node's compute loop calls it
  (src/plane.c:38-58 against load on the session thread, src/node.c:573-584),
  on activations rounded to fp16 as the head ships them (src/plane.c:259-263,
  fr_half/fr_unhalf in src/wire.c:46-67).
"""
import ctypes as C
import threading

import numpy as np
import pytest

import oracle
import vtable as vt
from fixtures import native_fixture, oracle_request

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not vt.available(), reason="oracle/_ref or libfr_hip.so not built")]

NATIVE_BYTES = 48 * (512 * (2 * 32 * 10 * 144 + 2560 * 17) + 3 * 2560 * 34)   # src/native.h:9-15 at H=2560
PHASES, TOTAL = 6, 5   # FR_METAL_PHASES, FR_METAL_TOTAL (src/metal.h:9-10)


class CostModel(C.Structure):     # fr_costmodel (src/backend.h:30-35)
    _fields_ = [("burst_max", C.c_uint), ("t0_ns", C.c_double), ("bw_eff", C.c_double),
                ("ns", C.c_double * 8), ("bytes", C.c_uint64 * 8)]


class BenchReport(C.Structure):   # fr_bench_report (src/bench.h:13-20)
    _fields_ = [("cost", CostModel), ("blocks", C.c_uint), ("samples", C.c_uint), ("burst_max", C.c_uint),
                ("selected_burst", C.c_uint), ("workers", C.c_uint), ("prefetch", C.c_uint),
                ("percentile", (((C.c_double * 2) * PHASES) * 4) * 2),
                ("mean", (C.c_double * 4) * 2), ("sustained_ratio", C.c_double), ("burst_slope", C.c_double),
                ("elapsed", C.c_double), ("rss_start", C.c_uint64), ("rss_end", C.c_uint64),
                ("barriers", C.c_uint64), ("working_set", C.c_uint64), ("resident_bytes", C.c_uint64),
                ("hot_allocations", C.c_uint64)]


def reference():
    vt.library()
    ref = C.CDLL(vt.REF_LIB, mode=C.RTLD_GLOBAL)
    ref.fr_bench_configure.argtypes = [C.c_uint, C.c_void_p]
    ref.fr_bench_last.argtypes = [C.POINTER(BenchReport)]
    return ref


def close_hook():
    fn = vt.library().fr_hip_backend_close
    fn.restype = C.c_int
    return fn


def test_close_hook_refuses_a_loaded_block():
    unit = np.zeros(NATIVE_BYTES, np.uint8)
    b = vt.backend()
    assert b.load(0, unit.ctypes.data, unit.nbytes) == vt.OK
    try:
        assert close_hook()() == vt.STATE
    finally:
        assert b.unload(0) == vt.OK
    assert close_hook()() == vt.OK
    assert close_hook()() == vt.OK


@pytest.mark.timeout(600)
def test_reference_bench_through_the_vtable(tmp_path, monkeypatch):
    """fr_hip.bench(4) with the reference's default 3 blocks: every sampled
    run() returns FR_OK, the percentiles are ordered and the fitted cost model
    is finite and positive. The p50/p99 the reference's timer took around
    run() are printed."""
    monkeypatch.chdir(tmp_path)        # the bench writes runs/bench-*.csv
    ref = reference()
    assert ref.fr_bench_configure(3, None) == vt.OK
    cost = CostModel()
    print("reference bench through fr_hip: 3 native blocks, bursts 1..4, 30 s sustained", flush=True)
    assert vt.backend().bench(4, C.addressof(cost)) == vt.OK
    rep = BenchReport()
    assert ref.fr_bench_last(C.byref(rep)) == vt.OK
    assert rep.blocks == 3 and rep.burst_max == 4 and rep.hot_allocations == 0
    assert np.isfinite(cost.bw_eff) and cost.bw_eff > 0 and cost.t0_ns >= 0
    for mode in range(2):
        for b in range(4):
            p50, p99 = rep.percentile[mode][b][TOTAL][0], rep.percentile[mode][b][TOTAL][1]
            assert 0 < p50 <= p99, (mode, b, p50, p99)
            print(f"{'reused' if mode else 'distinct'} burst {b + 1}: run() p50 {p50 / 1e3:.1f} us "
                  f"p99 {p99 / 1e3:.1f} us", flush=True)
    print(f"cost model: t0 {cost.t0_ns / 1e3:.1f} us, bw_eff {cost.bw_eff / 1e9:.1f} GB/s", flush=True)
    assert list((tmp_path / "runs").glob("bench-hip-*.csv"))
    assert close_hook()() == vt.OK


def test_run_on_a_compute_thread_with_fp16_activations():
    lay = oracle.layout(2560, oracle.FMT_NATIVE)
    data, gates, _ = native_fixture(lay)
    # Activations spanning normal and subnormal fp16, rounded to fp16 and back
    # (numpy's cast rounds to nearest even, as fr_half does for finite values
    # in range), signed zeros included.
    rng = np.random.default_rng(23)
    x = rng.standard_normal((8, 2560)) * np.exp2(rng.integers(-27, 6, (8, 2560)))
    x[:, :4] = [0.0, -0.0, 2.0 ** -24, -(2.0 ** -25) * 3]
    half = x.astype(np.float16)
    assert np.isfinite(half).all()
    xr = half.astype(np.float32)
    assert (xr != x.astype(np.float32)).any()
    experts = np.array([[(e + 7 * t) % 80 for e in range(10)] for t in range(8)], np.uint16)

    req = vt.Req()
    req.layer, req.burst = 47, 8
    np.frombuffer(req.expert, np.uint16).reshape(8, 10)[:] = experts
    np.frombuffer(req.gate, np.float32).reshape(8, 11)[:] = gates
    np.frombuffer(req.x, np.float32).reshape(8, 2560)[:] = xr

    b = vt.backend()
    assert b.load(19, data.ctypes.data, data.nbytes) == vt.OK   # loaded on this thread
    try:
        here = vt.Part()
        assert b.run(C.byref(req), C.byref(here)) == vt.OK
        there, rc = vt.Part(), []
        worker = threading.Thread(target=lambda: rc.append(b.run(C.byref(req), C.byref(there))))
        worker.start()
        worker.join(60)
        assert not worker.is_alive() and rc == [vt.OK]
    finally:
        assert b.unload(19) == vt.OK
    y_here = np.frombuffer(here.y, np.float32).reshape(8, 2560)
    y_there = np.frombuffer(there.y, np.float32).reshape(8, 2560)
    assert np.array_equal(y_here.view(np.uint32), y_there.view(np.uint32))
    blocks = [None] * 20
    blocks[19] = data
    rc, expect = oracle.ref_run(blocks, oracle.FMT_NATIVE, False, oracle_request(47, experts, gates, xr))
    assert rc == 0
    for t in range(8):
        rc, err = oracle.compare(expect[t], y_there[t])
        assert rc == 0 and err[0] <= 1e-5 and err[1] <= 1e-3, (t, err)


def test_hbm_capacity_for_the_node_share():
    """fr_hip_capacity: units that fit the device's free HBM plus those the
    engine holds, less the reserve, capped at 20 (the count a node would give
    selection_capacity, src/selection.c:227-244, for this backend)."""
    import fronk_amd as fa
    eng = fa.Engine(0)
    unit = fa.unit_bytes(2560, fa.FMT_NATIVE)
    for b in range(20):
        eng.release(b)
    rc, free, n = fa.capacity(2560, fa.FMT_NATIVE)
    assert rc == fa.OK and free > 0
    assert n == min(20, free // unit)
    rc, _, none = fa.capacity(2560, fa.FMT_NATIVE, reserve=free)
    assert rc == fa.OK and none == 0
    assert eng.reserve(3, 2560, fa.FMT_NATIVE) == fa.OK
    try:
        rc, free_after, n_after = fa.capacity(2560, fa.FMT_NATIVE)
        assert rc == fa.OK
        # the unit sits in HBM (the driver's free figure moves in its own
        # granules, and memory freed earlier may come back meanwhile) ...
        assert abs((free - free_after) - unit) <= 64 << 20
        assert n_after == min(20, (free_after + unit) // unit)   # ... and still counts
        rc, _, k = fa.capacity(2560, fa.FMT_NATIVE, reserve=free_after)
        assert rc == fa.OK and k == 1
    finally:
        assert eng.release(3) == fa.OK
