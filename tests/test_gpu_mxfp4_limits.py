"""MXFP4 blocks at the top of the E8M0 range, through run() against the
oracle's restatement of ref (backends/ref.c:57-98, fr_native_dot of
src/native.c:7-37, which decodes w = 2^(e-127) * code in fp32).

A code of magnitude >= 2 at e = 254, or >= 4 at e = 253, decodes to an
infinite weight: run() must return FR_NUMERIC with y untouched, whichever
kernel takes the request and even for a routed expert whose gate is 0
(src/backend.h:58-59). Codes of magnitude <= 1.5 at e = 254 decode to finite
weights: at gate 0 the expert adds nothing and run() succeeds, as ref does.
Every arithmetic follows the rule: F32 (decode and layer kernels), F64, the
ref-q8 arithmetic against the oracle's ref-q8, and - on the native units the
AVX2 backend takes - its q8_256 arithmetic.
"""
import ctypes as C

import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import oracle_request, slice_view, softmax_gates, sparse_unit
from test_gpu_parity import check_close

pytestmark = pytest.mark.gpu

H = 4096


@pytest.fixture(scope="module")
def eng():
    e = fa.Engine(0)
    yield e
    e.route(0)
    for b in range(20):
        e.release(b)


def run_into(y0, layer, experts, gates, x, mode):
    req, keep = fa.make_request(layer, experts, gates, x, mode)
    y = np.array(y0, np.float32, copy=True)
    rc = fa.lib().fr_hip_run(C.byref(req), fa.fptr(y))
    return rc, y


def set_block(view, off, e, mag_max):
    """Block at `off` (E8M0 byte, then 16 code bytes): exponent e, codes whose
    magnitude index (code & 7) is at most mag_max, the first one exactly it."""
    view[off] = e
    codes = view[off + 1:off + 17]
    lo, hi = codes & 15, codes >> 4
    lo = (lo & 8) | np.minimum(lo & 7, mag_max)
    hi = (hi & 8) | np.minimum(hi & 7, mag_max)
    lo[0] = mag_max
    view[off + 1:off + 17] = lo | (hi << 4)


@pytest.mark.parametrize("fmt,where", [(fa.FMT_NATIVE, "down"), (fa.FMT_MXFP4, "gate"), (fa.FMT_MXFP4, "down")])
def test_e8m0_overflow_matches_reference(eng, fmt, where):
    lay = oracle.layout(H, fmt)
    rng = np.random.default_rng(31 + fmt)
    experts = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
    seed = 515 + fmt
    units = []
    for b in range(2):
        u = sparse_unit(lay)
        for e in experts.ravel():
            slice_view(u, lay, 0, int(e))[:] = oracle.synth_slice(lay, seed, b, 0, int(e))
        units.append(u)
        assert eng.load_sparse(b, u, H, fmt, [(0, int(e)) for e in experts.ravel()]) == fa.OK
    try:
        gates = np.zeros((1, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 1)
        x = rng.standard_normal((1, H)).astype(np.float32)
        e3 = int(experts[0, 3])
        view = slice_view(units[1], lay, 0, e3)
        down = 2 * lay.proj
        off = down + 17 * 100 if where == "down" else 2176 * 5 + 17 * 9   # down row 100 / gate row 5 block 9
        saved = view[off:off + 17].copy()
        marker = np.full((1, H), -7.5, np.float32)
        cases = [(254, 4, False), (254, 6, False), (253, 6, False), (253, 7, True), (253, 5, False), (254, 3, True),
                 (254, 2, False)]
        for e, mag, zero_gate in cases:
            g = gates.copy()
            if zero_gate:
                g[0, 3] = 0.0
            set_block(view, off, e, mag)
            assert eng.refresh(1, units[1], 0, e3) == fa.OK
            req = oracle_request(0, experts, g, x)
            rc_ref, ref = oracle.ref_run(units + [None] * 18, fmt, False, req)
            rc_q8, ref_q8 = oracle.ref_run(units + [None] * 18, fmt, True, req)
            assert (rc_ref == 0) == (rc_q8 == 0), (e, mag)
            runs = [(0, fa.MODE_F32), (fa.ROUTE_NO_DECODE, fa.MODE_F32), (0, fa.MODE_F64), (0, fa.MODE_Q8),
                    (fa.ROUTE_NO_DECODE, fa.MODE_Q8)]
            if fmt == fa.FMT_NATIVE:
                runs.append((0, fa.MODE_Q8_256))
            for route, mode in runs:
                eng.route(route)
                print(f"fmt={fmt} {where} e={e} mag={mag} gate0={zero_gate} route={route} mode={mode} "
                      f"oracle rc={rc_ref}", flush=True)
                rc, y = run_into(marker, 0, experts, g, x, mode)
                eng.route(0)
                if rc_ref != 0:
                    assert rc == fa.NUMERIC, (e, mag, route, mode, rc)
                    assert np.array_equal(y, marker)
                elif mode == fa.MODE_Q8_256:
                    # The AVX2 backend's arithmetic, held to the tolerance the
                    # reference holds that backend to against ref.
                    assert rc == fa.OK, (e, mag, route, mode, rc)
                    rc2, err = oracle.compare(ref[0], y[0])
                    assert rc2 == 0 and err[0] <= 0.025 and err[1] <= 0.030, (e, mag, err)
                else:
                    assert rc == fa.OK, (e, mag, route, mode, rc)
                    check_close(ref_q8 if mode == fa.MODE_Q8 else ref, y, mode, (e, mag, route, mode))
        # The infinite-weight cases are the ones the reference rejects.
        view[off:off + 17] = saved
        assert eng.refresh(1, units[1], 0, e3) == fa.OK
        rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
    finally:
        eng.route(0)
        for b in range(2):
            eng.release(b)
