"""Device-side synthetic measurement data (fr_hip_synthetic).

The device generator must write, re-tiled, exactly the bytes that the oracle's
generator (fo_synth_slice) writes in the reference slice layout: a block filled
on the device is compared byte for byte with a block whose slices were
generated on the host and uploaded through the ordinary load path. Then a full
20-block layer share filled on the device is run end to end against the oracle
on the host-generated copy of the routed slices.
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import oracle_request, slice_view, softmax_gates, sparse_unit, zipf_routes
from test_gpu_parity import check_close

pytestmark = pytest.mark.gpu

H = 4096


@pytest.fixture(scope="module")
def eng():
    e = fa.Engine(0)
    yield e
    for b in range(20):
        e.release(b)


@pytest.mark.parametrize("fmt", [fa.FMT_Q4KT, fa.FMT_NATIVE, fa.FMT_Q8, fa.FMT_MXFP4])
def test_device_generator_matches_oracle_bytes(eng, fmt):
    lay = oracle.layout(H, fmt)
    seed = 0x5EED + fmt
    print(f"synthetic bytes fmt={fmt}", flush=True)
    assert eng.synthetic(6, H, fmt, 2, seed) == fa.OK
    assert eng.reserve(7, H, fmt) == fa.OK
    try:
        unit = sparse_unit(lay)
        for layer, e in [(0, 0), (1, 511), (1, 512), (0, 137)]:
            view = slice_view(unit, lay, layer, e)
            view[:] = oracle.synth_slice(lay, seed, 6, layer, e)
            assert eng.refresh(7, unit, layer, e) == fa.OK
            off = oracle.slice_offset(lay, layer, e)
            a = eng.read(6, off, view.size)
            b = eng.read(7, off, view.size)
            assert np.array_equal(a, b), (fmt, layer, e, int(np.argmax(a != b)))
        # Layers beyond the generated ones are not resident.
        assert eng.refresh(6, unit, 2, 0) == fa.INVALID
    finally:
        assert eng.release(6) == fa.OK
        assert eng.release(7) == fa.OK


def test_absent_layer_is_state(eng):
    assert eng.synthetic(2, H, fa.FMT_Q4KT, 1, 1) == fa.OK
    try:
        x = np.zeros((1, H), np.float32)
        gates = np.zeros((1, 11), np.float32)
        gates[0, :10] = 0.1
        rc, _ = eng.run(1, np.arange(10).reshape(1, 10), gates, x)
        assert rc == fa.STATE
        rc, _ = eng.run(0, np.arange(10).reshape(1, 10), gates, x)
        assert rc == fa.OK
    finally:
        eng.release(2)


@pytest.mark.parametrize("fmt", [fa.FMT_Q4KT, fa.FMT_MXFP4])
def test_layer_share_on_synthetic_blocks(eng, fmt):
    """The measurement workload itself: 20 owned slices of every expert, T=1
    with 10 uniform experts and a Zipf T=4 burst, against the oracle on the
    host-generated copies of the routed slices."""
    lay = oracle.layout(H, fmt)
    seed = 77 + fmt
    rng = np.random.default_rng(fmt)
    for b in range(20):
        assert eng.synthetic(b, H, fmt, 1, seed) == fa.OK
    try:
        cases = [rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10), zipf_routes(rng, 4)]
        used = sorted(set(np.concatenate([c.ravel() for c in cases]).tolist()))
        units = []
        for b in range(20):
            u = sparse_unit(lay)
            for e in used:
                slice_view(u, lay, 0, e)[:] = oracle.synth_slice(lay, seed, b, 0, e)
            units.append(u)
        for experts in cases:
            T = experts.shape[0]
            gates = np.zeros((T, 11), np.float32)
            gates[:, :10] = softmax_gates(rng, T)
            x = rng.standard_normal((T, H)).astype(np.float32)
            for mode in (fa.MODE_F32, fa.MODE_Q8):
                print(f"layer share fmt={fmt} T={T} mode={mode}", flush=True)
                rc, y = eng.run(0, experts, gates, x, mode)
                assert rc == fa.OK
                req = oracle_request(0, experts, gates, x)
                rc, ref = oracle.ref_run(units, fmt, mode == fa.MODE_Q8, req)
                assert rc == 0
                check_close(ref, y, mode, (fmt, T, mode))
    finally:
        for b in range(20):
            eng.release(b)


def plan_kind(eng, layer, experts, gates, x):
    plan, grid = eng.plan(layer, experts, gates, x, fa.MODE_F32)
    return int(np.frombuffer(plan[64:68].tobytes(), np.uint32)[0]), grid


@pytest.mark.parametrize("hidden", [4096, 2560])
def test_decode_kernel_and_layer_kernel_agree_with_oracle(eng, hidden, monkeypatch):
    """Single-token all-Q4_K requests run on the decode kernel (tasks of 8
    neurons, no h exchange); the same request forced onto the two-phase
    layer kernel must match the oracle as well."""
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    seed = 4242 + hidden
    rng = np.random.default_rng(hidden)
    for b in range(20):
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, seed) == fa.OK
    try:
        experts = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
        units = []
        for b in range(20):
            u = sparse_unit(lay)
            for e in experts.ravel():
                slice_view(u, lay, 0, int(e))[:] = oracle.synth_slice(lay, seed, b, 0, int(e))
            units.append(u)
        gates = np.zeros((1, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 1)
        x = rng.standard_normal((1, hidden)).astype(np.float32)
        req = oracle_request(0, experts, gates, x)
        rc, ref = oracle.ref_run(units, fa.FMT_Q4KT, False, req)
        assert rc == 0
        kind, grid = plan_kind(eng, 0, experts, gates, x)
        assert kind == 1 and 0 < grid <= 256, (kind, grid)
        print(f"decode kernel hidden={hidden} grid={grid}", flush=True)
        rc, y_dec = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
        check_close(ref, y_dec, fa.MODE_F32, ("decode", hidden))
        rc, again = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert np.array_equal(y_dec.view(np.uint32), again.view(np.uint32))
        monkeypatch.setenv("FRONK_HIP_NO_DECODE", "1")
        kind, grid = plan_kind(eng, 0, experts, gates, x)
        assert kind == 0
        print(f"layer kernel hidden={hidden} grid={grid}", flush=True)
        rc, y_lay = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
        check_close(ref, y_lay, fa.MODE_F32, ("layer", hidden))
    finally:
        for b in range(20):
            eng.release(b)


@pytest.mark.parametrize("burst", [2, 4, 8])
def test_decode_burst_rows_equal_single_token_runs(eng, burst):
    """Bursts of all-Q4_K routed requests also run on the decode kernel: each
    (token, pair) is a unit with its own partial, and a token's units are
    summed in the single-token order. Every row must match the oracle and be
    bit-identical to the same token run alone (the batching property of
    src/native.c:94-117, which the reference checks with memcmp)."""
    hidden, seed = 4096, 777
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    rng = np.random.default_rng(burst)
    for b in range(20):
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, seed) == fa.OK
    try:
        experts = zipf_routes(rng, burst)
        gates = np.zeros((burst, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, burst)
        x = rng.standard_normal((burst, hidden)).astype(np.float32)
        kind, grid = plan_kind(eng, 0, experts, gates, x)
        assert kind == 1 and 0 < grid <= 256, (kind, grid)
        print(f"decode burst={burst} grid={grid}", flush=True)
        rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
        units = []
        for b in range(20):
            u = sparse_unit(lay)
            for e in set(int(v) for v in experts.ravel()):
                slice_view(u, lay, 0, e)[:] = oracle.synth_slice(lay, seed, b, 0, e)
            units.append(u)
        rc, ref = oracle.ref_run(units, fa.FMT_Q4KT, False, oracle_request(0, experts, gates, x))
        assert rc == 0
        check_close(ref, y, fa.MODE_F32, ("burst", burst))
        for t in range(burst):
            rc, y1 = eng.run(0, experts[t:t + 1], gates[t:t + 1], x[t:t + 1], fa.MODE_F32)
            assert rc == fa.OK
            assert np.array_equal(y1[0].view(np.uint32), y[t].view(np.uint32)), f"token {t} differs from its T=1 run"
    finally:
        for b in range(20):
            eng.release(b)
