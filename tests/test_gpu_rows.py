"""decode_rows_kernel: single-token and burst requests whose units are all
row-format pairs - the reference's native units (Q4_K gate/up, MXFP4 down,
src/native.h:9-21), all-Q8_0 (also the shared expert), all-MXFP4 - run one
workgroup per (token, pair) unit and the fixed-order decode_reduce.

Each request is checked against the oracle's restatement of backends/ref.c
(F32 tolerance: rel. L2 1e-5, normalized max-abs 1e-3, as fr_compare reads
it), against the same request forced onto the two-phase layer kernel, run to
run bit for bit, and - for bursts - row by row bit for bit against the same
token run alone (the batching property of src/native.c:94-117).
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import oracle_request, slice_view, softmax_gates, sparse_unit, zipf_routes
from test_gpu_parity import check_close

pytestmark = pytest.mark.gpu

KIND_DECODE_ROWS = 2


@pytest.fixture(scope="module")
def eng():
    e = fa.Engine(0)
    yield e
    for b in range(20):
        e.release(b)


def plan_kind(eng, layer, experts, gates, x):
    plan, grid = eng.plan(layer, experts, gates, x, fa.MODE_F32)
    return int(np.frombuffer(plan[64:68].tobytes(), np.uint32)[0]), grid


def host_units(lay, seed, experts, shared):
    used = set(int(e) for e in np.asarray(experts).ravel()) | ({512} if shared else set())
    units = []
    for b in range(20):
        u = sparse_unit(lay)
        for e in used:
            slice_view(u, lay, 0, e)[:] = oracle.synth_slice(lay, seed, b, 0, e)
        units.append(u)
    return units


@pytest.mark.parametrize("fmt,hidden", [(fa.FMT_NATIVE, 4096), (fa.FMT_NATIVE, 2560), (fa.FMT_Q8, 4096),
                                        (fa.FMT_MXFP4, 4096)])
@pytest.mark.parametrize("shared", [False, True])
def test_rows_kernel_agrees_with_oracle_and_layer_kernel(eng, fmt, hidden, shared):
    lay = oracle.layout(hidden, fmt)
    seed = 9100 + 10 * fmt + hidden
    rng = np.random.default_rng(seed)
    for b in range(20):
        assert eng.synthetic(b, hidden, fmt, 1, seed) == fa.OK
    try:
        experts = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
        gates = np.zeros((1, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 1)
        gates[:, 10] = 0.5 if shared else 0.0
        x = rng.standard_normal((1, hidden)).astype(np.float32)
        rc, ref = oracle.ref_run(host_units(lay, seed, experts, shared), fmt, False,
                                 oracle_request(0, experts, gates, x))
        assert rc == 0
        kind, grid = plan_kind(eng, 0, experts, gates, x)
        assert kind == KIND_DECODE_ROWS and 0 < grid <= 256, (kind, grid)
        print(f"rows kernel fmt={fmt} hidden={hidden} shared={shared} grid={grid}", flush=True)
        rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
        check_close(ref, y, fa.MODE_F32, ("rows", fmt, hidden, shared))
        rc, again = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
        assert np.array_equal(y.view(np.uint32), again.view(np.uint32))
        eng.route(fa.ROUTE_NO_DECODE)
        kind, _ = plan_kind(eng, 0, experts, gates, x)
        assert kind == 0
        print(f"layer kernel fmt={fmt} hidden={hidden} shared={shared}", flush=True)
        rc, y_lay = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
        check_close(ref, y_lay, fa.MODE_F32, ("layer", fmt, hidden, shared))
    finally:
        eng.route(0)
        for b in range(20):
            eng.release(b)


@pytest.mark.parametrize("fmt,burst,shared_tokens", [(fa.FMT_NATIVE, 3, (1,)), (fa.FMT_Q8, 4, ()),
                                                     (fa.FMT_NATIVE, 8, (0,))])
def test_rows_burst_rows_equal_single_token_runs(eng, fmt, burst, shared_tokens):
    """The last case: 8 tokens x 10 experts x 20 blocks plus one token's
    shared expert on 20 blocks = 1,620 units."""
    hidden, seed = 4096, 4321 + fmt
    lay = oracle.layout(hidden, fmt)
    rng = np.random.default_rng(burst)
    for b in range(20):
        assert eng.synthetic(b, hidden, fmt, 1, seed) == fa.OK
    try:
        experts = zipf_routes(rng, burst)
        gates = np.zeros((burst, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, burst)
        for t in shared_tokens:
            gates[t, 10] = 0.25
        x = rng.standard_normal((burst, hidden)).astype(np.float32)
        kind, grid = plan_kind(eng, 0, experts, gates, x)
        assert kind == KIND_DECODE_ROWS and 0 < grid <= 256, (kind, grid)
        print(f"rows burst fmt={fmt} burst={burst} grid={grid}", flush=True)
        rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
        units = host_units(lay, seed, experts, bool(shared_tokens))
        rc, ref = oracle.ref_run(units, fmt, False, oracle_request(0, experts, gates, x))
        assert rc == 0
        check_close(ref, y, fa.MODE_F32, ("rows burst", fmt, burst))
        for t in range(burst):
            rc, y1 = eng.run(0, experts[t:t + 1], gates[t:t + 1], x[t:t + 1], fa.MODE_F32)
            assert rc == fa.OK
            assert np.array_equal(y1[0].view(np.uint32), y[t].view(np.uint32)), f"token {t} differs from its T=1 run"
    finally:
        for b in range(20):
            eng.release(b)


@pytest.mark.parametrize("fmt,modes", [(fa.FMT_Q8, (fa.MODE_F32, fa.MODE_Q8)),
                                       (fa.FMT_NATIVE, (fa.MODE_F32, fa.MODE_Q8_256))])
def test_rows_full_burst_with_shared_expert_stays_on_decode(eng, fmt, modes):
    """Eight tokens that all use the shared expert are the largest decode
    request: 8 x (10 + 1) x 20 = 1,760 units. It runs on the row-format decode
    kernel in every mode (F32 against the oracle, Q8 and the q8_256 arithmetic
    of the AVX2 backend included), and every row equals its token run alone
    bit for bit."""
    hidden, seed = 4096, 55 + fmt
    lay = oracle.layout(hidden, fmt)
    for b in range(20):
        assert eng.synthetic(b, hidden, fmt, 1, seed) == fa.OK
    try:
        rng = np.random.default_rng(8)
        experts = zipf_routes(rng, 8)
        gates = np.zeros((8, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 8)
        gates[:, 10] = 0.125
        x = rng.standard_normal((8, hidden)).astype(np.float32)
        for mode in modes:
            plan, grid = eng.plan(0, experts, gates, x, mode)
            head = np.frombuffer(plan[:80].tobytes(), np.uint32)
            assert int(head[16]) == KIND_DECODE_ROWS and int(head[3]) == 1760, (mode, head[16], head[3])
            print(f"full burst with shared expert fmt={fmt} mode={mode} grid={grid}", flush=True)
            rc, y = eng.run(0, experts, gates, x, mode)
            assert rc == fa.OK, (mode, rc)
            if mode == fa.MODE_F32:
                units = host_units(lay, seed, experts, True)
                rc, ref = oracle.ref_run(units, fmt, False, oracle_request(0, experts, gates, x))
                assert rc == 0
                check_close(ref, y, fa.MODE_F32, ("full burst", fmt))
            for t in range(8):
                rc, y1 = eng.run(0, experts[t:t + 1], gates[t:t + 1], x[t:t + 1], mode)
                assert rc == fa.OK
                assert np.array_equal(y1[0].view(np.uint32), y[t].view(np.uint32)), (mode, t)
    finally:
        for b in range(20):
            eng.release(b)


def q8_plan(eng, experts, gates, x):
    plan, grid = eng.plan(0, experts, gates, x, fa.MODE_Q8)
    head = np.frombuffer(plan[:80].tobytes(), np.uint32)
    return int(head[16]), int(head[2]), grid   # kind, mode, grid


@pytest.mark.parametrize("fmt,hidden,burst,shared_tokens", [
    (fa.FMT_NATIVE, 4096, 1, ()), (fa.FMT_NATIVE, 2560, 1, (0,)), (fa.FMT_Q8, 4096, 1, (0,)),
    (fa.FMT_NATIVE, 4096, 4, (1, 3)), (fa.FMT_Q8, 2560, 3, ())])
def test_rows_ref_q8(eng, fmt, hidden, burst, shared_tokens):
    """ref-q8 requests on row-format units with integer gate/up dots run on
    decode_rows_q8_kernel (x as two exact int8 digits, double after the
    integer dots): against the oracle's ref-q8 at the Q8 bar (1e-9), against
    layer_kernel's Q8 mode, bit for bit run to run, and every burst row bit
    for bit against its token run alone."""
    lay = oracle.layout(hidden, fmt)
    seed = 6100 + 10 * fmt + hidden + burst
    rng = np.random.default_rng(seed)
    for b in range(20):
        assert eng.synthetic(b, hidden, fmt, 1, seed) == fa.OK
    try:
        experts = zipf_routes(rng, burst) if burst > 1 else rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
        gates = np.zeros((burst, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, burst)
        for t in shared_tokens:
            gates[t, 10] = 0.5
        x = rng.standard_normal((burst, hidden)).astype(np.float32)
        kind, mode, grid = q8_plan(eng, experts, gates, x)
        assert kind == KIND_DECODE_ROWS and mode == fa.MODE_Q8, (kind, mode)
        print(f"rows ref-q8 fmt={fmt} hidden={hidden} burst={burst} shared={shared_tokens} grid={grid}", flush=True)
        rc, y = eng.run(0, experts, gates, x, fa.MODE_Q8)
        assert rc == fa.OK
        rc, ref = oracle.ref_run(host_units(lay, seed, experts, bool(shared_tokens)), fmt, True,
                                 oracle_request(0, experts, gates, x))
        assert rc == 0
        check_close(ref, y, fa.MODE_Q8, ("rows ref-q8", fmt, hidden, burst))
        rc, again = eng.run(0, experts, gates, x, fa.MODE_Q8)
        assert rc == fa.OK and np.array_equal(y.view(np.uint32), again.view(np.uint32))
        eng.route(fa.ROUTE_NO_DECODE)
        try:
            print(f"rows ref-q8 on the layer kernel fmt={fmt}", flush=True)
            rc, y_lay = eng.run(0, experts, gates, x, fa.MODE_Q8)
        finally:
            eng.route(0)
        assert rc == fa.OK
        check_close(y_lay, y, fa.MODE_Q8, ("rows ref-q8 vs layer", fmt, hidden, burst))
        for t in range(burst if burst > 1 else 0):
            rc, y1 = eng.run(0, experts[t:t + 1], gates[t:t + 1], x[t:t + 1], fa.MODE_Q8)
            assert rc == fa.OK
            assert np.array_equal(y1[0].view(np.uint32), y[t].view(np.uint32)), f"token {t} differs alone"
    finally:
        for b in range(20):
            eng.release(b)


def test_rows_ref_q8_mxfp4_takes_the_layer_kernel(eng):
    """MXFP4 gate/up rows dot in fp32: ref-q8 requests over them stay on the
    layer kernel's fp64 Q8 mode."""
    hidden, fmt, seed = 4096, fa.FMT_MXFP4, 61
    for b in range(2):
        assert eng.synthetic(b, hidden, fmt, 1, seed) == fa.OK
    try:
        rng = np.random.default_rng(2)
        experts = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
        gates = np.zeros((1, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 1)
        x = rng.standard_normal((1, hidden)).astype(np.float32)
        kind, mode, _ = q8_plan(eng, experts, gates, x)
        assert kind == 0 and mode == fa.MODE_Q8
    finally:
        for b in range(2):
            eng.release(b)
