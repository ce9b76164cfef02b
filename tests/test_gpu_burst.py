"""Bursts of two or more tokens on decode_burst_kernel.

A burst of all-Q4_K routed requests (F32, a node owning 12 or more blocks)
whose tokens share experts runs one workgroup turn per unique (expert, block)
pair: the pair's bytes are read once, and every token that routes to it is a
column pair (hi and lo parts of its operand) of f16 matrix-core products, for
gate/up and for the down. Each (token, pair) still gets its own partial,
summed per token in the reference's order by decode_reduce
(backends/ref.c:61-97). The route is taken by default from two routed tokens
per unique expert on average; FR_HIP_ROUTE_BURST forces it for the other
routings tested here.

Checked here: every row against the oracle at the F32 bar, run-to-run bit
identity, rows that permute bit for bit when the tokens do (a token's columns
do not depend on the others), the same burst on the unit route
(FR_HIP_ROUTE_NO_BURST, decode_kernel) with its rows bit-identical to the
tokens run alone (the batching property of src/native.c:94-117) and within
the F32 bar of the burst kernel, the default route choice, and the error
paths.
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import oracle_request, slice_view, softmax_gates, sparse_unit, zipf_routes
from test_gpu_parity import check_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = fa.Engine(0)
    yield e
    e.route(0)
    for b in range(20):
        e.release(b)


def routes(rng, burst, kind):
    if kind == "zipf":
        return zipf_routes(rng, burst)
    if kind == "same":   # every token on the same 10 experts, in its own order
        base = rng.choice(512, 10, replace=False)
        return np.stack([rng.permutation(base) for _ in range(burst)]).astype(np.uint16)
    ids = rng.choice(512, 10 * burst, replace=False)   # disjoint: no pair shared
    return ids.reshape(burst, 10).astype(np.uint16)


def host_blocks(lay, seed, blocks, experts):
    units = [None] * 20
    for b in blocks:
        u = sparse_unit(lay)
        for e in set(int(v) for v in np.asarray(experts).ravel()):
            slice_view(u, lay, 0, e)[:] = oracle.synth_slice(lay, seed, b, 0, e)
        units[b] = u
    return units


def plan_head(eng, experts, gates, x):
    plan, grid = eng.plan(0, experts, gates, x, fa.MODE_F32)
    return np.frombuffer(plan[:80].tobytes(), np.uint32), grid


def run_ok(eng, experts, gates, x):
    rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
    assert rc == fa.OK, rc
    return y


@pytest.mark.parametrize("burst,kind,hidden,nblocks", [(2, "zipf", 4096, 20), (4, "zipf", 4096, 20),
                                                       (8, "zipf", 4096, 20), (4, "same", 4096, 20),
                                                       (4, "disjoint", 4096, 20), (3, "zipf", 2560, 12),
                                                       (8, "same", 2560, 13)])
def test_burst_kernel(eng, burst, kind, hidden, nblocks):
    seed = 6060 + burst + hidden
    rng = np.random.default_rng(burst * 7 + hidden + nblocks)
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    blocks = sorted(rng.choice(20, nblocks, replace=False).tolist())
    for b in blocks:
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, seed) == fa.OK
    try:
        experts = routes(rng, burst, kind)
        gates = np.zeros((burst, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, burst)
        x = rng.standard_normal((burst, hidden)).astype(np.float32)
        unique = len(set(experts.ravel().tolist()))
        head, grid = plan_head(eng, experts, gates, x)
        want = fa.KIND_DECODE_BURST if 10 * burst >= 2 * unique else fa.KIND_DECODE
        assert int(head[16]) == want, (head[16], burst, unique)
        eng.route(fa.ROUTE_BURST)
        head, grid = plan_head(eng, experts, gates, x)
        assert int(head[16]) == fa.KIND_DECODE_BURST, head[16]
        assert int(head[3]) == unique * nblocks and 0 < grid <= 256, (head[3], grid)
        print(f"burst kernel: T={burst} {kind} hidden={hidden} blocks={nblocks} pairs={head[3]} grid={grid}",
              flush=True)
        y = run_ok(eng, experts, gates, x)
        units = host_blocks(lay, seed, blocks, experts)
        rc, ref = oracle.ref_run(units, fa.FMT_Q4KT, False, oracle_request(0, experts, gates, x))
        assert rc == 0
        check_close(ref, y, fa.MODE_F32, ("burst kernel", burst, kind, hidden))
        assert np.array_equal(run_ok(eng, experts, gates, x).view(np.uint32), y.view(np.uint32)), "repeat differs"
        perm = rng.permutation(burst)
        yp = run_ok(eng, experts[perm], gates[perm], x[perm])
        assert np.array_equal(yp.view(np.uint32), y[perm].view(np.uint32)), "rows do not permute with the tokens"
        eng.route(0)
        # The unit route: one (token, pair) unit per workgroup turn on
        # decode_kernel, each row bit-identical to its token run alone.
        eng.route(fa.ROUTE_NO_BURST)
        try:
            head_u, _ = plan_head(eng, experts, gates, x)
            assert int(head_u[16]) == fa.KIND_DECODE, head_u[16]
            print("unit route", flush=True)
            yu = run_ok(eng, experts, gates, x)
        finally:
            eng.route(0)
        check_close(ref, yu, fa.MODE_F32, ("unit route", burst, kind))
        check_close(yu.astype(np.float64), y, fa.MODE_F32, ("burst kernel vs unit route", burst, kind))
        for t in range(burst):
            y1 = run_ok(eng, experts[t:t + 1], gates[t:t + 1], x[t:t + 1])
            assert np.array_equal(y1[0].view(np.uint32), yu[t].view(np.uint32)), f"unit route: token {t} differs alone"
            check_close(y1.astype(np.float64), y[t:t + 1], fa.MODE_F32, ("burst row vs alone", t))
    finally:
        eng.route(0)
        for b in blocks:
            eng.release(b)


def test_burst_kernel_error_paths(eng):
    """A non-finite x, a gate/up d and a down d of one shared pair give
    FR_NUMERIC with y untouched; a zero-gate routed expert is still
    scale-checked (src/backend.h:58-59); the restored slice runs."""
    hidden, seed, nblocks = 4096, 7171, 12
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    rng = np.random.default_rng(71)
    for b in range(nblocks):
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, seed) == fa.OK
    try:
        experts = routes(rng, 4, "zipf")
        gates = np.zeros((4, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 4)
        x = rng.standard_normal((4, hidden)).astype(np.float32)
        eng.route(fa.ROUTE_BURST)
        head, _ = plan_head(eng, experts, gates, x)
        assert int(head[16]) == fa.KIND_DECODE_BURST
        print("burst error paths", flush=True)
        bad_x = x.copy()
        bad_x[2, 1000] = np.inf
        rc, y = eng.run(0, experts, gates, bad_x, fa.MODE_F32)
        assert rc == fa.NUMERIC and not y.any()
        e0 = int(experts[1, 4])
        unit = sparse_unit(lay)
        view = slice_view(unit, lay, 0, e0)
        view[:] = oracle.synth_slice(lay, seed, 5, 0, e0)
        good = view.copy()
        zero_gate = gates.copy()
        zero_gate[1, 4] = 0.0
        for off, g in ((1, gates), (2 * lay.proj + 1, gates), (1, zero_gate)):   # d high byte 0x7C -> inf
            view[:] = good
            view[off] = 0x7C
            assert eng.refresh(5, unit, 0, e0) == fa.OK
            rc, y = eng.run(0, experts, g, x, fa.MODE_F32)
            assert rc == fa.NUMERIC and not y.any(), off
        view[:] = good
        assert eng.refresh(5, unit, 0, e0) == fa.OK
        rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK and np.isfinite(y).all()
    finally:
        eng.route(0)
        for b in range(nblocks):
            eng.release(b)
