"""Every item of a decode launch on its own.

The decode kernels give each work item (a (token, expert, block) unit, or a
part of one on the split kernel) an fp32 partial of its own, which
decode_reduce sums per token in the reference's order. Here each item's
partial is read back (fr_hip_debug_partials) and compared with a float64
restatement of that item alone: the slice dequantized into dense matrices,
a and u of the item's neurons, h = SiLU(a)*u narrowed to fp32 as
backends/ref.c:80-83 does, times the token's gate through the down rows of
those neurons. A wrong item is then named exactly (token, expert, block,
part), instead of showing only as an error in the reduced y.

Covered: decode_kernel (one token, and a 4-token burst on the unit route),
decode_split_kernel with 2 and 4 items per unit, at hidden 4096 and 2560,
and decode_burst_kernel's (token, pair) partials.
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import dense_slice, slice_view, softmax_gates, sparse_unit, zipf_routes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = fa.Engine(0)
    yield e
    e.route(0)
    for b in range(20):
        e.release(b)


def item_reference(cache, units, lay, blocks, experts, gates, x, split):
    """[items][hidden] float64 in the kernels' numbering: token-major, the
    token's experts in request order, blocks ascending, then the unit's
    parts (8 * 4/split neurons each)."""
    T, H = x.shape
    per = 32 // split
    out = []
    for t in range(T):
        xt = x[t].astype(np.float64)
        for e in range(10):
            eid = int(experts[t, e])
            for b in blocks:
                if (b, eid) not in cache:
                    cache[(b, eid)] = dense_slice(slice_view(units[b], lay, 0, eid), lay, eid)
                Wg, Wu, Wd = cache[(b, eid)]
                a = (Wg @ xt).astype(np.float32).astype(np.float64)
                u = (Wu @ xt).astype(np.float32).astype(np.float64)
                sig = np.where(a >= 0, 1 / (1 + np.exp(-np.abs(a))), np.exp(-np.abs(a)) / (1 + np.exp(-np.abs(a))))
                h = (a * sig * u).astype(np.float32).astype(np.float64)
                for part in range(split):
                    n = slice(per * part, per * (part + 1))
                    out.append(float(gates[t, e]) * (Wd[:, n] @ h[n]))
    return np.array(out)


@pytest.mark.parametrize("hidden,nblocks,burst,route,want", [
    (4096, 12, 1, 0, fa.KIND_DECODE), (4096, 6, 1, 0, fa.KIND_DECODE_SPLIT), (4096, 3, 1, 0, fa.KIND_DECODE_SPLIT),
    (2560, 7, 1, 0, fa.KIND_DECODE_SPLIT), (2560, 12, 1, 0, fa.KIND_DECODE),
    (4096, 12, 4, fa.ROUTE_NO_BURST, fa.KIND_DECODE), (4096, 6, 4, 0, fa.KIND_DECODE_SPLIT),
    (4096, 12, 4, fa.ROUTE_BURST, fa.KIND_DECODE_BURST), (2560, 12, 3, fa.ROUTE_BURST, fa.KIND_DECODE_BURST)])
def test_each_decode_item_against_its_restatement(eng, hidden, nblocks, burst, route, want):
    seed = 9900 + hidden + nblocks + burst
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    rng = np.random.default_rng(seed)
    blocks = sorted(rng.choice(20, nblocks, replace=False).tolist())
    for b in blocks:
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, seed) == fa.OK
    try:
        experts = zipf_routes(rng, burst)
        gates = np.zeros((burst, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, burst)
        x = rng.standard_normal((burst, hidden)).astype(np.float32)
        eng.route(route)
        plan, grid = eng.plan(0, experts, gates, x, fa.MODE_F32)
        head = np.frombuffer(plan[:80].tobytes(), np.uint32)
        kind = int(head[16])
        assert kind == want, (kind, want)
        split = int(head[19]) if kind == fa.KIND_DECODE_SPLIT else 1
        print(f"items: hidden={hidden} blocks={nblocks} T={burst} kind={kind} split={split} grid={grid}", flush=True)
        rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
        assert rc == fa.OK
        count = burst * 10 * nblocks * split
        got = eng.partials(0, count)[:, :hidden].astype(np.float64)
        units = [None] * 20
        for b in blocks:
            u = sparse_unit(lay)
            for e in set(int(v) for v in experts.ravel()):
                slice_view(u, lay, 0, e)[:] = oracle.synth_slice(lay, seed, b, 0, e)
            units[b] = u
        ref = item_reference({}, units, lay, blocks, experts, gates, x, split)
        assert ref.shape == got.shape
        err = np.linalg.norm(got - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)
        worst = int(np.argmax(err))
        t, rest = divmod(worst, 10 * nblocks * split)
        e, rest = divmod(rest, nblocks * split)
        b, part = divmod(rest, split)
        # An item holds 8 to 32 neurons, so one neuron's fp32 rounding of a,
        # u and h (about 1e-6 relative where a nearly cancels) is not averaged
        # away as it is over a token's thousands of neurons: the bar per item
        # is 1e-4 (the wrong items this hunts for were off by 0.1 and more),
        # and the median item must meet the F32 bar of a whole token.
        assert err[worst] <= 1e-4, (f"item {worst}: token {t} expert {int(experts[t, e])} block {blocks[b]} "
                                    f"part {part}: rel. L2 {err[worst]:.3g}")
        assert float(np.median(err)) <= 1e-5, float(np.median(err))
    finally:
        eng.route(0)
        for b in blocks:
            eng.release(b)
