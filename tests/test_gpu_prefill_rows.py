"""Prefill chunks (fr_hip_run_batch) on the reference's own unit format and
with the shared expert.

Native units (Q4_K gate/up rows, MXFP4 down [H x 32], src/native.h:9-15) run
on the row-format prefill kernels; the shared expert (Q8_0, every unit
format's, backends/ref.c:68-73) has tiles of its own in either format; each
token's partials are summed in the reference's order, routed experts in
request order then the shared one (backends/ref.c:61-97). Row t must equal
what ref returns for token t (the reference serves a prompt as run() bursts
of at most 8, client/fronk_client.h:41-42): checked against the oracle on
host copies of the same slices, and against this library's run() bursts;
bit-for-bit properties at the full size (repeat, token permutation, doubled
gates); the reference's native fixture (src/native.c:66-76) at H=2560; and
the error paths.
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import native_fixture, oracle_request, slice_view, softmax_gates, sparse_unit, zipf_routes
from test_gpu_parity import check_close

pytestmark = pytest.mark.gpu

SEED = 0x5EED0007


@pytest.fixture(scope="module")
def eng():
    e = fa.Engine(0)
    yield e
    for b in range(20):
        e.release(b)


def load(eng, hidden, blocks, fmt, layers=1):
    for b in range(20):
        eng.release(b)
    for b in blocks:
        assert eng.synthetic(b, hidden, fmt, layers, SEED) == fa.OK


def oracle_rows(lay, fmt, blocks, layer, experts, gates, x):
    used = sorted(set(int(e) for e in np.asarray(experts).ravel()) | {oracle.SHARED})
    units = [None] * 20
    for b in blocks:
        u = sparse_unit(lay)
        for e in used:
            slice_view(u, lay, layer, e)[:] = oracle.synth_slice(lay, SEED, b, layer, e)
        units[b] = u
    rows = []
    for t0 in range(0, x.shape[0], 8):
        sl = slice(t0, min(t0 + 8, x.shape[0]))
        rc, ref = oracle.ref_run(units, fmt, False, oracle_request(layer, experts[sl], gates[sl], x[sl]))
        assert rc == 0
        rows.append(ref[:sl.stop - sl.start])
    return np.concatenate(rows)


def chunk(rng, tokens, hidden, pool, shared_every=0):
    experts = np.asarray(pool, np.uint16)[zipf_routes(rng, tokens, experts=len(pool))]
    gates = np.zeros((tokens, 11), np.float32)
    gates[:, :10] = softmax_gates(rng, tokens)
    if shared_every:
        gates[::shared_every, 10] = 0.5
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    return experts, gates, x


def run_ok(eng, layer, experts, gates, x):
    print(f"prefill rows tokens={x.shape[0]} hidden={x.shape[1]} shared={int((gates[:, 10] != 0).sum())}",
          flush=True)
    rc, y = eng.run_batch(layer, experts, gates, x)
    assert rc == fa.OK, rc
    return y


def run_bursts(eng, layer, experts, gates, x):
    out = []
    for t0 in range(0, x.shape[0], 8):
        rc, y = eng.run(layer, experts[t0:t0 + 8], gates[t0:t0 + 8], x[t0:t0 + 8], fa.MODE_F32)
        assert rc == fa.OK
        out.append(y)
    return np.concatenate(out)


@pytest.mark.parametrize("fmt,hidden,tokens,blocks,shared_every", [
    (fa.FMT_NATIVE, 2560, 40, (0, 7, 19), 0),
    (fa.FMT_NATIVE, 2560, 37, tuple(range(20)), 1),
    (fa.FMT_NATIVE, 4096, 24, (3, 11), 3),
    (fa.FMT_Q4KT, 4096, 33, (0, 5, 9, 13), 2),
])
def test_prefill_rows_match_oracle(eng, fmt, hidden, tokens, blocks, shared_every):
    """Hot experts span several 16-token tiles and cold ones hold a single
    token; the shared expert on every token, every third or every second
    (three shared tiles, one partial), or on none."""
    lay = oracle.layout(hidden, fmt)
    load(eng, hidden, blocks, fmt)
    rng = np.random.default_rng(hidden + tokens + fmt)
    pool = rng.choice(512, 40, replace=False)
    experts, gates, x = chunk(rng, tokens, hidden, pool, shared_every)
    y = run_ok(eng, 0, experts, gates, x)
    s = eng.sample()
    assert s.unique_experts == len(set(experts.ravel().tolist())) and s.blocks == len(blocks)
    ref = oracle_rows(lay, fmt, blocks, 0, experts, gates, x)
    check_close(ref, y, fa.MODE_F32, ("prefill rows", fmt, hidden, shared_every))
    check_close(run_bursts(eng, 0, experts, gates, x), y, fa.MODE_F32, ("prefill rows vs run", fmt, hidden))


def test_prefill_native_512_tokens_properties(eng):
    """512 tokens, uniform top-10 over 512 experts, the shared expert on every
    token, 20 owned native slices at H=2560 (the reference's width)."""
    hidden, tokens, layer = 2560, 512, 1
    lay = oracle.layout(hidden, fa.FMT_NATIVE)
    load(eng, hidden, range(20), fa.FMT_NATIVE, layers=2)
    rng = np.random.default_rng(2560)
    experts = np.stack([rng.choice(512, 10, replace=False) for _ in range(tokens)]).astype(np.uint16)
    gates = np.zeros((tokens, 11), np.float32)
    gates[:, :10] = softmax_gates(rng, tokens)
    gates[:, 10] = 0.5
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    y = run_ok(eng, layer, experts, gates, x)
    assert np.isfinite(y).all()
    assert np.array_equal(run_ok(eng, layer, experts, gates, x).view(np.uint32), y.view(np.uint32))
    perm = rng.permutation(tokens)
    yp = run_ok(eng, layer, experts[perm], gates[perm], x[perm])
    assert np.array_equal(yp.view(np.uint32), y[perm].view(np.uint32))
    y2 = run_ok(eng, layer, experts, 2 * gates, x)
    assert np.array_equal(y2.view(np.uint32), (2 * y).view(np.uint32))
    sample = np.arange(3, tokens, 71)
    ref = oracle_rows(lay, fa.FMT_NATIVE, range(20), layer, experts[sample], gates[sample], x[sample])
    check_close(ref, y[sample], fa.MODE_F32, "native prefill 512 sample")
    check_close(run_bursts(eng, layer, experts[:16], gates[:16], x[:16]), y[:16], fa.MODE_F32, "vs run")


def test_prefill_native_fixture(eng):
    """The reference's native self-test fixture (src/native.c:66-76): H=2560,
    block 19, experts 0..79 and the shared slice from LCG seed 7, 8 tokens,
    gates 0.0625 and shared 0.5; the distinct and the reused routing."""
    for b in range(20):
        eng.release(b)
    lay = oracle.layout(2560, oracle.FMT_NATIVE)
    data, gates, x = native_fixture(lay)
    assert eng.upload(19, data, 2560, fa.FMT_NATIVE) == fa.OK
    try:
        blocks = [None] * 20
        blocks[19] = data
        for reuse in (0, 1):
            experts = np.array([[e + (0 if reuse else t * 10) for e in range(10)] for t in range(8)], np.uint16)
            y = run_ok(eng, 47, experts, gates, x)
            rc, ref = oracle.ref_run(blocks, oracle.FMT_NATIVE, False, oracle_request(47, experts, gates, x))
            assert rc == 0
            check_close(ref, y, fa.MODE_F32, ("native fixture prefill", reuse))
    finally:
        eng.release(19)


def test_prefill_rows_error_paths(eng):
    """A non-finite x, a Q4_K gate d, an MXFP4 down exponent of 255 and a
    shared-expert Q8_0 d of inf each give FR_NUMERIC with y untouched; the
    restored slices run bit-identical to before."""
    hidden, blocks = 2560, (0, 1)
    lay = oracle.layout(hidden, fa.FMT_NATIVE)
    load(eng, hidden, blocks, fa.FMT_NATIVE)
    rng = np.random.default_rng(77)
    pool = rng.choice(512, 30, replace=False)
    experts, gates, x = chunk(rng, 20, hidden, pool, shared_every=2)
    y = run_ok(eng, 0, experts, gates, x)
    bad = x.copy()
    bad[7, 100] = np.inf
    rc, yb = eng.run_batch(0, experts, gates, bad)
    assert rc == fa.NUMERIC and not yb.any()
    e0 = int(experts[4, 2])
    unit = sparse_unit(lay)
    for e, off, val in ((e0, 1, 0x7C), (e0, 2 * lay.proj + 17 * 999, 255), (oracle.SHARED, 2 * lay.shared_proj + 1, 0x7C)):
        view = slice_view(unit, lay, 0, e)
        view[:] = oracle.synth_slice(lay, SEED, 1, 0, e)
        good = view.copy()
        view[off] = val
        assert eng.refresh(1, unit, 0, e) == fa.OK
        print(f"prefill rows error: expert {e} byte {off}", flush=True)
        rc, yb = eng.run_batch(0, experts, gates, x)
        assert rc == fa.NUMERIC and not yb.any(), (e, off)
        view[:] = good
        assert eng.refresh(1, unit, 0, e) == fa.OK
    assert np.array_equal(run_ok(eng, 0, experts, gates, x).view(np.uint32), y.view(np.uint32))
    # Blocks of two formats in one node are not a prefill chunk.
    assert eng.synthetic(2, hidden, fa.FMT_Q4KT, 1, SEED) == fa.OK
    assert eng.run_batch(0, experts, gates, x)[0] == fa.UNSUPPORTED
    eng.release(2)


def set_codes(view, off, e, mag_max, at=None):
    """Block at `off` (E8M0 byte, then 16 code bytes): exponent e, every code's
    magnitude index (code & 7) at most mag_max; with `at`, the low nibble of
    code byte `at` exactly mag_max."""
    view[off] = e
    codes = view[off + 1:off + 17]
    lo, hi = codes & 15, codes >> 4
    lo = (lo & 8) | np.minimum(lo & 7, mag_max)
    hi = (hi & 8) | np.minimum(hi & 7, mag_max)
    if at is not None:
        lo[at] = mag_max
    view[off + 1:off + 17] = lo | (hi << 4)


def test_prefill_rows_mx_exponent_edges(eng):
    """MXFP4 down exponents at both ends of the E8M0 range in one routed
    expert's slices (src/native.c:23-27), against the oracle, on tokens 0..7
    that route to that expert alone, so that its products are all of their
    y: every output row at exponent 0, 1, 2 or 63 (the kernel's exact slices
    for weights below 2^-63; 0 and 1 put code values below bf16's smallest
    normal), then at 64 or 65 (the lowest scaled inside the products); then
    rows at 253 with codes below 4 and at 254 with codes below 2 (finite
    weights); then 253 with a code of 4 and 254 with a code of 2, each placed
    in a later dword of the record, give FR_NUMERIC with y untouched."""
    hidden, blocks = 2560, (0, 1)
    lay = oracle.layout(hidden, fa.FMT_NATIVE)
    load(eng, hidden, blocks, fa.FMT_NATIVE)
    rng = np.random.default_rng(91)
    pool = rng.choice(512, 30, replace=False)
    experts, gates, x = chunk(rng, 24, hidden, pool, shared_every=2)
    e0 = int(experts[3, 1])
    for t in range(8):
        experts[t] = [e0] + [int(e) for e in experts[t] if e != e0][:9]
        gates[t] = 0.0
        gates[t, 0] = 0.7
    used = sorted(set(int(e) for e in experts.ravel()) | {oracle.SHARED})
    units = [None] * 20
    for b in blocks:
        u = sparse_unit(lay)
        for e in used:
            slice_view(u, lay, 0, e)[:] = oracle.synth_slice(lay, SEED, b, 0, e)
        units[b] = u
    views = [slice_view(units[b], lay, 0, e0) for b in blocks]
    goods = [v.copy() for v in views]
    down = 2 * lay.proj

    def refresh():
        for b in blocks:
            assert eng.refresh(b, units[b], 0, e0) == fa.OK

    def against_oracle(what, small):
        y = run_ok(eng, 0, experts, gates, x)
        rows = []
        for t0 in range(0, x.shape[0], 8):
            sl = slice(t0, t0 + 8)
            rc, ref = oracle.ref_run(units, fa.FMT_NATIVE, False, oracle_request(0, experts[sl], gates[sl], x[sl]))
            assert rc == 0
            rows.append(ref[:8])
        ref = np.concatenate(rows)
        assert np.abs(ref[:8]).max() < small   # tokens 0..7: the edited rows alone
        check_close(ref[:8], y[:8], fa.MODE_F32, (what, "tokens 0..7"))
        check_close(ref, y, fa.MODE_F32, what)
        check_close(run_bursts(eng, 0, experts, gates, x), y, fa.MODE_F32, (what, "vs run"))

    try:
        for exps, small in (((0, 1, 2, 63), 1e-10), ((64, 65), 1e-9)):
            for v in views:
                for row in range(hidden):
                    set_codes(v, down + 17 * row, exps[row % len(exps)], 7)
            refresh()
            against_oracle(f"exponents {exps}", small)
        for v, g in zip(views, goods):
            v[:] = g
        for v in views:
            for row, e, mag in ((200, 253, 5), (300, 254, 3), (301, 253, 5)):
                set_codes(v, down + 17 * row, e, mag)
        refresh()
        print("prefill rows MXFP4 exponents 253, 254 finite", flush=True)
        rc, y = eng.run_batch(0, experts, gates, x)
        rows = []
        for t0 in range(0, x.shape[0], 8):
            sl = slice(t0, t0 + 8)
            rc_ref, ref = oracle.ref_run(units, fa.FMT_NATIVE, False,
                                         oracle_request(0, experts[sl], gates[sl], x[sl]))
            rows.append((rc_ref, ref[:8]))
        if all(r == 0 for r, _ in rows):
            assert rc == fa.OK, rc
            check_close(np.concatenate([r for _, r in rows]), y, fa.MODE_F32, "exponents 253, 254")
        else:
            assert rc == fa.NUMERIC and not y.any(), rc
        for e, mag, at in ((253, 6, 9), (254, 4, 14)):
            for v, g in zip(views, goods):
                v[:] = g
            set_codes(views[1], down + 17 * 40, e, mag, at)
            refresh()
            print(f"prefill rows MXFP4 overflow e={e} code {mag} at byte {at}", flush=True)
            rc, yb = eng.run_batch(0, experts, gates, x)
            assert rc == fa.NUMERIC and not yb.any(), (e, mag, at, rc)
    finally:
        for v, g in zip(views, goods):
            v[:] = g
        refresh()
