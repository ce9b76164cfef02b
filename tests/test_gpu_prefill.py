"""Prefill chunks on matrix cores (fr_hip_run_batch).

The reference has no multi-token path beyond run()'s burst of at most 8: its
client cuts a prompt into bursts (client/fronk_client.h:41-42) and each burst
is run() (backends/ref.c:57-98). So row t of a chunk must equal, within the F32
tolerance, what ref returns for token t: checked against the oracle's
restatement of ref on host copies of the same synthetic slices, and against
this library's own run() on the same tokens. At the full 512-token size,
size-independent properties hold bit for bit: a repeat run is identical,
permuting the tokens permutes the rows, and doubling every gate doubles every
output (a power of two commutes with every rounding on the path).
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import oracle_request, slice_view, softmax_gates, sparse_unit, zipf_routes
from test_gpu_parity import check_close

pytestmark = pytest.mark.gpu

SEED = 0x5EED0005


@pytest.fixture(scope="module")
def eng():
    e = fa.Engine(0)
    yield e
    for b in range(20):
        e.release(b)


def load(eng, hidden, blocks, layers=1, fmt=fa.FMT_Q4KT):
    for b in range(20):
        eng.release(b)
    for b in blocks:
        assert eng.synthetic(b, hidden, fmt, layers, SEED) == fa.OK


def host_units(lay, blocks, layer, experts):
    """Sparse host copies of the owned synthetic blocks (None where a block is
    not owned) holding the slices of `experts` at `layer`."""
    used = sorted(set(int(e) for e in np.asarray(experts).ravel()))
    units = [None] * 20
    for b in blocks:
        u = sparse_unit(lay)
        for e in used:
            slice_view(u, lay, layer, e)[:] = oracle.synth_slice(lay, SEED, b, layer, e)
        units[b] = u
    return units


def oracle_rows(lay, blocks, layer, experts, gates, x):
    units = host_units(lay, blocks, layer, experts)
    rows = []
    for t0 in range(0, x.shape[0], 8):
        sl = slice(t0, min(t0 + 8, x.shape[0]))
        rc, ref = oracle.ref_run(units, fa.FMT_Q4KT, False, oracle_request(layer, experts[sl], gates[sl], x[sl]))
        assert rc == 0
        rows.append(ref[:sl.stop - sl.start])
    return np.concatenate(rows)


def chunk(rng, tokens, hidden, pool=None):
    """Top-10 routes per token. With a pool, Zipf(1.1) popularity over it, so
    that hot experts take several 16-token tiles and cold ones a single token."""
    if pool is None:
        experts = np.stack([rng.choice(512, 10, replace=False) for _ in range(tokens)]).astype(np.uint16)
    else:
        experts = np.asarray(pool, np.uint16)[zipf_routes(rng, tokens, experts=len(pool))]
    gates = np.zeros((tokens, 11), np.float32)
    gates[:, :10] = softmax_gates(rng, tokens)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    return experts, gates, x


def run_ok(eng, layer, experts, gates, x):
    print(f"prefill tokens={x.shape[0]} hidden={x.shape[1]} layer={layer}", flush=True)
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


@pytest.mark.parametrize("hidden,tokens,blocks", [
    (4096, 40, tuple(range(20))),
    (2560, 24, (0, 7, 19)),
    (2304, 24, (0, 5, 19)),
])
def test_prefill_rows_match_oracle(eng, hidden, tokens, blocks):
    """Hot experts span several tiles, cold ones hold one token; at hidden 2560
    and 2304 only 3 slices are owned, and at 2304 (9 super-blocks) the last
    down workgroup (512 outputs) has idle wavefronts."""
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    load(eng, hidden, blocks)
    rng = np.random.default_rng(hidden + tokens)
    pool = rng.choice(512, 40, replace=False)
    experts, gates, x = chunk(rng, tokens, hidden, pool)
    counts = np.bincount(experts.ravel(), minlength=512)
    assert counts.max() > 16 and counts[counts > 0].min() < 16   # several tiles, and partial ones
    y = run_ok(eng, 0, experts, gates, x)
    s = eng.sample()
    assert s.unique_experts == len(set(experts.ravel().tolist())) and s.blocks == len(blocks)
    ref = oracle_rows(lay, blocks, 0, experts, gates, x)
    check_close(ref, y, fa.MODE_F32, ("prefill", hidden))
    check_close(run_bursts(eng, 0, experts, gates, x), y, fa.MODE_F32, ("prefill vs run", hidden))


def test_prefill_512_tokens_properties(eng):
    """The chunk size of the prefill workload: 512 tokens, uniform top-10 over
    512 experts, 20 owned slices, hidden 4096, layer 1."""
    hidden, tokens, layer = 4096, 512, 1
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    load(eng, hidden, range(20), layers=2)
    rng = np.random.default_rng(512)
    experts, gates, x = chunk(rng, tokens, hidden)
    y = run_ok(eng, layer, experts, gates, x)
    assert np.isfinite(y).all()
    again = run_ok(eng, layer, experts, gates, x)
    assert np.array_equal(y.view(np.uint32), again.view(np.uint32))
    perm = rng.permutation(tokens)
    yp = run_ok(eng, layer, experts[perm], gates[perm], x[perm])
    assert np.array_equal(yp.view(np.uint32), y[perm].view(np.uint32))
    y2 = run_ok(eng, layer, experts, 2 * gates, x)
    assert np.array_equal(y2.view(np.uint32), (2 * y).view(np.uint32))
    sample = np.arange(0, tokens, 64)
    ref = oracle_rows(lay, range(20), layer, experts[sample], gates[sample], x[sample])
    check_close(ref, y[sample], fa.MODE_F32, "prefill 512 sample")
    check_close(run_bursts(eng, layer, experts[:16], gates[:16], x[:16]), y[:16], fa.MODE_F32, "prefill vs run")


def test_prefill_48_layers_resident(eng):
    """The resident node of the prefill workload: 48 layers of 20 owned
    blocks in HBM (108.7 GB), a 512-token chunk on the last layer, whose
    slices sit at the top of each block's 5.4 GB. Sampled rows against the
    oracle; every row finite; a repeat is bit-identical."""
    hidden, tokens, layer = 4096, 512, 47
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    print("prefill: 20 blocks x 48 layers resident", flush=True)
    load(eng, hidden, range(20), layers=48)
    try:
        rng = np.random.default_rng(4847)
        experts, gates, x = chunk(rng, tokens, hidden)
        y = run_ok(eng, layer, experts, gates, x)
        assert np.isfinite(y).all()
        assert np.array_equal(run_ok(eng, layer, experts, gates, x).view(np.uint32), y.view(np.uint32))
        sample = np.arange(5, tokens, 73)
        ref = oracle_rows(lay, range(20), layer, experts[sample], gates[sample], x[sample])
        check_close(ref, y[sample], fa.MODE_F32, "prefill layer 47 of 48")
    finally:
        for b in range(20):
            eng.release(b)


def test_prefill_error_paths(eng):
    hidden = 4096
    load(eng, hidden, (0, 1))
    rng = np.random.default_rng(5)
    experts, gates, x = chunk(rng, 20, hidden)
    y = run_ok(eng, 0, experts, gates, x)
    assert eng.run_batch(0, experts[:0], gates[:0], x[:0])[0] == fa.INVALID
    dup = experts.copy()
    dup[3, 1] = dup[3, 0]
    assert eng.run_batch(0, dup, gates, x)[0] == fa.INVALID
    big = experts.copy()
    big[2, 4] = 512
    assert eng.run_batch(0, big, gates, x)[0] == fa.INVALID
    assert eng.run_batch(0, experts, gates, x, fa.MODE_F64)[0] == fa.UNSUPPORTED
    assert eng.run_batch(1, experts, gates, x)[0] == fa.STATE
    assert eng.run_batch(0, experts, gates, x[:, :2560])[0] == fa.INVALID
    bad = x.copy()
    bad[7, 100] = np.inf
    rc, yb = eng.run_batch(0, experts, gates, bad)
    assert rc == fa.NUMERIC and not yb.any()
    # The status word is cleared per launch: the next good chunk succeeds.
    assert np.array_equal(run_ok(eng, 0, experts, gates, x).view(np.uint32), y.view(np.uint32))
    assert eng.synthetic(2, hidden, fa.FMT_Q8, 1, SEED) == fa.OK
    assert eng.run_batch(0, experts, gates, x)[0] == fa.UNSUPPORTED
    eng.release(2)


def test_prefill_large_down_scales(eng):
    """Down super-blocks whose d is 4 or more in magnitude (4, -5, 6, 100, and
    65504, the largest fp16) in one expert's slice: the down kernel takes those
    slices on its scaled path; rows against the oracle and against run()."""
    hidden, blocks = 4096, (0, 1)
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    load(eng, hidden, blocks)
    rng = np.random.default_rng(4444)
    pool = rng.choice(512, 30, replace=False)
    experts, gates, x = chunk(rng, 24, hidden, pool)
    e0 = int(experts[2, 3])
    units = host_units(lay, blocks, 0, experts)
    view = slice_view(units[1], lay, 0, e0)
    good = view.copy()
    for neuron, sb, d in ((5, 3, 0x4400), (17, 9, 0xC500), (0, 0, 0x4600), (31, 15, 0x5640), (12, 6, 0x7BFF)):
        off = 2 * lay.proj + neuron * lay.down_row + 144 * sb
        view[off:off + 2] = np.array([d], np.uint16).view(np.uint8)
    try:
        assert eng.refresh(1, units[1], 0, e0) == fa.OK
        y = run_ok(eng, 0, experts, gates, x)
        rows = []
        for t0 in range(0, x.shape[0], 8):
            sl = slice(t0, t0 + 8)
            rc, ref = oracle.ref_run(units, fa.FMT_Q4KT, False, oracle_request(0, experts[sl], gates[sl], x[sl]))
            assert rc == 0
            rows.append(ref[:8])
        check_close(np.concatenate(rows), y, fa.MODE_F32, "prefill large down scales")
        check_close(run_bursts(eng, 0, experts, gates, x), y, fa.MODE_F32, "prefill large down scales vs run")
    finally:
        view[:] = good
        assert eng.refresh(1, units[1], 0, e0) == fa.OK
