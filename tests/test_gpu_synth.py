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


def km_tiles(ref, hidden):
    """The matrix-core tiles of a Q4KT slice's gate/up rows, restated from the
    layout description: ref holds the 32 gate and 32 up rows in the reference
    layout (row = nsb super-blocks of [d, dmin, 12 scale bytes, 128 nibble
    bytes]; element j of a super-block is byte 32*(j//64) + j%32, high nibble
    when j%64 >= 32). Per super-block: [4 row-blocks][16 rows][16 B] headers,
    then [4 row-blocks][2 parts][64 lanes][16 B] nibbles; row i < 8 of
    row-block rb is gate row 8rb+i, row i >= 8 is up row 8rb+i-8; lane
    16kg+i of part p holds sub-block 4p+kg of row i as 4 words, word u with
    positions 8u..8u+3 in the low nibbles and 8u+4..8u+7 in the high ones."""
    nsb = hidden // 256
    rows = ref[:64 * 144 * nsb].reshape(64, nsb, 144)
    j = np.arange(256)
    q = (rows[:, :, 16 + 32 * (j // 64) + j % 32] >> (4 * ((j % 64) // 32))) & 15   # [row][sb][256]
    out = np.zeros(9216 * nsb, np.uint8)
    u, b = np.meshgrid(np.arange(4), np.arange(4), indexing="ij")
    for sb in range(nsb):
        blk = out[9216 * sb:9216 * (sb + 1)]
        for rb in range(4):
            for i in range(16):
                r = 8 * rb + i if i < 8 else 32 + 8 * rb + i - 8
                blk[16 * (16 * rb + i):16 * (16 * rb + i) + 16] = rows[r, sb, :16]
                for p in range(2):
                    for kg in range(4):
                        v = q[r, sb, 32 * (4 * p + kg):32 * (4 * p + kg) + 32]
                        base = 1024 + 2048 * rb + 1024 * p + 16 * (16 * kg + i)
                        blk[base:base + 16] = (v[8 * u + b] | (v[8 * u + 4 + b] << 4)).reshape(16)
    return out


def test_q4kt_gate_up_tiles_match_layout(eng):
    """The re-tiler's matrix-core tiles of the Q4KT gate/up rows, byte for
    byte, against the layout restated above, on random slice bytes."""
    lay = oracle.layout(H, fa.FMT_Q4KT)
    rng = np.random.default_rng(77)
    assert eng.reserve(7, H, fa.FMT_Q4KT) == fa.OK
    try:
        unit = sparse_unit(lay)
        for layer, e in [(0, 5), (3, 400)]:
            view = slice_view(unit, lay, layer, e)
            view[:] = rng.integers(0, 256, view.size, dtype=np.uint8)
            assert eng.refresh(7, unit, layer, e) == fa.OK
            got = eng.read(7, oracle.slice_offset(lay, layer, e), 2 * lay.proj)
            want = km_tiles(view, H)
            assert np.array_equal(got, want), (layer, e, int(np.argmax(got != want)))
    finally:
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
def test_decode_kernel_and_layer_kernel_agree_with_oracle(eng, hidden):
    """Single-token all-Q4_K requests run on decode_kernel + decode_reduce;
    the same request routed to the two-phase layer_kernel must match the
    oracle as well, and each route repeats bit for bit."""
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
        for route, want in [(0, fa.KIND_DECODE), (fa.ROUTE_NO_DECODE, fa.KIND_LAYER)]:
            eng.route(route)
            kind, grid = plan_kind(eng, 0, experts, gates, x)
            assert kind == want, (route, kind)
            print(f"route={route} kind={kind} hidden={hidden} grid={grid}", flush=True)
            rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
            assert rc == fa.OK
            check_close(ref, y, fa.MODE_F32, ("route", route, hidden))
            rc, again = eng.run(0, experts, gates, x, fa.MODE_F32)
            assert rc == fa.OK
            assert np.array_equal(y.view(np.uint32), again.view(np.uint32))
    finally:
        eng.route(0)
        for b in range(20):
            eng.release(b)


@pytest.mark.parametrize("burst", [2, 3, 4, 5, 8])
def test_decode_burst_rows_equal_single_token_runs(eng, burst):
    """Bursts of all-Q4_K routed requests on the unit route
    (FR_HIP_ROUTE_NO_BURST): decode_kernel with each (token, pair) a unit with
    its own partial, a token's units summed in the single-token order. Every
    row must match the oracle and be bit-identical to the same token run alone
    (the batching property of src/native.c:94-117, which the reference checks
    with memcmp). The default route of these bursts, decode_burst_kernel, is
    tested in test_gpu_burst.py."""
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
        eng.route(fa.ROUTE_NO_BURST)
        kind, grid = plan_kind(eng, 0, experts, gates, x)
        assert kind == fa.KIND_DECODE and 0 < grid <= 256, (kind, grid)
        print(f"decode burst={burst} grid={grid}", flush=True)
        rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
        eng.route(0)
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
        eng.route(0)
        for b in range(20):
            eng.release(b)


def q8_plan(eng, experts, gates, x):
    plan, grid = eng.plan(0, experts, gates, x, fa.MODE_Q8)
    head = np.frombuffer(plan[:80].tobytes(), np.uint32)
    return int(head[16]), int(head[2]), grid   # kind, mode, grid


@pytest.mark.parametrize("hidden", [4096, 2560])
def test_ref_q8_decode_kernel(eng, hidden):
    """ref-q8 requests on all-Q4_K units run on decode_q8_kernel: x as two
    exact int8 digits per value, the matrix-core dots, everything after them
    in double. A single token and a Zipf burst against the oracle's ref-q8
    at the Q8 bar (1e-9), against the same requests on layer_kernel's Q8 mode,
    a bit-identical repeat, and every burst row bit-identical to its token
    run alone."""
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    seed = 8080 + hidden
    rng = np.random.default_rng(hidden + 1)
    for b in range(20):
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, seed) == fa.OK
    try:
        single = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
        burst = zipf_routes(rng, 4)
        used = sorted(set(np.concatenate([single.ravel(), burst.ravel()]).tolist()))
        units = []
        for b in range(20):
            u = sparse_unit(lay)
            for e in used:
                slice_view(u, lay, 0, e)[:] = oracle.synth_slice(lay, seed, b, 0, e)
            units.append(u)
        for experts in (single, burst):
            T = experts.shape[0]
            gates = np.zeros((T, 11), np.float32)
            gates[:, :10] = softmax_gates(rng, T)
            x = rng.standard_normal((T, hidden)).astype(np.float32)
            x[0, :64] *= 1e-37   # a group whose scale is subnormal
            kind, mode, grid = q8_plan(eng, experts, gates, x)
            assert kind == fa.KIND_DECODE and mode == fa.MODE_Q8, (kind, mode)
            print(f"ref-q8 decode hidden={hidden} T={T} grid={grid}", flush=True)
            rc, y = eng.run(0, experts, gates, x, fa.MODE_Q8)
            assert rc == fa.OK
            rc, ref = oracle.ref_run(units, fa.FMT_Q4KT, True, oracle_request(0, experts, gates, x))
            assert rc == 0
            check_close(ref, y, fa.MODE_Q8, ("ref-q8 decode", hidden, T))
            rc, again = eng.run(0, experts, gates, x, fa.MODE_Q8)
            assert rc == fa.OK and np.array_equal(y.view(np.uint32), again.view(np.uint32))
            eng.route(fa.ROUTE_NO_DECODE)
            try:
                print(f"ref-q8 layer kernel hidden={hidden} T={T}", flush=True)
                rc, yl = eng.run(0, experts, gates, x, fa.MODE_Q8)
            finally:
                eng.route(0)
            assert rc == fa.OK
            check_close(yl, y, fa.MODE_Q8, ("ref-q8 decode vs layer kernel", hidden, T))
            for t in range(T if T > 1 else 0):
                rc, y1 = eng.run(0, experts[t:t + 1], gates[t:t + 1], x[t:t + 1], fa.MODE_Q8)
                assert rc == fa.OK
                assert np.array_equal(y1[0].view(np.uint32), y[t].view(np.uint32)), f"token {t} differs alone"
    finally:
        for b in range(20):
            eng.release(b)


def test_ref_q8_inexact_weights_run_on_layer_kernel(eng):
    """A super-block whose d and dmin exponents are far apart has float
    weights the reference rounds (src/native.c:22); the decode kernel flags
    it and run() repeats the request on layer_kernel, which decodes every
    weight as the reference does: the result meets the oracle at the Q8 bar,
    after two launches."""
    hidden, seed = 4096, 9090
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    rng = np.random.default_rng(9)
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
        e0 = int(experts[0, 0])
        view = slice_view(units[3], lay, 0, e0)
        view[0:4] = np.frombuffer(np.array([0x3FFF, 0x03FF], np.uint16).tobytes(), np.uint8)   # d 1.999, dmin subnormal
        assert eng.refresh(3, units[3], 0, e0) == fa.OK
        gates = np.zeros((1, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 1)
        x = rng.standard_normal((1, hidden)).astype(np.float32)
        before = eng.sample().runs
        print("ref-q8 inexact header", flush=True)
        rc, y = eng.run(0, experts, gates, x, fa.MODE_Q8)
        assert rc == fa.OK
        assert eng.sample().runs - before == 2
        rc, ref = oracle.ref_run(units, fa.FMT_Q4KT, True, oracle_request(0, experts, gates, x))
        assert rc == 0
        check_close(ref, y, fa.MODE_Q8, "ref-q8 inexact header")
    finally:
        for b in range(20):
            eng.release(b)


def test_ref_q8_decode_error_paths(eng):
    """decode_q8_kernel: a non-finite gate/up d, a non-finite down d and x at
    FLT_MAX give FR_NUMERIC with y untouched; the restored slice runs."""
    hidden, seed = 4096, 3131
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    rng = np.random.default_rng(31)
    for b in range(2):
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, seed) == fa.OK
    try:
        experts = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
        gates = np.zeros((1, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 1)
        x = rng.standard_normal((1, hidden)).astype(np.float32)
        e0 = int(experts[0, 3])
        unit = sparse_unit(lay)
        view = slice_view(unit, lay, 0, e0)
        view[:] = oracle.synth_slice(lay, seed, 1, 0, e0)
        good = view.copy()
        print("ref-q8 decode error paths", flush=True)
        rc, y = eng.run(0, experts, gates, np.full((1, hidden), np.finfo(np.float32).max, np.float32), fa.MODE_Q8)
        assert rc == fa.NUMERIC
        for off in (1, 2 * lay.proj + 1):   # high byte of a gate row's d, of a down row's d: 0x7C -> inf
            view[:] = good
            view[off] = 0x7C
            assert eng.refresh(1, unit, 0, e0) == fa.OK
            rc, y = eng.run(0, experts, gates, x, fa.MODE_Q8)
            assert rc == fa.NUMERIC and not y.any(), off
        view[:] = good
        assert eng.refresh(1, unit, 0, e0) == fa.OK
        rc, y = eng.run(0, experts, gates, x, fa.MODE_Q8)
        assert rc == fa.OK and np.isfinite(y).all()
    finally:
        for b in range(2):
            eng.release(b)


SPLIT_GRID = [(n, 4 if n <= 5 else 2 if n <= 11 else 1, h) for h in (4096, 2560) for n in range(1, 13)]


@pytest.mark.parametrize("nblocks,split,hidden", SPLIT_GRID)
def test_split_units_for_few_blocks(eng, nblocks, split, hidden):
    """A node that owns at most 5 (11) blocks splits each all-Q4_K unit into
    4 (2) items of fewer row-blocks (decode_split_kernel): a single token
    against the oracle and the layer kernel, bit for bit run to run, and a
    4-token burst whose rows are bit-identical to the tokens run alone (the
    split depends on the owned blocks only). Every block count 1..12 at
    hidden 4096 and 2560 (where three of the eight wavefronts own no
    super-block): a regression grid over both split kernels and the
    unsplit decode_kernel."""
    seed = 5150 + nblocks
    lay = oracle.layout(hidden, fa.FMT_Q4KT)
    rng = np.random.default_rng(nblocks)
    blocks = sorted(rng.choice(20, nblocks, replace=False).tolist())
    for b in blocks:
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, seed) == fa.OK
    try:
        burst = zipf_routes(rng, 4)
        single = burst[:1]
        units = [None] * 20
        for b in blocks:
            u = sparse_unit(lay)
            for e in set(int(v) for v in burst.ravel()):
                slice_view(u, lay, 0, e)[:] = oracle.synth_slice(lay, seed, b, 0, e)
            units[b] = u
        gates = np.zeros((4, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 4)
        x = rng.standard_normal((4, hidden)).astype(np.float32)
        plan, grid = eng.plan(0, single, gates[:1], x[:1], fa.MODE_F32)
        head = np.frombuffer(plan[:80].tobytes(), np.uint32)
        want = fa.KIND_DECODE if split == 1 else fa.KIND_DECODE_SPLIT
        assert int(head[16]) == want and (split == 1 or int(head[19]) == split), (head[16], head[19])
        assert grid == min(256, 10 * nblocks * split) or split == 1, grid
        print(f"split units: {nblocks} blocks, split {split}, grid {grid}", flush=True)
        rc, y = eng.run(0, single, gates[:1], x[:1], fa.MODE_F32)
        assert rc == fa.OK
        rc, ref = oracle.ref_run(units, fa.FMT_Q4KT, False, oracle_request(0, single, gates[:1], x[:1]))
        assert rc == 0
        check_close(ref, y, fa.MODE_F32, ("split", nblocks))
        rc, again = eng.run(0, single, gates[:1], x[:1], fa.MODE_F32)
        assert rc == fa.OK and np.array_equal(y.view(np.uint32), again.view(np.uint32))
        eng.route(fa.ROUTE_NO_DECODE)
        try:
            rc, y_lay = eng.run(0, single, gates[:1], x[:1], fa.MODE_F32)
        finally:
            eng.route(0)
        assert rc == fa.OK
        check_close(ref, y_lay, fa.MODE_F32, ("split vs layer", nblocks))
        # Unsplit bursts default to decode_burst_kernel (test_gpu_burst.py);
        # the unit route keeps burst rows bit-identical to single tokens.
        eng.route(fa.ROUTE_NO_BURST if split == 1 else 0)
        try:
            rc, yb = eng.run(0, burst, gates, x, fa.MODE_F32)
        finally:
            eng.route(0)
        assert rc == fa.OK
        rc, refb = oracle.ref_run(units, fa.FMT_Q4KT, False, oracle_request(0, burst, gates, x))
        assert rc == 0
        check_close(refb, yb, fa.MODE_F32, ("split burst", nblocks))
        for t in range(4):
            rc, y1 = eng.run(0, burst[t:t + 1], gates[t:t + 1], x[t:t + 1], fa.MODE_F32)
            assert rc == fa.OK
            assert np.array_equal(y1[0].view(np.uint32), yb[t].view(np.uint32)), f"token {t} differs alone"
    finally:
        for b in blocks:
            eng.release(b)
