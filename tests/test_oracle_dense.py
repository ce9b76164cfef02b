"""Pins of the oracle's run() that do not go through its own loops.

1. Closed forms after tests/test_backend.c:113-161: Q4_0 slices whose gate and
   up rows are one-hot (weight 1.0 at column 0) with x[0] = 1 give a = u = 1,
   h = SiLU(1) = 1/(1+e^-1); a one-hot down row puts gate*SiLU(1) in y[0], so
   routed + shared gates and extra blocks add up as whole multiples.
2. Dense float64 restatement with numpy for every unit format, including
   the H=4096 ones the reference never runs (Q4_K with the transposed down,
   all-Q8_0, all-MXFP4): each row is dequantized (fo_dequant_row, pinned by
   the decoder KATs), the slice becomes dense matrices, and y is computed with
   matrix products in a different summation order, keeping the reference's
   narrowing points (a, u and h to fp32, backends/ref.c:76-95).
"""
import math

import numpy as np
import pytest

import oracle
from fixtures import dense_slice, fill_experts, oracle_request, slice_view, softmax_gates, sparse_unit

SILU1 = 1.0 / (1.0 + math.exp(-1.0))


def q4_0_row(n, hot=None):
    """Q4_0 row of n weights, all 0 except 1.0 at column `hot`."""
    groups = np.zeros((n // 32, 18), np.uint8)
    groups[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    groups[:, 2:] = 0x88                  # q = 8 -> (8 - 8) * 1.0 = 0
    if hot is not None:
        g, j = divmod(hot, 32)
        b = 2 + (j % 16)
        if j < 16:
            groups[g, b] = (groups[g, b] & 0xF0) | 9
        else:
            groups[g, b] = (groups[g, b] & 0x0F) | (9 << 4)
    return groups.ravel()


def one_hot_slice(lay):
    """Neuron 0: gate and up rows one-hot at column 0, down row 0 one-hot at
    neuron 0; everything else zero."""
    H = lay.hidden
    rows = [q4_0_row(H, 0 if n == 0 else None) for n in range(32)]
    gate = np.concatenate(rows)
    down = np.concatenate([q4_0_row(32, 0 if d == 0 else None) for d in range(H)])
    return np.concatenate([gate, gate, down])


def run_ref(units, fmt, layer, experts, gates, x, q8=False):
    req = oracle_request(layer, experts, gates, x)
    rc, y = oracle.ref_run(units, fmt, q8, req)
    assert rc == 0
    return y


def test_silu_closed_forms():
    lay = oracle.layout(2560, oracle.FMT_LEGACY)
    H, layer = 2560, 5
    s = one_hot_slice(lay)
    assert s.size == lay.slice
    u0, u1 = sparse_unit(lay), sparse_unit(lay)
    for u in (u0, u1):
        for e in (7, oracle.SHARED):
            slice_view(u, lay, layer, e)[:] = s
    x = np.zeros((8, H), np.float32)
    x[:, 0] = 1.0
    experts = np.array([[7] + list(range(100, 109))] * 8, np.uint16)
    gates = np.zeros((8, 11), np.float32)
    gates[:, 0] = 3.0
    # routed 3 alone, then + shared 2, then two blocks
    y = run_ref([u0] + [None] * 19, oracle.FMT_LEGACY, layer, experts[:1], gates[:1], x[:1])
    assert y[0, 0] == np.float32(3 * SILU1) and not np.any(y[0, 1:])
    gates[:, 10] = 2.0
    y = run_ref([u0] + [None] * 19, oracle.FMT_LEGACY, layer, experts[:1], gates[:1], x[:1])
    assert y[0, 0] == np.float32(5 * SILU1)
    y = run_ref([u0, u1] + [None] * 18, oracle.FMT_LEGACY, layer, experts, gates, x)
    assert y.shape == (8, H)
    assert np.all(y[:, 0] == np.float32(10 * SILU1)) and not np.any(y[:, 1:])
    # a routed expert with gate 0 still runs (and contributes nothing)
    gates[:, 0] = 0.0
    y = run_ref([u0] + [None] * 19, oracle.FMT_LEGACY, layer, experts[:1], gates[:1], x[:1])
    assert y[0, 0] == np.float32(2 * SILU1)


def dense_run(units, lay, layer, experts, gates, x):
    T, H = x.shape
    y = np.zeros((T, H))
    cache = {}
    for t in range(T):
        for e in range(11):
            shared = e == 10
            if shared and gates[t, e] == 0:
                continue
            eid = oracle.SHARED if shared else int(experts[t, e])
            for b, u in enumerate(units):
                if u is None:
                    continue
                key = (b, eid)
                if key not in cache:
                    cache[key] = dense_slice(slice_view(u, lay, layer, eid), lay, eid)
                Wg, Wu, Wd = cache[key]
                a = (Wg @ x[t].astype(np.float64)).astype(np.float32).astype(np.float64)
                uu = (Wu @ x[t].astype(np.float64)).astype(np.float32).astype(np.float64)
                sig = np.where(a >= 0, 1 / (1 + np.exp(-np.abs(a))), np.exp(-np.abs(a)) / (1 + np.exp(-np.abs(a))))
                h = (a * sig * uu).astype(np.float32).astype(np.float64)
                y[t] += float(gates[t, e]) * (Wd @ h)
    return y.astype(np.float32)


@pytest.mark.parametrize("hidden,fmt", [(2560, oracle.FMT_LEGACY), (2560, oracle.FMT_NATIVE), (4096, oracle.FMT_Q4KT),
                                        (4096, oracle.FMT_Q8), (4096, oracle.FMT_MXFP4), (4096, oracle.FMT_NATIVE)])
def test_dense_restatement(hidden, fmt):
    lay = oracle.layout(hidden, fmt)
    rng = np.random.default_rng(hidden + fmt)
    layer = 11
    experts = np.stack([rng.choice(512, 10, replace=False) for _ in range(2)]).astype(np.uint16)
    used = sorted(set(experts.ravel().tolist()) | {oracle.SHARED})
    units = [None] * 20
    for b in (2, 13):
        u = sparse_unit(lay)
        fill_experts(u, lay, layer, used, seed=b + 10 * fmt)
        units[b] = u
    gates = np.zeros((2, 11), np.float32)
    gates[:, :10] = softmax_gates(rng, 2)
    gates[1, 10] = 0.5
    x = rng.standard_normal((2, hidden)).astype(np.float32)
    ref = run_ref(units, fmt, layer, experts, gates, x)
    dense = dense_run(units, lay, layer, experts, gates, x)
    for t in range(2):
        rc, err = oracle.compare(dense[t], ref[t])
        assert rc == 0 and err[0] < 1e-9 and err[1] < 1e-8, (t, err)
