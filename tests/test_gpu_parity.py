"""End-to-end parity of the single-launch layer kernel with the oracle.

Every test runs the HIP path through the C ABI (fr_hip_run) and compares it
with the restated reference run() (backends/ref.c:57-98) on the same bytes.
Tolerances (per token, fr_compare metrics of src/backend.c:74-92):
  F32 mode vs ref     relative L2 <= 1e-5 and normalized max <= 1e-3
  F64 mode vs ref     relative L2 <= 1e-9 (fp64 arithmetic, other order)
  Q8  mode vs ref-q8  relative L2 <= 1e-9 (bit-exact quantizers, fp64)
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import fill_experts, oracle_request, softmax_gates, sparse_unit, zipf_routes

pytestmark = pytest.mark.gpu

TOL = {fa.MODE_F32: (1e-5, 1e-3), fa.MODE_F64: (1e-9, 1e-8), fa.MODE_Q8: (1e-9, 1e-8)}


@pytest.fixture(scope="module")
def eng():
    e = fa.Engine(0)
    yield e
    for b in range(20):
        e.release(b)


def check_close(ref, got, mode, what=""):
    l2, mx = TOL[mode]
    for t in range(ref.shape[0]):
        rc, err = oracle.compare(ref[t], got[t])
        assert rc == 0, what
        assert err[0] <= l2 and err[1] <= mx, (what, t, err)


def run_both(eng, blocks, fmt, layer, experts, gates, x, mode):
    # Name the case before the launch so that a failure that ends the process
    # still says which one it was.
    print(f"case fmt={fmt} layer={layer} burst={x.shape[0]} hidden={x.shape[1]} mode={mode} "
          f"experts={np.asarray(experts).ravel()[:4].tolist()}...", flush=True)
    rc, y = eng.run(layer, experts, gates, x, mode)
    assert rc == fa.OK, (rc, mode)
    req = oracle_request(layer, experts, gates, x)
    rc, ref = oracle.ref_run(blocks, fmt, mode == fa.MODE_Q8, req)
    assert rc == 0
    return ref, y


@pytest.mark.parametrize("fmt", [fa.FMT_Q4KT, fa.FMT_Q8, fa.FMT_MXFP4, fa.FMT_NATIVE])
def test_h4096_baseline_distributions(eng, fmt):
    """Measurement-config weights at H=4096: 10 experts of 512, softmax gates,
    x ~ N(0,1), two owned blocks, T=1 and a Zipf T=4 burst."""
    lay = oracle.layout(4096, fmt)
    rng = np.random.default_rng(100 + fmt)
    layer = 5
    experts1 = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
    experts4 = zipf_routes(rng, 4)
    used = sorted(set(experts1.ravel()) | set(experts4.ravel()))
    units = {}
    for b in (3, 17):
        u = sparse_unit(lay)
        fill_experts(u, lay, layer, used, seed=b * 1000 + fmt)
        assert eng.load_sparse(b, u, 4096, fmt, [(layer, e) for e in used]) == fa.OK
        units[b] = u
    blocks = [units.get(b) for b in range(20)]
    try:
        for experts in (experts1, experts4):
            T = experts.shape[0]
            gates = np.zeros((T, 11), np.float32)
            gates[:, :10] = softmax_gates(rng, T)
            x = rng.standard_normal((T, 4096)).astype(np.float32)
            for mode in (fa.MODE_F32, fa.MODE_F64, fa.MODE_Q8):
                ref, y = run_both(eng, blocks, fmt, layer, experts, gates, x, mode)
                check_close(ref, y, mode, (fmt, T, mode))
    finally:
        for b in units:
            assert eng.release(b) == fa.OK


def test_legacy_golden_corpus(eng):
    """The reference's committed golden partials (tests/vectors/*) through the
    GPU legacy Q4_0 path: F64 within the reference reproducibility tolerance,
    F32 within the measurement tolerance."""
    import ctypes as C
    import os
    from test_oracle_golden import build_vector, golden_values, GOLDEN
    for index in range(8):
        req, mask, name, blocks, _ = build_vector(index)
        loaded = []
        used = sorted(set(int(e) for e in req.experts()[:req.burst].ravel()) | {512})
        for b in range(20):
            if blocks[b] is not None:
                # Only the fixture's slices are materialized: copy just those.
                assert eng.load_sparse(b, blocks[b], 2560, fa.FMT_LEGACY, [(req.layer, e) for e in used]) == fa.OK
                loaded.append(b)
        try:
            _, gold = golden_values(os.path.join(GOLDEN, name + ".txt"), req.burst)
            T = req.burst
            experts = req.experts()[:T]
            gates = req.gates()[:T]
            x = req.xs()[:T, :2560]
            for mode, limit in [(fa.MODE_F64, oracle.REFERENCE_TOLERANCE), (fa.MODE_F32, (1e-5, 1e-3, 0.9999))]:
                rc, y = eng.run(req.layer, experts, gates, x, mode)
                assert rc == fa.OK
                for t in range(T):
                    rc, err = oracle.compare(gold[t], y[t])
                    assert rc == 0 and oracle.conforms(err, limit), (name, mode, t, err)
        finally:
            for b in loaded:
                assert eng.release(b) == fa.OK


def test_state_errors(eng):
    rc, _ = eng.run(0, np.arange(10).reshape(1, 10), np.zeros((1, 11), np.float32), np.zeros((1, 4096), np.float32))
    assert rc == fa.STATE
