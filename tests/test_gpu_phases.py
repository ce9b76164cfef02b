"""fr_hip_run's phase sample (fr_hip_phase_get), after the Metal backend's
encode/queue/gpu/return split (src/metal.h:9-15, backends/metal.m:572-585):
the host phases are taken on every call and add up to at most the call; the
GPU phase is measured only while phase events are on, and lies inside the
call."""
import numpy as np
import pytest

import fronk_amd as fa
from fixtures import softmax_gates

pytestmark = pytest.mark.gpu


def test_run_phases():
    eng = fa.Engine(0)
    hidden, nblocks = 4096, 4
    rng = np.random.default_rng(5)
    for b in range(nblocks):
        assert eng.synthetic(b, hidden, fa.FMT_Q4KT, 1, 77) == fa.OK
    try:
        experts = rng.choice(512, 10, replace=False).astype(np.uint16)[None]
        gates = np.zeros((1, 11), np.float32)
        gates[:, :10] = softmax_gates(rng, 1)
        x = rng.standard_normal((1, hidden)).astype(np.float32)
        print("phases: events off", flush=True)
        _, runs0 = eng.phases()
        for _ in range(3):
            rc, y = eng.run(0, experts, gates, x, fa.MODE_F32)
            assert rc == fa.OK
        ph, runs = eng.phases()
        assert runs == runs0 + 3
        for k in ("plan", "enqueue", "wait", "total"):
            assert ph[k] > 0, (k, ph)
        assert ph["gpu"] == 0 and ph["overhead"] == ph["total"], ph
        assert ph["plan"] + ph["enqueue"] + ph["wait"] <= ph["total"], ph
        print("phases: events on", flush=True)
        eng.phase_events(True)
        try:
            rc, y2 = eng.run(0, experts, gates, x, fa.MODE_F32)
            assert rc == fa.OK
        finally:
            eng.phase_events(False)
        assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
        ph, _ = eng.phases()
        assert 0 < ph["gpu"] < ph["total"], ph
        assert abs(ph["overhead"] - (ph["total"] - ph["gpu"])) < 1e-6 * ph["total"], ph
        # A call that fails before its kernels (a layer the blocks do not
        # hold) leaves the sample as it was.
        rc, _ = eng.run(1, experts, gates, x, fa.MODE_F32)
        assert rc == fa.STATE
        assert eng.phases() == (ph, runs + 1)
    finally:
        for b in range(nblocks):
            eng.release(b)
