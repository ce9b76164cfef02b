"""The reference's native self-test fixture (src/native.c:66-135) on the GPU.

H=2560 native unit in block 19: experts 0..79 and the shared slice, LCG data,
every burst 1..8 with distinct and reused routing, in each arithmetic mode;
plus run-to-run determinism, burst invariance and the atomic-failure paths.
Tolerances as in test_gpu_parity.
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import native_fixture
from test_gpu_parity import check_close, run_both

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    return fa.Engine(0)


@pytest.fixture(scope="module")
def native2560(eng):
    """The reference native self-test fixture at H=2560 in block 19."""
    lay = oracle.layout(2560, oracle.FMT_NATIVE)
    data, gates, x = native_fixture(lay)
    assert eng.upload(19, data, 2560, fa.FMT_NATIVE) == fa.OK
    blocks = [None] * 20
    blocks[19] = data
    yield lay, data, gates, x, blocks
    assert eng.release(19) == fa.OK


@pytest.mark.parametrize("mode", [fa.MODE_F32, fa.MODE_F64, fa.MODE_Q8])
def test_native_fixture_all_bursts(eng, native2560, mode):
    """fr_native_self_test's request grid (src/native.c:77-93): distinct and
    reused routing, bursts 1..8, shared expert at gate 0.5."""
    lay, data, gates, x, blocks = native2560
    for reuse in (0, 1):
        for burst in range(1, 9):
            experts = np.array([[e + (0 if reuse else t * 10) for e in range(10)] for t in range(burst)])
            ref, y = run_both(eng, blocks, oracle.FMT_NATIVE, 47, experts, gates[:burst], x[:burst], mode)
            check_close(ref, y, mode, (reuse, burst))


def test_native_fixture_deterministic_and_burst_invariant(eng, native2560):
    lay, data, gates, x, blocks = native2560
    experts = np.array([[e + t * 3 for e in range(10)] for t in range(8)])
    rc, y8 = eng.run(47, experts, gates, x, fa.MODE_F32)
    assert rc == fa.OK
    rc, again = eng.run(47, experts, gates, x, fa.MODE_F32)
    assert np.array_equal(y8.view(np.uint32), again.view(np.uint32)), "run-to-run bits differ"
    same = 0
    for t in range(8):
        rc, y1 = eng.run(47, experts[t:t + 1], gates[t:t + 1], x[t:t + 1], fa.MODE_F32)
        assert rc == fa.OK
        same += np.array_equal(y1[0].view(np.uint32), y8[t].view(np.uint32))
        check_close(y1, y8[t:t + 1], fa.MODE_F32)
    # The request runs on the row-format decode kernel: (token, pair) units
    # summed per token in a fixed order, so every burst row is bit-identical
    # to its single-token run (src/native.c:94-117 checks this with memcmp).
    plan, _ = eng.plan(47, experts, gates, x, fa.MODE_F32)
    assert int(np.frombuffer(plan[64:68].tobytes(), np.uint32)[0]) == 2
    assert same == 8


@pytest.mark.parametrize("mode", [fa.MODE_F32, fa.MODE_Q8])
def test_native_error_paths(eng, native2560, mode):
    """x at FLT_MAX, a non-finite Q4_K d, an E8M0 255 down scale and a
    non-finite shared-expert Q8_0 scale each give FR_NUMERIC (the F32 and
    the ref-q8 row-format decode kernels), and the restored units run."""
    lay, data, gates, x, blocks = native2560
    experts = np.arange(10).reshape(1, 10)
    print(f"native error paths mode={mode}", flush=True)
    rc, y = eng.run(47, experts, gates[:1], np.full((1, 2560), np.finfo(np.float32).max, np.float32), mode)
    assert rc == fa.NUMERIC
    for off, val in [(oracle.slice_offset(lay, 47, 0) + 1, 0x7C),
                     (oracle.slice_offset(lay, 47, 0) + 2 * lay.proj, 255),
                     (oracle.slice_offset(lay, 47, 512) + 1, 0x7C)]:
        saved = data[off]
        data[off] = val
        layer, expert = 47, (512 if off >= oracle.slice_offset(lay, 47, 512) else 0)
        assert eng.refresh(19, data, layer, expert) == fa.OK
        rc, _ = eng.run(47, experts, gates[:1], x[:1], mode)
        assert rc == fa.NUMERIC, off
        data[off] = saved
        assert eng.refresh(19, data, layer, expert) == fa.OK
    rc, _ = eng.run(47, experts, gates[:1], x[:1], mode)
    assert rc == fa.OK
