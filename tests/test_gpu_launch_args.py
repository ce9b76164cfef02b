"""The decode launches take the plan header's fields and token table from the
host plan as kernel arguments: a host plan whose token table does not lie
within it is refused before any launch (FR_INVALID from fr_hip_launch and
fr_hip_launch_static alike), and the same plan, restored, runs and matches
run() bit for bit, for one token and for a 4-token Zipf burst (four entries
in the token table)."""
import ctypes as C

import numpy as np
import pytest

import fronk_amd as fa
from fixtures import softmax_gates, zipf_routes

pytestmark = pytest.mark.gpu

H = 4096
GROUPS_OFF = 11   # word index of groups_off in the 80-byte plan header
TOTAL = 13        # word index of total


def launch(lib, plan, dplan, stream, T):
    rc = lib.fr_hip_launch(plan.ctypes.data, C.c_void_p(dplan.data_ptr()), stream)
    if rc != fa.OK:
        return rc, None
    y = np.zeros(T * H, np.float32)
    st = C.c_uint(0)
    assert lib.fr_hip_last_output(stream, fa.fptr(y), T * H, C.byref(st)) == fa.OK
    assert st.value == 0
    return rc, y.reshape(T, H)


def test_header_args_refused_and_restored():
    import torch
    lib = fa.lib()
    eng = fa.Engine(0)
    rng = np.random.default_rng(9090)
    s = torch.cuda.Stream()
    sp = C.c_void_p(s.cuda_stream)
    ydev = torch.zeros((H,), dtype=torch.float32, device="cuda")
    sdev = torch.zeros((1,), dtype=torch.int32, device="cuda")
    for b in range(20):
        assert eng.synthetic(b, H, fa.FMT_Q4KT, 1, 9100 + b) == fa.OK
    try:
        for T in (1, 4):
            experts = zipf_routes(rng, T) if T > 1 else rng.choice(512, 10, replace=False).astype(np.uint16)[None]
            gates = np.zeros((T, 11), np.float32)
            gates[:, :10] = softmax_gates(rng, T)
            x = rng.standard_normal((T, H)).astype(np.float32)
            plan, grid = eng.plan(0, experts, gates, x, fa.MODE_F32)
            head = plan[:80].view(np.uint32)
            dplan = torch.from_numpy(plan.copy()).to("cuda")
            print(f"launch args T={T}: kind {int(head[16])}, {int(head[3])} pairs, grid {grid}", flush=True)
            assert int(head[16]) in (fa.KIND_DECODE, fa.KIND_DECODE_SPLIT, fa.KIND_DECODE_ROWS, fa.KIND_DECODE_BURST)
            good = head.copy()
            for bad_off in (int(head[TOTAL]), int(head[TOTAL]) - 4, 8):
                head[GROUPS_OFF] = bad_off
                assert lib.fr_hip_launch(plan.ctypes.data, C.c_void_p(dplan.data_ptr()), sp) == fa.INVALID, bad_off
                if T == 1:
                    assert lib.fr_hip_launch_static(plan.ctypes.data, C.c_void_p(dplan.data_ptr()),
                                                    C.c_void_p(ydev.data_ptr()), C.c_void_p(sdev.data_ptr()),
                                                    sp) == fa.INVALID, bad_off
            head[:] = good
            rc, y = launch(lib, plan, dplan, sp, T)
            assert rc == fa.OK
            rc2, yr = eng.run(0, experts, gates, x, fa.MODE_F32)
            assert rc2 == fa.OK
            assert np.array_equal(y.view(np.uint32), np.asarray(yr, np.float32).reshape(T, H).view(np.uint32)), T
    finally:
        for b in range(20):
            eng.release(b)
