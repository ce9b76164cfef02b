"""fr_hip_launch_static: the launch that allocates nothing (for callers under
graph capture or in loops that forbid hipMalloc). Its unit partials live in
the library's static device array; y and the status word are the caller's.

Checked against the engine's own launch of the same plan (fr_hip_launch +
fr_hip_last_output) bit for bit, on calls in a row with fewer owned blocks
each: 20 (decode_kernel, 200 units), 10 (units split in 2: 200 items) and 3
(split in 4: 120 items), and on the error path; plans it does not run return
FR_UNSUPPORTED. Then the reference's own unit format with the shared expert
(decode_rows_kernel, 220 units), and the launch captured in a graph and
replayed with new plans.
"""
import ctypes as C

import numpy as np
import pytest

import fronk_amd as fa
from fixtures import softmax_gates, zipf_routes

pytestmark = pytest.mark.gpu

H = 4096


def device_plan(plan):
    import torch
    return torch.from_numpy(plan.copy()).to("cuda")


def engine_launch(lib, plan, dplan, stream):
    assert lib.fr_hip_launch(plan.ctypes.data, C.c_void_p(dplan.data_ptr()), stream) == fa.OK
    y = np.zeros(H, np.float32)
    st = C.c_uint(0)
    assert lib.fr_hip_last_output(stream, fa.fptr(y), H, C.byref(st)) == fa.OK
    return y, st.value


def static_launch(lib, plan, dplan, ydev, sdev, stream):
    import torch
    rc = lib.fr_hip_launch_static(plan.ctypes.data, C.c_void_p(dplan.data_ptr()), C.c_void_p(ydev.data_ptr()),
                                  C.c_void_p(sdev.data_ptr()), stream)
    if rc != fa.OK:
        return rc, None, None
    torch.cuda.synchronize()
    return rc, ydev.cpu().numpy().copy(), int(sdev.cpu().numpy()[0])


def test_static_launch_matches_engine_launch():
    import torch
    lib = fa.lib()
    eng = fa.Engine(0)
    rng = np.random.default_rng(77)
    s = torch.cuda.Stream()
    sp = C.c_void_p(s.cuda_stream)
    # The caller's outputs, filled with garbage that the launch must replace.
    ydev = torch.full((H,), float("nan"), dtype=torch.float32, device="cuda")
    sdev = torch.full((1,), 0x5A5A, dtype=torch.int32, device="cuda")
    for b in range(20):
        assert eng.synthetic(b, H, fa.FMT_Q4KT, 1, 4040 + b) == fa.OK
    try:
        for call, blocks in enumerate((20, 10, 3)):
            for b in range(blocks, 20):
                eng.release(b)
            experts = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
            gates = np.zeros((1, 11), np.float32)
            gates[:, :10] = softmax_gates(rng, 1)
            x = rng.standard_normal((1, H)).astype(np.float32)
            plan, grid = eng.plan(0, experts, gates, x, fa.MODE_F32)
            head = plan[:80].view(np.uint32)
            npairs = int(head[3])
            assert npairs == 10 * blocks
            assert int(head[16]) == (fa.KIND_DECODE if blocks > 11 else fa.KIND_DECODE_SPLIT)
            dplan = device_plan(plan)
            print(f"static launch call {call}: {npairs} units, grid {grid}", flush=True)
            rc, ys, st = static_launch(lib, plan, dplan, ydev, sdev, sp)
            assert rc == fa.OK and st == 0, (rc, st)
            ye, ste = engine_launch(lib, plan, dplan, sp)
            assert ste == 0
            assert np.array_equal(ys.view(np.uint32), ye.view(np.uint32)), call
        # Error path: an fp32 overflow sets the status word; then a clean
        # call clears it.
        print("static launch error path", flush=True)
        big = np.full((1, H), 3e38, np.float32)
        plan, _ = eng.plan(0, experts, gates, big, fa.MODE_F32)
        rc, _, st = static_launch(lib, plan, device_plan(plan), ydev, sdev, sp)
        assert rc == fa.OK and st != 0
        plan, _ = eng.plan(0, experts, gates, x, fa.MODE_F32)
        dplan = device_plan(plan)
        rc, ys, st = static_launch(lib, plan, dplan, ydev, sdev, sp)
        assert rc == fa.OK and st == 0
        ye, _ = engine_launch(lib, plan, dplan, sp)
        assert np.array_equal(ys.view(np.uint32), ye.view(np.uint32))
        # Plans it does not run: a 4-token burst, a layer_kernel plan.
        ex4 = zipf_routes(rng, 4)
        g4 = np.zeros((4, 11), np.float32)
        g4[:, :10] = softmax_gates(rng, 4)
        plan4, _ = eng.plan(0, ex4, g4, rng.standard_normal((4, H)).astype(np.float32), fa.MODE_F32)
        assert lib.fr_hip_launch_static(plan4.ctypes.data, C.c_void_p(device_plan(plan4).data_ptr()),
                                        C.c_void_p(ydev.data_ptr()), C.c_void_p(sdev.data_ptr()), sp) == fa.UNSUPPORTED
        planf, _ = eng.plan(0, experts, gates, x, fa.MODE_F64)
        assert lib.fr_hip_launch_static(planf.ctypes.data, C.c_void_p(device_plan(planf).data_ptr()),
                                        C.c_void_p(ydev.data_ptr()), C.c_void_p(sdev.data_ptr()), sp) == fa.UNSUPPORTED
    finally:
        for b in range(20):
            eng.release(b)


def test_static_launch_rows_kernel_and_graph_replays():
    """The reference's own unit format (Q4_K gate/up, MXFP4 down) with the
    shared expert: 220 units on decode_rows_kernel, static launch against the
    engine launch bit for bit. Then the static launch captured once in a
    graph on a side stream and replayed three times, each time with a new
    plan of the same shape copied into the captured plan buffer and eager work
    of the program between the replays: every replay equals the engine's
    launch of its plan bit for bit."""
    import torch
    lib = fa.lib()
    eng = fa.Engine(0)
    rng = np.random.default_rng(78)
    s = torch.cuda.Stream()
    sp = C.c_void_p(s.cuda_stream)
    ydev = torch.full((H,), float("nan"), dtype=torch.float32, device="cuda")
    sdev = torch.full((1,), 0x5A5A, dtype=torch.int32, device="cuda")
    for b in range(20):
        assert eng.synthetic(b, H, fa.FMT_NATIVE, 1, 5050 + b) == fa.OK
    try:
        def request():
            experts = rng.choice(512, 10, replace=False).astype(np.uint16).reshape(1, 10)
            gates = np.zeros((1, 11), np.float32)
            gates[:, :10] = softmax_gates(rng, 1)
            gates[0, 10] = 0.5
            return experts, gates, rng.standard_normal((1, H)).astype(np.float32)

        plan, grid = eng.plan(0, *request(), fa.MODE_F32)
        head = plan[:80].view(np.uint32)
        assert int(head[16]) == fa.KIND_DECODE_ROWS and int(head[3]) == 220, (head[16], head[3])
        dplan = device_plan(plan)
        print(f"static launch, native units with the shared expert: grid {grid}", flush=True)
        rc, ys, st = static_launch(lib, plan, dplan, ydev, sdev, sp)
        assert rc == fa.OK and st == 0, (rc, st)
        ye, _ = engine_launch(lib, plan, dplan, sp)
        assert np.array_equal(ys.view(np.uint32), ye.view(np.uint32))

        # Capture: one static launch into a graph on the side stream.
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
            assert lib.fr_hip_launch_static(plan.ctypes.data, C.c_void_p(dplan.data_ptr()),
                                            C.c_void_p(ydev.data_ptr()), C.c_void_p(sdev.data_ptr()),
                                            C.c_void_p(s.cuda_stream)) == fa.OK
        torch.cuda.synchronize()
        for rep in range(3):
            nplan, ngrid = eng.plan(0, *request(), fa.MODE_F32)
            assert ngrid == grid and nplan.size == plan.size
            dplan.copy_(torch.from_numpy(nplan.copy()))
            filler = torch.randn(1 << 20, device="cuda").sum()   # the program's own eager work
            torch.cuda.synchronize()
            print(f"graph replay {rep}", flush=True)
            g.replay()
            torch.cuda.synchronize()
            got = ydev.cpu().numpy().copy()
            assert int(sdev.cpu().numpy()[0]) == 0
            want, _ = engine_launch(lib, nplan, dplan, sp)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
            del filler
    finally:
        for b in range(20):
            eng.release(b)
