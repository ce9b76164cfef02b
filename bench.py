#!/usr/bin/env python3
"""Layer-share measurement of the expert neuron-slice path on one MI355X.

A step is one layer call of the node backend's run() (src/backend.h:63): the
launch of one decode kernel over every (token, routed expert, owned 32-neuron
slice) unit of a request, then its fixed-order reduction kernel (the Q4_K
workloads run decode_kernel, the Q8_0 / MXFP4 / native ones
decode_rows_kernel). Default workload: 512 experts x 20 owned slices resident at
hidden=4096, all Q4_K (down stored transposed), one token, 10 experts drawn
uniformly without replacement, gates = softmax of N(0,1) logits, x ~ N(0,1).
Weights are synthetic (seeded, generated on the device), resident in HBM
before timing; calls rotate over 8 resident layers so that the working set
between reuses is far beyond the 256 MB Infinity Cache. Each step's launch
plan (routing, gates, x) is also resident in HBM when timing starts.

stdout: exactly one JSON line. Everything else goes to stderr.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload q4k]
                  [--cpu-seconds S] [--no-cpu] [--blocks N] [--mode f32]
                  workloads: q4k (the default), mtp4 (4-token Zipf burst),
                  q8, mxfp4 (all-Q8_0 / all-MXFP4 shares), native (Q4_K
                  gate/up with an MXFP4 down); --blocks N owns N of the 20
                  slices (1: config 1), --mode q8 / q8_256 runs the ref-q8 /
                  AVX2 arithmetic (either skips the other legs)
  python bench.py --workload prefill   a step is one 48-layer chunk of 512
                                        tokens through fr_hip_run_batch
                                        (prefill_native: the reference's own
                                        units with the shared expert)
  python bench.py --copy-kernel BYTES   plain device copy, for scaling the
                                        FETCH_SIZE/WRITE_SIZE counters
  python bench.py --traffic-summary FETCH WRITE COPY_FETCH COPY_WRITE
                  --copy-kernel BYTES [--workload q4k]
                                        (no GPU) writes
                                        profiles/decode_<workload>_traffic.json
                                        from four rocprofv3 --pmc output
                                        directories: the workload's FETCH_SIZE
                                        and WRITE_SIZE runs and the copy
                                        kernel's; the headline line then
                                        reports those bytes as roofline.traffic
                                        while the kernel source is the one
                                        counted
"""
import argparse
import ctypes as C
import csv
import glob
import hashlib
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "quantized-weight GB/s (% HBM peak) + MoE layer-share tokens/s, 1 MI355X"
HBM_PEAK_GBS = 8000.0
HIDDEN = 4096
SLICES = 20
LAYERS = 8
SEED = 0x4652_4F4E_4B00_0002

WORKLOADS = {
    "q4k": dict(fmt="FMT_Q4KT", burst=1, routing="uniform",
                text="MoE layer-share decode: 10 of 512 experts x 20 owned slices x 32 neurons, hidden 4096, "
                     "Q4_K gate/up/down (down stored transposed), 1 token"),
    "q8": dict(fmt="FMT_Q8", burst=1, routing="uniform",
               text="MoE layer-share decode: 10 of 512 experts x 20 slices, hidden 4096, Q8_0 gate/up/down, 1 token"),
    "mxfp4": dict(fmt="FMT_MXFP4", burst=1, routing="uniform",
                  text="MoE layer-share decode: 10 of 512 experts x 20 slices, hidden 4096, MXFP4 gate/up/down, "
                       "1 token"),
    "native": dict(fmt="FMT_NATIVE", burst=1, routing="uniform",
                   text="MoE layer-share decode: 10 of 512 experts x 20 slices, hidden 4096, Q4_K gate/up, "
                        "MXFP4 down [H x 32], 1 token"),
    "mtp4": dict(fmt="FMT_Q4KT", burst=4, routing="zipf",
                 text="MoE layer-share burst: 4 tokens, per-token top-10 of 512 under Zipf(1.1), 20 slices, "
                      "hidden 4096, Q4_K (down transposed); bytes counted once per unique expert"),
    "shared4": dict(fmt="FMT_Q4KT", burst=4, routing="shared",
                    text="MoE layer-share burst: 4 tokens routed to the same 10 of 512 experts (each in its own "
                         "order), 20 slices, hidden 4096, Q4_K (down transposed); bytes counted once per unique "
                         "expert"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def softmax_gates(rng, burst):
    logits = rng.standard_normal((burst, 10))
    g = np.exp(logits - logits.max(axis=1, keepdims=True))
    out = np.zeros((burst, 11), np.float32)
    out[:, :10] = g / g.sum(axis=1, keepdims=True)
    return out


def draw_routes(rng, burst, routing, zipf_perm, zipf_p):
    if routing == "uniform":
        return np.stack([rng.choice(512, 10, replace=False) for _ in range(burst)]).astype(np.uint16)
    if routing == "shared":
        base = rng.choice(512, 10, replace=False)
        return np.stack([rng.permutation(base) for _ in range(burst)]).astype(np.uint16)
    return np.stack([zipf_perm[rng.choice(512, 10, replace=False, p=zipf_p)] for _ in range(burst)]).astype(np.uint16)


def make_requests(n, burst, routing, seed):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(512)
    p = 1.0 / np.arange(1, 513) ** 1.1
    p /= p.sum()
    reqs = []
    for i in range(n):
        experts = draw_routes(rng, burst, routing, perm, p)
        gates = softmax_gates(rng, burst)
        x = rng.standard_normal((burst, HIDDEN)).astype(np.float32)
        reqs.append((i % LAYERS, experts, gates, x))
    return reqs


def algorithmic_bytes(fa, fmt, experts, gates, blocks=SLICES):
    """Weight bytes read once per unique (expert, owned slice) over `blocks`
    owned slices, plus x and y (4*T*H bytes each)."""
    T = experts.shape[0]
    lay_slice, lay_shared = slice_sizes(fa, fmt)
    unique = len(set(int(e) for e in experts.ravel()))
    weights = unique * blocks * lay_slice
    if np.any(gates[:, 10] != 0):
        weights += blocks * lay_shared
    return weights, weights + 8 * T * HIDDEN


def slice_sizes(fa, fmt):
    # Slice sizes follow from the unit size: 48 layers x (512 routed + shared).
    routed = {fa.FMT_Q4KT: 221184, fa.FMT_Q8: 417792, fa.FMT_MXFP4: 208896, fa.FMT_NATIVE: 217088}[fmt]
    shared = 3 * (HIDDEN // 32) * 34 * 32
    assert fa.unit_bytes(HIDDEN, fmt) == 48 * (512 * routed + shared)
    return routed, shared


def grid_kernels(lib, plan):
    """The kernels one launch of this plan runs (plan header fields `kind` and `mode`)."""
    head = np.frombuffer(plan[:80].tobytes(), np.uint32)
    kind, mode = int(head[16]), int(head[2])
    if mode == 2 and kind in (1, 2):
        return ("decode_q8_kernel" if kind == 1 else "decode_rows_q8_kernel") + " + decode_reduce"
    if mode == 3 and kind == 2:
        return "decode_rows_q8_kernel (q8_256) + decode_reduce"
    return {1: "decode_kernel + decode_reduce", 2: "decode_rows_kernel + decode_reduce",
            3: "decode_split_kernel + decode_reduce", 4: "decode_burst_kernel + decode_reduce"}.get(kind, "layer_kernel")


def plan_slices(plan):
    """(device address, bytes) of every unit of a layer plan: the plan header's
    pair count (byte 12) and pair table offset (byte 40), 48-byte pair
    descriptors with the slice address at 0 and the gate-row bytes at 8 (a
    Q4_K slice is three such projections)."""
    npairs = int(np.frombuffer(plan[12:16].tobytes(), np.uint32)[0])
    off = int(np.frombuffer(plan[40:44].tobytes(), np.uint32)[0])
    desc = np.frombuffer(plan[off:off + 48 * npairs].tobytes(), np.uint8).reshape(npairs, 48)
    addr = desc[:, 0:8].copy().view(np.uint64).ravel()
    proj = desc[:, 8:12].copy().view(np.uint32).ravel().astype(np.uint64)
    return addr, 3 * proj


def cut_pieces(addr, length, parts):
    """Each (address, length) range cut into `parts` 16-byte aligned pieces."""
    out = []
    for a, n in zip(addr.tolist(), length.tolist()):
        step = ((n + parts - 1) // parts + 15) // 16 * 16
        for p in range(parts):
            lo = p * step
            if lo < n:
                out.append((a + lo, min(step, n - lo)))
    return np.array(out, np.uint64).reshape(-1, 2)


def time_probe(lib, tables, threads, depth, reps, sink, stream):
    """Events around `reps` probe launches on `stream`, rotating over the
    device piece tables; returns microseconds per launch."""
    import torch
    sptr = C.c_void_p(stream.cuda_stream)

    def go(i):
        t = tables[i % len(tables)]
        fa_rc = lib.fr_hip_stream_probe(C.c_void_p(t.data_ptr()), t.shape[0], threads, depth,
                                        C.c_void_p(sink.data_ptr()), sptr)
        if fa_rc != 0:
            raise RuntimeError(f"fr_hip_stream_probe failed with {fa_rc}")

    for i in range(len(tables)):
        go(i)
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(reps):
            go(i)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):   # replay() runs on the current stream
        g.replay()
        stream.synchronize()
        ev0.record(stream)
        g.replay()
        ev1.record(stream)
    stream.synchronize()
    return ev0.elapsed_time(ev1) * 1e3 / reps


def stream_ceiling(eng, lib, plans, sweep, reps=200):
    """Achievable read bandwidth for the decode workload: the probe reading
    (a) the same scattered per-unit slices as the layer plans `plans` and
    (b) one contiguous buffer of the same size per call, rotated over 8
    buffers (beyond the 256 MB Infinity Cache), over `sweep` = [(pieces per
    slice or total pieces, threads, depth)]. Returns the table and the best
    rate of each kind."""
    import torch
    slices = [plan_slices(p) for p in plans]
    total = int(slices[0][1].sum())
    stream = torch.cuda.Stream()
    sink = torch.zeros(16 * 8192, dtype=torch.int32, device="cuda")
    region = torch.empty(8 * ((total + 4095) // 4096 * 4096), dtype=torch.uint8, device="cuda")
    region.fill_(7)
    base = region.data_ptr()
    rows, best = [], {}
    for kind, parts, threads, depth in sweep:
        tables = []
        for i, (addr, length) in enumerate(slices[:8]):
            if kind == "scattered":
                pc = cut_pieces(addr, length, parts)
            else:
                start = base + i * ((total + 4095) // 4096 * 4096)
                pc = cut_pieces(np.array([start], np.uint64), np.array([total], np.uint64), parts)
            tables.append(torch.from_numpy(pc.view(np.int64).copy()).to("cuda"))
        us = time_probe(lib, tables, threads, depth, reps, sink, stream)
        gbs = total / (us * 1e-6) / 1e9
        rows.append({"kind": kind, "workgroups": int(tables[0].shape[0]), "threads": threads,
                     "depth": depth, "in_flight_kib_per_wg": threads * depth * 16 // 1024,
                     "us": round(us, 3), "gbs": round(gbs, 1)})
        log(f"stream {kind:10s} wg={rows[-1]['workgroups']:5d} threads={threads:4d} depth={depth} "
            f"{us:8.3f} us {gbs:8.1f} GB/s")
        if gbs > best.get(kind, {}).get("gbs", 0):
            best[kind] = rows[-1]
    return rows, best, total


def bench_stream(args):
    """--workload stream: the achievable-bandwidth sweep over the decode
    workload's own slices and over a contiguous buffer of the same size."""
    import torch
    import fronk_amd as fa
    lib = fa.lib()
    eng = fa.Engine(0)
    for b in range(SLICES):
        fa.check(eng.synthetic(b, HIDDEN, fa.FMT_Q4KT, LAYERS, SEED), "fr_hip_synthetic")
    reqs = make_requests(8, 1, "uniform", SEED + 1)
    plans = [eng.plan(*r, fa.MODE_F32)[0] for r in reqs]
    sweep = [("scattered", p, t, d) for p in (1, 2, 4) for t in (256, 512, 1024) for d in (1, 2, 4)]
    sweep += [("contiguous", g, t, d) for g in (200, 256, 512, 1024) for t in (256, 512, 1024) for d in (1, 2, 4)]
    rows, best, total = stream_ceiling(eng, lib, plans, sweep)
    for b in range(SLICES):
        eng.release(b)
    sc = best["scattered"]
    print(json.dumps({
        "metric": "achievable HBM read GB/s (streaming probe over the decode slices)",
        "value": sc["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": 64, "warmup": 8,
        "ms_per_step": round(sc["us"] * 1e-3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u8", "data": "synthetic",
        "config": {"workload": "read the 200 Q4_K slices (221,184 B) of a 10-of-512 x 20-slice layer share, "
                               "or one contiguous buffer of the same size, rotated over 8 layers",
                   "bytes_per_call": total},
        "best": best, "sweep": rows, "peak": HBM_PEAK_GBS,
    }), flush=True)


def copy_kernel(nbytes):
    import torch
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "launches": 5}))


def cpu_baseline(fa, eng, fmt, reqs, budget_s):
    """The oracle's scalar restatement of the reference ref backend
    (backends/ref.c:57-98), one host thread, on a bounded sample of the same
    requests; the GPU's outputs for the same requests are compared with it."""
    import oracle
    from fixtures import host_units
    lay = oracle.layout(HIDDEN, fmt)
    done, seconds, wbytes = 0, 0.0, 0
    worst = [0.0, 0.0, 0.0, 0.0]   # rel. L2, normalized max, absolute max-abs, max |y_ref|
    for layer, experts, gates, x in reqs:
        units = host_units(lay, SEED, layer, experts)
        req = oracle.Req()
        req.layer, req.burst, req.hidden = layer, experts.shape[0], HIDDEN
        req.experts()[:req.burst] = experts
        req.gates()[:req.burst] = gates
        req.xs()[:req.burst, :HIDDEN] = x
        t0 = time.perf_counter()
        rc, ref = oracle.ref_run(units, fmt, False, req)
        seconds += time.perf_counter() - t0
        if rc != 0:
            raise RuntimeError(f"oracle ref_run failed with {rc}")
        rc, y = eng.run(layer, experts, gates, x, fa.MODE_F32)
        if rc != fa.OK:
            raise RuntimeError(f"fr_hip_run failed with {rc}")
        for t in range(req.burst):
            rc, err = oracle.compare(ref[t], y[t])
            worst = [max(worst[0], err[0]), max(worst[1], err[1]),
                     max(worst[2], float(np.max(np.abs(y[t].astype(np.float64) - ref[t])))),
                     max(worst[3], float(np.max(np.abs(ref[t]))))]
        wbytes += algorithmic_bytes(fa, fmt, experts, gates)[0]
        done += 1
        del units
        if seconds >= budget_s:
            break
    return {
        "value": wbytes / seconds / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"{done} calls of this workload through the oracle's scalar restatement of ref "
                  f"(backends/ref.c:57-98), 1 thread, {seconds:.1f} s",
        "tokens_per_s": done * reqs[0][1].shape[0] / seconds,
        "gpu_vs_oracle": {"rel_l2_max": worst[0], "normalized_max": worst[1], "abs_max": worst[2],
                          "ref_abs_max": worst[3], "calls": done},
    }


PREFILL_LAYERS = 48
PREFILL_TOKENS = 512
MFMA_F16_PEAK_TFLOPS = 2500.0   # dense f16/bf16 matrix cores (the prefill GEMMs' instructions)
PREFILL_TEXT = ("Resident node prefill: 48 layers x 512 experts x 640 intermediate x hidden 4096, all Q4_K "
                "(down transposed, 108.7 GB in HBM); a chunk of 512 tokens, top-10 of 512 uniform per token per "
                "layer, through fr_hip_run_batch (f16 matrix cores on exact operands and exactly split x and h, fp32 "
                "accumulation)")
PREFILL_NATIVE_TEXT = ("Resident node prefill on the reference's own units: 48 layers x 512 experts x hidden 4096, "
                       "Q4_K gate/up rows, MXFP4 down, Q8_0 shared expert (106.7 GB in HBM); a chunk of 512 tokens, "
                       "top-10 of 512 uniform per token per layer and the shared expert at gate 0.5 on every token, "
                       "through fr_hip_run_batch (f16 matrix cores for gate/up, bf16 matrix cores for the downs, on exact "
                       "operands and exactly split x and h)")


def prefill_requests(rng, layers, tokens, shared=0.0):
    reqs = []
    for layer in range(layers):
        experts = np.argsort(rng.random((tokens, 512)), axis=1)[:, :10].astype(np.uint16)
        gates = softmax_gates(rng, tokens)
        gates[:, 10] = shared
        reqs.append((layer, experts, gates, rng.standard_normal((tokens, HIDDEN)).astype(np.float32)))
    return reqs


def prefill_cpu_baseline(fa, y0, req, budget_s, fmt=None):
    """Bursts of 8 tokens of the chunk's layer 0 (the reference client's cut,
    client/fronk_client.h:41-42) through the oracle's scalar restatement of
    ref (backends/ref.c:57-98), one host thread; bytes are each burst's unique
    experts x 20 slices. The chunk's GPU rows are compared with it."""
    import oracle
    from fixtures import host_units, oracle_request
    fmt = fa.FMT_Q4KT if fmt is None else fmt
    lay = oracle.layout(HIDDEN, fmt)
    layer, experts, gates, x = req
    done, seconds, wbytes, worst = 0, 0.0, 0, [0.0, 0.0, 0.0, 0.0]
    for t0 in range(0, experts.shape[0], 8):
        sl = slice(t0, t0 + 8)
        units = host_units(lay, SEED, layer, experts[sl])
        t1 = time.perf_counter()
        rc, ref = oracle.ref_run(units, fmt, False, oracle_request(layer, experts[sl], gates[sl], x[sl]))
        seconds += time.perf_counter() - t1
        if rc != 0:
            raise RuntimeError(f"oracle ref_run failed with {rc}")
        for t in range(ref.shape[0]):
            rc, err = oracle.compare(ref[t], y0[t0 + t])
            worst = [max(worst[0], err[0]), max(worst[1], err[1]),
                     max(worst[2], float(np.max(np.abs(y0[t0 + t].astype(np.float64) - ref[t])))),
                     max(worst[3], float(np.max(np.abs(ref[t]))))]
        wbytes += len(set(experts[sl].ravel().tolist())) * SLICES * lay.slice
        if np.any(gates[sl, 10] != 0):
            wbytes += SLICES * lay.shared_slice
        done += ref.shape[0]
        del units
        if seconds >= budget_s:
            break
    return {
        "value": wbytes / seconds / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"{done} tokens of layer 0 in bursts of 8 through the oracle's scalar restatement of ref "
                  f"(backends/ref.c:57-98), 1 thread, {seconds:.1f} s",
        "tokens_per_s": done / seconds,
        "gpu_vs_oracle": {"rel_l2_max": worst[0], "normalized_max": worst[1], "abs_max": worst[2],
                          "ref_abs_max": worst[3], "tokens": done},
    }


def prefill_leg(fa, lib, eng, steps, warmup, fmt=None, shared=0.0):
    """Config 5 on the device: 48 layers x 20 blocks of synthetic Q4_K resident,
    one 512-token chunk per step through fr_hip_batch_launch, timed with
    events on the launch stream (fmt: the unit format, Q4_K-T by default;
    shared: the shared expert's gate on every token, 0 for none). Returns the
    measures and the first layer's request (for the CPU leg); the blocks stay
    resident for the caller."""
    import torch
    fmt = fa.FMT_Q4KT if fmt is None else fmt
    t0 = time.perf_counter()
    for b in range(SLICES):
        fa.check(eng.synthetic(b, HIDDEN, fmt, PREFILL_LAYERS, SEED), "fr_hip_synthetic")
    log(f"resident: {SLICES} blocks x {PREFILL_LAYERS} layers generated in {time.perf_counter() - t0:.1f} s")
    reqs = prefill_requests(np.random.default_rng(SEED + 5), PREFILL_LAYERS, PREFILL_TOKENS, shared)
    slice_bytes, shared_bytes = slice_sizes(fa, fmt)
    cap = lib.fr_hip_batch_plan_bytes(PREFILL_TOKENS, HIDDEN)
    stride = (cap + 255) // 256 * 256
    host = np.zeros((PREFILL_LAYERS, stride), np.uint8)
    wts = np.zeros(PREFILL_LAYERS)
    for i, (layer, experts, gates, x) in enumerate(reqs):
        plan = eng.batch_plan(layer, experts, gates, x)
        host[i, :plan.size] = plan
        wts[i] = len(set(experts.ravel().tolist())) * SLICES * slice_bytes + (SLICES * shared_bytes if shared else 0)
    dev = torch.from_numpy(host).to("cuda")
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    hptr, dptr, sptr = host.ctypes.data, dev.data_ptr(), C.c_void_p(stream.cuda_stream)

    def chunk():
        for i in range(PREFILL_LAYERS):
            rc = lib.fr_hip_batch_launch(C.c_void_p(hptr + i * stride), C.c_void_p(dptr + i * stride), sptr)
            if rc != fa.OK:
                raise RuntimeError(f"fr_hip_batch_launch failed with {rc}")

    for _ in range(warmup):
        chunk()
    stream.synchronize()
    log(f"warm: {warmup} chunks")
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(steps):
            chunk()
        ev1.record(stream)
    stream.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    chunk_ms = ev0.elapsed_time(ev1) / steps
    log(f"timed: {steps} chunks, {chunk_ms:.3f} ms per chunk")
    status = C.c_uint(0)
    fa.check(lib.fr_hip_batch_output(sptr, None, 0, C.byref(status)), "fr_hip_batch_output")
    if status.value:
        raise RuntimeError(f"prefill kernels reported status {status.value}")

    # Split per launch: prefill_gate_up + prefill_down ("main") and the whole
    # launch, from events on the launch stream over one more chunk.
    fa.check(lib.fr_hip_timing(PREFILL_LAYERS), "fr_hip_timing")
    chunk()
    main_ms, total_ms, counted = C.c_double(), C.c_double(), C.c_uint()
    fa.check(lib.fr_hip_timing_read(C.byref(main_ms), C.byref(total_ms), C.byref(counted)), "fr_hip_timing_read")

    alg = wts.sum() + PREFILL_LAYERS * 8.0 * PREFILL_TOKENS * HIDDEN   # weights once per unique expert, x and y
    achieved = alg / (chunk_ms * 1e-3) / 1e9
    experts_per_token = 11 if shared else 10
    flops = PREFILL_LAYERS * 2.0 * PREFILL_TOKENS * experts_per_token * SLICES * 3 * 32 * HIDDEN   # multiply-adds x 2
    tflops = flops / (chunk_ms * 1e-3) / 1e12
    traffic, traffic_note = None, "counted for the Q4_K-T prefill only"
    if fmt == fa.FMT_Q4KT and not shared:
        traffic, traffic_note = counted_traffic(os.path.join(ROOT, "profiles", "prefill_traffic.json"))
    return {
        "wall_s": wall, "steps": steps, "warmup": warmup, "weights": float(wts.sum()),
        "chunk_ms": chunk_ms, "achieved": achieved, "tflops": tflops, "traffic": traffic,
        "traffic_note": traffic_note,
        "main_us": main_ms.value * 1e3 / counted.value, "launch_us": total_ms.value * 1e3 / counted.value,
    }, reqs[0]


def bench_prefill(args):
    import torch  # noqa: F401  (before the library: one HIP runtime)
    import fronk_amd as fa
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    steps = args.steps if args.steps is not None else 3
    warmup = args.warmup if args.warmup is not None else 1
    lib = fa.lib()
    eng = fa.Engine(0)
    native = args.workload == "prefill_native"
    fmt, shared = (fa.FMT_NATIVE, 0.5) if native else (fa.FMT_Q4KT, 0.0)
    m, req0 = prefill_leg(fa, lib, eng, steps, warmup, fmt, shared)
    cpu = None
    if not args.no_cpu:
        layer, experts, gates, x = req0
        rc, y0 = eng.run_batch(layer, experts, gates, x)
        fa.check(rc, "fr_hip_run_batch")
        cpu = prefill_cpu_baseline(fa, y0, req0, args.cpu_seconds, fmt)
    for b in range(SLICES):
        eng.release(b)
    chunk_ms = m["chunk_ms"]
    out = {
        "metric": METRIC,
        "value": round(m["weights"] * steps / m["wall_s"] / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(m["wall_s"] * 1e3 / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded device generator; Q4_K d/dmin fp16 U[1e-3,1e-2], x ~ N(0,1))",
        "config": {"workload": PREFILL_NATIVE_TEXT if native else PREFILL_TEXT, "hidden": HIDDEN, "experts": 512,
                   "active_experts": 10, "shared_gate": shared, "slices": SLICES, "tokens": PREFILL_TOKENS,
                   "layers": PREFILL_LAYERS, "format": "NATIVE" if native else "Q4KT", "mode": "f32"},
        "hbm_frac": round(m["weights"] * steps / m["wall_s"] / 1e9 / HBM_PEAK_GBS, 4),
        "tokens_per_s_per_layer": round(PREFILL_TOKENS / (chunk_ms * 1e-3 / PREFILL_LAYERS), 1),
        "chunk_ms": round(chunk_ms, 4),
        "layer_us": round(chunk_ms * 1e3 / PREFILL_LAYERS, 2),
        "kernel_split_us": {"gate_up+down": round(m["main_us"], 2), "launch": round(m["launch_us"], 2),
                            "note": "per layer launch, events on the launch stream, one extra chunk"},
        "weight_bytes_per_chunk": m["weights"],
        "roofline": {"bound": "hbm", "achieved": round(m["achieved"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(m["achieved"] / HBM_PEAK_GBS, 4), "traffic": m["traffic"],
                     "traffic_note": "HBM bytes per layer launch: " + m["traffic_note"],
                     "kernel": ("prefill_split + prefill_gate_up_rows<Q4_K> + prefill_gate_up_rows<Q8_0> + "
                                "prefill_down_rows<MXFP4> + prefill_down_rows<Q8_0> + prefill_reduce per layer"
                                if native else
                                "prefill_split + prefill_gate_up + prefill_down + prefill_reduce per layer")},
        "mfma": {"achieved": round(m["tflops"], 2), "peak": MFMA_F16_PEAK_TFLOPS,
                 "unit": "TFLOP/s (useful multiply-adds x 2 against the dense f16/bf16 matrix-core peak)",
                 "frac": round(m["tflops"] / MFMA_F16_PEAK_TFLOPS, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def percentiles(ns):
    """p50 and p99 as the reference's bench takes them (src/bench.c:432-436):
    sorted[(n+1)/2-1] and sorted[(99n+99)/100-1]."""
    v = sorted(ns)
    n = len(v)
    return v[(n + 1) // 2 - 1], v[(99 * n + 99) // 100 - 1]


def time_run_calls(call, count, warmup=512, samples=1024):
    """The reference's run() timing protocol (src/bench.c:352-377): `warmup`
    untimed calls, then a monotonic timer around each of `samples` calls.
    `call(i)` makes the i-th call and raises on failure. Returns the per-call
    times in microseconds."""
    for i in range(warmup):
        call(i % count)
    out = np.zeros(samples)
    clock = time.perf_counter_ns
    for k in range(samples):
        i = (warmup + k) % count
        t0 = clock()
        call(i)
        out[k] = (clock() - t0) * 1e-3
    return out


KERNEL_SOURCE = os.path.join(ROOT, "fronk_amd", "csrc", "fronk_hip.hip")


def source_sha256():
    with open(KERNEL_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def counted_traffic(tfile):
    """HBM bytes per launch from a traffic summary, or (None, why) when the
    summary is missing or was counted on another kernel source."""
    if not os.path.exists(tfile):
        return None, "no counter summary"
    t = json.load(open(tfile))
    if t.get("kernel_source_sha256") != source_sha256():
        return None, "counter summary taken on another kernel source"
    return t.get("hbm_bytes_per_launch"), (f"FETCH_SIZE + WRITE_SIZE per launch, copy-calibrated, counted on kernel "
                                           f"source sha256 {t['kernel_source_sha256'][:16]}")


def kernel_short(name):
    m = re.search(r"::([A-Za-z_0-9]+(?:<[^>(]*>)?)\(", name)
    return m.group(1) if m else name.split("(")[0].strip()


def counter_medians(d):
    """{kernel: ({counter: median value per dispatch}, dispatches)} from a
    rocprofv3 --pmc output directory (one row per dispatch and counter)."""
    vals = {}
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for row in csv.DictReader(open(f)):
            k = vals.setdefault(kernel_short(row["Kernel_Name"]), {})
            k.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
    return {k: ({c: float(np.median(v)) for c, v in cs.items()}, max(len(v) for v in cs.values()))
            for k, cs in vals.items()}


def traffic_summary(args):
    """profiles/decode_<workload>_traffic.json (prefill_traffic.json for the
    prefill chunk) from the counter runs: each decode (prefill) kernel's
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch, medians), scaled by what the
    same counters read for the copy kernel of known size; a launch is one
    decode call (one layer of a prefill chunk: the chunk's mean)."""
    fetch_dir, write_dir, copy_fetch, copy_write = args.traffic_summary
    nbytes = args.copy_kernel
    if nbytes <= 0:
        raise SystemExit("--traffic-summary needs --copy-kernel BYTES (the size the copy runs used)")
    cf = counter_medians(copy_fetch)["__amd_rocclr_copyBuffer"][0]["FETCH_SIZE"]
    cw = counter_medians(copy_write)["__amd_rocclr_copyBuffer"][0]["WRITE_SIZE"]
    fs, ws = nbytes / (cf * 1024), nbytes / (cw * 1024)
    f, w = counter_medians(fetch_dir), counter_medians(write_dir)
    import fronk_amd as fa
    prefill = args.workload == "prefill"
    if prefill:
        text = (f"one layer launch of a prefill chunk: {PREFILL_TOKENS} tokens x {PREFILL_LAYERS} resident layers, "
                f"top-10 of 512 uniform, {SLICES} slices, hidden {HIDDEN}, Q4_K (down transposed)")
        prefix, per_launch = "prefill_", 1
        slice_bytes = slice_sizes(fa, fa.FMT_Q4KT)[0]
        routes = prefill_requests(np.random.default_rng(SEED + 5), PREFILL_LAYERS, PREFILL_TOKENS)
        alg = (sum(len(set(r[1].ravel().tolist())) * SLICES * slice_bytes for r in routes) +
               PREFILL_LAYERS * 8.0 * PREFILL_TOKENS * HIDDEN) / PREFILL_LAYERS
    else:
        spec = WORKLOADS[args.workload]
        text, prefix, per_launch = spec["text"], "decode_", 1
        reqs = make_requests(64, spec["burst"], spec["routing"], SEED + 1)
        alg = np.mean([algorithmic_bytes(fa, getattr(fa, spec["fmt"]), r[1], r[2])[1] for r in reqs])
    out = {"workload": args.workload, "text": text, "kernel_source_sha256": source_sha256(),
           "fetch_scale": round(fs, 5), "write_scale": round(ws, 5), "copy_bytes": nbytes}
    total = 0.0
    for k in sorted(f):
        if not k.startswith(prefix) or k not in w:
            continue
        fk, wk = f[k][0]["FETCH_SIZE"], w[k][0]["WRITE_SIZE"]
        rd, wr = fk * 1024 * fs, wk * 1024 * ws
        out[k] = {"fetch_kib_per_dispatch": round(fk, 1), "write_kib_per_dispatch": round(wk, 1),
                  "fetch_bytes": int(round(rd)), "write_bytes": int(round(wr)), "dispatches": f[k][1]}
        total += (rd + wr) * per_launch
    out["algorithmic_bytes_per_launch"] = int(round(float(alg)))
    out["hbm_bytes_per_launch"] = int(round(total))
    path = os.path.join(ROOT, "profiles", "prefill_traffic.json" if prefill else
                        f"decode_{args.workload}_traffic.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1)
    log(f"wrote {path}: {out['hbm_bytes_per_launch']} HBM bytes per launch, "
        f"{out['hbm_bytes_per_launch'] / out['algorithmic_bytes_per_launch']:.3f}x the algorithmic bytes")


def run_leg(fa, lib, reqs, weight_bytes, warmup=512, samples=1024, mode=None):
    """fr_hip_run timed the reference's way over prepared requests (layers
    rotating as the requests do); ctypes call overhead is inside the timer."""
    prepared = [fa.make_request(*r, fa.MODE_F32 if mode is None else mode) for r in reqs]
    y = np.zeros((8, HIDDEN), np.float32)
    yp = fa.fptr(y)
    run = lib.fr_hip_run

    def call(i):
        rc = run(C.byref(prepared[i][0]), yp)
        if rc != fa.OK:
            raise RuntimeError(f"fr_hip_run failed with {rc}")

    us = time_run_calls(call, len(prepared), warmup, samples)
    p50, p99 = percentiles(us)
    burst = reqs[0][1].shape[0]
    return {"p50_us": round(p50, 2), "p99_us": round(p99, 2), "mean_us": round(float(us.mean()), 2),
            "warmup": warmup, "samples": samples,
            "run_tokens_per_s": round(burst * samples / (us.sum() * 1e-6), 1),
            "gbs_at_p50": round(weight_bytes / (p50 * 1e-6) / 1e9, 2),
            "timer": "perf_counter_ns around each fr_hip_run call (ctypes call included), "
                     "512 warm-ups first (src/bench.c:352-377)",
            "phases_us": run_phases(fa, lib, call, len(prepared))}


def run_phases(fa, lib, call, count, samples=256):
    """The library's own phase sample of run() (fr_hip_phase_get), medians
    over `samples` calls: the host phases without events, then the GPU phase
    (and TOTAL - GPU) over as many calls with events around the launches."""
    ns = (C.c_double * len(fa.PHASES))()
    runs = C.c_uint64()

    def sweep(events):
        fa.check(lib.fr_hip_phase_events(1 if events else 0), "fr_hip_phase_events")
        rows = []
        for k in range(samples):
            call(k % count)
            fa.check(lib.fr_hip_phase_get(ns, C.byref(runs)), "fr_hip_phase_get")
            rows.append(list(ns))
        fa.check(lib.fr_hip_phase_events(0), "fr_hip_phase_events")
        return np.median(np.array(rows), axis=0) * 1e-3

    host, ev = sweep(False), sweep(True)
    out = {name: round(float(host[i]), 2) for i, name in enumerate(fa.PHASES) if name in ("plan", "enqueue", "wait",
                                                                                         "total")}
    out.update({"gpu_with_events": round(float(ev[3]), 2), "overhead_with_events": round(float(ev[4]), 2),
                "total_with_events": round(float(ev[5]), 2), "samples": samples,
                "source": "fr_hip_phase_get medians (host clock; GPU phase from two HIP events, a second pass)"})
    return out


class Launches:
    """A workload's launch plans resident in HBM and enqueued with fr_hip_launch
    on one stream."""

    def __init__(self, fa, lib, eng, fmt, reqs, blocks=SLICES, mode=None):
        import torch
        self.fa, self.lib = fa, lib
        n = len(reqs)
        burst = reqs[0][1].shape[0]
        cap = lib.fr_hip_plan_bytes(burst, HIDDEN)
        self.stride = (cap + 255) // 256 * 256
        self.host = np.zeros((n, self.stride), np.uint8)
        self.alg = np.zeros(n)
        self.wts = np.zeros(n)
        self.grid = 0
        for i, (layer, experts, gates, x) in enumerate(reqs):
            plan, self.grid = eng.plan(layer, experts, gates, x, fa.MODE_F32 if mode is None else mode)
            self.host[i, :plan.size] = plan
            self.wts[i], self.alg[i] = algorithmic_bytes(fa, fmt, experts, gates, blocks)
        self.dev = torch.from_numpy(self.host).to("cuda")
        self.stream = torch.cuda.Stream()
        torch.cuda.synchronize()
        self.hptr, self.dptr = self.host.ctypes.data, self.dev.data_ptr()
        self.sptr = C.c_void_p(self.stream.cuda_stream)
        self.kernels = grid_kernels(lib, self.host[0])

    def enqueue(self, i):
        rc = self.lib.fr_hip_launch(C.c_void_p(self.hptr + i * self.stride), C.c_void_p(self.dptr + i * self.stride),
                                    self.sptr)
        if rc != self.fa.OK:
            raise RuntimeError(f"fr_hip_launch failed with {rc}")

    def timed(self, first, last):
        """Events around launches first..last-1 on the launch stream; returns
        (wall seconds, ms per launch). Checks the last launch's status."""
        import torch
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        with torch.cuda.stream(self.stream):
            ev0.record(self.stream)
            for i in range(first, last):
                self.enqueue(i)
            ev1.record(self.stream)
        self.stream.synchronize()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        status = C.c_uint(0)
        self.fa.check(self.lib.fr_hip_last_output(self.sptr, None, 0, C.byref(status)), "fr_hip_last_output")
        if status.value:
            raise RuntimeError(f"decode kernels reported status {status.value}")
        return wall, ev0.elapsed_time(ev1) / (last - first)

    def split(self, first, count):
        """Main kernel and whole launch in microseconds from events between
        the kernels of `count` more launches (the markers add a little)."""
        fa, lib = self.fa, self.lib
        fa.check(lib.fr_hip_timing(count), "fr_hip_timing")
        for i in range(first, first + count):
            self.enqueue(i)
        main_ms, total_ms, counted = C.c_double(), C.c_double(), C.c_uint()
        fa.check(lib.fr_hip_timing_read(C.byref(main_ms), C.byref(total_ms), C.byref(counted)),
                 "fr_hip_timing_read")
        return main_ms.value * 1e3 / counted.value, total_ms.value * 1e3 / counted.value


def decode_leg(fa, lib, eng, key, steps, warmup, seed, blocks=SLICES, mode=None):
    """One decode workload with its `blocks` owned slices already resident:
    `warmup` then `steps` pipelined launches (F32 unless `mode`). Returns the
    extra-key record."""
    wl = WORKLOADS[key]
    fmt = getattr(fa, wl["fmt"])
    reqs = make_requests(warmup + steps, wl["burst"], wl["routing"], seed)
    L = Launches(fa, lib, eng, fmt, reqs, blocks, mode)
    for i in range(warmup):
        L.enqueue(i)
    wall, ms = L.timed(warmup, warmup + steps)
    alg = float(L.alg[warmup:].mean())
    wts = float(L.wts[warmup:].mean())
    achieved = alg / (ms * 1e-3) / 1e9
    return {"workload": wl["text"], "kernel": L.kernels, "launches": steps, "kernel_us": round(ms * 1e3, 3),
            "weight_bytes_per_call": wts, "algorithmic_bytes_per_call": alg,
            "gbs": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(wl["burst"] * steps / wall, 1)}


def host_info():
    """The GPU box's host as the CPU baseline sees it: nproc, the affinity set,
    lscpu's model / cores / threads, and the thread share this pool allows."""
    info = {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Thread(s) per core", "Core(s) per socket", "Socket(s)", "CPU(s)",
                             "L3 cache"):
                info["lscpu_" + k.strip().lower().replace("(s)", "s").replace(" ", "_")] = v.strip()
    except (OSError, ValueError):
        pass
    # One GPU's share of the box's CPUs: worker pools stay within 16 threads.
    info["share"] = min(info["affinity"], 16)
    return info


NATIVE_H = 2560
NATIVE_LAYERS = 8
NATIVE_EXPERTS = 80   # experts 0..79 carry data (fr_native_fixture), as in the reference's fixture


def native_routes(passes):
    """The reference bench's routing (src/bench.c:279-284) over the filled
    experts: layer = pass % L, experts base..base+9 with base = (pass / L) * 41,
    here modulo the 80 filled experts and 8 filled layers."""
    out = []
    for p in range(passes):
        base = (p // NATIVE_LAYERS) * 41 % NATIVE_EXPERTS
        out.append((p % NATIVE_LAYERS, np.array([(base + e) % NATIVE_EXPERTS for e in range(10)], np.uint16)))
    return out


def native_inputs():
    """The reference bench's request values (src/bench.c:347-351): routed gates
    0.0625, shared 0.5, x[d] = ((37 d) % 257 - 128) / 128."""
    g = np.full(11, 0.0625, np.float32)
    g[10] = 0.5
    x = np.array([((d * 37) % 257 - 128) / 128 for d in range(NATIVE_H)], np.float32)
    return g, x


def cpu_reference_leg(fa, lib, eng, passes=1024):
    """CPU baseline: the reference's own AVX2 backend (backends/avx2.c, the
    fr_avx2 vtable) compiled from its sources into oracle/_ref, swept over the
    reference's worker choices {1, cores/2, cores-1, cores, logical}
    (backends/avx2.c:747) within this box's thread share and prefetch {0, 2},
    each point timed the reference's way (512 warm-ups, 256 samples, p50/p99).
    The shape is the reference's own: H = 2560 (src/model.h:16), native units
    (Q4_K gate/up, MXFP4 down, Q8_0 shared), 10 routed + the shared expert,
    20 owned blocks, layers rotating over 8 filled layers. The same bytes and
    requests then run through fr_hip_run on the GPU with the same protocol.
    Bytes per call follow the reference's byte model (src/bench.c:158-162)."""
    import oracle
    import vtable
    if not os.path.exists(oracle.REF_PATH):
        return None
    ref = C.CDLL(oracle.REF_PATH, mode=C.RTLD_GLOBAL)
    ref.fr_native_fixture.argtypes = [C.c_void_p, C.c_uint, C.c_uint32]
    avx2 = vtable.Backend.in_dll(ref, "fr_avx2")
    lay = oracle.layout(NATIVE_H, oracle.FMT_NATIVE)
    t0 = time.perf_counter()
    units = []
    for b in range(SLICES):
        u = np.zeros(lay.block, np.uint8)
        for layer in range(NATIVE_LAYERS):
            ref.fr_native_fixture(u.ctypes.data, layer, 7 + 1009 * b + 31 * layer)
        units.append(u)
    log(f"cpu leg: {SLICES} native units x {NATIVE_LAYERS} layers filled in {time.perf_counter() - t0:.1f} s")
    g, x = native_inputs()
    routes = native_routes(passes)
    reqs = []
    for layer, experts in routes:
        q = vtable.Req()
        q.layer, q.burst = layer, 1
        for j in range(10):
            q.expert[0][j] = int(experts[j])
        for j in range(11):
            q.gate[0][j] = float(g[j])
        C.memmove(q.x[0], x.ctypes.data, 4 * NATIVE_H)
        reqs.append(q)
    call_bytes = SLICES * (10 * lay.slice + lay.shared_slice)
    part = vtable.Part()

    def call(i):
        if avx2.run(C.byref(reqs[i]), C.byref(part)) != 0:
            raise RuntimeError("fr_avx2 run failed")

    info = host_info()
    tpc = 1
    try:
        tpc = max(1, int(info.get("lscpu_threads_per_core", "1")))
    except ValueError:
        pass
    logical = info["share"]
    cores = max(1, logical // tpc)
    choices = []
    for w in (1, max(1, cores // 2), max(1, cores - 1), cores, logical):
        if w not in choices:
            choices.append(w)
    sweep, best = [], None
    for workers in choices:
        for prefetch in (0, 2):
            ref.fr_avx2_set_tuning(C.c_uint(SLICES), C.c_uint(1), C.c_uint(workers), C.c_uint(prefetch))
            if ref.fr_avx2_configure(C.c_uint(SLICES), C.c_uint(1)) != 0:
                raise RuntimeError("fr_avx2_configure failed")
            for b in range(SLICES):
                if avx2.load(b, units[b].ctypes.data, lay.block) != 0:
                    raise RuntimeError("fr_avx2 load failed")
            us = time_run_calls(call, len(reqs), 512, 256)
            for b in range(SLICES):
                avx2.unload(b)
            p50, p99 = percentiles(us)
            row = {"workers": workers, "prefetch": prefetch, "p50_us": round(p50, 2), "p99_us": round(p99, 2),
                   "gbs_at_p50": round(call_bytes / (p50 * 1e-6) / 1e9, 2)}
            log(f"avx2 workers={workers:3d} prefetch={prefetch} p50 {p50:9.2f} us p99 {p99:9.2f} us "
                f"{row['gbs_at_p50']:8.2f} GB/s")
            sweep.append(row)
            if best is None or p50 < best["p50_us"]:
                best = row
    ref.fr_avx2_close()

    # The same units and requests on the GPU through fr_hip_run.
    t0 = time.perf_counter()
    for b in range(SLICES):
        fa.check(eng.reserve(b, NATIVE_H, fa.FMT_NATIVE), "fr_hip_reserve")
        for layer in range(NATIVE_LAYERS):
            for e in list(range(NATIVE_EXPERTS)) + [512]:
                fa.check(eng.refresh(b, units[b], layer, e), "fr_hip_refresh")
    log(f"gpu same shape: slices copied in {time.perf_counter() - t0:.1f} s")
    gpu_reqs = [(layer, experts.reshape(1, 10), g.reshape(1, 11), x.reshape(1, NATIVE_H)) for layer, experts in routes]
    prepared = [fa.make_request(*r, fa.MODE_F32) for r in gpu_reqs]
    y = np.zeros((8, NATIVE_H), np.float32)
    yp = fa.fptr(y)

    def gcall(i):
        rc = lib.fr_hip_run(C.byref(prepared[i][0]), yp)
        if rc != fa.OK:
            raise RuntimeError(f"fr_hip_run failed with {rc}")

    us = time_run_calls(gcall, len(prepared), 512, 1024)
    for b in range(SLICES):
        eng.release(b)
    gp50, gp99 = percentiles(us)
    return {
        "value": best["gbs_at_p50"], "unit": "GB/s", "cores": best["workers"], "kind": "reference",
        "sample": f"backends/avx2.c built from the reference sources (oracle/_ref): {NATIVE_H}-wide native layer "
                  f"share (Q4_K gate/up, MXFP4 down, Q8_0 shared), 10 routed + shared x {SLICES} blocks, "
                  f"{NATIVE_LAYERS} layers rotating; per point 512 warm-ups + 256 timed run() calls, "
                  f"{call_bytes} B per call (src/bench.c:158-162); best of the worker/prefetch sweep",
        "p50_us": best["p50_us"], "p99_us": best["p99_us"], "prefetch": best["prefetch"],
        "host": info, "sweep": sweep,
        "gpu_same_shape": {"p50_us": round(gp50, 2), "p99_us": round(gp99, 2),
                           "gbs_at_p50": round(call_bytes / (gp50 * 1e-6) / 1e9, 2),
                           "vs_cpu_p50": round(best["p50_us"] / gp50, 2),
                           "note": "fr_hip_run on the same units and requests, 512 warm-ups + 1024 samples"},
    }


def sustained_read(lib, gib=1, reps=20):
    """The probe over one contiguous buffer of `gib` GiB per launch (far past
    the 256 MB Infinity Cache and every launch-size effect): the box's
    sustained HBM read rate, best of a few workgroup counts and depths."""
    import torch
    nbytes = gib << 30
    stream = torch.cuda.Stream()
    sink = torch.zeros(16 * 8192, dtype=torch.int32, device="cuda")
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.fill_(3)
    best = None
    for parts, depth in ((4096, 4), (8192, 4), (8192, 2)):
        pc = cut_pieces(np.array([buf.data_ptr()], np.uint64), np.array([nbytes], np.uint64), parts)
        table = torch.from_numpy(pc.view(np.int64).copy()).to("cuda")
        us = time_probe(lib, [table], 1024, depth, reps, sink, stream)
        gbs = nbytes / (us * 1e-6) / 1e9
        log(f"stream sustained {gib} GiB wg={parts} depth={depth} {us:9.1f} us {gbs:8.1f} GB/s")
        if best is None or gbs > best["gbs"]:
            best = {"gbs": round(gbs, 1), "us": round(us, 1), "workgroups": parts, "threads": 1024, "depth": depth,
                    "bytes": nbytes}
    del buf
    return best


def achievable_leg(eng, lib, plans):
    """Achievable HBM read rate for the headline calls: the streaming probe
    over the same scattered slices and over a contiguous buffer of the same
    size (best of a short sweep of pieces, threads and depth), and the
    sustained rate of a 1 GiB read."""
    sweep = [("scattered", p, t, d) for p in (1, 2) for t in (512, 1024) for d in (2, 4)]
    sweep += [("contiguous", g, t, d) for g in (512, 1024) for t in (512, 1024) for d in (2, 4)]
    rows, best, total = stream_ceiling(eng, lib, plans, sweep)
    out = {k: {"gbs": v["gbs"], "us": v["us"], "workgroups": v["workgroups"], "threads": v["threads"],
               "depth": v["depth"]} for k, v in best.items()}
    out["sustained_1gib"] = sustained_read(lib)
    return out, total


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="q4k",
                    choices=sorted(WORKLOADS) + ["prefill", "prefill_native", "stream", "run"])
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the other configs' legs")
    ap.add_argument("--copy-kernel", type=int, default=0)
    ap.add_argument("--traffic-summary", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"))
    ap.add_argument("--blocks", type=int, default=SLICES,
                    help="owned slices of the measured leg (1..20; config 1 is 1); other values skip the other legs")
    ap.add_argument("--mode", default="f32", choices=["f32", "q8", "q8_256"],
                    help="arithmetic of the measured leg; other than f32 skips the other legs")
    args = ap.parse_args()
    if not 1 <= args.blocks <= SLICES:
        ap.error("--blocks is 1..20")
    if args.blocks != SLICES or args.mode != "f32":
        args.no_extra = args.no_cpu = True
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the layer share is built and timed on a "
              "single MI355X, and its multi-GPU sharding is a design, not a measured path.", file=sys.stderr)
        sys.exit(2)
    if args.traffic_summary:
        traffic_summary(args)
        return
    if args.copy_kernel:
        copy_kernel(args.copy_kernel)
        return
    if args.workload in ("prefill", "prefill_native"):
        bench_prefill(args)
        return
    if args.workload == "stream":
        bench_stream(args)
        return
    if args.steps is None:
        args.steps = 1000
    if args.warmup is None:
        args.warmup = 200

    import torch  # noqa: F401  (before the library: one HIP runtime)
    import fronk_amd as fa
    sys.path.insert(0, os.path.join(ROOT, "tests"))

    key = "q4k" if args.workload == "run" else args.workload
    wl = WORKLOADS[key]
    fmt = getattr(fa, wl["fmt"])
    burst = wl["burst"]
    lib = fa.lib()
    eng = fa.Engine(0)
    mode = {"f32": fa.MODE_F32, "q8": fa.MODE_Q8, "q8_256": fa.MODE_Q8_256}[args.mode]
    t0 = time.perf_counter()
    for b in range(args.blocks):
        fa.check(eng.synthetic(b, HIDDEN, fmt, LAYERS, SEED), "fr_hip_synthetic")
    log(f"resident: {args.blocks} blocks x {LAYERS} layers generated in {time.perf_counter() - t0:.1f} s")

    if args.workload == "run":
        # run() alone, the reference's way: for kernel traces of run() calls.
        reqs = make_requests(1024, burst, wl["routing"], SEED + 1)
        wts = float(np.mean([algorithmic_bytes(fa, fmt, r[1], r[2], args.blocks)[0] for r in reqs]))
        rec = run_leg(fa, lib, reqs, wts, mode=mode)
        for b in range(SLICES):
            eng.release(b)
        print(json.dumps({"workload": wl["text"], "run": rec}), flush=True)
        return

    n = args.warmup + args.steps
    reqs = make_requests(n, burst, wl["routing"], SEED + 1)
    L = Launches(fa, lib, eng, fmt, reqs, args.blocks, mode)
    # The streaming ceiling first: about a second of GPU work right before
    # the timed launches, so that they run at the clocks of a busy GPU
    # rather than those of one that idled while the plans were built.
    ceiling, ceiling_bytes = achievable_leg(eng, lib, [L.host[i % n, :] for i in range(args.warmup, args.warmup + 8)])
    for i in range(args.warmup):
        L.enqueue(i)
    L.stream.synchronize()
    wall, kernel_ms = L.timed(args.warmup, n)
    timed = slice(args.warmup, n)
    ms_per_step = wall * 1e3 / args.steps
    weight_gbs = L.wts[timed].sum() / wall / 1e9
    alg_per_launch = float(L.alg[timed].mean())

    # Roofline: algorithmic bytes over the launch's own time, from the HIP
    # events around the timed region on the launch stream. A single-token
    # Q4_K launch is decode_kernel followed by decode_reduce (its fixed-order
    # partial sum); their rocprofv3 averages add up to this figure. The split
    # between them comes from a second pass with events between the kernels.
    achieved = alg_per_launch / (kernel_ms * 1e-3) / 1e9
    main_us, launch_us = L.split(args.warmup, min(args.steps, 500))
    log(f"headline: {kernel_ms * 1e3:.3f} us per launch, {achieved:.1f} GB/s")

    run_rec = run_leg(fa, lib, reqs[:1024], float(L.wts[:1024].mean()), mode=mode)
    log(f"run(): p50 {run_rec['p50_us']} us p99 {run_rec['p99_us']} us")

    traffic, traffic_note = None, f"counted only for the default {SLICES}-slice f32 workloads"
    if args.blocks == SLICES and args.mode == "f32":   # the counted workload
        traffic, traffic_note = counted_traffic(os.path.join(ROOT, "profiles", f"decode_{key}_traffic.json"))

    scalar = None
    if not args.no_cpu:
        scalar = cpu_baseline(fa, eng, fmt, reqs[args.warmup:], args.cpu_seconds)

    extra = {}
    if not args.no_extra and key == "q4k":
        extra["config4_mtp4"] = decode_leg(fa, lib, eng, "mtp4", 300, 50, SEED + 4)
        extra["burst4_shared_experts"] = decode_leg(fa, lib, eng, "shared4", 300, 50, SEED + 11)
        q8 = decode_leg(fa, lib, eng, "q4k", 100, 20, SEED + 5, mode=fa.MODE_Q8)
        q8["workload"] = ("config 2 in the ref-q8 arithmetic (the hip-q8 table: x and h through "
                          "fr_q8_activation, fp64 sums)")
        extra["config2_ref_q8"] = q8
        for b in range(1, SLICES):
            eng.release(b)
        one = decode_leg(fa, lib, eng, "q4k", 300, 50, SEED + 6, blocks=1)
        one["workload"] = ("config 1, latency: one owned Q4_K slice (block 0 only) x the 10 routed experts every "
                           "request carries, hidden 4096, 1 token")
        r1 = make_requests(1024, 1, "uniform", SEED + 7)
        one["run"] = run_leg(fa, lib, r1, 10 * slice_sizes(fa, fa.FMT_Q4KT)[0])
        extra["config1_latency"] = one
        eng.release(0)
        for name, k in (("config3a_q8", "q8"), ("config3b_mxfp4", "mxfp4"), ("native_h4096", "native")):
            f = getattr(fa, WORKLOADS[k]["fmt"])
            for b in range(SLICES):
                fa.check(eng.synthetic(b, HIDDEN, f, LAYERS, SEED), "fr_hip_synthetic")
            extra[name] = decode_leg(fa, lib, eng, k, 300, 50, SEED + 8)
            if k == "native":   # the reference's own unit format in the ref-q8 arithmetic (hip-q8)
                nq8 = decode_leg(fa, lib, eng, k, 100, 20, SEED + 9, mode=fa.MODE_Q8)
                nq8["workload"] = ("native units (Q4_K gate/up, MXFP4 down) at hidden 4096 in the ref-q8 "
                                   "arithmetic (the hip-q8 table), 10 of 512 x 20 slices, 1 token")
                extra["native_ref_q8"] = nq8
                n256 = decode_leg(fa, lib, eng, k, 100, 20, SEED + 10, mode=fa.MODE_Q8_256)
                n256["workload"] = ("native units (Q4_K gate/up, MXFP4 down) at hidden 4096 in the AVX2 "
                                    "backend's arithmetic (the hip-q8-256 table: x per 256 and h per 32 "
                                    "through quantize8, integer dots), 10 of 512 x 20 slices, 1 token")
                extra["native_q8_256"] = n256
            for b in range(SLICES):
                eng.release(b)
        m, _ = prefill_leg(fa, lib, eng, 2, 1)
        for b in range(SLICES):
            eng.release(b)
        extra["config5_prefill"] = {
            "workload": PREFILL_TEXT, "chunks": 2, "chunk_ms": round(m["chunk_ms"], 3),
            "layer_us": round(m["chunk_ms"] * 1e3 / PREFILL_LAYERS, 2),
            "weight_bytes_per_chunk": m["weights"], "gbs": round(m["achieved"], 1),
            "frac": round(m["achieved"] / HBM_PEAK_GBS, 4),
            "tokens_per_s_per_layer": round(PREFILL_TOKENS / (m["chunk_ms"] * 1e-3 / PREFILL_LAYERS), 1),
            "algorithmic_tflops": round(m["tflops"], 2)}
        m, _ = prefill_leg(fa, lib, eng, 2, 1, fa.FMT_NATIVE, 0.5)
        for b in range(SLICES):
            eng.release(b)
        extra["config5_prefill_native"] = {
            "workload": PREFILL_NATIVE_TEXT, "chunks": 2, "chunk_ms": round(m["chunk_ms"], 3),
            "layer_us": round(m["chunk_ms"] * 1e3 / PREFILL_LAYERS, 2),
            "weight_bytes_per_chunk": m["weights"], "gbs": round(m["achieved"], 1),
            "frac": round(m["achieved"] / HBM_PEAK_GBS, 4),
            "tokens_per_s_per_layer": round(PREFILL_TOKENS / (m["chunk_ms"] * 1e-3 / PREFILL_LAYERS), 1),
            "algorithmic_tflops": round(m["tflops"], 2)}
        for k2, v in extra.items():
            log(f"{k2}: {v.get('kernel_us', v.get('chunk_ms'))} {v.get('gbs')} GB/s")
    else:
        for b in range(SLICES):
            eng.release(b)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_reference_leg(fa, lib, eng)

    out = {
        "metric": METRIC,
        "value": round(weight_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if args.mode == "f32" else "i8+f64",
        "data": "synthetic (seeded device generator; Q4_K d/dmin fp16 U[1e-3,1e-2], x ~ N(0,1))",
        "config": {"workload": wl["text"] if args.blocks == SLICES else
                   wl["text"].replace(f"{SLICES} owned slices", f"{args.blocks} owned slices")
                             .replace(f"{SLICES} slices", f"{args.blocks} slices"),
                   "hidden": HIDDEN, "experts": 512, "active_experts": 10,
                   "slices": args.blocks, "burst": burst, "format": wl["fmt"][4:], "mode": args.mode,
                   "layers_rotated": LAYERS},
        "hbm_frac": round(weight_gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(burst * args.steps / wall, 1),
        "kernel_us": round(kernel_ms * 1e3, 3),
        "kernel_split_us": {"main": round(main_us, 3), "rest": round(launch_us - main_us, 3),
                            "note": "events between the kernels of each launch, second pass"},
        "weight_bytes_per_call": float(L.wts[timed].mean()),
        "grid": L.grid,
        "run": run_rec,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_note": traffic_note,
                     "achievable": {"gbs": ceiling["scattered"]["gbs"],
                                    "frac_of_achievable": round(achieved / ceiling["scattered"]["gbs"], 4),
                                    "probe": ceiling, "bytes_per_call": ceiling_bytes,
                                    "note": "streaming probe over the same scattered slices (and a contiguous "
                                            "buffer of the same size), best of a short sweep"},
                     "kernel": L.kernels},
        "cpu_baseline": cpu,
        "cpu_scalar_port": scalar,
        "configs": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
