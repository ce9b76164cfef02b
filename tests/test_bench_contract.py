"""bench.py's contract on the CPU: it measures one GPU only and refuses
--gpus N > 1 with a message and no JSON line, and its algorithmic byte model
uses the slice sizes of the oracle's layout (src/native.h:9-21 restated), so
that `value` and `roofline.achieved` count each weight byte once per call."""
import os
import subprocess
import sys

import numpy as np
import pytest

import fronk_amd as fa
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert r.stdout == ""
    assert "one GPU" in r.stderr


@pytest.mark.parametrize("fmt", [fa.FMT_Q4KT, fa.FMT_Q8, fa.FMT_MXFP4, fa.FMT_NATIVE])
def test_slice_sizes_match_the_oracle_layout(fmt):
    lay = oracle.layout(bench.HIDDEN, fmt)
    routed, shared = bench.slice_sizes(fa, fmt)
    assert routed == lay.slice
    assert shared == lay.shared_slice


@pytest.mark.parametrize("fmt,per_call", [(fa.FMT_Q4KT, 44_236_800), (fa.FMT_Q8, 83_558_400),
                                          (fa.FMT_MXFP4, 41_779_200), (fa.FMT_NATIVE, 43_417_600)])
def test_single_token_byte_model(fmt, per_call):
    """10 distinct experts x 20 slices, no shared expert: the per-call weight
    bytes of the layer share (the figures of the workload table)."""
    experts = np.arange(10, dtype=np.uint16).reshape(1, 10)
    gates = np.zeros((1, 11), np.float32)
    gates[0, :10] = 0.1
    weights, total = bench.algorithmic_bytes(fa, fmt, experts, gates)
    assert weights == per_call
    assert total == per_call + 8 * bench.HIDDEN
    # The shared expert adds its 20 slices once, whatever the burst.
    gates[0, 10] = 0.5
    w_shared, _ = bench.algorithmic_bytes(fa, fmt, experts, gates)
    assert w_shared == per_call + bench.SLICES * oracle.layout(bench.HIDDEN, fmt).shared_slice


def test_burst_counts_unique_experts_once():
    experts = np.array([[e for e in range(10)], [e for e in range(5, 15)]], np.uint16)
    gates = np.zeros((2, 11), np.float32)
    weights, total = bench.algorithmic_bytes(fa, fa.FMT_Q4KT, experts, gates)
    assert weights == 15 * bench.SLICES * 221_184
    assert total == weights + 8 * 2 * bench.HIDDEN
