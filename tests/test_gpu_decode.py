"""Bit-exact decode and quantization on the GPU.

The device decoder that the fp64 and q8 paths use (and that the re-tiled
layout feeds) must reproduce the reference's per-weight decode
(src/native.c:13-31, src/q4.c:29-31) bit for bit, and the device activation
quantizer must reproduce fr_q8_activation (src/q4.c:37-61) bit for bit.
"""
import numpy as np
import pytest

import fronk_amd as fa
import oracle
from fixtures import baseline_row

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    return fa.Engine(0)


def special_row(rng, typ, n, finite=True):
    """Random row with the edge scales the reference tests: subnormal and zero
    fp16 scales, negative scales, E8M0 0 (2^-127) and 254. With `finite`, the
    E8M0 254 block's codes have magnitude <= 1.5 (weights below 2^128);
    otherwise they are random, and some decode to infinity."""
    per, size = {oracle.Q4_K: (256, 144), oracle.Q8_0: (32, 34), oracle.MXFP4: (32, 17), oracle.Q4_0: (32, 18)}[typ]
    b = baseline_row(rng, typ, n).reshape(-1, size)
    nb = b.shape[0]
    if typ == oracle.MXFP4:
        b[0, 0], b[1 % nb, 0] = 0, 254
        if finite:
            b[1 % nb, 1:] &= 0xBB   # clear bit 2 of both nibbles: magnitude index <= 3
    else:
        b[0, 0:2] = [0x01, 0x00]          # smallest subnormal
        b[1 % nb, 0:2] = [0x00, 0x80]     # -0
        b[2 % nb, 0:2] = [0xff, 0x83]     # negative subnormal
        b[3 % nb, 0:2] = [0x00, 0x7b]     # large finite
        if typ == oracle.Q4_K:
            b[0, 2:4] = [0xff, 0x03]
    return b.reshape(-1)


@pytest.mark.parametrize("typ", [oracle.Q4_K, oracle.Q8_0, oracle.MXFP4, oracle.Q4_0])
@pytest.mark.parametrize("n", [2560, 4096])
def test_dequant_rows_bit_exact(eng, typ, n):
    """Every weight bit for bit, infinities included; FR_NUMERIC exactly when
    a weight is not finite (the rows fr_native_dot rejects, src/native.c:7-37)."""
    rng = np.random.default_rng(typ * 100 + n)
    for trial in range(4):
        row = special_row(rng, typ, n, finite=trial < 3) if trial else baseline_row(rng, typ, n)
        rc, got = eng.dequant(typ, row, n)
        want = oracle.dequant(row, typ, n)
        assert rc == (fa.OK if np.all(np.isfinite(want)) else fa.NUMERIC), (typ, n, trial, rc)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (typ, n, trial)


@pytest.mark.parametrize("typ", [oracle.Q4_K, oracle.Q8_0, oracle.MXFP4, oracle.Q4_0])
def test_dequant_rejects_nonfinite_scale(eng, typ):
    rng = np.random.default_rng(5)
    row = baseline_row(rng, typ, 4096)
    if typ == oracle.MXFP4:
        row[17 * 5] = 255
    else:
        row[1] = 0x7c
    rc, _ = eng.dequant(typ, row, 4096)
    assert rc == fa.NUMERIC


@pytest.mark.parametrize("e,code,ok", [(254, 0x4, False), (254, 0xB, True), (253, 0x6, False), (253, 0xD, True)])
def test_dequant_mxfp4_top_exponents(eng, e, code, ok):
    """E8M0 254 with code 4 (2.0) and 253 with code 6 (4.0) decode to 2^128:
    infinite, FR_NUMERIC; 254 with code 11 (-1.5) and 253 with code 13 (-3.0)
    stay finite."""
    rng = np.random.default_rng(6)
    row = baseline_row(rng, oracle.MXFP4, 4096).reshape(-1, 17)
    row[3, 0] = e
    row[3, 1:] = 0x11 if ok else 0x00
    row[3, 5] = code | (1 << 4)
    rc, got = eng.dequant(oracle.MXFP4, row.reshape(-1), 4096)
    want = oracle.dequant(row.reshape(-1), oracle.MXFP4, 4096)
    assert rc == (fa.OK if ok else fa.NUMERIC)
    assert np.all(np.isfinite(want)) == ok
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt,hidden", [(oracle.FMT_NATIVE, 2560), (oracle.FMT_NATIVE, 4096),
                                        (oracle.FMT_Q4KT, 4096), (oracle.FMT_Q8, 4096),
                                        (oracle.FMT_MXFP4, 4096), (oracle.FMT_LEGACY, 2560)])
def test_dequant_down_bit_exact(eng, fmt, hidden):
    lay = oracle.layout(hidden, fmt)
    rng = np.random.default_rng(fmt * 7 + hidden)
    if lay.down_transposed:
        rows = [baseline_row(rng, lay.down_type, hidden) for _ in range(32)]
        down = np.concatenate(rows)
        rowb = len(rows[0])
        want = np.stack([oracle.dequant(down[n * rowb:(n + 1) * rowb], lay.down_type, hidden) for n in range(32)]).T
    else:
        down = baseline_row(rng, lay.down_type, 32 * hidden)
        rowb = down.size // hidden
        want = np.stack([oracle.dequant(down[d * rowb:(d + 1) * rowb], lay.down_type, 32) for d in range(hidden)])
    rc, got = eng.dequant_down(fmt, down, hidden)
    assert rc == fa.OK
    assert np.array_equal(np.ascontiguousarray(got).view(np.uint32), np.ascontiguousarray(want).view(np.uint32))


def test_quantize_bit_exact(eng):
    rng = np.random.default_rng(3)
    cases = [rng.standard_normal(4096).astype(np.float32),
             (rng.standard_normal(4096) * 1e-30).astype(np.float32),
             (rng.standard_normal(4096) * 1e30).astype(np.float32),
             np.zeros(4096, np.float32)]
    ties = np.zeros(4096, np.float32)
    ties[:7] = [127, .5, 1.5, 2.5, -.5, -1.5, -2.5]
    ties[64:66] = [254, 3]
    ties[128] = np.finfo(np.float32).max
    ties[192] = 2.0 ** -149
    ties[256] = 2.0 ** -125
    cases.append(ties)
    for x in cases:
        rc, want = oracle.q8_activation(x)
        assert rc == 0
        for regs in (False, True):   # q8_group and q8_regs64
            rc, got = eng.quantize(x, regs)
            assert rc == fa.OK
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), regs
    # The 32-value hidden-slice form.
    for x in [rng.standard_normal(32).astype(np.float32) * 1e4, ties[:32].copy()]:
        rc, got = eng.quantize(x)
        assert rc == fa.OK
        assert np.array_equal(got.view(np.uint32), oracle.q8_activation(x)[1].view(np.uint32))


def test_ref_q8_decode_kernels_quantizers_bit_exact(eng):
    """The quantizers the ref-q8 decode kernels run themselves: x staged as two
    exact digits per value (s*k + u*r) in decode_q8_kernel's layout (form 0)
    and decode_rows_q8_kernel's lane-major layout (form 1), with the exact sum
    of each 32-value sub-block, and their h quantizer (form 2), each bit-exact
    against fr_q8_activation (src/q4.c:37-61) - including a 64-value group
    whose scale is subnormal - and a non-finite x as FR_NUMERIC. The staged
    digits are integers, so a value the reference quantizes to -0.0 is staged
    as k = 0 and comes back +0.0: those are compared as values (equal), every
    other value bit for bit."""
    import math
    rng = np.random.default_rng(41)
    sub = (rng.standard_normal(4096) * 1e-39).astype(np.float32)   # max/127 below 2^-126: subnormal scales
    ties = np.zeros(4096, np.float32)
    ties[:7] = [127, .5, 1.5, 2.5, -.5, -1.5, -2.5]
    ties[64:66] = [254, 3]
    ties[128] = np.finfo(np.float32).max
    ties[192] = 2.0 ** -149
    ties[256] = 2.0 ** -125
    mixed = rng.standard_normal(4096).astype(np.float32)
    mixed[640:704] *= np.float32(1e-38)
    cases = [rng.standard_normal(4096).astype(np.float32), sub, ties, mixed,
             (rng.standard_normal(2560) * 1e4).astype(np.float32), np.zeros(128, np.float32)]
    for i, x in enumerate(cases):
        rc, want = oracle.q8_activation(x)
        assert rc == 0
        exact = [math.fsum(want[32 * s:32 * s + 32].astype(np.float64)) for s in range(x.size // 32)]
        for form in (0, 1):
            print(f"staged quantizer case {i} form {form} n={x.size}", flush=True)
            rc, got, sums = eng.quantize_staged(x, form)
            assert rc == fa.OK, (i, form, rc)
            nz = want != 0
            assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32)), (i, form)
            assert np.all(got[~nz] == 0), (i, form)
            assert np.array_equal(sums, np.array(exact)), (i, form)
    bad = cases[0].copy()
    bad[777] = np.nan
    for form in (0, 1):
        rc, _, _ = eng.quantize_staged(bad, form)
        assert rc == fa.NUMERIC, form
    for h in [(rng.standard_normal(32) * 1e4).astype(np.float32), ties[:32].copy(), sub[:32].copy(),
              np.zeros(32, np.float32)]:
        rc, got, _ = eng.quantize_staged(h, 2)
        assert rc == fa.OK
        assert np.array_equal(got.view(np.uint32), oracle.q8_activation(h)[1].view(np.uint32))
