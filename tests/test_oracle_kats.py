"""Known-answer tests that pin each oracle primitive independently.

Restated from the reference's own unit tests (tests/test_q4.c, tests/test_native.c,
tests/test_backend.c) plus closed forms the mathematics fixes. None of these
recomputes the oracle's formula: each answer comes from an independent
construction (bit-level IEEE decoding, one-hot basis vectors, analytic SiLU).
"""
import ctypes as C
import math
import struct

import numpy as np
import pytest

import oracle


def f16_closed_form(i):
    e, m = (i >> 10) & 31, i & 1023
    if e == 31:
        return math.nan if m else (-math.inf if i & 0x8000 else math.inf)
    v = math.ldexp(1.0 + m / 1024, e - 15) if e else math.ldexp(m, -24)
    return -v if i & 0x8000 else v


def test_f16_all_codes():
    """All 65,536 encodings incl. signed zero, subnormals and specials (tests/test_q4.c:12-20)."""
    lib = oracle.lib()
    for i in range(65536):
        got = lib.fo_f16(i)
        want = f16_closed_form(i)
        if math.isnan(want):
            assert math.isnan(got)
        else:
            assert got == want and math.copysign(1, got) == (-1 if i & 0x8000 else 1), i
    # numpy's independent binary16 decoder agrees bit for bit.
    codes = np.arange(65536, dtype=np.uint16)
    ours = np.array([lib.fo_f16(int(c)) for c in codes[::97]], np.float32)
    ref = codes[::97].view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    assert np.array_equal(ours[~np.isnan(ours)], ref[~np.isnan(ref)])


def test_q4_0_nibble_basis():
    """Low nibble = column j, high nibble = j+16, levels q-8 (tests/test_q4.c:21-38)."""
    q = np.zeros(37, np.uint8)[1:]          # deliberately unaligned
    q[1] = 0x3C                              # d = 1
    for i in range(16):
        q[2 + i] = i | ((15 - i) << 4)
    lib = oracle.lib()
    out = C.c_double()
    for i in range(32):
        x = np.zeros(64, np.float32)
        x[i] = 1
        assert lib.fo_q4_dot(oracle.u8ptr(q), oracle.fptr(x), 32, C.byref(out)) == 0
        assert out.value == (i - 8 if i < 16 else 23 - i)
    x = np.zeros(64, np.float32)
    x[31] = 1
    q[1] = 0xBC
    assert lib.fo_q4_dot(oracle.u8ptr(q), oracle.fptr(x), 32, C.byref(out)) == 0 and out.value == 8
    q[0], q[1] = 1, 0
    assert lib.fo_q4_dot(oracle.u8ptr(q), oracle.fptr(x), 32, C.byref(out)) == 0 and out.value == -8 * 2.0 ** -24
    q[0], q[1] = 0, 0x7C
    out.value = 123
    assert lib.fo_q4_dot(oracle.u8ptr(q), oracle.fptr(x), 32, C.byref(out)) == oracle.NUMERIC and out.value == 123
    assert lib.fo_q4_dot(oracle.u8ptr(q), oracle.fptr(x), 31, C.byref(out)) == oracle.INVALID
    q[:] = 0
    q[1] = q[19] = 0x3C
    q[2], q[20] = 9, 7
    x = np.zeros(64, np.float32)
    x[0], x[32] = 2, 3
    assert lib.fo_q4_dot(oracle.u8ptr(q), oracle.fptr(x), 64, C.byref(out)) == 0 and out.value == -1


def test_q8_activation_kats():
    """tests/test_q4.c:39-57: nearest-even ties, 64+32 groups, in place, zeros,
    FLT_MAX, underflow, reciprocal overflow, NaN, shape."""
    x = np.zeros(96, np.float32)
    x[:7] = [127, .5, 1.5, 2.5, -.5, -1.5, -2.5]
    x[64], x[65] = 254, 3
    rc, out = oracle.q8_activation(x)
    assert rc == 0
    assert list(out[:7]) == [127, 0, 2, 2, 0, -2, -2] and out[64] == 254 and out[65] == 4
    inplace = x.copy()
    assert oracle.lib().fo_q8_activation(oracle.fptr(inplace), oracle.fptr(inplace), 96) == 0
    assert np.array_equal(inplace, out)
    rc, out = oracle.q8_activation(np.zeros(96, np.float32))
    assert rc == 0 and not out.any()
    big = np.zeros(32, np.float32)
    big[0] = np.finfo(np.float32).max
    rc, out = oracle.q8_activation(big)
    assert rc == 0 and np.isfinite(out[0]) and out[0] > np.finfo(np.float32).max * np.float32(0.99)
    tiny = np.zeros(32, np.float32)
    tiny[0] = 2.0 ** -149
    rc, out = oracle.q8_activation(tiny)
    assert rc == 0 and out[0] == 0
    tiny[0] = 2.0 ** -125
    rc, out = oracle.q8_activation(tiny)
    assert rc == 0 and np.isfinite(out[0]) and out[0] > 0
    tiny[0] = np.nan
    assert oracle.q8_activation(tiny)[0] == oracle.NUMERIC
    assert oracle.lib().fo_q8_activation(oracle.fptr(tiny), oracle.fptr(tiny), 31) == oracle.INVALID


def test_quantize8_closed_forms():
    """AVX2 quantize8 (backends/avx2.c:184-203): RNE ties, int16 sums per 32,
    a zero group gives d = 0 and zero codes, and a subnormal group whose
    multiplier overflows saturates to -128 through the packs."""
    x = np.zeros(256, np.float32)
    x[:6] = [127, 0.5, 1.5, 2.5, -0.5, -2.5]
    q, d, s = oracle.quantize8(x, 256)
    assert d[0] == np.float32(127) / np.float32(127)
    assert list(q[:6]) == [127, 0, 2, 2, 0, -2]
    assert s[0] == 127 + 0 + 2 + 2 + 0 - 2 and not s[1:].any()
    q, d, s = oracle.quantize8(np.zeros(32, np.float32), 32)
    assert d[0] == 0 and not q.any() and s[0] == 0
    sub = np.zeros(32, np.float32)
    sub[0] = 2.0 ** -140                     # 127/amax overflows to inf
    q, d, s = oracle.quantize8(sub, 32)
    # x*inf = inf and 0*inf = NaN both convert to INT32_MIN and pack to -128;
    # 32 * INT32_MIN wraps to 0 in the int32 sum.
    assert (q == -128).all() and s[0] == 0


def q4k_basis_block():
    """Super-block with d = 1, dmin = .5, scales {1,2,3,4,17,34,51,63} and mins
    {63,51,34,17,4,3,2,1} packed per the 6-bit layout (tests/test_native.c:7-10)."""
    sc = [1, 2, 3, 4, 17, 34, 51, 63]
    mi = [63, 51, 34, 17, 4, 3, 2, 1]
    q = np.zeros(144, np.uint8)
    q[1], q[3] = 0x3C, 0x38
    for g in range(4):
        q[4 + g] = sc[g] | ((sc[g + 4] >> 4) << 6)
        q[8 + g] = mi[g] | ((mi[g + 4] >> 4) << 6)
        q[12 + g] = (sc[g + 4] & 15) | ((mi[g + 4] & 15) << 4)
    for j in range(128):
        q[16 + j] = (j % 16) | ((15 - j % 16) << 4)
    return q, sc, mi


def test_q4k_all_lanes():
    """Every sub-block scale/min, both nibbles, all 256 lanes (tests/test_native.c:7-17)."""
    q, sc, mi = q4k_basis_block()
    for j in range(256):
        x = np.zeros(256, np.float32)
        x[j] = 1
        g = j // 32
        v = 15 - j % 16 if g % 2 else j % 16
        rc, y = oracle.native_dot(q, oracle.Q4_K, x)
        assert rc == 0 and y == sc[g] * v - .5 * mi[g], j
    w = oracle.dequant(q, oracle.Q4_K, 256)
    assert np.array_equal(w, np.array([sc[j // 32] * (15 - j % 16 if (j // 32) % 2 else j % 16) - .5 * mi[j // 32]
                                       for j in range(256)], np.float32))
    q[1] = 0x7C
    assert oracle.native_dot(q, oracle.Q4_K, np.ones(256, np.float32))[0] == oracle.NUMERIC
    q[1] = 0x3C
    assert oracle.native_dot(q, oracle.Q4_K, np.ones(256, np.float32), 32)[0] == oracle.INVALID


def test_mxfp4_lut_signs_order():
    """E2M1 values, sign, nibble order, E8M0 0 -> 2^-127, 255 refused
    (tests/test_native.c:19-27)."""
    values = [0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6]
    mx = np.zeros(17, np.uint8)
    mx[0] = 127
    for j in range(16):
        mx[j + 1] = j | ((15 - j) << 4)
    for j in range(32):
        x = np.zeros(32, np.float32)
        x[j] = 1
        rc, y = oracle.native_dot(mx, oracle.MXFP4, x)
        assert rc == 0 and y == values[j if j < 16 else 31 - j]
    x = np.zeros(32, np.float32)
    x[2] = 1
    mx[0] = 0
    rc, y = oracle.native_dot(mx, oracle.MXFP4, x)
    assert rc == 0 and y == math.ldexp(1, -127)
    mx[0] = 255
    assert oracle.native_dot(mx, oracle.MXFP4, x)[0] == oracle.NUMERIC


def test_q8_0_signed_byte():
    """d = .5, byte 128 -> -64 (tests/test_native.c:28-29)."""
    sh = np.zeros(34, np.uint8)
    sh[1], sh[4] = 0x38, 128
    x = np.zeros(32, np.float32)
    x[2] = 1
    rc, y = oracle.native_dot(sh, oracle.Q8_0, x)
    assert rc == 0 and y == -64


@pytest.mark.parametrize("hidden", [2560, 4096])
def test_layout_totals(hidden):
    """The native unit ends exactly with the shared slice of layer 47
    (tests/test_native.c:31); sizes of every format."""
    for fmt in [oracle.FMT_NATIVE, oracle.FMT_Q4KT, oracle.FMT_Q8, oracle.FMT_MXFP4]:
        lay = oracle.layout(hidden, fmt)
        assert oracle.slice_offset(lay, 47, 512) + lay.shared_slice == lay.block
    lay = oracle.layout(2560, oracle.FMT_NATIVE)
    assert lay.slice == 135680 and lay.layer == 69729280 and lay.block == 3347005440
    leg = oracle.layout(2560, oracle.FMT_LEGACY)
    assert leg.block == 3404021760
    q4kt = oracle.layout(4096, oracle.FMT_Q4KT)
    assert q4kt.slice == 221184 and oracle.layout(4096, oracle.FMT_NATIVE).slice == 217088
    assert oracle.layout(4096, oracle.FMT_Q8).slice == 417792
    assert oracle.layout(4096, oracle.FMT_MXFP4).slice == 208896


def test_compare_edge_cases():
    """tests/test_backend.c:166-182."""
    a = np.array([1, 2, -3], np.float32)
    rc, e = oracle.compare(a, a)
    assert rc == 0 and e[0] == 0 and e[1] == 0 and e[2] > 0.999999999999
    rc, e = oracle.compare(a, -a)
    assert e[0] == 2 and e[1] == 2 and e[2] < -.9999 and not oracle.conforms(e, oracle.BACKEND_TOLERANCE)
    z = np.zeros(3, np.float32)
    rc, e = oracle.compare(z, z)
    assert oracle.conforms(e, oracle.BACKEND_TOLERANCE)
    s = z.copy()
    s[0] = 2.0 ** -149
    rc, e = oracle.compare(z, s)
    assert not oracle.conforms(e, oracle.BACKEND_TOLERANCE)
    rc, e = oracle.compare(a, z)
    assert e[2] == 0 and not oracle.conforms(e, oracle.BACKEND_TOLERANCE)
    assert oracle.compare(a, np.array([1, np.nan, 3], np.float32))[0] == oracle.NUMERIC
    t = oracle.BACKEND_TOLERANCE
    assert oracle.conforms(t, t)
    assert not oracle.conforms((np.nextafter(t[0], 1), 0, 1), t)
    assert not oracle.conforms((0, np.nextafter(t[1], 1), 1), t)
    assert not oracle.conforms((0, 0, np.nextafter(t[2], 0)), t)
