"""The synthetic measurement generator of the oracle (fo_synth_*).

The generator is not a reference function; it writes the measurement
configurations' distributions. What pins it:
  * fo_synth_scale against numpy's float64 -> float16 cast (round to nearest
    even, an independent implementation) on random and boundary inputs;
  * every field of every block type lies in its stated range and the
    nibble/code/int8 histograms cover their whole alphabets;
  * byte-wise generation equals slice-wise generation, and the bytes depend on
    every key field (seed, block, layer, expert).
"""
import numpy as np
import pytest

import oracle

H = 4096


def scale_value(h):
    u = np.float64(h >> 40) * 2.0 ** -24
    return np.float16(np.float64(1e-3) + np.float64(9e-3) * u)


def test_scale_rounding_matches_numpy():
    rng = np.random.default_rng(5)
    hs = [int(v) for v in rng.integers(0, 2 ** 63, 4000, dtype=np.int64)] + [0, (1 << 64) - 1, 1 << 40, (1 << 63)]
    for h in hs:
        got = oracle.synth_scale(h)
        want = int(scale_value(h).view(np.uint16))
        assert got == want, hex(h)


def test_scale_boundary_ties():
    # Search for u where the fp64 value sits exactly on a binary16 midpoint is
    # impractical; instead check the whole top-24-bit range on a stride that
    # visits every binade of the output and both ends.
    for top in list(range(0, 1 << 24, 4099)) + [(1 << 24) - 1]:
        h = top << 40
        assert oracle.synth_scale(h) == int(scale_value(h).view(np.uint16))


def q4k_fields(row):
    sb = row.reshape(-1, 144)
    d = sb[:, 0:2].copy().view(np.float16).ravel()
    dmin = sb[:, 2:4].copy().view(np.float16).ravel()
    return d, dmin, sb[:, 4:16], sb[:, 16:]


def in_scale_range(v):
    lo, hi = np.float16(1e-3), np.float16(1e-2)
    return np.all((v >= lo) & (v <= hi))


@pytest.mark.parametrize("fmt", [oracle.FMT_Q4KT, oracle.FMT_NATIVE, oracle.FMT_Q8, oracle.FMT_MXFP4])
def test_slice_distributions(fmt):
    lay = oracle.layout(H, fmt)
    s = oracle.synth_slice(lay, 99, 4, 7, 300)
    assert s.size == lay.slice
    gu = s[:2 * lay.proj]
    dn = s[2 * lay.proj:]
    if fmt in (oracle.FMT_Q4KT, oracle.FMT_NATIVE):
        d, dmin, scales, nib = q4k_fields(gu)
        assert in_scale_range(d) and in_scale_range(dmin)
        assert len(np.unique(d)) > 50
        q = np.concatenate([nib & 15, nib >> 4]).ravel()
        assert np.bincount(q, minlength=16).min() > 0.9 * q.size / 16
        six = np.concatenate([(scales[:, :8] & 63).ravel(), (scales[:, 8:] & 15).ravel()])
        assert six.max() == 63 and np.bincount(scales[:, :8].ravel() & 63, minlength=64).min() > 0
    if fmt == oracle.FMT_Q4KT:
        d, dmin, _, _ = q4k_fields(dn)
        assert in_scale_range(d) and in_scale_range(dmin)
    if fmt == oracle.FMT_Q8:
        for part in (gu, dn):
            b = part.reshape(-1, 34)
            d = b[:, 0:2].copy().view(np.float16).ravel()
            assert in_scale_range(d)
            q = b[:, 2:].view(np.int8).ravel()
            assert q.min() == -127 and q.max() == 127
            counts = np.bincount(q.astype(np.int64) + 127, minlength=255)
            assert counts.size == 255 and counts.min() > 0.8 * q.size / 255
    if fmt in (oracle.FMT_MXFP4, oracle.FMT_NATIVE):
        parts = [dn] if fmt == oracle.FMT_NATIVE else [gu, dn]
        for part in parts:
            b = part.reshape(-1, 17)
            e = b[:, 0]
            assert e.min() == 118 and e.max() == 130 and len(np.unique(e)) == 13
            codes = np.concatenate([b[:, 1:] & 15, b[:, 1:] >> 4]).ravel()
            assert np.bincount(codes, minlength=16).min() > 0.9 * codes.size / 16


def test_shared_slice_is_q8():
    lay = oracle.layout(H, oracle.FMT_Q4KT)
    s = oracle.synth_slice(lay, 99, 0, 0, 512)
    assert s.size == lay.shared_slice
    b = s.reshape(-1, 34)
    assert in_scale_range(b[:, 0:2].copy().view(np.float16).ravel())
    assert b[:, 2:].view(np.int8).min() >= -127


def test_bytewise_equals_slicewise_and_keys_matter():
    import ctypes as C
    lay = oracle.layout(H, oracle.FMT_Q4KT)
    s = oracle.synth_slice(lay, 3, 2, 1, 9)
    key = oracle.lib().fo_synth_key(3, 2, 1, 9)
    rng = np.random.default_rng(0)
    for o in rng.integers(0, lay.slice, 200):
        assert oracle.lib().fo_synth_byte(C.byref(lay), key, 9, int(o)) == s[o]
    for args in [(4, 2, 1, 9), (3, 3, 1, 9), (3, 2, 2, 9), (3, 2, 1, 10)]:
        other = oracle.synth_slice(lay, *args)
        assert np.mean(other != s) > 0.5, args
    assert np.array_equal(oracle.synth_slice(lay, 3, 2, 1, 9), s)
