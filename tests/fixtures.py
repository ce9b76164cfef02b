"""Shared synthetic inputs for the parity tests (not collected by pytest).

Units are sparse: np.zeros maps pages lazily, so a 48-layer unit of several GB
costs memory only for the slices a test fills.
"""
import numpy as np

import oracle

TYPE_BYTES = {oracle.Q4_K: (256, 144), oracle.Q8_0: (32, 34), oracle.MXFP4: (32, 17), oracle.Q4_0: (32, 18)}


def half_bits(v):
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def baseline_row(rng, typ, n):
    """One row of n weights with the measurement distributions: Q4_K nibbles
    and 6-bit scales/mins uniform, fp16 d/dmin uniform in [1e-3, 1e-2]; Q8_0
    int8 uniform in [-127, 127] with fp16 d in [1e-3, 1e-2]; MXFP4 codes uniform
    over 16 with E8M0 uniform in [118, 130]; Q4_0 random signed d."""
    per, size = TYPE_BYTES[typ]
    nb = n // per
    b = rng.integers(0, 256, (nb, size), dtype=np.uint8)
    if typ == oracle.Q4_K:
        d = half_bits(rng.uniform(1e-3, 1e-2, (nb, 2)))
        b[:, 0:4] = d.view(np.uint8).reshape(nb, 4)
    elif typ == oracle.Q8_0:
        b[:, 0:2] = half_bits(rng.uniform(1e-3, 1e-2, nb)).view(np.uint8).reshape(nb, 2)
        b[:, 2:] = (rng.integers(-127, 128, (nb, 32)).astype(np.int8)).view(np.uint8)
    elif typ == oracle.MXFP4:
        b[:, 0] = rng.integers(118, 131, nb)
    else:
        b[:, 0:2] = half_bits(rng.uniform(1e-3, 1e-2, nb) * rng.choice([-1, 1], nb)).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def fill_baseline_slice(view, lay, expert, rng):
    """Write one slice (routed or shared) of `lay` with baseline_row rows."""
    shared = expert == oracle.SHARED
    gu = lay.shared_gu_type if shared else lay.gu_type
    dn = lay.shared_down_type if shared else lay.down_type
    H = lay.hidden
    row = oracle.lib().fo_row_bytes(gu, H)
    off = 0
    for _ in range(64):
        view[off:off + row] = baseline_row(rng, gu, H)
        off += row
    if not shared and lay.down_transposed:
        drow = oracle.lib().fo_row_bytes(dn, H)
        for _ in range(32):
            view[off:off + drow] = baseline_row(rng, dn, H)
            off += drow
    else:
        drow = oracle.lib().fo_row_bytes(dn, 32)
        view[off:off + H * drow] = baseline_row(rng, dn, 32 * H)
        off += H * drow
    assert off == (lay.shared_slice if shared else lay.slice)


def sparse_unit(lay):
    return np.zeros(lay.block, np.uint8)


def slice_view(unit, lay, layer, expert):
    off = oracle.slice_offset(lay, layer, expert)
    size = lay.shared_slice if expert == oracle.SHARED else lay.slice
    return unit[off:off + size]


def fill_experts(unit, lay, layer, experts, seed):
    rng = np.random.default_rng(seed)
    for e in experts:
        fill_baseline_slice(slice_view(unit, lay, layer, e), lay, e, rng)


def softmax_gates(rng, burst, k=10):
    logits = rng.standard_normal((burst, k)).astype(np.float64)
    g = np.exp(logits - logits.max(axis=1, keepdims=True))
    return (g / g.sum(axis=1, keepdims=True)).astype(np.float32)


def zipf_routes(rng, burst, s=1.1, experts=512, k=10):
    """Per-token top-k without replacement under Zipf(s) popularity over a
    seeded permutation of the experts."""
    perm = rng.permutation(experts)
    w = 1.0 / np.arange(1, experts + 1) ** s
    w /= w.sum()
    return np.stack([perm[rng.choice(experts, k, replace=False, p=w)] for _ in range(burst)]).astype(np.uint16)


def oracle_request(layer, experts, gates, x):
    req = oracle.Req()
    burst, hidden = x.shape
    req.layer, req.burst, req.hidden = layer, burst, hidden
    req.experts()[:burst] = experts
    req.gates()[:burst] = gates
    req.xs()[:burst, :hidden] = x
    return req


def native_fixture(lay, layer=47):
    """The reference's native fixture recipe (src/native.c:66-76): experts
    0..79 and the shared slice filled from LCG seed 7, then 8 tokens of x =
    (r % 257 - 128)/128 and gates 0.0625 (shared 0.5)."""
    data = sparse_unit(lay)
    seed = 7
    for e in range(81):
        eid = oracle.SHARED if e == 80 else e
        seed = oracle.fill_slice(slice_view(data, lay, layer, eid), lay, eid, seed)
    gates = np.full((8, 11), 0.0625, np.float32)
    gates[:, 10] = 0.5
    H = lay.hidden
    x = np.zeros((8, H), np.float32)
    lib = oracle.lib()
    import ctypes as C
    s = C.c_uint32(seed)
    for t in range(8):
        for j in range(H):
            v = lib.fo_lcg(C.byref(s))
            x[t, j] = np.float32((v % 257) - 128) / np.float32(128)
    return data, gates, x


def host_units(lay, seed, layer, experts, blocks=20):
    """Sparse host copies of the device's synthetic blocks 0..blocks-1 holding
    just the slices of `experts` (and the shared slice) at `layer`."""
    used = sorted(set(int(e) for e in np.asarray(experts).ravel()) | {oracle.SHARED})
    units = []
    for b in range(blocks):
        u = sparse_unit(lay)
        for e in used:
            slice_view(u, lay, layer, e)[:] = oracle.synth_slice(lay, seed, b, layer, e)
        units.append(u)
    return units


def dense_slice(view, lay, expert):
    """(Wg, Wu, Wd) float64 of one slice; Wd is [H x 32] in every format."""
    H = lay.hidden
    shared = expert == oracle.SHARED
    gu = lay.shared_gu_type if shared else lay.gu_type
    dn = lay.shared_down_type if shared else lay.down_type
    row = oracle.lib().fo_row_bytes(gu, H)
    proj = lay.shared_proj if shared else lay.proj
    Wg = np.stack([oracle.dequant(view[n * row:(n + 1) * row], gu, H) for n in range(32)]).astype(np.float64)
    Wu = np.stack([oracle.dequant(view[proj + n * row:proj + (n + 1) * row], gu, H) for n in range(32)]).astype(np.float64)
    base = view[2 * proj:]
    if not shared and lay.down_transposed:
        drow = oracle.lib().fo_row_bytes(dn, H)
        Wd = np.stack([oracle.dequant(base[n * drow:(n + 1) * drow], dn, H) for n in range(32)]).astype(np.float64).T
    else:
        drow = oracle.lib().fo_row_bytes(dn, 32)
        Wd = np.stack([oracle.dequant(base[d * drow:(d + 1) * drow], dn, 32) for d in range(H)]).astype(np.float64)
    return Wg, Wu, Wd
