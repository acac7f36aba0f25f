"""Pins of the oracle's integer and scalar primitives against facts that do not
come from the oracle itself: published constants, known answers, closed forms."""
import math

import numpy as np
import pytest

from common import spec_cfg0


def lowbias32_np(x):
    x = np.asarray(x, np.uint64) & 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x ^= x >> 15
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    x ^= x >> 16
    return x.astype(np.uint32)


def lowbias32_inverse(x):
    # published inverse of lowbias32 (C. Wellons, hash-prospector): an independent
    # check of both multiplier constants of ffnerf_OG.cl:296-300
    x = np.asarray(x, np.uint64) & 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x43021123) & 0xFFFFFFFF
    x ^= (x >> 15) ^ (x >> 30)
    x = (x * 0x1D69E2A5) & 0xFFFFFFFF
    x ^= x >> 16
    return x.astype(np.uint32)


def test_hash_u32_is_lowbias32(ora):
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.integers(0, 2 ** 32, 4000, dtype=np.uint64), [0, 1, 2, 0xFFFFFFFF, 0x80000000]])
    got = np.array([ora.hash_u32(int(v)) for v in xs], np.uint32)
    assert np.array_equal(lowbias32_inverse(got), xs.astype(np.uint32))
    assert np.array_equal(got, lowbias32_np(xs))


def test_xorshift32_marsaglia_known_answer(ora):
    # G. Marsaglia, "Xorshift RNGs" (2003): y = 2463534242, (13, 17, 5) -> 723471715
    assert ora.lib().ora_xorshift32(2463534242) == 723471715
    # rand01 takes the low 24 bits of the new state (ffnerf_OG.cl:303-311)
    assert ora.lib().ora_rand01_first(2463534242) == np.float32((723471715 & 0xFFFFFF) / 16777216.0)


def test_det_pow_within_one_ulp(ora):
    rng = np.random.default_rng(1)
    xs = np.concatenate([np.exp(rng.uniform(-30, 8, 20000)), [1.0, 2.0, 0.5, 1e-30, 3.4e25]]).astype(np.float32)
    got = np.array([ora.det_powr(float(x), 1.3) for x in xs], np.float32)
    ref = np.power(xs.astype(np.float64), np.float64(np.float32(1.3)))
    ulp = np.abs(got.astype(np.float64) - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 1.0, ulp.max()
    assert np.mean(got == ref.astype(np.float32)) > 0.999


def test_det_log_exp_closed_forms(ora):
    L = ora.lib()
    for x in (1.0, 2.0, 0.5, 10.0, 1e-300, 1e300, 3.0):
        assert L.ora_det_log(x) == pytest.approx(math.log(x), rel=2e-16, abs=2e-16)
    for z in (0.0, 1.0, -1.0, 50.0, -600.0, 0.3465):
        assert L.ora_det_exp(z) == pytest.approx(math.exp(z), rel=4e-16)
    assert L.ora_det_log(1.0) == 0.0
    assert L.ora_det_exp(0.0) == 1.0


def _aabb(ora, o, d, bmin, bmax):
    f = lambda v: np.ascontiguousarray(v, np.float32)
    t0 = np.zeros(1, np.float32)
    t1 = np.zeros(1, np.float32)
    hit = ora.lib().ora_ray_aabb(ora.fptr(f(o)), ora.fptr(f(d)), ora.fptr(f(bmin)), ora.fptr(f(bmax)),
                                 ora.fptr(t0), ora.fptr(t1))
    return hit, float(t0[0]), float(t1[0])


def test_ray_aabb_slab_cases(ora):
    bmin, bmax = [0, 0, 0], [1, 1, 1]
    # axis-parallel ray: zero direction components take the 1/0 = INF branch
    hit, t0, t1 = _aabb(ora, [-1.0, 0.5, 0.5], [1.0, 0.0, 0.0], bmin, bmax)
    assert hit and t0 == 1.0 and t1 == 2.0
    # diagonal through the corners
    s = 1 / math.sqrt(3)
    hit, t0, t1 = _aabb(ora, [-1, -1, -1], [s, s, s], bmin, bmax)
    assert hit and t0 == pytest.approx(math.sqrt(3), rel=1e-6) and t1 == pytest.approx(2 * math.sqrt(3), rel=1e-6)
    # miss
    hit, _, _ = _aabb(ora, [-1.0, 2.0, 0.5], [1.0, 0.0, 0.0], bmin, bmax)
    assert not hit
    # origin inside: t0 < 0 < t1
    hit, t0, t1 = _aabb(ora, [0.5, 0.5, 0.5], [0.0, 0.0, -1.0], bmin, bmax)
    assert hit and t0 == -0.5 and t1 == 0.5


def test_scan_trees_match_prefix_sums_for_addition(ora):
    # addition is commutative: the reference's tree order must give the exact
    # exclusive prefix for integer-valued floats
    for n in (1, 2, 4, 8, 16, 32, 64):
        a = np.arange(1, n + 1, dtype=np.float32)
        b = a.copy()
        ora.lib().ora_scan_excl_f(ora.fptr(b), n)
        assert np.array_equal(b, np.concatenate([[0], np.cumsum(a)[:-1]]).astype(np.float32))
        c = a.copy()
        assert ora.lib().ora_reduce_sum_f(ora.fptr(c), n) == a.sum()


def _emulate_reference_aff_scan(a, b):
    """The reference's Blelloch loop (ffnerf_OG.cl:715-735) on affine maps in
    float64, written as an independent emulation of its index arithmetic."""
    n = len(a)
    s = [(a[i], b[i]) for i in range(n)]
    comb = lambda L, R: (R[0] * L[0], R[0] * L[1] + R[1])
    st = 1
    while st < n:
        for lid in range(n):
            idx = (lid + 1) * (st << 1) - 1
            if idx < n:
                s[idx] = comb(s[idx - st], s[idx])
        st <<= 1
    s[n - 1] = (1.0, 0.0)
    st = n >> 1
    while st >= 1:
        for lid in range(n):
            idx = (lid + 1) * (st << 1) - 1
            if idx < n:
                t = s[idx - st]
                s[idx - st] = s[idx]
                s[idx] = comb(t, s[idx])
        if st == 1:
            break
        st >>= 1
    return s


def test_aff_scan_reproduces_reference_operand_order(ora):
    """The reference's down-sweep composes non-commuting affine maps out of
    order at prefixes 3, 5, 6, 7, 9, ...; the oracle must do the same."""
    n = 16
    rng = np.random.default_rng(3)
    a = rng.uniform(0.2, 0.9, n).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    aa, bb = a.copy(), b.copy()
    ta = np.zeros(1, np.float32)
    tb = np.zeros(1, np.float32)
    ora.lib().ora_scan_excl_aff_rev(ora.fptr(aa), ora.fptr(bb), n, ora.fptr(ta), ora.fptr(tb))
    emu = _emulate_reference_aff_scan(a.astype(np.float64), b.astype(np.float64))
    assert np.allclose(aa, [e[0] for e in emu], rtol=1e-6)
    assert np.allclose(bb, [e[1] for e in emu], rtol=1e-5, atol=1e-6)
    # the true exclusive prefix (maps applied in index order) differs exactly where predicted
    true = [(1.0, 0.0)]
    for i in range(n - 1):
        A, B = true[-1]
        true.append((a[i] * A, a[i] * B + b[i]))
    wrong = [i for i in range(n) if abs(true[i][1] - bb[i]) > 1e-5]
    assert wrong == [3, 5, 6, 7, 9, 10, 11, 12, 13, 14, 15]


def test_sh_basis_orthonormal(ora):
    # real SH of degree <= 3 (ffnerf_OG.cl:572-602) are orthonormal on the sphere
    n = 20000
    i = np.arange(n) + 0.5
    phi = np.arccos(1 - 2 * i / n)
    th = np.pi * (1 + 5 ** 0.5) * i
    dirs = np.stack([np.cos(th) * np.sin(phi), np.sin(th) * np.sin(phi), np.cos(phi)], 1).astype(np.float32)
    Y = np.zeros((n, 16), np.float32)
    for k in range(n):
        ora.lib().ora_sh_encode(ora.fptr(np.ascontiguousarray(dirs[k])), ora.fptr(Y[k]))
    gram = (Y.astype(np.float64).T @ Y.astype(np.float64)) * (4 * np.pi / n)
    assert np.allclose(gram, np.eye(16), atol=2e-3)


def test_decay_expectation_and_paths(ora):
    """decay_occ_grid_in-st.cl: E[q'] = q*d for every nibble of an unchanged
    word; a raised nibble keeps its proposal; q = 1 stays."""
    n = 20000
    d = 0.9
    q24 = int(round(d * (1 << 24)))
    for q in (2, 5, 9, 16):
        word = sum((q - 1) << (4 * s) for s in range(8))
        occ_in = np.full(n, word, np.uint32)
        occ_st = occ_in.copy()
        ora.occ_decay(occ_in, occ_st, q24, seed=77)
        assert np.array_equal(occ_in, occ_st)
        nib = np.stack([((occ_in >> (4 * s)) & 0xF) + 1 for s in range(8)], 1).astype(np.float64)
        assert abs(nib.mean() - q * d) < 0.01
        assert set(np.unique(nib)).issubset({math.floor(q * d), math.floor(q * d) + 1})
    # mixed word: nibble 0 raised by a proposal (kept), nibble 1 equal (decays), q=1 nibble fixed
    win = np.full(n, 0x00000053, np.uint32)  # nibbles: q=4, q=6, rest q=1
    wst = np.full(n, 0x0000005A, np.uint32)  # nibble 0 raised to q=11
    ora.occ_decay(win, wst, q24, seed=5)
    assert np.all((wst & 0xF) == 0xA)
    assert np.all((wst >> 8) == 0)
    q1 = ((wst >> 4) & 0xF) + 1
    assert abs(q1.mean() - 6 * d) < 0.02


def test_adam_step_one_closed_form(ora):
    # first Adam step from zero state: m = (1-b1) g, v = (1-b2) g^2 (weight_update.cl:177-201)
    rng = np.random.default_rng(2)
    g = rng.normal(size=1000).astype(np.float32)
    p = rng.normal(size=1000).astype(np.float32)
    p0 = p.copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    b1, b2, eps, lr = 0.9, 0.99, 1e-15, 1e-2
    ora.adam(p, m, v, g, lr, b1, b2, eps)
    exp = p0 - lr * (1 - b1) * g / (np.sqrt((1 - b2) * g.astype(np.float64) ** 2) + eps)
    assert np.allclose(p, exp, rtol=1e-6, atol=1e-7)
    assert np.allclose(m, (1 - b1) * g, rtol=1e-6)


def test_binary16_rounding_matches_numpy(ora):
    """The oracle's float32 -> binary16 rounding (fp16 tables) against numpy's astype(float16), which rounds
    to nearest even: every finite half round-trips, the midpoints between neighbours (ties) go to the even
    one, and random floats over the whole range (subnormals, overflow to infinity) agree."""
    lib = ora.lib()
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    h = bits.view(np.float16)
    finite = np.isfinite(h)
    f32 = h.astype(np.float32)
    for b, v in zip(bits[finite], f32[finite]):
        assert lib.ora_f32_to_f16_bits(float(v)) == int(b)
        assert np.float32(lib.ora_f16_bits_to_f32(int(b))).view(np.uint32) == v.view(np.uint32)
    pos = np.sort(f32[finite & (f32 >= 0)]).astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)          # exact in float32
    rng = np.random.default_rng(7)
    rand = np.concatenate([rng.uniform(-7e4, 7e4, 20000), rng.standard_normal(20000) * 1e-5,
                           rng.standard_normal(20000) * 1e-7, [65519.99, 65520.0, -65520.0, 1e-8, 5.96e-8, 2.98e-8]])
    for v in np.concatenate([mids, -mids[:2000], rand.astype(np.float32)]):
        with np.errstate(over="ignore"):  # values past 65520 become infinity, as intended
            want = np.float32(v).astype(np.float16).view(np.uint16)
        assert lib.ora_f32_to_f16_bits(float(v)) == int(want), v
