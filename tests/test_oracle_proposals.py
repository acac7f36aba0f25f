"""Pins of the oracle's occupancy proposals (ora_occ_propose_ray,
ffnerf_OG.cl:1640-1821) and of the sampler's proposal weights
(ora_sample_ray, ffnerf_OG.cl:1140-1206) by what the mathematics fixes:

- a transmittance that is linear in t makes the reference's interpolation at
  the cell faces exact, so each run's predicted absorption has a closed form
  (cell faces from a brute-force point-in-box scan along the ray); the
  stochastic rounding to 1/16 levels must land on the floor or ceiling of
  16 * pred, with mean 16 * pred over seeds;
- the keep probability's closed form against the keep frequency over seeds
  (a ray inside the distance where near-camera proposals are thinned);
- the marched proposal pass cuts a ray's samples into runs itself: fed a
  resampled ray's samples, its runs are the resampler's run flags, so it raises
  the grid exactly as the resampled pass with those flags does;
- a ray through two occupancy levels: systematic resampling puts
  S * P(first half) samples (to within one) into the first half, where
  P = 0.3 * 1/2 + 0.7 * w_a / (w_a + w_b), w = (rho dt)^1.3 -- in float64,
  checked against exponents and mixtures that a plausible mistake would use.
"""
import ctypes as C

import numpy as np
import pytest

from common import spec_cfg0

BOX_LO, BOX_HI, G = 0.0, 1.0, 32  # spec_cfg0: unit box, 32 occupancy words per axis (64 subcells)


def _propose(ora, cfg, ray, S, seed, Ts, DTs, Tr, T_final, flags, occ_in, occ_st):
    lib = ora.lib()
    f = ora.fptr
    lib.ora_occ_propose_ray(C.byref(cfg), f(np.ascontiguousarray(ray, np.float32)), 0, S, seed & 0xFFFFFFFF,
                            f(Ts), f(DTs), f(Tr), C.c_float(T_final), ora.uptr(flags), ora.uptr(occ_in),
                            ora.uptr(occ_st))


def _cell_sub(x):
    """(cell index, subcell, distance of the position to the nearest cell/subcell boundary in grid units)."""
    gpos = (np.asarray(x, np.float64) - BOX_LO) / (BOX_HI - BOX_LO) * G
    i = np.floor(gpos).astype(int)
    f = gpos - i
    sub = int((f[0] >= 0.5) + 2 * (f[1] >= 0.5) + 4 * (f[2] >= 0.5))
    margin = float(np.min(np.minimum(np.abs(f - 0.5), np.minimum(f, 1.0 - f))))
    return int(i[0] + G * (i[1] + G * i[2])), sub, tuple(i), margin


def _cell_faces_brute(o, d, ijk, lo_t, hi_t, step=2e-6):
    """First and last t in [lo_t, hi_t] where o + t d lies in the cell: a scan of points, not the slab."""
    t = np.arange(lo_t, hi_t, step)
    x = o[None, :] + t[:, None] * d[None, :]
    cmin = BOX_LO + np.array(ijk) * (BOX_HI - BOX_LO) / G
    cmax = cmin + (BOX_HI - BOX_LO) / G
    inside = np.all((x >= cmin) & (x <= cmax), axis=1)
    k = np.flatnonzero(inside)
    return t[k[0]], t[k[-1]]


def _ray_setup(o, d, t_start, h, S):
    o = np.asarray(o, np.float64)
    d = np.asarray(d, np.float64)
    d = d / np.linalg.norm(d)
    ts = (t_start + (np.arange(S) + 0.5) * h).astype(np.float32)
    x = o[None, :] + ts.astype(np.float64)[:, None] * d[None, :]
    keys, margins = [], []
    for s in range(S):
        cell, sub, ijk, mg = _cell_sub(x[s])
        keys.append((cell, sub, ijk))
        margins.append(mg)
    flags = np.zeros(2, np.uint32)
    for s in range(S):
        if s == 0 or keys[s][:2] != keys[s - 1][:2]:
            flags[s >> 5] |= np.uint32(1 << (s & 31))
    ray = np.zeros(8, np.float32)
    ray[:3], ray[3], ray[4:7] = o, 1.0, d
    return ray, ts, keys, float(min(margins)), flags


def _runs(flags, S):
    starts = [s for s in range(S) if (int(flags[s >> 5]) >> (s & 31)) & 1]
    return [(a, starts[i + 1] if i + 1 < len(starts) else S) for i, a in enumerate(starts)]


def _pred_closed_form(o, d, ts, T_of, T_final, run, ijk, S, t_near):
    """pred of the run [lid, nxt) with a linear transmittance T_of(t): the reference interpolates Tr between
    the samples around each cell face, which is exact for a linear T, so T_enter = T(clamp(t_enter, t_prev,
    t_cur)) and T_exit = T(clamp(t_exit, t_last, t_next)) (T_final past the last run)."""
    lid, nxt = run
    span = 0.2
    t_in, t_out = _cell_faces_brute(o, d, ijk, float(ts[lid]) - span, float(ts[lid]) + span)
    t_in = max(t_in, t_near)
    t_prev, t_cur = float(ts[max(lid - 1, 0)]), float(ts[lid])
    T_enter = T_of(min(max(t_in, t_prev), t_cur)) if lid > 0 else T_of(t_cur)
    if nxt < S:
        t_last, t_next = float(ts[nxt - 1]), float(ts[nxt])
        T_exit = T_of(min(max(t_out, t_last), t_next))
    else:
        T_exit = T_final
    return min(1.0, max(0.0, (T_enter - T_exit) / T_enter))


def test_proposal_levels_match_the_closed_form(ora):
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    S, h = 32, 0.011
    # an oblique ray through the box, all samples beyond the thinning distance (keep probability 1)
    ray, ts, keys, margin, flags = _ray_setup((-0.8, 0.131, 0.262), (1.0, 0.31, 0.17), 1.02, h, S)
    assert margin > 5e-4, margin  # no sample within float rounding (~1e-5 grid units) of a cell or subcell boundary
    o, d = ray[:3].astype(np.float64), ray[4:7].astype(np.float64)
    slope = 2.7
    T_of = lambda t: 1.0 - slope * (t - float(ts[0]))
    Tr = np.array([T_of(float(t)) for t in ts], np.float32)
    T_final = T_of(float(ts[-1]) + h)
    assert T_final > 0.03
    DTs = np.full(S, h, np.float32)
    runs = _runs(flags, S)
    assert len(runs) >= 8
    occ_in = np.zeros(G ** 3, np.uint32)  # level 1 everywhere: every run with 16 pred > 1 proposes
    preds = {r: _pred_closed_form(o, d, ts, T_of, T_final, r, keys[r[0]][2], S, spec["t_near"]) for r in runs}
    n_seeds = 2000
    q_sum = {r: 0.0 for r in runs}
    for seed in range(n_seeds):
        st = occ_in.copy()
        _propose(ora, cfg, ray, S, 0x1000 + 7919 * seed, ts, DTs, Tr, np.float32(T_final), flags, occ_in, st)
        for r in runs:
            cell, sub, _ = keys[r[0]]
            q = int((st[cell] >> (4 * sub)) & 0xF) + 1
            p16 = 16.0 * preds[r]
            if abs(p16 - 1.0) <= 1e-3:  # within rounding of the proposal threshold: either outcome
                continue
            if p16 < 1.0:
                assert q == 1, (r, q, p16)
                continue
            lo, hi = np.floor(p16 - 1e-4), np.floor(p16 + 1e-4) + 1
            assert lo <= q <= min(hi, 16), (r, q, p16)
            q_sum[r] += q
    proposing = [r for r in runs if 16.0 * preds[r] > 1.0 + 1e-3]
    assert len(proposing) >= 10
    for r in proposing:
        p16 = min(16.0 * preds[r], 16.0)
        frac = p16 - np.floor(p16)
        sd = np.sqrt(frac * (1 - frac) / n_seeds) + 1e-9
        assert abs(q_sum[r] / n_seeds - p16) <= 5 * sd + 1e-6, (r, q_sum[r] / n_seeds, p16)


def test_keep_probability_matches_the_closed_form(ora):
    """Rays closer than half the box diagonal D keep a proposal with probability
    f = (tl^2 + tl + 1/3) / (Dl^2 + Dl + 1/3), tl = t / lambda, Dl = D / lambda, lambda = x extent / G."""
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    S, h = 16, 0.009
    ray, ts, keys, margin, flags = _ray_setup((0.05, 0.5 + 0.13 / 64, 0.5 + 0.29 / 64), (1.0, 0.02, 0.01), 0.33, h, S)
    assert margin > 5e-4, margin
    slope = 6.0  # steep: runs predicting 16 pred >= 2 raise the level-1 grid whenever they are kept
    T_of = lambda t: 1.0 - slope * (t - float(ts[0]))
    Tr = np.array([T_of(float(t)) for t in ts], np.float32)
    T_final = np.float32(T_of(float(ts[-1]) + h))
    assert T_final > 0.0
    DTs = np.full(S, h, np.float32)
    runs = _runs(flags, S)
    lam = (BOX_HI - BOX_LO) / G
    D = 0.5 * np.sqrt(3.0) * (BOX_HI - BOX_LO)
    Dl = D / lam
    occ_in = np.zeros(G ** 3, np.uint32)
    n_seeds = 4000
    kept = {r: 0 for r in runs}
    for seed in range(n_seeds):
        st = occ_in.copy()
        _propose(ora, cfg, ray, S, 0xABC000 + 104729 * seed, ts, DTs, Tr, T_final, flags, occ_in, st)
        for r in runs:
            cell, sub, _ = keys[r[0]]
            kept[r] += int(((st[cell] >> (4 * sub)) & 0xF) != 0)
    checked = 0
    for r in runs:
        o, d = ray[:3].astype(np.float64), ray[4:7].astype(np.float64)
        if 16.0 * _pred_closed_form(o, d, ts, T_of, float(T_final), r, keys[r[0]][2], S, spec["t_near"]) < 2.001:
            continue
        tl = float(ts[r[0]]) / lam
        f = min(1.0, (tl * tl + tl + 1 / 3) / (Dl * Dl + Dl + 1 / 3))
        assert f < 0.5
        sd = np.sqrt(f * (1 - f) / n_seeds)
        assert abs(kept[r] / n_seeds - f) <= 5 * sd, (r, kept[r] / n_seeds, f)
        checked += 1
    assert checked >= 4


def _two_level_ray_counts(ora, qa, qb, S, seeds, do_train):
    """Samples of a ray along +x through the unit box whose first half (x < 1/2) has occupancy nibble qa - 1
    and second half qb - 1; returns the number of samples in the first half per seed."""
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    idx = np.arange(G ** 3)
    ix = idx % G
    occ = np.where(ix < G // 2, np.uint32(0x11111111 * (qa - 1)), np.uint32(0x11111111 * (qb - 1))).astype(np.uint32)
    ray = np.array([-1.0, 0.5 + 0.37 / 64, 0.5 + 0.21 / 64, 1.0, 1.0, 0.0, 0.0, 0.0], np.float32)
    counts = []
    for sd in seeds:
        Ts, DTs, _ = ora.sample_ray(cfg, ray, 0, S, sd, occ, do_train)
        x = ray[0] + Ts.astype(np.float64)
        assert np.all(DTs > 0)
        counts.append(int(np.sum(x < 0.5)))
    return np.array(counts)


def _p_first_half(qa, qb, gamma=1.3, uniform=0.3, infer=False, rho_min=1.0, rho_max=16.0):
    def q_eff(q):  # nibble + 1 in training; max(nibble - 2, 0) in inference
        return max(q - 3, 0) if infer else q
    ra, rb = (rho_min + (rho_max - rho_min) * q_eff(q) / 16.0 for q in (qa, qb))
    act_a, act_b = (1.0 if q_eff(q) > 0 else 0.0 for q in (qa, qb))
    if infer:
        ra, rb = ra * act_a, rb * act_b
    wa, wb = ra ** gamma if ra > 0 else 0.0, rb ** gamma if rb > 0 else 0.0
    n_act = act_a + act_b if infer else 2.0
    uni_a = (act_a if infer else 1.0) / n_act
    return uniform * uni_a + (1.0 - uniform) * wa / (wa + wb)


@pytest.mark.parametrize("qa,qb,do_train", [(16, 1, True), (1, 16, True), (9, 3, True), (13, 6, True),
                                            (13, 5, False), (11, 3, False)])
def test_sampler_weights_two_level_ray(ora, qa, qb, do_train):
    S = 64
    seeds = [3, 17, 256, 9001, 0xBEEF, 123457]
    counts = _two_level_ray_counts(ora, qa, qb, S, seeds, do_train)
    p = _p_first_half(qa, qb, infer=not do_train)
    # systematic resampling puts floor or ceil of S * P(first half) samples into a contiguous candidate range
    assert np.all(np.abs(counts - S * p) <= 1.0 + 1e-3), (counts, S * p)
    # the check has the power to tell the reference's constants from plausible mistakes
    if do_train and qa != qb:
        for wrong in (_p_first_half(qa, qb, gamma=1.0), _p_first_half(qa, qb, uniform=0.5),
                      _p_first_half(qa, qb, uniform=0.7)):
            if abs(S * wrong - S * p) > 2.5:
                assert np.any(np.abs(counts - S * wrong) > 1.0 + 1e-3)


def test_sampler_weights_have_power():
    """At least the (16, 1) ray separates gamma 1.3 from 1.0 and the 0.3/0.7 mixture from 0.5/0.5."""
    p = _p_first_half(16, 1)
    assert abs(64 * p - 64 * _p_first_half(16, 1, gamma=1.0)) > 2.0
    assert abs(64 * p - 64 * _p_first_half(16, 1, uniform=0.5)) > 2.0


def test_marched_runs_are_the_samplers_runs(ora):
    """ora_occ_propose_marched_ray finds the runs of one (cell, subcell) in a ray's samples by itself.  Fed the
    samples of resampled rays (every sample active, so that both passes see the same samples), it must raise
    occ_st exactly as ora_occ_propose_ray does with the resampler's own run flags (the key of the reference's
    sampler), for transmittances that fall along the ray and low occupancy levels (many proposals)."""
    from common import look_at_rays
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    rng = np.random.default_rng(17)
    S = 64
    occ_in = (rng.integers(0, 3, (G ** 3, 8)).astype(np.uint32) << (4 * np.arange(8, dtype=np.uint32))).sum(
        axis=1).astype(np.uint32)
    rays = look_at_rays(300, spec, seed=18, miss_frac=0.0)
    compared = raised = multi = 0
    for r, ray in enumerate(rays):
        seed = 0xC0FFEE + 31 * r
        Ts, DTs, flags = ora.sample_ray(cfg, ray, r, S, seed, occ_in, True)
        if not (DTs > 0).all():
            continue
        Tr = np.cumprod(np.concatenate([[1.0], rng.uniform(0.6, 1.0, S - 1)])).astype(np.float32)
        T_final = np.float32(Tr[-1] * rng.uniform(0.5, 1.0))
        a, b = occ_in.copy(), occ_in.copy()
        _propose(ora, cfg, ray, S, seed, Ts, DTs, Tr, T_final, flags, occ_in, a)  # as ray 0
        ora.lib().ora_occ_propose_marched_ray(C.byref(cfg), ora.fptr(np.ascontiguousarray(ray, np.float32)), 0, S,
                                              seed, ora.fptr(Ts), ora.fptr(Tr), C.c_float(T_final),
                                              ora.uptr(occ_in), ora.uptr(b))
        assert np.array_equal(a, b), r
        compared += 1
        raised += int((a != occ_in).sum())
        multi += int(len(_runs(flags, S)) < S)
    assert compared > 100 and raised > 200 and multi > 50, (compared, raised, multi)
