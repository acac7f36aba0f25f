"""Pins of the oracle's occupancy bitfield, DDA marcher and early-terminated
render (the specification of the HIP marcher; the reference has no marcher).

The marcher is checked against an independent point-test brute force (every
lattice point classified by the cell that contains it), against closed forms
(full grid: every lattice point in [t0, t1); empty grid: nothing), and for
truncation and ordering invariants.  The render is checked against the
closed form of a constant field."""
import ctypes as C

import numpy as np
import pytest

from common import look_at_rays, random_params, spec_cfg0
from oracle import oracle as ora


def np_bitfield(occ, G, q_min):
    """Independent numpy restatement of the bitfield definition."""
    R = 2 * G
    z, y, x = np.meshgrid(np.arange(R), np.arange(R), np.arange(R), indexing="ij")
    word = occ[(x >> 1) + G * ((y >> 1) + G * (z >> 1))]
    sub = (x & 1) | ((y & 1) << 1) | ((z & 1) << 2)
    q = ((word >> (4 * sub).astype(np.uint32)) & 0xF) + 1
    flat = (q >= q_min).reshape(-1)
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    idx = np.nonzero(flat)[0]
    np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits


def point_test_samples(ray, bits, R, bmin, bmax, t_near, dt, max_steps):
    """Lattice points whose point o + t d lies in an occupied cell (floor and clamp), in float32."""
    f = np.float32
    o, d = ray[:3].astype(f), ray[4:7].astype(f)
    t0t1 = aabb(o, d, bmin, bmax)
    if t0t1 is None:
        return np.zeros(0, f)
    t0, t1 = max(t0t1[0], f(t_near)), t0t1[1]
    if not t1 > t0:
        return np.zeros(0, f)
    inv = (f(R) / (bmax - bmin)).astype(f)
    out, k = [], 0
    while True:
        tk = f(t0 + f(f(k) + f(0.5)) * f(dt))
        if not tk < t1:
            break
        p = (o + tk * d).astype(f)
        c = np.clip(np.floor(((p - bmin) * inv).astype(f)).astype(np.int64), 0, R - 1)
        i = c[0] + R * (c[1] + R * c[2])
        if (bits[i >> 5] >> np.uint32(i & 31)) & 1:
            out.append(tk)
        k += 1
    return np.array(out[:max_steps], f)


def aabb(o, d, bmin, bmax):
    f = np.float32
    with np.errstate(divide="ignore", invalid="ignore"):
        invd = np.where(d != 0, f(1) / d, f(np.inf)).astype(f)
        tb = ((bmin - o) * invd).astype(f)
        tt = ((bmax - o) * invd).astype(f)
    tmin = np.max(np.minimum(tb, tt))
    tmax = np.min(np.maximum(tb, tt))
    if tmax < tmin:
        return None
    return f(tmin), f(tmax)


def lattice(t0, t1, dt):
    f = np.float32
    out, k = [], 0
    while True:
        tk = f(f(t0) + f(f(k) + f(0.5)) * f(dt))
        if not tk < t1:
            return np.array(out, f)
        out.append(tk)
        k += 1


SPEC = spec_cfg0(occ_G=16)
BMIN, BMAX = np.zeros(3, np.float32), np.ones(3, np.float32)


def test_bitfield_matches_numpy_definition():
    rng = np.random.default_rng(3)
    G = 8
    occ = rng.integers(0, 2 ** 32, G ** 3, dtype=np.uint64).astype(np.uint32)
    for q_min in (1, 3, 9, 16, 17):
        np.testing.assert_array_equal(ora.occ_bitfield(occ, G, q_min), np_bitfield(occ, G, q_min))
    assert ora.occ_bitfield(occ, G, 1).tolist() == [0xFFFFFFFF] * (16 ** 3 // 32)
    assert not ora.occ_bitfield(occ, G, 17).any()


def _shell_bits(R, r0=0.3, half=0.06, seed=0):
    rng = np.random.default_rng(seed)
    c = (np.arange(R) + 0.5) / R
    z, y, x = np.meshgrid(c, c, c, indexing="ij")
    rad = np.sqrt((x - 0.5) ** 2 + (y - 0.5) ** 2 + (z - 0.5) ** 2)
    occ = (np.abs(rad - r0) <= half) | (rng.random((R, R, R)) < 0.02)
    flat = occ.reshape(-1)
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    idx = np.nonzero(flat)[0]
    np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits


def test_march_agrees_with_point_test_brute_force():
    R, dt, max_steps = 32, np.float32(np.sqrt(3.0) / 200), 4096
    bits = _shell_bits(R)
    cfg = ora.make_cfg(SPEC)
    m = ora.march_cfg(R, dt, max_steps)
    rays = look_at_rays(300, SPEC, seed=5)
    total, differ = 0, 0
    for r in rays:
        t = ora.march_ray(cfg, m, bits, r)
        ref = point_test_samples(r, bits, R, BMIN, BMAX, SPEC["t_near"], dt, max_steps)
        total += max(len(ref), 1)
        differ += len(set(t.tolist()) ^ set(ref.tolist()))
        assert np.all(np.diff(t) > 0)
    assert total > 3000
    # the two definitions differ only for lattice points on a cell face (rounding of the point test)
    assert differ <= 0.002 * total, (differ, total)


def test_march_full_and_empty_grids_closed_form():
    R, dt = 32, np.float32(0.0123)
    full = np.full((R ** 3) // 32, 0xFFFFFFFF, np.uint32)
    empty = np.zeros_like(full)
    cfg = ora.make_cfg(SPEC)
    m = ora.march_cfg(R, dt, 100000)
    for r in look_at_rays(200, SPEC, seed=7):
        o, d = r[:3], r[4:7]
        tt = aabb(o, d, BMIN, BMAX)
        t = ora.march_ray(cfg, m, full, r)
        if tt is None or not min(tt[1], np.float32(SPEC["t_far"])) > max(tt[0], np.float32(SPEC["t_near"])):
            assert len(t) == 0
            continue
        t0, t1 = max(tt[0], np.float32(SPEC["t_near"])), tt[1]
        np.testing.assert_array_equal(t, lattice(t0, t1, dt))
        assert len(ora.march_ray(cfg, m, empty, r)) == 0


def test_march_truncation_is_a_prefix():
    R, dt = 32, np.float32(np.sqrt(3.0) / 300)
    bits = _shell_bits(R, seed=2)
    cfg = ora.make_cfg(SPEC)
    for r in look_at_rays(100, SPEC, seed=9):
        full = ora.march_ray(cfg, ora.march_cfg(R, dt, 100000), bits, r)
        for ms in (1, 5, 17):
            part = ora.march_ray(cfg, ora.march_cfg(R, dt, ms), bits, r)
            np.testing.assert_array_equal(part, full[:ms])


def _const_field_params(spec, b0, cbias):
    p = random_params(spec, seed=0)
    for k in list(p):
        if k.startswith(("W", "b", "m", "v")) and not k.startswith(("m_", "v_")):
            p[k][...] = 0.0
    p["bd_out"][0] = b0
    p["bc_out"][:] = cbias
    return p


def test_render_constant_field_closed_form():
    spec = SPEC
    b0, cb = 1.3, np.array([0.4, -0.7, 1.9], np.float32)
    p = _const_field_params(spec, b0, cb)
    model = ora.OracleModel(spec, p)
    # sigma and rgb of the constant field through the oracle's own MLP (any encoding gives the same)
    sig, rgb = C.c_float(), np.zeros(3, np.float32)
    a0 = np.zeros(spec["n_levels"] * spec["f_per_level"], np.float32)
    d = np.array([0.0, 0.0, 1.0], np.float32)
    ora.lib().ora_mlp_forward(C.byref(model.cfg), C.byref(model._params()), ora.fptr(a0), ora.fptr(d), 1.0,
                              C.byref(sig), ora.fptr(rgb), None)
    sigma = np.float32(sig.value)
    assert abs(sigma - np.log1p(np.exp(1.3))) < 1e-5
    R = 32
    full = np.full((R ** 3) // 32, 0xFFFFFFFF, np.uint32)
    dt = np.float32(0.01)
    for T_stop in (0.0, 0.2):
        m = ora.march_cfg(R, dt, 100000, T_stop=T_stop)
        rays = look_at_rays(40, spec, seed=11, miss_frac=0.0)
        out, used = model.render(rays, full, m)
        alpha = np.float32(1) - np.exp(np.float32(max(min(-sigma * dt, 18.0), -5.0)))
        for r, ray in enumerate(rays):
            n_lat = len(ora.march_ray(model.cfg, m, full, ray))
            n = n_lat
            if T_stop > 0:
                # first j (1-based) with (1 - alpha)^j < T_stop
                n = min(n_lat, int(np.floor(np.log(T_stop) / np.log1p(-float(alpha)))) + 1)
            assert used[r] == n
            Tn = (1.0 - float(alpha)) ** n
            np.testing.assert_allclose(out[r, 3], Tn, rtol=1e-5)
            np.testing.assert_allclose(out[r, :3], rgb * (1.0 - Tn), rtol=1e-5, atol=1e-7)


def test_marched_compositing_matches_autograd(ora):
    """ora_composite_marched (the marched training step's compositing, loss gradient and backward) against
    float64 autograd of the same function: alpha = 1 - exp(-sigma dt), front-to-back weights, the
    Charbonnier loss sqrt(r^2 + 1e-6) at the composited colour plus background, stopping after the sample
    that leaves T < T_stop; dL/dsigma adds the density penalty regu on every composited sample, and the
    samples after the stop get no gradient."""
    import torch
    rng = np.random.default_rng(9)
    for case in range(40):
        n = int(rng.integers(1, 90))
        dt = np.float32(rng.uniform(0.005, 0.03))
        sig = rng.uniform(0.0, 4.5 / dt, n).astype(np.float32) * (rng.random(n) < 0.5)  # sigma dt < 5: no clamp
        rgb = rng.uniform(0.05, 0.95, (n, 3)).astype(np.float32)
        bg = rng.uniform(0, 1, 3).astype(np.float32) * (case % 2)
        tg = rng.uniform(0, 1, 3).astype(np.float32)
        T_stop = np.float32([0.0, 1e-4, 1e-2][case % 3])
        regu = np.float32(5e-3) * dt / np.float32(128)
        used, Tr, dLds, dLdc, Cf, T_end = ora.composite_marched(sig, rgb, dt, T_stop, bg, tg, regu)
        s = torch.tensor(sig.astype(np.float64), requires_grad=True)
        c = torch.tensor(rgb.astype(np.float64), requires_grad=True)
        alpha = 1.0 - torch.exp(-s * float(dt))
        T = torch.cumprod(torch.cat([torch.ones(1, dtype=torch.float64), 1.0 - alpha]), 0)
        stop = n
        Td = T.detach().numpy()
        for j in range(n):  # the same rule in float64
            if Td[j + 1] < float(T_stop):
                stop = j + 1
                break
        if abs(Td[stop] - float(T_stop)) < 1e-5 and stop < n:
            continue  # within rounding of the threshold: either stop is right
        assert used == stop, (case, used, stop)
        C = (T[:stop, None] * alpha[:stop, None] * c[:stop]).sum(0) + T[stop] * torch.tensor(bg, dtype=torch.float64)
        loss = torch.sqrt((C - torch.tensor(tg, dtype=torch.float64)) ** 2 + 1e-6).sum()
        loss.backward()
        g_s = s.grad.numpy().copy()
        g_s[:stop] += float(regu)
        g_c = c.grad.numpy()
        scale = max(np.abs(g_s).max(), 1e-12)
        assert np.abs(dLds - g_s).max() <= 2e-4 * scale + 1e-9, (case, np.abs(dLds - g_s).max(), scale)
        assert np.abs(dLdc - g_c).max() <= 2e-4 * max(np.abs(g_c).max(), 1e-12) + 1e-9, case
        assert np.allclose(Cf, C.detach().numpy(), rtol=1e-5, atol=1e-6)
        assert np.all(dLds[stop:] == 0) and np.all(dLdc[stop:] == 0)
