"""Pins of the oracle's importance resampler (ffnerf_OG.cl:1002-1250): closed
forms for uniform occupancy, invariants of systematic resampling, and the
no-hit / inference special cases."""
import numpy as np
import pytest

from common import look_at_rays, random_params, spec_cfg0


def _cands(spec, ray, ray_id, S, seed):
    """Independent restatement of the stratified candidates t_k."""
    from test_oracle_primitives import lowbias32_np
    o, d = ray[:3].astype(np.float32), ray[4:7].astype(np.float32)
    lo, hi = np.array(spec["box_min"], np.float32), np.array(spec["box_max"], np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(d != 0, np.float32(1) / d, np.float32(np.inf)).astype(np.float32)
        tb, tt = (lo - o) * inv, (hi - o) * inv
    t0 = np.float32(max(np.nanmax(np.fmin(tb, tt)), np.float32(spec["t_near"])))
    t1 = np.float32(min(np.nanmin(np.fmax(tb, tt)), np.float32(spec["t_far"])))
    if not t1 > t0:
        return None
    t0 = np.float32(t0 + np.float32(1e-6))
    lid = np.arange(S, dtype=np.uint64)
    st = lowbias32_np(np.uint64(seed) ^ np.uint64((ray_id * 747796405) & 0xFFFFFFFF) ^ ((lid * 2891336453) & 0xFFFFFFFF))
    st = st.astype(np.uint64)
    st ^= (st << 13) & 0xFFFFFFFF
    st ^= st >> 17
    st ^= (st << 5) & 0xFFFFFFFF
    r = ((st & 0xFFFFFF).astype(np.float32) * np.float32(1 / 16777216)).astype(np.float32)
    u = ((lid.astype(np.float32) + r) * np.float32(1.0 / S)).astype(np.float32)
    return (t0 + (np.float32(t1) - t0) * u).astype(np.float32), t0, np.float32(t1)


@pytest.mark.parametrize("S", [64, 32, 16, 8, 1])
def test_sampler_invariants(ora, S):
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    p = random_params(spec, seed=1)
    rays = look_at_rays(200, spec, seed=2, miss_frac=0.2)
    seed = 0xC0FFEE
    for r in range(rays.shape[0]):
        Ts, DTs, flags = ora.sample_ray(cfg, rays[r], r, S, seed, p["occ_in"], True)
        c = _cands(spec, rays[r], r, S, seed)
        bits = [(int(flags[i >> 5]) >> (i & 31)) & 1 for i in range(S)]
        if c is None:
            assert np.all(Ts == 0) and np.all(DTs == 0) and all(bits)
            continue
        cand, t0, t1 = c
        assert np.all(np.diff(Ts) >= 0)                       # systematic resampling keeps order
        assert np.isin(Ts, cand).all()                        # every sample is a candidate
        dtb = np.float32(np.clip(np.float32((t1 - t0) * np.float32(1.0 / S)), spec["dt_min"], spec["dt_max"]))
        assert np.all(DTs == dtb)
        assert bits[0] == 1
        for i in range(1, S):                                 # a repeated sample never starts a run
            if Ts[i] == Ts[i - 1]:
                assert bits[i] == 0


def test_uniform_occupancy_keeps_the_strata(ora):
    """All nibbles equal: p_i = 1/S exactly, the CDF is (i+1)/S and systematic
    resampling returns candidate i for sample i (u0 > 0)."""
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    occ = np.full(spec["occ_G"] ** 3, 0x77777777, np.uint32)
    rays = look_at_rays(100, spec, seed=3, miss_frac=0.0)
    for S in (64, 16):
        for r in range(rays.shape[0]):
            Ts, _, _ = ora.sample_ray(cfg, rays[r], r, S, 99, occ, True)
            cand, _, _ = _cands(spec, rays[r], r, S, 99)
            assert np.array_equal(Ts, cand)


def test_inference_with_empty_grid_piles_on_the_last_stratum(ora):
    """do_train=0 and every nibble <= 2: nothing is active, p = 0.3/S, so every
    u_k above 0.3 maps past the CDF end to the last candidate (reference quirk)."""
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    occ = np.full(spec["occ_G"] ** 3, 0x22222222, np.uint32)
    rays = look_at_rays(20, spec, seed=4, miss_frac=0.0)
    S = 64
    for r in range(rays.shape[0]):
        Ts, _, _ = ora.sample_ray(cfg, rays[r], r, S, 7, occ, False)
        cand, _, _ = _cands(spec, rays[r], r, S, 7)
        assert np.sum(Ts == cand[-1]) >= int(0.69 * S)


def test_importance_concentrates_samples_in_occupied_cells(ora):
    spec = spec_cfg0()
    G = spec["occ_G"]
    cfg = ora.make_cfg(spec)
    occ = np.zeros(G ** 3, np.uint32)  # q = 1 everywhere
    idx = np.arange(G ** 3)
    ix, iy, iz = idx % G, (idx // G) % G, idx // (G * G)
    ball = ((ix - G / 2 + 0.5) ** 2 + (iy - G / 2 + 0.5) ** 2 + (iz - G / 2 + 0.5) ** 2) < (0.25 * G) ** 2
    occ[ball] = 0xFFFFFFFF  # q = 16 inside the ball
    rays = look_at_rays(200, spec, seed=5, miss_frac=0.0)
    flat = np.zeros_like(occ)

    def frac_inside(grid):
        inside = 0
        for r in range(rays.shape[0]):
            Ts, _, _ = ora.sample_ray(cfg, rays[r], r, 64, 11, grid, True)
            x = rays[r, :3] + Ts[:, None] * rays[r, 4:7]
            inside += int(np.sum(np.linalg.norm(x - 0.5, axis=1) < 0.25))
        return inside / (64 * rays.shape[0])

    # rho = rho_min + (rho_max - rho_min) q/16: 16x the weight inside the ball
    assert frac_inside(occ) > 2.0 * frac_inside(flat)
