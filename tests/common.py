"""Shared fixtures for the tests: model specs at the BASELINE shapes, seeded
rays through the scene box, random parameters and occupancy grids."""
from __future__ import annotations

import numpy as np

M, D_OUT, C_IN, C_OUT = 64, 16, 32, 3
LAYERS = ["Wd_in", "Wd_01", "Wd_12", "Wd_out", "Wc_in", "Wc_01", "Wc_12", "Wc_23", "Wc_out"]
BIASES = ["bd_0", "bd_1", "bd_2", "bd_out", "bc_0", "bc_1", "bc_2", "bc_3", "bc_out"]


def resolutions(L, base=16.0, finest=None, growth=None):
    out = []
    for l in range(L):
        r = base * growth ** l if growth is not None else base * (finest / base) ** (0.0 if L == 1 else l / (L - 1))
        out.append(max(2, int(np.rint(r))))
    return out


def spec_cfg0(**kw):
    """BASELINE configs[0] shapes: L=8, F=2, T=2^14, base 16 growth 1.5, ND=1, NC=2, 64^3 occupancy."""
    s = dict(n_levels=8, f_per_level=2, log2_T=[14] * 8, res=resolutions(8, 16.0, growth=1.5), nd=1, nc=2,
             occ_G=32, box_min=[0.0, 0.0, 0.0], box_max=[1.0, 1.0, 1.0], rho_min=1.0, rho_max=16.0,
             dt_min=1.0 / 8192, dt_max=12.8 / 64 / 6, t_near=0.3, t_far=1e9, background=0, hash_opt=1)
    s.update(kw)
    return s


def spec_cfg1(**kw):
    """BASELINE configs[1] shapes: L=16, F=2, T=2^19, 16 -> 2048, 128^3 occupancy (G=64)."""
    s = spec_cfg0(n_levels=16, log2_T=[19] * 16, res=resolutions(16, 16.0, finest=2048.0), occ_G=64)
    s.update(kw)
    return s


def spec_ref(**kw):
    """The reference's compiled-in shape: L=16, F=4, per-level T, 16 -> 1024, ND=NC=2, box [-3,3]."""
    s = dict(n_levels=16, f_per_level=4, log2_T=[13, 13, 13, 13, 15, 15, 15, 15, 17, 17, 17, 17, 18, 18, 19, 19],
             res=resolutions(16, 16.0, finest=1024.0), nd=2, nc=2, occ_G=32, box_min=[-3.0] * 3, box_max=[3.0] * 3,
             rho_min=1.0, rho_max=16.0, dt_min=6.0 / 8192, dt_max=12.8 / 64 / 6 * 6.0, t_near=0.3, t_far=1e9,
             background=0, hash_opt=0)
    s.update(kw)
    return s


def table_floats(spec):
    return int(sum(1 << int(t) for t in spec["log2_T"])) * int(spec["f_per_level"])


def layer_shapes(spec):
    LF = spec["n_levels"] * spec["f_per_level"]
    shp = {"Wd_in": (M, LF), "Wd_out": (D_OUT, M), "Wc_in": (M, C_IN), "Wc_out": (C_OUT, M)}
    if spec["nd"] >= 2:
        shp["Wd_01"] = (M, M)
    if spec["nd"] >= 3:
        shp["Wd_12"] = (M, M)
    if spec["nc"] >= 2:
        shp["Wc_01"] = (M, M)
    if spec["nc"] >= 3:
        shp["Wc_12"] = (M, M)
    if spec["nc"] >= 4:
        shp["Wc_23"] = (M, M)
    return shp


def random_params(spec, seed=0, table_scale=0.5, occ_mode="random"):
    """Parameters with enough signal that every code path is exercised
    (table values ~U(+-table_scale), He-normal weights, random occupancy)."""
    rng = np.random.default_rng(seed)
    p = {"table": rng.uniform(-table_scale, table_scale, table_floats(spec)).astype(np.float32)}
    for wn, sh in layer_shapes(spec).items():
        p[wn] = (rng.normal(0, 1, sh) * np.sqrt(2.0 / sh[1])).astype(np.float32)
        bn = BIASES[LAYERS.index(wn)]
        p[bn] = rng.normal(0, 0.1, sh[0]).astype(np.float32)
        for pre in ("m", "v"):
            p[pre + wn] = np.zeros(sh, np.float32)
            p[pre + bn] = np.zeros(sh[0], np.float32)
    p["bd_out"][0] = 1.0
    p["m_table"] = np.zeros_like(p["table"])
    p["v_table"] = np.zeros_like(p["table"])
    n = spec["occ_G"] ** 3
    if occ_mode == "random":
        p["occ_in"] = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    else:
        p["occ_in"] = np.full(n, 0xEEEEEEEE, np.uint32)
    p["occ_st"] = p["occ_in"].copy()
    return p


def look_at_rays(n, spec, seed=0, radius=1.5, miss_frac=0.1):
    """Rays from cameras on a sphere around the box centre aimed near the centre;
    a fraction aimed away so that they miss the box."""
    rng = np.random.default_rng(seed)
    bmin, bmax = np.array(spec["box_min"], np.float64), np.array(spec["box_max"], np.float64)
    c = 0.5 * (bmin + bmax)
    ext = float(np.max(bmax - bmin))
    v = rng.normal(size=(n, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    o = c + v * radius * ext
    tgt = c + rng.uniform(-0.3, 0.3, (n, 3)) * ext
    d = tgt - o
    k = int(n * miss_frac)
    d[:k] = -d[:k]
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    rays = np.zeros((n, 8), np.float32)
    rays[:, :3] = o
    rays[:, 3] = 1.0
    rays[:, 4:7] = d
    return rays


def sphere_targets(rays, spec):
    """Targets of the BASELINE analytic scene (sigma=50 ball r=0.25 at the box centre, colour = position)
    -- closed-form chord integral on black.  Works for the unit box."""
    o, d = rays[:, :3].astype(np.float64), rays[:, 4:7].astype(np.float64)
    c = 0.5 * (np.array(spec["box_min"]) + np.array(spec["box_max"]))
    r, sig = 0.25, 50.0
    oc = o - c
    b = np.sum(oc * d, 1)
    cc = np.sum(oc * oc, 1) - r * r
    disc = b * b - cc
    out = np.zeros((rays.shape[0], 4), np.float32)
    hit = disc > 0
    sq = np.sqrt(np.where(hit, disc, 0))
    ta, tb = -b - sq, -b + sq
    ta = np.maximum(ta, 0.0)
    ell = np.maximum(tb - ta, 0.0)
    xa = o + ta[:, None] * d
    e = np.exp(-sig * ell)
    C = xa * (1 - e)[:, None] + d * ((1 - e * (1 + sig * ell)) / sig)[:, None]
    out[:, :3] = np.where(hit[:, None], C, 0.0)
    return out


def default_scalars(**kw):
    s = dict(lr=1e-2, lr_t=1e-2 * np.sqrt(1 - 0.99) / (1 - 0.9), color_rel_lr=1.0, sh_multiplier=1.0,
             occ_strength=1.0, beta1=0.9, beta2=0.99, eps=1e-15, rng_seed=12345, do_train=1)
    s.update(kw)
    return s


def cfg4_shell_bitfield(R, seed=4, radius=0.3, thickness=0.02, noise=0.007):
    """BASELINE configs[4]'s occupancy field: the cells whose centre lies within thickness/2 of a sphere of the
    given radius about the box centre, plus seeded isolated cells (a `noise` fraction), about 3 % set at
    R = 256.  R^3 bits, x fastest, 32 per word.  Returns (bits, fraction set)."""
    rng = np.random.default_rng(seed)
    c = (np.arange(R, dtype=np.float32) + 0.5) / R
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    yy, xx = np.meshgrid(c, c, indexing="ij")
    n_set = 0
    for z in range(R):  # slab by slab to bound host memory
        rad = np.sqrt((xx - 0.5) ** 2 + (yy - 0.5) ** 2 + (c[z] - 0.5) ** 2)
        occ = (np.abs(rad - radius) <= 0.5 * thickness) | (rng.random((R, R)) < noise)
        idx = np.nonzero(occ.reshape(-1))[0].astype(np.int64) + z * R * R
        n_set += idx.size
        np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits, n_set / R ** 3


def cfg3_points(n, dist, seed=1):
    """BASELINE configs[3]'s query points in the unit box: (a) "uniform", or (b) "shell": 90 % on a spherical
    shell of radius 0.25 +- 0.01 about the centre, 10 % uniform, shuffled."""
    rng = np.random.default_rng(seed)
    if dist == "uniform":
        return rng.random((n, 3), dtype=np.float32)
    k = n // 10
    v = rng.normal(size=(n - k, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    r = rng.uniform(0.24, 0.26, (n - k, 1))
    x = np.concatenate([0.5 + v * r, rng.random((k, 3))]).astype(np.float32)
    return x[rng.permutation(n)]
