"""Pins of the oracle's hash-grid encoding (ffnerf_OG.cl:1286-1364) and its
backward (ffnerf_OG.cl:2090-2173) by properties the trilinear interpolation and
the linear structure of the encoding fix, independent of the oracle's code."""
import numpy as np

from common import spec_cfg0, spec_ref, table_floats


def _pts(n, spec, seed, margin=0.0):
    rng = np.random.default_rng(seed)
    lo, hi = np.array(spec["box_min"]), np.array(spec["box_max"])
    return (lo + (hi - lo) * rng.uniform(margin, 1 - margin, (n, 3))).astype(np.float32)


def corners_np(spec, x):
    """Independent numpy statement of the corner math: index and weight of the
    8 corners of every level (float32 arithmetic, no fused ops)."""
    x = np.asarray(x, np.float32)
    lo, hi = np.array(spec["box_min"], np.float32), np.array(spec["box_max"], np.float32)
    p = np.clip((x - lo) / (hi - lo), np.float32(0), np.float32(1) - np.float32(1e-6)).astype(np.float32)
    F = spec["f_per_level"]
    off = np.concatenate([[0], np.cumsum([1 << t for t in spec["log2_T"]])[:-1]]).astype(np.uint64)
    idx = np.zeros((x.shape[0], spec["n_levels"], 8), np.uint64)
    w = np.zeros((x.shape[0], spec["n_levels"], 8), np.float32)
    for l in range(spec["n_levels"]):
        R = spec["res"][l]
        u = (p * np.float32(R)).astype(np.float32)
        i0 = np.clip(np.floor(u).astype(np.int64), 0, R - 2)
        f = (u - i0.astype(np.float32)).astype(np.float32)
        for c in range(8):
            dx, dy, dz = c & 1, (c >> 1) & 1, (c >> 2) & 1
            wx = f[:, 0] if dx else np.float32(1) - f[:, 0]
            wy = f[:, 1] if dy else np.float32(1) - f[:, 1]
            wz = f[:, 2] if dz else np.float32(1) - f[:, 2]
            w[:, l, c] = (wx * wy).astype(np.float32) * wz
            h = (((i0[:, 0] + dx) * 73856093) ^ ((i0[:, 1] + dy) * 19349663) ^ ((i0[:, 2] + dz) * 83492791)
                 ^ (l * 2654435761)) & 0xFFFFFFFF
            h ^= h >> 16
            h = (h * 0x7FEB352D) & 0xFFFFFFFF
            h ^= h >> 15
            h = (h * 0x846CA68B) & 0xFFFFFFFF
            h ^= h >> 16
            idx[:, l, c] = (off[l] + (h & ((1 << spec["log2_T"][l]) - 1))) * F
    return idx.astype(np.uint32), w


def test_corner_indices_and_weights_bit_exact(ora):
    for spec in (spec_cfg0(), spec_ref()):
        cfg = ora.make_cfg(spec)
        x = _pts(3000, spec, 1, margin=-0.05)  # includes points outside the box (clamped)
        table = np.zeros(table_floats(spec), np.float32)
        _, idx, w = ora.hash_encode(cfg, table, x, with_idx=True)
        idx_np, w_np = corners_np(spec, x)
        assert np.array_equal(idx, idx_np)
        assert np.array_equal(w, w_np)


def test_partition_of_unity_and_top_cell_extrapolation(ora):
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    table = np.ones(table_floats(spec), np.float32)
    x = _pts(2000, spec, 2)
    x[:50] = 1.0  # the box's top corner: the last cell's weights extrapolate, f in [1, 2)
    a0, _, w = ora.hash_encode(cfg, table, x, with_idx=True)
    assert np.allclose(a0, 1.0, atol=2e-6)
    assert np.allclose(w.sum(-1), 1.0, atol=2e-6)
    assert (w[:50, :, 7] > 1.0).all()  # corner (1,1,1) weight f^3 with f > 1
    # (1-f) < 0 on every axis: w_000 = (1-f)^3 < 0 and w_100 = f (1-f)^2 > 0
    assert (w[:50, :, 0] < 0).all() and (w[:50, :, 1] > 0).all()


def test_one_hot_table_returns_summed_corner_weight(ora):
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    x = _pts(500, spec, 3)
    idx, w = corners_np(spec, x)
    F = spec["f_per_level"]
    for l in (0, 5, 7):
        target = int(idx[7, l, 3])  # an entry touched by point 7
        table = np.zeros(table_floats(spec), np.float32)
        table[target + 1] = 1.0  # feature 1 of that entry
        a0 = ora.hash_encode(cfg, table, x)
        exp = np.where(idx[:, l, :] == target, w[:, l, :], 0).sum(1)
        assert np.allclose(a0[:, l * F + 1], exp, atol=1e-7)
        assert np.allclose(a0[:, l * F + 0], 0.0)


def test_backward_is_adjoint_of_forward(ora):
    """encode is linear in the table, so <encode(T), g> = <T, backward(g)>."""
    for spec in (spec_cfg0(), spec_ref()):
        cfg = ora.make_cfg(spec)
        rng = np.random.default_rng(4)
        x = _pts(1500, spec, 5)
        LF = spec["n_levels"] * spec["f_per_level"]
        T = rng.normal(size=table_floats(spec)).astype(np.float32)
        g = rng.normal(size=(1500, LF)).astype(np.float32)
        a0 = ora.hash_encode(cfg, T, x).astype(np.float64)
        grad = ora.hash_backward(cfg, x, g, table_floats(spec))
        lhs = float((a0 * g).sum())
        rhs = float((T.astype(np.float64) * grad).sum())
        assert abs(lhs - rhs) <= 1e-4 * (abs(lhs) + 1.0)
        # and the scatter conserves mass: each level receives sum(g) (weights sum to 1)
        F = spec["f_per_level"]
        for l in range(spec["n_levels"]):
            lo = sum(1 << t for t in spec["log2_T"][:l]) * F
            hi = lo + (1 << spec["log2_T"][l]) * F
            assert abs(grad[lo:hi].sum() - g[:, l * F:(l + 1) * F].astype(np.float64).sum()) < 1e-3


def test_backward_skips_non_finite(ora):
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    x = _pts(10, spec, 6)
    g = np.ones((10, 16), np.float32)
    g[3, 5] = np.nan
    g[4, 0] = np.inf
    grad = ora.hash_backward(cfg, x, g, table_floats(spec))
    assert np.isfinite(grad).all()
