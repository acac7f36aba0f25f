"""GPU parity of the occupancy bitfield, the DDA marcher with compaction and
the early-terminated render, through the C ABI, against the oracle."""
import numpy as np
import pytest

from common import look_at_rays, random_params, spec_cfg0
from oracle import oracle as ora

pytestmark = pytest.mark.gpu

SPEC = spec_cfg0(occ_G=16)


@pytest.fixture(scope="module")
def gm():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    from gpu_helpers import GpuModel
    p = random_params(SPEC, seed=1)
    return GpuModel(SPEC, p), p


def shell_bits(R, seed=0, frac=0.02, half_width=0.06):
    rng = np.random.default_rng(seed)
    c = (np.arange(R) + 0.5) / R
    z, y, x = np.meshgrid(c, c, c, indexing="ij")
    rad = np.sqrt((x - 0.5) ** 2 + (y - 0.5) ** 2 + (z - 0.5) ** 2)
    occ = (np.abs(rad - 0.3) <= half_width) | (rng.random((R, R, R)) < frac)
    idx = np.nonzero(occ.reshape(-1))[0]
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits


def test_bitfield_bit_exact(gm):
    g, _ = gm
    rng = np.random.default_rng(4)
    for G in (8, 16, 20):
        occ = rng.integers(0, 2 ** 32, G ** 3, dtype=np.uint64).astype(np.uint32)
        for q_min in (1, 4, 12, 17):
            print(f"[bitfield] G={G} q_min={q_min}", flush=True)
            np.testing.assert_array_equal(g.bitfield(occ, G, q_min), ora.occ_bitfield(occ, G, q_min))


def special_rays(R):
    """Rays the walk finds hard: axis-aligned (two direction components zero), along face diagonals and the
    space diagonal from origins on cell corners (boundary crossings at equal times on two or three axes), and
    from inside the box (the walk starts in the cell of t_near)."""
    rays = []
    dirs = [(1, 0, 0), (0, -1, 0), (0, 0, 1), (1, 1, 0), (0, -1, 1), (1, 1, 1), (-1, 1, -1), (1, 2, 0), (3, 1, 2)]
    rng = np.random.default_rng(R)
    for d in dirs:
        d = np.array(d, np.float64)
        d /= np.linalg.norm(d)
        for _ in range(12):
            corner = rng.integers(0, R + 1, 3) / R  # a cell corner inside or on the box
            for o in (corner - 2.0 * d, corner - 0.5 * d, corner):
                r = np.zeros(8, np.float32)
                r[:3] = o
                r[3] = 1.0
                r[4:7] = d
                rays.append(r)
    return np.array(rays, np.float32)


# (R, max_steps, random-cell fraction, shell half width): the sparse fields leave most 8^3 blocks empty, so
# the walk crosses them in one step; R = 44 has partial blocks at the grid's far faces
@pytest.mark.parametrize("R,max_steps,frac,hw", [(32, 4096, 0.02, 0.06), (32, 7, 0.02, 0.06), (64, 300, 0.02, 0.06),
                                                 (64, 4096, 0.0, 0.03), (44, 4096, 0.0003, 0.02),
                                                 (128, 9, 0.0, 0.02)])
def test_march_bit_exact(gm, R, max_steps, frac, hw):
    import ffn_lib as fl
    g, _ = gm
    bits = shell_bits(R, seed=R, frac=frac, half_width=hw)
    dt = np.float32(np.sqrt(3.0) / 256)
    rays = np.concatenate([look_at_rays(1500, SPEC, seed=R + max_steps), special_rays(R)])
    print(f"[march] R={R} max_steps={max_steps} frac={frac} hw={hw}", flush=True)
    counts, offsets, samples, ids, total = g.march(rays, bits, fl.march_params(R, dt, max_steps))
    cfg = ora.make_cfg(SPEC)
    m = ora.march_cfg(R, dt, max_steps)
    ref = [ora.march_ray(cfg, m, bits, r) for r in rays]
    np.testing.assert_array_equal(counts, [len(t) for t in ref])
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.uint32))
    assert total == int(counts.sum()) and total > 200
    for r, t in enumerate(ref):
        sl = slice(int(offsets[r]), int(offsets[r]) + len(t))
        np.testing.assert_array_equal(samples[sl, 3], t)
        o, d = rays[r, :3], rays[r, 4:7]
        np.testing.assert_array_equal(samples[sl, :3], (o[None, :] + t[:, None] * d[None, :]).astype(np.float32))
        assert np.all(ids[sl] == r)


def test_march_capacity_bound(gm):
    import ffn_lib as fl
    g, _ = gm
    R = 32
    bits = shell_bits(R, seed=3)
    rays = look_at_rays(500, SPEC, seed=21)
    dt = np.float32(np.sqrt(3.0) / 256)
    mp = fl.march_params(R, dt, 4096)
    c_full, o_full, s_full, _, total = g.march(rays, bits, mp)
    cap = total // 3
    c, o, s, ids, total2 = g.march(rays, bits, mp, capacity=cap)
    assert total2 == total
    np.testing.assert_array_equal(s[:cap], s_full[:cap])


def test_render_matches_oracle():
    import ffn_lib as fl
    from gpu_helpers import GpuModel
    p = random_params(SPEC, seed=2)
    p["bd_out"][0] = 6.0  # dense enough that rays terminate inside the marched samples
    g = GpuModel(SPEC, p)
    R = 32
    bits = shell_bits(R, seed=8, frac=0.05)
    rays = look_at_rays(400, SPEC, seed=31, miss_frac=0.05)
    dt = np.float32(np.sqrt(3.0) / 128)
    model = ora.OracleModel(SPEC, p)
    for T_stop in (1e-4, 0.3):
        print(f"[render] T_stop={T_stop}", flush=True)
        ref, used_ref = model.render(rays, bits, ora.march_cfg(R, dt, 512, T_stop=T_stop))
        out, used = g.render(rays, bits, fl.march_params(R, dt, 512, T_stop=T_stop, chunk=16))
        out2, used2 = g.render(rays, bits, fl.march_params(R, dt, 512, T_stop=T_stop, chunk=512))
        # chunking does not change anything: every sample is shaded and composited in the same order
        np.testing.assert_array_equal(out, out2)
        np.testing.assert_array_equal(used, used2)
        # the termination index can move by one where T crosses T_stop within rounding
        assert np.mean(used == used_ref) > 0.99
        same = used == used_ref
        np.testing.assert_allclose(out[same], ref[same], rtol=1e-3, atol=2e-5)
        assert used_ref.sum() > 2000
        if T_stop > 0.1:
            assert np.any(used_ref < [len(ora.march_ray(model.cfg, ora.march_cfg(R, dt, 512), bits, r))
                                      for r in rays])


def test_render_one_walk_equals_two_walks(monkeypatch):
    """Each render round walks its rays once into per-ray chunks of slots when num_rays * chunk samples fit
    FFN_MARCH_SLOT_BUDGET_MB, else counts then emits: the same image and samples used, bit for bit."""
    import ffn_lib as fl
    from gpu_helpers import GpuModel
    p = random_params(SPEC, seed=5)
    p["bd_out"][0] = 6.0
    R = 32
    bits = shell_bits(R, seed=9, frac=0.05)
    rays = look_at_rays(700, SPEC, seed=33, miss_frac=0.05)
    dt = np.float32(np.sqrt(3.0) / 128)
    for chunk in (16, 512):
        print(f"[render one/two walks] chunk={chunk}", flush=True)
        res = []
        for budget in ("8192", "0"):
            monkeypatch.setenv("FFN_MARCH_SLOT_BUDGET_MB", budget)
            res.append(GpuModel(SPEC, p).render(rays, bits, fl.march_params(R, dt, 512, T_stop=1e-2, chunk=chunk)))
        np.testing.assert_array_equal(res[0][0], res[1][0])
        np.testing.assert_array_equal(res[0][1], res[1][1])
        assert res[0][1].sum() > 2000


def test_march_block_skip_changes_no_sample(gm, monkeypatch):
    """The walk crosses empty 8^3 blocks in one step (a block summary of the bitfield, used when at least half
    the blocks are empty): the counts, samples and ray ids are bit-identical with the summary off
    (FFN_MARCH_BLOCKS=0) on a 256^3 field (a thin shell and sparse random cells, most blocks empty) with ordinary
    and tie-prone rays, and against the oracle; the render's image and samples used as well."""
    import ffn_lib as fl
    g, _ = gm
    R = 256
    bits = shell_bits(R, seed=41, frac=0.0003, half_width=0.01)
    # most 8^3 blocks are empty, so the walk takes the block summary (it does when at least half are)
    idx = np.arange(R ** 3, dtype=np.int64)
    occ = ((bits[idx >> 5] >> (idx & 31).astype(np.uint32)) & 1).astype(bool).reshape(R // 8, 8, R // 8, 8, R // 8, 8)
    assert occ.any(axis=(1, 3, 5)).mean() < 0.3
    dt = np.float32(np.sqrt(3.0) / 1024)
    rays = np.concatenate([look_at_rays(3000, SPEC, seed=42), special_rays(R)])
    mp = fl.march_params(R, dt, 1024)
    print(f"[march blocks on/off] R={R} rays={len(rays)}", flush=True)
    res = []
    for env in ("1", "0"):
        monkeypatch.setenv("FFN_MARCH_BLOCKS", env)
        res.append(g.march(rays, bits, mp))
    for a, b in zip(res[0], res[1]):
        np.testing.assert_array_equal(a, b)
    counts, offsets, samples = res[0][0], res[0][1], res[0][2]
    assert res[0][4] > 10000
    cfg = ora.make_cfg(SPEC)
    m = ora.march_cfg(R, dt, 1024)
    for r in range(0, len(rays), 7):
        t = ora.march_ray(cfg, m, bits, rays[r])
        assert counts[r] == len(t)
        np.testing.assert_array_equal(samples[int(offsets[r]):int(offsets[r]) + len(t), 3], t)
    # the render's rounds resume each ray from its saved walk state: the same image and samples used
    out = []
    for env in ("1", "0"):
        monkeypatch.setenv("FFN_MARCH_BLOCKS", env)
        out.append(g.render(rays, bits, fl.march_params(R, dt, 1024, T_stop=1e-2, chunk=16)))
    np.testing.assert_array_equal(out[0][0], out[1][0])
    np.testing.assert_array_equal(out[0][1], out[1][1])
