"""GPU parity of libffnerf_hip.so against the CPU oracle on the same seeded
inputs.  Bit-exact where the north star asks for it (sample times, run flags,
hash indices and encodings, occupancy words, Adam of a given gradient); fp32
tolerances elsewhere (the MLP runs as MFMA tiles, so its sums associate
differently).  The train-step comparisons and how every difference is
accounted for are described in tests/parity.py."""
import numpy as np
import pytest

from common import (default_scalars, look_at_rays, random_params, spec_cfg0, spec_cfg1, spec_ref, sphere_targets,
                    table_floats)
from parity import compare_step

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gh():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a visible GPU")
    import gpu_helpers
    return gpu_helpers


def _flag_bits(flags, S):
    return [[(int(f[i >> 5]) >> (i & 31)) & 1 for i in range(S)] for f in flags]


@pytest.mark.parametrize("S", [64, 32, 16, 8, 4, 2, 1])
@pytest.mark.parametrize("do_train", [1, 0])
def test_sampler_bit_exact(gh, ora, S, do_train):
    print(f"[case] sampler S={S} do_train={do_train}", flush=True)
    spec = spec_cfg0()
    p = random_params(spec, seed=11)
    m = gh.GpuModel(spec, p)
    rays = look_at_rays(257, spec, seed=12, miss_frac=0.2)
    seed = 0x9E3779B9
    Ts, DTs, flags = m.sample(rays, S, seed, do_train)
    cfg = ora.make_cfg(spec)
    for r in range(rays.shape[0]):
        t_o, dt_o, f_o = ora.sample_ray(cfg, rays[r], r, S, seed, p["occ_in"], do_train)
        assert np.array_equal(Ts[r], t_o), r
        assert np.array_equal(DTs[r], dt_o), r
        mask = (1 << S) - 1 if S < 64 else 0xFFFFFFFFFFFFFFFF
        g64 = (int(flags[r, 0]) | (int(flags[r, 1]) << 32)) & mask
        o64 = (int(f_o[0]) | (int(f_o[1]) << 32)) & mask
        assert g64 == o64, r


@pytest.mark.parametrize("which", ["cfg0", "cfg1", "ref"])
def test_hash_forward_bit_exact(gh, ora, which):
    print(f"[case] hash fwd {which}", flush=True)
    spec = {"cfg0": spec_cfg0, "cfg1": spec_cfg1, "ref": spec_ref}[which]()
    p = random_params(spec, seed=21)
    m = gh.GpuModel(spec, p)
    rng = np.random.default_rng(22)
    lo, hi = np.array(spec["box_min"]), np.array(spec["box_max"])
    x = (lo + (hi - lo) * rng.uniform(-0.05, 1.05, (20000, 3))).astype(np.float32)
    x[:16] = hi  # the top face: extrapolated last cell
    a0_g, idx_g = m.encode(x, with_idx=True)
    a0_o, idx_o, _ = ora.hash_encode(ora.make_cfg(spec), p["table"], x, with_idx=True)
    assert np.array_equal(idx_g, idx_o)
    assert np.array_equal(a0_g.view(np.uint32), a0_o.view(np.uint32))


@pytest.mark.parametrize("which", ["cfg0", "ref"])
def test_hash_backward_matches_oracle(gh, ora, which):
    print(f"[case] hash bwd {which}", flush=True)
    spec = {"cfg0": spec_cfg0, "ref": spec_ref}[which]()
    p = random_params(spec, seed=31)
    m = gh.GpuModel(spec, p)
    rng = np.random.default_rng(32)
    lo, hi = np.array(spec["box_min"]), np.array(spec["box_max"])
    n = 30000
    x = (lo + (hi - lo) * rng.uniform(0, 1, (n, 3))).astype(np.float32)
    LF = spec["n_levels"] * spec["f_per_level"]
    g = rng.normal(size=(n, LF)).astype(np.float32)
    g[5, 3] = np.nan  # dropped, like the reference's isfinite guard
    grad_g = m.encode_bwd(x, g, table_floats(spec))
    grad_o = ora.hash_backward(ora.make_cfg(spec), x, g, table_floats(spec))
    scale = np.abs(grad_o).max()
    assert np.isfinite(grad_g).all()
    assert np.abs(grad_g - grad_o).max() <= 1e-5 * scale
    touched_g, touched_o = grad_g != 0, grad_o != 0
    assert (touched_g == touched_o).mean() > 0.9999


def _ray_walk_points(rng, lo, hi, n_rays, per_ray):
    """Points that walk along rays in small steps, so consecutive samples share cells at the coarse levels
    (runs of every length, longer than one merge group)."""
    o = lo + (hi - lo) * rng.uniform(0.2, 0.8, (n_rays, 1, 3))
    d = rng.normal(size=(n_rays, 1, 3))
    d /= np.linalg.norm(d, axis=2, keepdims=True)
    t = np.cumsum(rng.uniform(0.0, 0.006, (n_rays, per_ray, 1)), axis=1)
    return np.clip(o + t * d * (hi - lo), lo, hi).reshape(-1, 3).astype(np.float32)


@pytest.mark.parametrize("case", ["f1", "one_partial_round", "wide_table", "runs", "runs_f4"])
def test_hash_backward_shapes(gh, ora, case):
    """The scatter's edge shapes: one feature per level (8192-entry buckets), fewer samples than one emit
    round, 2^22-entry levels (1024 buckets per level: the widest run table and emit stage), and samples
    along rays (consecutive samples in one cell are merged before the scatter; zero-gradient samples inside
    the runs break them), at two and four features per level."""
    print(f"[case] hash bwd shape {case}", flush=True)
    rng = np.random.default_rng(34)
    if case == "f1":
        spec, n = spec_cfg0(f_per_level=1), 20000
    elif case == "one_partial_round":
        spec, n = spec_cfg0(), 1000
    elif case == "wide_table":
        spec, n = spec_cfg0(n_levels=2, log2_T=[22, 22], res=[256.0, 2048.0]), 50000
    else:
        spec = spec_cfg0(f_per_level=4 if case == "runs_f4" else 2)
        n = 96 * 64 + 37
    p = random_params(spec, seed=33)
    m = gh.GpuModel(spec, p)
    lo, hi = np.array(spec["box_min"]), np.array(spec["box_max"])
    if case.startswith("runs"):
        x = np.concatenate([_ray_walk_points(rng, lo, hi, 96, 64), _ray_walk_points(rng, lo, hi, 1, 37)])
        x[100:140] = x[100]  # one point repeated over a whole merge group and more
    else:
        x = (lo + (hi - lo) * rng.uniform(0, 1, (n, 3))).astype(np.float32)
    LF = spec["n_levels"] * spec["f_per_level"]
    g = rng.normal(size=(n, LF)).astype(np.float32)
    if case.startswith("runs"):
        g[::7] = 0.0
    grad_g = m.encode_bwd(x, g, table_floats(spec))
    grad_o = ora.hash_backward(ora.make_cfg(spec), x, g, table_floats(spec))
    scale = np.abs(grad_o).max()
    assert np.isfinite(grad_g).all()
    assert np.abs(grad_g - grad_o).max() <= 1e-5 * scale
    assert ((grad_g != 0) == (grad_o != 0)).mean() > 0.9999
    if case == "f1":  # and the forward of the same shape, bit-exact
        a0_g, idx_g = m.encode(x[:5000], with_idx=True)
        a0_o, idx_o, _ = ora.hash_encode(ora.make_cfg(spec), p["table"], x[:5000], with_idx=True)
        assert np.array_equal(idx_g, idx_o)
        assert np.array_equal(a0_g.view(np.uint32), a0_o.view(np.uint32))


def test_hash_backward_too_wide_is_an_error(gh):
    """F = 4 with 2^22-entry levels needs an emit stage larger than a CU's LDS: the scatter refuses the
    shape before launching its kernels (an error with a message, no silent return)."""
    import ffn_lib as fl
    print("[case] hash bwd too wide", flush=True)
    spec = spec_cfg0(n_levels=2, f_per_level=4, log2_T=[22, 22], res=[256.0, 2048.0])
    m = gh.GpuModel(spec, random_params(spec, seed=35))
    x = np.random.default_rng(36).uniform(0.0, 1.0, (1000, 3)).astype(np.float32)
    g = np.ones((1000, 8), np.float32)
    with pytest.raises(fl.FfnError, match="ffn_hash_encode_bwd"):
        m.encode_bwd(x, g, table_floats(spec))


def test_train_step_with_unbuilt_scatter_changes_nothing(gh):
    """A training step whose table shape the scatter does not support is refused before its first launch:
    no colour, occupancy proposal, table or MLP update is written (a step is applied whole or not at all)."""
    import ffn_lib as fl
    print("[case] train step refused for an unbuilt scatter shape", flush=True)
    spec = spec_cfg0(n_levels=4, f_per_level=4, log2_T=[22, 14, 14, 14], res=[32.0, 64.0, 128.0, 256.0])
    m = gh.GpuModel(spec, random_params(spec, seed=37))
    before = m.state()
    rays = look_at_rays(64, spec, seed=38)
    with pytest.raises(fl.FfnError, match="scatter is not built"):
        m.train_step(rays, sphere_targets(rays, spec), 64, default_scalars(), taps=False)
    after = m.state()
    for k in before:
        assert np.array_equal(before[k].view(np.uint32), after[k].view(np.uint32)), k


def test_occ_decay_bit_exact(gh, ora):
    import ctypes
    import torch
    import ffn_lib as fl
    print("[case] occ decay", flush=True)
    rng = np.random.default_rng(41)
    n = 64 ** 3
    win = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    wst = win.copy()
    raise_ = rng.random(n) < 0.3
    wst[raise_] |= rng.integers(0, 2 ** 32, int(raise_.sum()), dtype=np.uint64).astype(np.uint32)
    for q24, seed in ((int(round(0.9 * (1 << 24))), 1234), (int(round(0.95 * (1 << 24))), 99), (1 << 24, 7), (0, 3)):
        gi, gs = gh.to_dev(win), gh.to_dev(wst)
        fl.check(fl.load().ffn_occ_decay(fl.ptr(gi), fl.ptr(gs), n, q24, seed, fl.stream_ptr()), "decay")
        torch.cuda.synchronize()
        oi, os_ = win.copy(), wst.copy()
        ora.occ_decay(oi, os_, q24, seed)
        assert np.array_equal(gh.to_np(gi, np.uint32), oi)
        assert np.array_equal(gh.to_np(gs, np.uint32), os_)


def test_adam_bit_exact(gh, ora):
    import torch
    import ffn_lib as fl
    print("[case] adam", flush=True)
    rng = np.random.default_rng(51)
    n = 1_000_003
    p, m, v = (rng.normal(size=n).astype(np.float32) for _ in range(3))
    v = np.abs(v)
    g = (rng.normal(size=n) * (rng.random(n) < 0.3)).astype(np.float32)
    t = [gh.to_dev(a) for a in (p, m, v, g)]
    fl.check(fl.load().ffn_adam(*[fl.ptr(x) for x in t], n, 0.01, 0.9, 0.99, 1e-15, 1, fl.stream_ptr()), "adam")
    torch.cuda.synchronize()
    ora.adam(p, m, v, g, 0.01, 0.9, 0.99, 1e-15)
    assert np.array_equal(gh.to_np(t[0]), p)
    assert np.array_equal(gh.to_np(t[1]), m)
    assert np.array_equal(gh.to_np(t[2]), v)
    assert not gh.to_np(t[3]).any()  # gradient cleared in the same pass


def _compare_step(spec, p, rays, tg, S, sc, gh, ora, check_params=True):
    m, o, stats = compare_step(spec, p, rays, tg, S, sc, gh, ora, check_params=check_params)
    print("parity:", {k: v for k, v in stats.items() if not k.startswith("g")}, flush=True)
    return m, o


@pytest.mark.parametrize("S", [64, 32, 16, 8, 4, 2, 1])
def test_train_step_cfg0_adam(gh, ora, S):
    print(f"[case] train step cfg0 adam S={S}", flush=True)
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=61)
    rays = look_at_rays(96 * 64 // S, spec, seed=62, miss_frac=0.1)
    tg = sphere_targets(rays, spec)
    _compare_step(spec, p, rays, tg, S, default_scalars(), gh, ora)


@pytest.mark.parametrize("S", [64, 16])
def test_train_step_empty_tiles_match_full_path(gh, ora, S):
    """Tiles whose samples are all inactive (rays that miss the box) skip the MLP when no taps are
    requested; the step must leave exactly the state and colours of the full path (which the other step
    tests check against the oracle)."""
    print(f"[case] train step empty tiles S={S}", flush=True)
    spec = spec_cfg0(hash_opt=1, background=2)
    p = random_params(spec, seed=81)
    rays = look_at_rays(96 * 64 // S, spec, seed=82, miss_frac=0.4)
    tg = sphere_targets(rays, spec)
    full = gh.GpuModel(spec, p)
    fast = gh.GpuModel(spec, p)
    out_full, _ = full.train_step(rays, tg, S, default_scalars(), taps=True)
    out_fast, _ = fast.train_step(rays, tg, S, default_scalars(), taps=False)
    assert np.array_equal(out_full.view(np.uint32), out_fast.view(np.uint32))
    sf, ss = full.state(), fast.state()
    assert set(sf) == set(ss)
    for k in sf:
        assert np.array_equal(sf[k].view(np.uint32), ss[k].view(np.uint32)), k


def test_train_step_empty_grid_proposals(gh, ora):
    print("[case] train step proposals", flush=True)
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=71)
    p["occ_in"][:] = 0
    p["occ_st"][:] = 0
    p["bd_out"][0] = 4.0
    rays = look_at_rays(128, spec, seed=72, miss_frac=0.0)
    tg = sphere_targets(rays, spec)
    m, o = _compare_step(spec, p, rays, tg, 64, default_scalars(), gh, ora)
    assert not np.array_equal(o.p["occ_st"], p["occ_st"])


def test_train_step_many_proposals(gh, ora):
    """Occupancy levels 1..8 in every subcell and a dense field (density bias 8), so that many runs absorb
    enough light to propose: the proposals (including the kernels' exact early out for runs whose
    transmittance drop cannot exceed the cell's smallest level) must match the oracle, which evaluates
    every run in full."""
    print("[case] train step many proposals", flush=True)
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=151)
    rng = np.random.default_rng(152)
    nib = rng.integers(0, 8, (p["occ_in"].size, 8)).astype(np.uint32)
    occ = np.zeros(p["occ_in"].size, np.uint32)
    for q in range(8):
        occ |= nib[:, q] << np.uint32(4 * q)
    p["occ_in"][:] = occ.reshape(p["occ_in"].shape)
    p["occ_st"][:] = p["occ_in"]
    p["bd_out"][0] = 8.0
    rays = look_at_rays(256, spec, seed=153, miss_frac=0.0)
    tg = sphere_targets(rays, spec)
    m, o = _compare_step(spec, p, rays, tg, 64, default_scalars(), gh, ora)
    changed = int((o.p["occ_st"] != p["occ_st"]).sum())
    print(f"occupancy words raised by the oracle's proposals: {changed}", flush=True)
    assert changed > 50


@pytest.mark.parametrize("bg", [1, 2])
def test_train_step_backgrounds_and_sgd(gh, ora, bg):
    print(f"[case] train step sgd bg={bg}", flush=True)
    spec = spec_cfg0(hash_opt=0, background=bg)
    p = random_params(spec, seed=81)
    rays = look_at_rays(64, spec, seed=82, miss_frac=0.2)
    tg = sphere_targets(rays, spec)
    _compare_step(spec, p, rays, tg, 64, default_scalars(lr=0.05), gh, ora)


def test_train_step_reference_shape(gh, ora):
    """The reference's compiled-in shape: L=16, F=4 (LF=64), per-level T, ND=NC=2, SGD table."""
    print("[case] train step reference shape", flush=True)
    spec = spec_ref(hash_opt=0)
    p = random_params(spec, seed=91)
    rays = look_at_rays(48, spec, seed=92, miss_frac=0.1, radius=1.2)
    tg = np.random.default_rng(93).uniform(0, 1, (48, 4)).astype(np.float32)
    _compare_step(spec, p, rays, tg, 64, default_scalars(lr=0.01, lr_t=0.01, beta2=0.999, eps=1e-6), gh, ora)


def test_render_mode(gh, ora):
    print("[case] render", flush=True)
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=101)
    rays = look_at_rays(64, spec, seed=102)
    tg = np.zeros((64, 4), np.float32)
    m, o = _compare_step(spec, p, rays, tg, 64, default_scalars(do_train=0), gh, ora)
    st = m.state()
    for k in ("table", "Wd_in", "Wc_out", "occ_in", "occ_st"):
        assert np.array_equal(st[k], p[k]), k


@pytest.mark.parametrize("mlp_precision", [0, 1])
def test_train_step_deterministic(gh, mlp_precision):
    """Two runs of the same step from the same state leave bit-identical state and colours: the scatter
    sums in fixed point (order-free), the MLP weight gradients are summed over the block partials in a
    fixed order, and the occupancy proposals only take maxima.  The batch (cfg1 shapes, 4096 rays x 64
    samples) spans many MLP blocks and scatter chunks, so any order-dependent sum would show."""
    print(f"[case] train step determinism mlp_precision={mlp_precision}", flush=True)
    spec = spec_cfg1(hash_opt=1, mlp_precision=mlp_precision)
    p = random_params(spec, seed=101)
    rays = look_at_rays(4096, spec, seed=102, miss_frac=0.1)
    tg = sphere_targets(rays, spec)
    runs = []
    for _ in range(2):
        m = gh.GpuModel(spec, p)
        out, _ = m.train_step(rays, tg, 64, default_scalars(), taps=False)
        out2, _ = m.train_step(rays, tg, 64, default_scalars(rng_seed=7), taps=False)
        runs.append((out, out2, m.state()))
        del m
    (a1, a2, sa), (b1, b2, sb) = runs
    assert np.array_equal(a1.view(np.uint32), b1.view(np.uint32))
    assert np.array_equal(a2.view(np.uint32), b2.view(np.uint32))
    assert set(sa) == set(sb)
    for k in sa:
        assert np.array_equal(sa[k].view(np.uint32), sb[k].view(np.uint32)), k


def test_hash_scatter_full_size_adjoint(gh):
    """The scatter at the benchmark's full size, 2^24 samples (2^18 rays x 64 points walking along each
    ray, clamped into the box) on the cfg1/cfg2 table (16 levels of 2^19 entries): 16384 emit rounds per
    level in one level group, which the oracle comparisons (tens of thousands of points) do not reach.
    Size-independent properties of the linear map table -> encoding and its adjoint, summed in float64:
      <encode(x; T), g> = <T, encode_bwd(x, g)>   (adjoint identity),
      sum(encode_bwd(x, g)) = sum(g)              (the eight trilinear weights sum to one).
    Positive T and g keep both sums free of cancellation, so fp32 rounding stays near 1e-7."""
    import torch
    import ffn_lib as fl
    print("[case] hash scatter full size adjoint", flush=True)
    spec = spec_cfg1(hash_opt=1)
    p = random_params(spec, seed=111)
    p["table"] = np.random.default_rng(112).uniform(0.5, 1.5, p["table"].shape).astype(np.float32)
    m = gh.GpuModel(spec, p)
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(113)
    n_rays, S = 1 << 18, 64
    lo = torch.tensor(spec["box_min"], dtype=torch.float32, device=dev)
    hi = torch.tensor(spec["box_max"], dtype=torch.float32, device=dev)
    o = lo + (hi - lo) * (0.2 + 0.6 * torch.rand((n_rays, 1, 3), generator=gen, device=dev))
    d = torch.randn((n_rays, 1, 3), generator=gen, device=dev)
    d = d / d.norm(dim=2, keepdim=True)
    t = torch.cumsum(0.02 * torch.rand((n_rays, S, 1), generator=gen, device=dev), dim=1)
    x = torch.minimum(torch.maximum(o + t * d * (hi - lo), lo), hi).reshape(-1, 3).contiguous()
    n = x.shape[0]
    LF = spec["n_levels"] * spec["f_per_level"]
    a0 = torch.empty((n, LF), dtype=torch.float32, device=dev)
    fl.check(m.lib.ffn_hash_encode_fwd(m.h.h, fl.ptr(x), n, fl.ptr(a0), None, fl.stream_ptr()), "encode fwd")
    g = 0.5 + torch.rand((n, LF), generator=gen, device=dev)
    G = torch.zeros(table_floats(spec), dtype=torch.float32, device=dev)
    fl.check(m.lib.ffn_hash_encode_bwd(m.h.h, fl.ptr(x), fl.ptr(g), n, fl.ptr(G), fl.stream_ptr()), "encode bwd")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(G).all())
    lhs = sum(float((a0[i:i + (1 << 22)].double() * g[i:i + (1 << 22)].double()).sum()) for i in range(0, n, 1 << 22))
    rhs = float((m.t["table"].double() * G.double()).sum())
    gsum = sum(float(g[i:i + (1 << 22)].double().sum()) for i in range(0, n, 1 << 22))
    Gsum = float(G.double().sum())
    print(f"adjoint rel {abs(lhs - rhs) / lhs:.2e}  weight-sum rel {abs(Gsum - gsum) / gsum:.2e}", flush=True)
    assert abs(lhs - rhs) <= 2e-6 * lhs
    assert abs(Gsum - gsum) <= 2e-6 * gsum


def test_scatter_level_groups_bit_identical(gh, monkeypatch):
    """A pair budget smaller than one step's pairs splits the levels into groups (one emit and one reduce
    launch per group, the pair buffer reused).  At FFN_BIN_BUDGET_MB=64, 2^18 points on 16 levels of 2^19
    entries need 256 rounds x 8640 slots x 10 B = 22 MB per level, so three levels per group and six
    groups; the per-level fixed-point sums do not depend on the grouping, so the table gradient must equal
    the single-group one bit for bit."""
    print("[case] scatter level groups", flush=True)
    spec = spec_cfg1(hash_opt=1)
    p = random_params(spec, seed=121)
    rng = np.random.default_rng(122)
    lo, hi = np.array(spec["box_min"]), np.array(spec["box_max"])
    x = _ray_walk_points(rng, lo, hi, 4096, 64)
    LF = spec["n_levels"] * spec["f_per_level"]
    g = rng.normal(size=(x.shape[0], LF)).astype(np.float32)
    m = gh.GpuModel(spec, p)
    one_group = m.encode_bwd(x, g, table_floats(spec))
    monkeypatch.setenv("FFN_BIN_BUDGET_MB", "64")
    grouped = m.encode_bwd(x, g, table_floats(spec))
    monkeypatch.delenv("FFN_BIN_BUDGET_MB")
    assert np.abs(one_group).max() > 0
    assert np.array_equal(one_group.view(np.uint32), grouped.view(np.uint32))


@pytest.mark.parametrize("case", ["uniform22", "rays22", "cfg2_shape"])
def test_scatter_walk64_bit_identical(gh, ora, monkeypatch, case):
    """The reduce walks 64 rounds per wavefront step (a binary search finds each lane's run) where a level
    has many buckets (2^22 entries: 512 buckets, runs of a few pair blocks) or the batch has at least 1024
    emit rounds (the benchmark shape's 16 levels of 2^19), 16 rounds otherwise.  Its fixed-point sums are
    exact, so the table gradient equals the 16-round walk's (FFN_REDUCE_WALK64=0) bit for bit, with runs of
    every length (points along rays at a coarse level, uniform points at a fine one); the 2^22 cases are the
    oracle's float64 sums as well."""
    print(f"[case] scatter walk64 {case}", flush=True)
    if case == "cfg2_shape":
        spec = spec_cfg1(hash_opt=1)
    else:
        spec = spec_cfg0(n_levels=2, log2_T=[22, 22], res=[64.0, 2048.0])
    p = random_params(spec, seed=141)
    rng = np.random.default_rng(142)
    lo, hi = np.array(spec["box_min"]), np.array(spec["box_max"])
    if case == "uniform22":
        x = (lo + (hi - lo) * rng.uniform(0, 1, (70000, 3))).astype(np.float32)
    else:
        x = _ray_walk_points(rng, lo, hi, 1024 if case == "rays22" else 16400, 64)  # cfg2_shape: 1025 rounds
    LF = spec["n_levels"] * spec["f_per_level"]
    g = rng.normal(size=(x.shape[0], LF)).astype(np.float32)
    m = gh.GpuModel(spec, p)
    w64 = m.encode_bwd(x, g, table_floats(spec))
    monkeypatch.setenv("FFN_REDUCE_WALK64", "0")
    w16 = m.encode_bwd(x, g, table_floats(spec))
    monkeypatch.delenv("FFN_REDUCE_WALK64")
    assert np.abs(w64).max() > 0
    assert np.array_equal(w64.view(np.uint32), w16.view(np.uint32))
    if case != "cfg2_shape":
        grad_o = ora.hash_backward(ora.make_cfg(spec), x, g, table_floats(spec))
        assert np.abs(w64 - grad_o).max() <= 1e-5 * np.abs(grad_o).max()


def test_stage_times(gh):
    """ffn_set_profiling / ffn_stage_times (the reference's profiling queue and event_ms,
    ffnerf_tools.py:11-13,127-138): with profiling on, each stage of a training step is bracketed by
    events on the caller's stream; two steps give two launches of every stage, positive times, and a reset
    empties the record."""
    print("[case] stage times", flush=True)
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=131)
    rays = look_at_rays(256, spec, seed=132, miss_frac=0.1)
    tg = sphere_targets(rays, spec)
    m = gh.GpuModel(spec, p)
    m.h.set_profiling(True)
    m.h.stage_times(reset=True)
    for _ in range(2):
        m.train_step(rays, tg, 64, default_scalars(), taps=False)
    st = m.h.stage_times(reset=True)
    for s in ("sample", "hash_fwd", "mlp", "hash_bwd", "mlp_adam"):
        assert st[s][1] == 2 and st[s][0] > 0.0, (s, st[s])
    assert st["table_adam"][1] == 0  # the table Adam is fused into the scatter's reduce
    assert all(n == 0 for _, n in m.h.stage_times(reset=True).values())
    m.h.set_profiling(False)
    m.train_step(rays, tg, 64, default_scalars(), taps=False)
    assert all(n == 0 for _, n in m.h.stage_times(reset=True).values())


@pytest.mark.parametrize("mlp_precision", [0, 1])
def test_headline_shape_sixteen_steps(gh, ora, mlp_precision):
    """The benchmark's model shape (L=16, F=2, T=2^19 per level, 16 -> 2048, 128^3 occupancy, Adam on table
    and MLPs) at 512 rays x 64 samples per step, over 16 steps with a fresh batch and seed each step and
    the bias-corrected Adam step of each step count; the occupancy decay (0.95) runs after step 16, as the
    trainer schedules it.  Every step starts both implementations from the restatement's state (so rounding
    differences do not compound through Adam) and is checked as in tests/parity.py; the decay is bit-exact."""
    import torch
    import ffn_lib as fl
    print(f"[case] headline shape 16 steps mlp_precision={mlp_precision}", flush=True)
    spec = spec_cfg1(hash_opt=1, mlp_precision=mlp_precision)
    state = random_params(spec, seed=201)
    # occupancy levels 1..6 and a denser field (density bias 4), so that runs absorb enough light to propose
    # every step and the decay after step 16 merges raised words (occ_st != occ_in)
    rng = np.random.default_rng(202)
    nib = rng.integers(0, 6, (state["occ_in"].size, 8)).astype(np.uint32)
    state["occ_in"] = np.bitwise_or.reduce(nib << (4 * np.arange(8, dtype=np.uint32)), axis=1).astype(np.uint32)
    state["occ_st"] = state["occ_in"].copy()
    state["bd_out"][0] = 4.0
    b1, b2, lr = 0.9, 0.99, 1e-2
    raised = 0
    for step in range(1, 17):
        rays = look_at_rays(512, spec, seed=300 + step, miss_frac=0.1)
        lr_t = lr * np.sqrt(1.0 - b2 ** step) / (1.0 - b1 ** step)
        sc = default_scalars(lr_t=lr_t, rng_seed=0x5EED0000 + step)
        m, o, stats = compare_step(spec, state, rays, sphere_targets(rays, spec), 64, sc, gh, ora)
        print(f"step {step}:", {k: v for k, v in stats.items() if not k.startswith("g")}, flush=True)
        raised += stats["occ_raised"]
        state = {k: v.copy() for k, v in o.p.items()}
        del m
    assert raised > 100, raised
    q24, seed = int(round(0.95 * (1 << 24))), 0xDECA1
    gi, gs = gh.to_dev(state["occ_in"]), gh.to_dev(state["occ_st"])
    n = state["occ_in"].size
    fl.check(fl.load().ffn_occ_decay(fl.ptr(gi), fl.ptr(gs), n, q24, seed, fl.stream_ptr()), "decay")
    torch.cuda.synchronize()
    oi, os_ = state["occ_in"].copy(), state["occ_st"].copy()
    ora.occ_decay(oi, os_, q24, seed)
    assert not np.array_equal(os_, state["occ_st"])
    assert (state["occ_in"] != state["occ_st"]).sum() > 100  # the merge path of the decay
    assert np.array_equal(gh.to_np(gi, np.uint32), oi)
    assert np.array_equal(gh.to_np(gs, np.uint32), os_)


def _f16_params(spec, seed, **kw):
    p = random_params(spec, seed=seed, **kw)
    p["table"] = p["table"].astype(np.float16).astype(np.float32)  # binary16 values (stored exactly as fp16)
    return p


@pytest.mark.parametrize("which", ["cfg0", "cfg3"])
def test_hash_fp16_table_forward_bit_exact(gh, ora, which):
    """A binary16 table widens exactly: the encodings and indices are bit-identical to
    the oracle's over the same values."""
    print(f"[case] hash fwd fp16 table {which}", flush=True)
    spec = spec_cfg0(table_dtype=1) if which == "cfg0" else spec_cfg1(table_dtype=1, log2_T=[22] * 16)
    p = _f16_params(spec, seed=211)
    m = gh.GpuModel(spec, p)
    rng = np.random.default_rng(212)
    x = rng.uniform(-0.05, 1.05, (20000, 3)).astype(np.float32)
    x[:16] = 1.0
    a0_g, idx_g = m.encode(x, with_idx=True)
    a0_o, idx_o, _ = ora.hash_encode(ora.make_cfg(spec), p["table"], x, with_idx=True)
    assert np.array_equal(idx_g, idx_o)
    assert np.array_equal(a0_g.view(np.uint32), a0_o.view(np.uint32))


@pytest.mark.parametrize("which", ["cfg0", "cfg3"])
def test_hash_fp16_table_backward(gh, ora, which):
    """The scatter into a binary16 gradient table: every entry is its exact sum rounded once to nearest even,
    so it is within one binary16 ulp of the oracle's float64 sum (and the touched entries agree)."""
    print(f"[case] hash bwd fp16 table {which}", flush=True)
    spec = spec_cfg0(table_dtype=1) if which == "cfg0" else spec_cfg1(table_dtype=1, log2_T=[22] * 16)
    m = gh.GpuModel(spec, _f16_params(spec, seed=221))
    rng = np.random.default_rng(222)
    n = 30000
    x = rng.uniform(0, 1, (n, 3)).astype(np.float32)
    LF = spec["n_levels"] * spec["f_per_level"]
    g = rng.normal(size=(n, LF)).astype(np.float32)
    grad_g = m.encode_bwd(x, g, table_floats(spec)).astype(np.float64)
    grad_o = ora.hash_backward(ora.make_cfg(spec), x, g, table_floats(spec))
    with np.errstate(over="ignore"):
        ulp16 = np.spacing(np.abs(grad_o).astype(np.float16)).astype(np.float64)
    err = np.abs(grad_g - grad_o)
    assert (err <= ulp16 + 1e-6 * np.abs(grad_o).max()).all(), float((err - ulp16).max())
    assert ((grad_g != 0) == (grad_o != 0)).mean() > 0.9999


@pytest.mark.parametrize("hash_opt,mlp_precision", [(1, 0), (0, 0), (1, 1)])
def test_train_step_fp16_table(gh, ora, hash_opt, mlp_precision):
    """Training steps on a binary16 table (Adam with fp32 moments, or the reference SGD), fp32 and fp16 MLPs,
    against the oracle's binary16 table semantics (tests/parity.py)."""
    print(f"[case] train step fp16 table hash_opt={hash_opt} mlp={mlp_precision}", flush=True)
    spec = spec_cfg0(hash_opt=hash_opt, mlp_precision=mlp_precision, table_dtype=1)
    p = _f16_params(spec, seed=231)
    rays = look_at_rays(96, spec, seed=232, miss_frac=0.1)
    m, o = _compare_step(spec, p, rays, sphere_targets(rays, spec), 64, default_scalars(lr=0.05), gh, ora)
    assert not np.array_equal(m.state()["table"], p["table"])


def test_dense_level_copies_change_no_bit(gh, monkeypatch):
    """The gather reads the coarse levels from dense vertex copies (levels with R^3 <= FFN_DENSE_MAX_CELLS):
    encodings, hash indices and a whole training step are bit-identical with the copies off (0), at the
    default and with every level of the cfg0 shape dense."""
    print("[case] dense level copies on/off", flush=True)
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=201)
    rays = look_at_rays(128, spec, seed=202, miss_frac=0.1)
    tg = sphere_targets(rays, spec)
    x = np.random.default_rng(203).uniform(-0.1, 1.1, (5000, 3)).astype(np.float32)
    res = []
    for cells in ("0", str(1 << 21), str(1 << 30)):
        monkeypatch.setenv("FFN_DENSE_MAX_CELLS", cells)
        m = gh.GpuModel(spec, p)
        enc, idx = m.encode(x, with_idx=True)
        enc_plain = m.encode(x)  # the dense path without the index tap
        np.testing.assert_array_equal(enc_plain, enc)
        out, _ = m.train_step(rays, tg, 64, default_scalars())
        res.append((enc, idx, out, m.state()))
    for r in res[1:]:
        np.testing.assert_array_equal(r[0], res[0][0])
        np.testing.assert_array_equal(r[1], res[0][1])
        np.testing.assert_array_equal(r[2], res[0][2])
        for k in res[0][3]:
            np.testing.assert_array_equal(r[3][k], res[0][3][k], err_msg=k)
