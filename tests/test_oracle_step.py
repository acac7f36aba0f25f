"""Pins of the oracle's compositing, MLP and full training step against
torch float64 autograd (a library routine) and closed forms."""
import numpy as np
import pytest
import torch

from common import (BIASES, LAYERS, default_scalars, layer_shapes, look_at_rays, random_params, spec_cfg0,
                    sphere_targets, table_floats)


def _composite(ora, cfg, sig, rgb, dts, tgt, S, do_train=1, seed=5):
    out = np.zeros(4, np.float32)
    Tr = np.zeros(S, np.float32)
    Tf = np.zeros(1, np.float32)
    dLdc = np.zeros(3 * S, np.float32)
    dLds = np.zeros(S, np.float32)
    f = lambda a: np.ascontiguousarray(a, np.float32)
    ora.lib().ora_composite_ray(ora.byref(cfg) if hasattr(ora, "byref") else __import__("ctypes").byref(cfg), 0, S,
                                seed, do_train, ora.fptr(f(sig)), ora.fptr(f(rgb)), ora.fptr(f(dts)),
                                ora.fptr(f(tgt)), ora.fptr(out), ora.fptr(Tr), ora.fptr(Tf), ora.fptr(dLdc),
                                ora.fptr(dLds))
    return out, Tr, float(Tf[0]), dLdc.reshape(S, 3), dLds


def _torch_composite(sig, rgb, dt, tgt, bg):
    sig = torch.tensor(sig, dtype=torch.float64, requires_grad=True)
    rgb = torch.tensor(rgb, dtype=torch.float64, requires_grad=True)
    alpha = 1 - torch.exp(-sig * dt)
    T = torch.cumprod(torch.cat([torch.ones(1, dtype=torch.float64), 1 - alpha[:-1]]), 0)
    C = (T * alpha)[:, None].mul(rgb).sum(0) + T[-1] * (1 - alpha[-1]) * torch.tensor(bg, dtype=torch.float64)
    eps2 = float(np.float32(1e-3) * np.float32(1e-3))
    L = torch.sqrt((C - torch.tensor(tgt, dtype=torch.float64)) ** 2 + eps2).sum()
    L.backward()
    return C.detach().numpy(), T.detach().numpy(), sig.grad.numpy(), rgb.grad.numpy()


@pytest.mark.parametrize("bg_mode", [0, 1])
def test_composite_constant_ray_matches_autograd(ora, bg_mode):
    """Constant sigma and colour along the ray: the affine maps commute, so the
    reference's scan order gives the true gradient (plus the density penalty)."""
    S = 64
    cfg = ora.make_cfg(spec_cfg0(background=bg_mode))
    sig = np.full(S, 3.0, np.float32)
    rgb = np.tile(np.array([0.2, 0.5, 0.9], np.float32), (S, 1))
    dts = np.full(S, 0.01, np.float32)
    tgt = np.array([0.3, 0.1, 0.6, 0.0], np.float32)
    out, Tr, Tf, dLdc, dLds = _composite(ora, cfg, sig, rgb.reshape(-1), dts, tgt, S)
    bg = [1.0, 1.0, 1.0] if bg_mode == 1 else [0.0, 0.0, 0.0]
    C, T, gsig, grgb = _torch_composite(sig, rgb, 0.01, tgt[:3], bg)
    a = 1 - np.exp(-3.0 * 0.01)
    assert np.allclose(out[:3], np.clip(C, 0, 1), atol=2e-6)
    assert np.allclose(C[:3] - np.array(bg) * (1 - a) ** S, rgb[0] * (1 - (1 - a) ** S), atol=2e-6)
    assert np.allclose(Tr, T, rtol=1e-5)  # float32 alpha, 64 products
    assert Tf == pytest.approx((1 - a) ** S, rel=1e-5)
    assert np.allclose(dLdc, grgb, rtol=1e-5, atol=1e-8)
    regu = 5e-3 * 0.01 / S
    assert np.allclose(dLds - regu, gsig, rtol=1e-4, atol=1e-7)


def test_composite_general_colour_gradient(ora):
    """dL/dc_s = T_s alpha_s dL/dC holds for any ray (no scan ordering involved)."""
    S = 32
    rng = np.random.default_rng(0)
    cfg = ora.make_cfg(spec_cfg0())
    sig = rng.uniform(0, 20, S).astype(np.float32)
    rgb = rng.uniform(0, 1, (S, 3)).astype(np.float32)
    dts = np.full(S, 0.02, np.float32)
    tgt = np.array([0.3, 0.1, 0.6, 0.0], np.float32)
    _, Tr, _, dLdc, _ = _composite(ora, cfg, sig, rgb.reshape(-1), dts, tgt, S)
    C, T, _, grgb = _torch_composite(sig, rgb, 0.02, tgt[:3], [0, 0, 0])
    assert np.allclose(Tr, T, rtol=1e-5)
    assert np.allclose(dLdc, grgb, rtol=1e-4, atol=1e-8)


def _torch_mlp(spec, p, a0, dirs, sh_mult):
    """The reference MLP (ffnerf_OG.cl:1373-1466) in float64 torch."""
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in p.items()
         if k in LAYERS or k in BIASES}
    x = torch.tensor(a0, dtype=torch.float64, requires_grad=True)
    h = torch.relu(x @ t["Wd_in"].T + t["bd_0"])
    if spec["nd"] >= 2:
        h = torch.relu(h @ t["Wd_01"].T + t["bd_1"])
    dout = h @ t["Wd_out"].T + t["bd_out"]
    d = torch.tensor(dirs, dtype=torch.float64)
    X, Y, Z = d[:, 0], d[:, 1], d[:, 2]
    sh = torch.stack([
        torch.full_like(X, 0.28209479177387814), 0.4886025119029199 * Y, 0.4886025119029199 * Z,
        0.4886025119029199 * X, 1.0925484305920792 * X * Y, 1.0925484305920792 * Y * Z,
        0.31539156525252005 * (3 * Z * Z - 1), 1.0925484305920792 * X * Z, 0.5462742152960396 * (X * X - Y * Y),
        0.5900435899266435 * Y * (3 * X * X - Y * Y), 2.890611442640554 * X * Y * Z,
        0.4570457994644658 * Y * (5 * Z * Z - 1), 0.3731763325901154 * (5 * Z * Z * Z - 3 * Z),
        0.4570457994644658 * X * (5 * Z * Z - 1), 1.445305721320277 * Z * (X * X - Y * Y),
        0.5900435899266435 * X * (X * X - 3 * Y * Y)], 1) * sh_mult
    c = torch.relu(torch.cat([dout, sh], 1) @ t["Wc_in"].T + t["bc_0"])
    if spec["nc"] >= 2:
        c = torch.relu(c @ t["Wc_01"].T + t["bc_1"])
    cout = c @ t["Wc_out"].T + t["bc_out"]
    return t, x, dout, cout


def test_mlp_forward_matches_torch(ora):
    spec = spec_cfg0()
    cfg = ora.make_cfg(spec)
    p = random_params(spec, seed=3)
    model = ora.OracleModel(spec, p)
    P = model._params()
    rng = np.random.default_rng(1)
    a0 = rng.normal(0, 0.5, (64, 16)).astype(np.float32)
    dirs = rng.normal(size=(64, 3))
    dirs = (dirs / np.linalg.norm(dirs, axis=1, keepdims=True)).astype(np.float32)
    _, _, dout, cout = _torch_mlp(spec, p, a0, dirs, 0.7)
    import ctypes
    for i in range(64):
        sig = np.zeros(1, np.float32)
        rgb = np.zeros(3, np.float32)
        do = np.zeros(16, np.float32)
        ora.lib().ora_mlp_forward(ctypes.byref(cfg), ctypes.byref(P), ora.fptr(np.ascontiguousarray(a0[i])),
                                  ora.fptr(np.ascontiguousarray(dirs[i])), 0.7, ora.fptr(sig), ora.fptr(rgb),
                                  ora.fptr(do))
        assert np.allclose(do, dout[i].detach().numpy(), rtol=1e-5, atol=1e-5)
        ref_sig = np.log1p(np.exp(np.clip(dout[i, 0].item(), -10, 10)))
        assert sig[0] == pytest.approx(ref_sig, rel=1e-5)
        ref_rgb = 1 / (1 + np.exp(-np.clip(0.5 * cout[i].detach().numpy(), -18, 18)))
        assert np.allclose(rgb, ref_rgb, rtol=1e-5, atol=1e-6)


def _small_step(ora, hash_opt, S=16, n_rays=24, seed=7, occ_word=None, **sc):
    spec = spec_cfg0(hash_opt=hash_opt)
    p = random_params(spec, seed=seed)
    if occ_word is not None:
        p["occ_in"][:] = occ_word
        p["occ_st"][:] = occ_word
        p["bd_out"][0] = 4.0
    model = ora.OracleModel(spec, p)
    rays = look_at_rays(n_rays, spec, seed=seed, miss_frac=0.15)
    tg = sphere_targets(rays, spec)
    before = {k: v.copy() for k, v in model.p.items()}
    out, taps = model.train_step(rays, tg, S, default_scalars(**sc), taps=True)
    return spec, rays, before, model, out, taps


def test_step_weight_gradients_match_autograd(ora):
    """The reference backward is the chain rule through the MLP from the output
    deltas f_vol*dL/dc*s(1-s)/2 and f_vol*dL/dsigma*softplus'(clamp(dout0,+-18))
    (ffnerf_OG.cl:1863-1891): differentiating <delta, outputs> with autograd must
    give the same weight gradients and dL/da0."""
    spec, rays, before, model, out, taps = _small_step(ora, hash_opt=1)
    S = 16
    N = rays.shape[0] * S
    dirs = np.repeat(rays[:, 4:7], S, axis=0)
    t, x, dout, cout = _torch_mlp(spec, before, taps["a0"], dirs, 1.0)
    Ts, DTs = taps["Ts"].astype(np.float64), taps["DTs"].astype(np.float64)
    D = 0.5 * np.sqrt(3.0)
    num = Ts * Ts + Ts * DTs + DTs * DTs / 3
    den = D * D + D * DTs + DTs * DTs / 3
    xg = Ts / D
    gate = np.where(xg >= 1, 1.0, np.power(np.maximum(xg, 1e-12), 0.2))
    fvol = gate * num / den
    rgb = 1 / (1 + np.exp(-np.clip(0.5 * cout.detach().numpy(), -18, 18)))
    d_cout = fvol[:, None] * taps["dL_dc"] * rgb * (1 - rgb) * 0.5
    z = np.clip(dout[:, 0].detach().numpy(), -18, 18)
    d_dout0 = fvol * taps["dL_dsigma"] / (1 + np.exp(-z))
    surrogate = (torch.tensor(d_cout) * cout).sum() + (torch.tensor(d_dout0) * dout[:, 0]).sum()
    surrogate.backward()
    for wn in layer_shapes(spec):
        bn = BIASES[LAYERS.index(wn)]
        gw, gb = t[wn].grad.numpy(), t[bn].grad.numpy()
        scale = np.abs(gw).max() + 1e-30
        assert np.abs(taps["g" + wn] - gw).max() <= 2e-4 * scale, wn
        assert np.abs(taps["g" + bn] - gb).max() <= 2e-4 * (np.abs(gb).max() + 1e-30), bn
    gx = x.grad.numpy()
    assert np.abs(taps["dL_da0"] - gx).max() <= 2e-4 * (np.abs(gx).max() + 1e-30)
    # table gradient is the scatter of dL/da0 (the scatter itself is pinned by the adjoint test)
    T32 = taps["Ts"].reshape(-1, S)  # float32, as the kernel forms x = o + t d
    x_s = rays[:, None, :3] + T32[..., None] * rays[:, None, 4:7]
    g_scatter = ora.hash_backward(model.cfg, x_s.reshape(-1, 3).astype(np.float32), taps["dL_da0"], table_floats(spec))
    assert np.allclose(taps["g_table"], g_scatter, rtol=1e-5, atol=1e-9 * np.abs(g_scatter).max())


def test_step_adam_first_step_closed_form(ora):
    spec, rays, before, model, out, taps = _small_step(ora, hash_opt=1)
    sc = default_scalars()
    for wn in layer_shapes(spec):
        g = taps["g" + wn].astype(np.float64)
        exp = before[wn] - sc["lr_t"] * (1 - sc["beta1"]) * g / (np.sqrt((1 - sc["beta2"]) * g * g) + sc["eps"])
        lr_cmp = sc["lr_t"] * (sc["color_rel_lr"] if wn.startswith("Wc") else 1.0)
        exp = before[wn] - lr_cmp * (1 - sc["beta1"]) * g / (np.sqrt((1 - sc["beta2"]) * g * g) + sc["eps"])
        assert np.allclose(model.p[wn], exp, rtol=1e-5, atol=1e-7), wn
    g = taps["g_table"].astype(np.float64)
    exp = before["table"] - sc["lr_t"] * (1 - sc["beta1"]) * g / (np.sqrt((1 - sc["beta2"]) * g * g) + sc["eps"])
    assert np.allclose(model.p["table"], exp, rtol=1e-5, atol=1e-7)


def test_step_reference_sgd_table_update(ora):
    """hash_opt=0: table += -lr 2^(-0.1 l) 0.5 * scatter(dL/da0) (ffnerf_OG.cl:2107-2169)."""
    spec, rays, before, model, out, taps = _small_step(ora, hash_opt=0)
    S = 16
    sc = default_scalars()
    L, F = spec["n_levels"], spec["f_per_level"]
    scale = np.array(ora.lvl_lr_scale(L), np.float32)
    g = taps["dL_da0"].reshape(-1, L, F) * (-np.float32(sc["lr"]) * scale[None, :, None] * 0.5)
    Ts = taps["Ts"].reshape(-1, S)
    x_s = (rays[:, None, :3] + Ts[..., None] * rays[:, None, 4:7]).reshape(-1, 3).astype(np.float32)
    upd = ora.hash_backward(model.cfg, x_s, g.reshape(-1, L * F).astype(np.float32), table_floats(spec))
    delta = model.p["table"].astype(np.float64) - before["table"]
    assert np.allclose(delta, upd, atol=2e-7 * max(1.0, np.abs(before["table"]).max()))


def test_step_proposals_only_raise_the_grid(ora):
    spec, rays, before, model, out, taps = _small_step(ora, hash_opt=1, n_rays=64, S=64, occ_word=0)
    st0, st1 = before["occ_st"], model.p["occ_st"]
    assert not np.array_equal(st0, st1)
    for s in range(8):
        n0 = (st0 >> (4 * s)) & 0xF
        n1 = (st1 >> (4 * s)) & 0xF
        assert np.all(n1 >= n0)
    assert np.array_equal(model.p["occ_in"], before["occ_in"])


def test_render_mode_changes_nothing(ora):
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=9)
    model = ora.OracleModel(spec, p)
    before = {k: v.copy() for k, v in model.p.items()}
    rays = look_at_rays(16, spec, seed=9)
    out, _ = model.train_step(rays, np.zeros((16, 4), np.float32), 64, default_scalars(do_train=0))
    for k, v in before.items():
        assert np.array_equal(v, model.p[k]), k
    assert np.all(out[:, 3] == 0.0)
    out_t, _ = model.train_step(rays, np.zeros((16, 4), np.float32), 64, default_scalars(do_train=1))
    assert np.all(out_t[:, 3] == 4.0)


def _shell_bits(R, seed=0, frac=0.2):
    rng = np.random.default_rng(seed)
    c = (np.arange(R) + 0.5) / R
    z, y, x = np.meshgrid(c, c, c, indexing="ij")
    rad = np.sqrt((x - 0.5) ** 2 + (y - 0.5) ** 2 + (z - 0.5) ** 2)
    occ = (np.abs(rad - 0.3) <= 0.08) | (rng.random((R, R, R)) < frac)
    idx = np.nonzero(occ.reshape(-1))[0]
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits


@pytest.mark.parametrize("T_stop", [0.0, 1e-2])
def test_marched_step_is_the_composition_of_pinned_parts(ora, T_stop):
    """ora_train_step_marched is the march (ora_march_ray), the encoding at the marched positions
    (ora_hash_encode), the reference MLP (torch float64), the marched compositing and its backward
    (ora_composite_marched, pinned against autograd in test_oracle_march) and the reference backward from the
    output deltas with dt = the march step and t = the sample time (autograd of the surrogate, as for the
    resampled step), then the scatter of dL/da0 (ora_hash_backward)."""
    spec = spec_cfg0(hash_opt=1, occ_G=16)
    p = random_params(spec, seed=21)
    p["bd_out"][0] = 8.0
    model = ora.OracleModel(spec, {k: v.copy() for k, v in p.items()})
    rays = look_at_rays(40, spec, seed=22, miss_frac=0.1)
    tg = sphere_targets(rays, spec)
    R = 32
    bits = _shell_bits(R, seed=23)
    dt = np.float32(np.sqrt(3.0) / 128)
    m = ora.march_cfg(R, dt, 128, T_stop=T_stop)
    sc = default_scalars(occ_strength=0.0)
    out, used, taps = model.train_step_marched(rays, tg, bits, m, sc)
    # the march and the encodings
    ts = [ora.march_ray(model.cfg, m, bits, r) for r in rays]
    counts = np.array([t.size for t in ts])
    assert counts.sum() == taps["Ts"].size and counts.sum() > 500
    np.testing.assert_array_equal(taps["Ts"], np.concatenate(ts))
    x = np.concatenate([(r[None, :3] + t[:, None] * r[None, 4:7]).astype(np.float32) for r, t in zip(rays, ts)])
    a0 = ora.hash_encode(model.cfg, p["table"], x)
    np.testing.assert_array_equal(taps["a0"].view(np.uint32), a0.view(np.uint32))
    # the MLP outputs
    dirs = np.repeat(rays[:, 4:7], counts, axis=0)
    t, xa, dout, cout = _torch_mlp(spec, p, a0, dirs, sc["sh_multiplier"])
    sig_ref = np.log1p(np.exp(np.clip(dout[:, 0].detach().numpy(), -10, 10)))
    rgb_ref = 1 / (1 + np.exp(-np.clip(0.5 * cout.detach().numpy(), -18, 18)))
    assert np.allclose(taps["sigma"], sig_ref, rtol=1e-5, atol=1e-6)
    assert np.allclose(taps["rgb"], rgb_ref, rtol=1e-5, atol=1e-6)
    # per ray: compositing and its backward are ora_composite_marched on those outputs
    regu = np.float32(5e-3) * dt / np.float32(128)
    off = np.concatenate([[0], np.cumsum(counts)])
    for r in range(rays.shape[0]):
        sl = slice(off[r], off[r + 1])
        u, Tr, dLds, dLdc, Cf, T_end = ora.composite_marched(taps["sigma"][sl], taps["rgb"][sl], dt, m.T_stop,
                                                             np.zeros(3, np.float32), tg[r, :3], regu)
        assert u == used[r]
        np.testing.assert_array_equal(taps["dL_dsigma"][sl], dLds)
        np.testing.assert_array_equal(taps["dL_dc"][sl], dLdc)
        np.testing.assert_array_equal(out[r, :3], np.clip(Cf, 0, 1))
        assert out[r, 3] == 4.0
    if T_stop > 0:
        assert (used < counts).sum() >= 3  # some rays stop early
    else:
        np.testing.assert_array_equal(used, counts)
    # the backward from the output deltas (dt = the march step, t = the sample time)
    Ts = taps["Ts"].astype(np.float64)
    DT = float(dt)
    D = 0.5 * np.sqrt(3.0)
    num = Ts * Ts + Ts * DT + DT * DT / 3
    den = D * D + D * DT + DT * DT / 3
    xg = Ts / D
    fvol = np.where(xg >= 1, 1.0, np.power(np.maximum(xg, 1e-12), 0.2)) * num / den
    d_cout = fvol[:, None] * taps["dL_dc"] * rgb_ref * (1 - rgb_ref) * 0.5
    z = np.clip(dout[:, 0].detach().numpy(), -18, 18)
    d_dout0 = fvol * taps["dL_dsigma"] / (1 + np.exp(-z))
    ((torch.tensor(d_cout) * cout).sum() + (torch.tensor(d_dout0) * dout[:, 0]).sum()).backward()
    for wn in layer_shapes(spec):
        bn = BIASES[LAYERS.index(wn)]
        gw, gb = t[wn].grad.numpy(), t[bn].grad.numpy()
        assert np.abs(taps["g" + wn] - gw).max() <= 2e-4 * (np.abs(gw).max() + 1e-30), wn
        assert np.abs(taps["g" + bn] - gb).max() <= 2e-4 * (np.abs(gb).max() + 1e-30), bn
    gx = xa.grad.numpy()
    assert np.abs(taps["dL_da0"] - gx).max() <= 2e-4 * (np.abs(gx).max() + 1e-30)
    g_scatter = ora.hash_backward(model.cfg, x, taps["dL_da0"], table_floats(spec))
    assert np.allclose(taps["g_table"], g_scatter, rtol=1e-5, atol=1e-9 * np.abs(g_scatter).max())


@pytest.mark.parametrize("hash_opt", [1, 0])
def test_fp16_table_step_reduces_to_the_fp32_step(ora, hash_opt):
    """A binary16 table holds values that float32 represents exactly, so the fp16-table step computes every
    encoding, MLP output and gradient exactly as the fp32 step does on the same values; only the table's
    update differs: Adam (fp32 moments) rounds the fp32 step's result to binary16 once, and the reference SGD
    rounds the table plus the entry's summed update once (the fp32 step adds the contributions one by
    one).  The binary16 rounding itself is pinned against numpy (test_binary16_rounding_matches_numpy)."""
    spec32 = spec_cfg0(hash_opt=hash_opt)
    spec16 = spec_cfg0(hash_opt=hash_opt, table_dtype="fp16")
    p = random_params(spec32, seed=31)
    p["table"] = p["table"].astype(np.float16).astype(np.float32)
    rays = look_at_rays(24, spec32, seed=32, miss_frac=0.15)
    tg = sphere_targets(rays, spec32)
    sc = default_scalars(occ_strength=0.0)
    m32 = ora.OracleModel(spec32, {k: v.copy() for k, v in p.items()})
    m16 = ora.OracleModel(spec16, {k: v.copy() for k, v in p.items()})
    out32, t32 = m32.train_step(rays, tg, 16, sc, taps=True)
    out16, t16 = m16.train_step(rays, tg, 16, sc, taps=True)
    np.testing.assert_array_equal(out32, out16)
    for k in ("a0", "sigma", "rgb", "dL_dsigma", "dL_dc", "dL_da0"):
        np.testing.assert_array_equal(t32[k], t16[k], err_msg=k)
    for k in p:
        if k in ("table", "m_table", "v_table"):
            continue
        np.testing.assert_array_equal(m32.p[k], m16.p[k], err_msg=k)
    if hash_opt == 1:
        np.testing.assert_array_equal(m16.p["m_table"], m32.p["m_table"])
        np.testing.assert_array_equal(m16.p["v_table"], m32.p["v_table"])
        np.testing.assert_array_equal(m16.p["table"], m32.p["table"].astype(np.float16).astype(np.float32))
    else:
        L, F = spec32["n_levels"], spec32["f_per_level"]
        scale = np.array(ora.lvl_lr_scale(L), np.float32)
        g = t32["dL_da0"].reshape(-1, L, F) * (-np.float32(sc["lr"]) * scale[None, :, None] * 0.5)
        Ts = t32["Ts"].reshape(-1, 16)
        x_s = (rays[:, None, :3] + Ts[..., None] * rays[:, None, 4:7]).reshape(-1, 3).astype(np.float32)
        upd = ora.hash_backward(m32.cfg, x_s, g.reshape(-1, L * F).astype(np.float32), table_floats(spec32))
        exp = (p["table"].astype(np.float64) + upd).astype(np.float32)
        # float64 sum, one rounding to float32, then to binary16: within one binary16 ulp of the exact rounding
        got, ref = m16.p["table"], exp.astype(np.float16).astype(np.float32)
        ulp16 = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
        assert np.all(np.abs(got - ref) <= ulp16), np.abs(got - ref).max()
        assert np.mean(got == ref) > 0.999
