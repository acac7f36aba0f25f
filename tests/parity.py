"""One training step of libffnerf_hip.so compared with the CPU restatement
(oracle/) from the same state, for the GPU parity tests.

What is compared, and how every difference is accounted for:
- bit-exact: sample times, dt, run flags, hash encodings, occ_in;
- ReLU branches: the restatement takes every hidden unit's branch from the
  GPU's ReLU tap (``relu_in``) and reports its own sign of the same
  pre-activation.  Units whose branch differs ("flips") are counted, and each
  must lie within rounding of zero: |pre-activation| <= ``flip_z`` of the
  layer's largest.  With the branches matched, the remaining differences are
  rounding, held to the path's tolerance everywhere (no per-sample allowance);
- occupancy proposals: the restatement's proposal pass fed with the GPU's own
  transmittances (``Tr``, ``T_final`` taps) must reproduce the GPU's occ_st
  word for word.  (Fed with its own transmittances, which differ by rounding,
  a proposal whose stochastic threshold falls between the two values may
  differ; those words are counted and reported);
- Adam: the GPU's updated parameter, m and v are Adam of the GPU's own summed
  gradient bit for bit (``ora.adam`` on the tapped gradient).  Against the
  restatement's parameters, the entries whose update differs by more than
  the path's tolerance are counted and bounded in number (0.1 % of a layer,
  at least 4 entries, on the fp32 path; 10 % on the fp16 path), each is at
  most two Adam steps, and
  each has a gradient within the layer's gradient tolerance (a gradient
  within rounding of zero, where Adam's step is sign-like, or a cancelling
  first moment);
- reference SGD on the table: every entry within the tolerance of the largest
  update, plus the rounding of the restatement's one-at-a-time adds (n/2 + 1
  ulps for n contributions);
- binary16 tables (table_dtype fp16): both sides widen the stored values
  exactly, so the encodings stay bit-exact; each entry's update is rounded to
  nearest even once per step on both sides (Adam of the GPU's own gradient
  bit for bit after that rounding; SGD within one binary16 ulp).
"""
from __future__ import annotations

import numpy as np

from common import BIASES, LAYERS, layer_shapes

# tolerances per MLP path (fp32 MFMA; fp16/bf16 MFMA).  The counted allowances (ReLU flips, Adam updates
# outside the tolerance) sit 5-10x above the largest counts the GPU suite produces (fp32: at most 1.7e-6 of
# the units flip, at most 2e-6 of a table's entries or one entry of an MLP layer move apart; fp16: 9.3e-5 of
# the units with |pre-activation| <= 3.3e-4 of the layer's largest, 4.8 % of a layer's entries); the kernels
# are deterministic, so the suite reproduces those counts exactly
TOL = {
    0: dict(fwd=1e-4, out=1e-4, loss=1e-3, grad=1e-3, table=1e-3, flip_z=1e-5, flip_frac=2e-5, undet_frac=1e-3),
    1: dict(fwd=1e-2, out=1e-2, loss=1e-2, grad=1e-2, table=1e-2, flip_z=3e-3, flip_frac=1e-3, undet_frac=0.10),
}


def _maxrel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / (np.abs(b).max() + 1e-30))


def _normrel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))


def unpack_relu(words: np.ndarray) -> np.ndarray:
    """[N][14] u32 ReLU words -> bool [N][7][64] (hidden layer h, unit n)."""
    w = np.ascontiguousarray(words, np.uint32).reshape(-1, 14)
    bits = np.unpackbits(w.view(np.uint8), axis=1, bitorder="little")
    return bits.reshape(-1, 7, 64).astype(bool)


def hidden_layers(spec):
    return list(range(int(spec["nd"]))) + [3 + i for i in range(int(spec["nc"]))]


def _check_relu(spec, G, O, tol, stats):
    flips = unpack_relu(G["relu"] ^ O["relu_out"])
    pre = O["preact"]
    hl = hidden_layers(spec)
    units = pre.shape[0] * len(hl) * 64
    n = int(flips.sum())
    zrel = 0.0
    for h in hl:
        f = flips[:, h, :]
        if f.any():
            zrel = max(zrel, float(np.abs(pre[:, h, :][f]).max() / (np.abs(pre[:, h, :]).max() + 1e-30)))
    unused = [h for h in range(7) if h not in hl]
    assert not flips[:, unused, :].any()
    stats["relu_flips"] = n
    stats["relu_units"] = units
    stats["flip_z_max"] = zrel
    assert n <= tol["flip_frac"] * units, (n, units)
    assert zrel <= tol["flip_z"], zrel


def _check_adam(name, p0, m0, v0, g_gpu, g_ora, st_g, st_o, lr, sc, tol, frac, ora, stats, f16=False):
    """p, m, v of the GPU = Adam(p0, m0, v0, g_gpu) exactly; against the restatement by count and size."""
    mk, vk = ("m_" + name, "v_" + name) if name == "table" else ("m" + name, "v" + name)
    pe, me, ve = p0.copy(), m0.copy(), v0.copy()
    ora.adam(pe, me, ve, np.ascontiguousarray(g_gpu, np.float32), lr, sc["beta1"], sc["beta2"], sc["eps"])
    if f16:  # a binary16 table takes the update rounded to nearest even
        pe = pe.astype(np.float16).astype(np.float32)
    assert np.array_equal(st_g[name].view(np.uint32), pe.view(np.uint32)), name
    assert np.array_equal(st_g[mk].view(np.uint32), me.view(np.uint32)), name
    assert np.array_equal(st_g[vk].view(np.uint32), ve.view(np.uint32)), name
    g_gpu = np.asarray(g_gpu, np.float64).ravel()
    g_ora = np.asarray(g_ora, np.float64).ravel()
    d_g = (st_g[name].astype(np.float64) - p0).ravel()
    d_o = (st_o[name].astype(np.float64) - p0).ravel()
    ulp = np.spacing(np.abs(st_o[name]).astype(np.float16 if f16 else np.float32)).astype(np.float64).ravel()
    err = np.abs(d_g - d_o)
    out = err > tol * np.abs(d_o) + 4.0 * ulp  # updates that differ by more than the path's tolerance
    n_out = int(out.sum())
    stats.setdefault("adam_outliers", {})[name] = (n_out, g_gpu.size)
    assert n_out <= max(4, frac * g_gpu.size), (name, n_out, g_gpu.size)
    if n_out:
        # Adam is exact (above), so an update moves only with its gradient: each outlier's gradient is within
        # the layer's gradient tolerance (an entry whose gradient is within rounding of zero, where Adam's
        # first step is sign-like, or whose first moment cancels), and no outlier exceeds two Adam steps
        assert (np.abs(g_gpu - g_ora) <= tol * np.abs(g_ora).max())[out].all(), name
        step_max = max(np.abs(d_o).max(), np.abs(d_g).max())
        assert err[out].max() <= 2.0 * step_max + 4.0 * ulp[out].max(), name


def compare_step(spec, p, rays, tg, S, sc, gh, ora, check_params=True):
    """Run one step on the GPU and on the restatement from state p; check as described in the module
    docstring.  Returns (gpu model, oracle model, stats)."""
    prec = int(spec.get("mlp_precision", 0))
    tol = TOL[prec]
    f16 = spec.get("table_dtype", 0) in (1, "fp16")
    if f16:
        assert np.array_equal(p["table"], p["table"].astype(np.float16).astype(np.float32)), "table not binary16"
    m = gh.GpuModel(spec, p)
    o = ora.OracleModel(spec, {k: v.copy() for k, v in p.items()})
    out_g, G = m.train_step(rays, tg, S, sc, taps=True)
    out_o, O = o.train_step(rays, tg, S, sc, taps=True, relu_in=G["relu"], C_in=G["C"])
    stats = {}
    # sampling and encoding: bit-exact whatever the MLP precision
    assert np.array_equal(G["Ts"], O["Ts"])
    assert np.array_equal(G["DTs"], O["DTs"])
    assert np.array_equal(G["flags"], O["flags"])
    assert np.array_equal(G["a0"].view(np.uint32), O["a0"].view(np.uint32))
    _check_relu(spec, G, O, tol, stats)
    # forward and compositing
    for k in ("sigma", "rgb", "Tr", "T_final"):
        stats[k] = _maxrel(G[k], O[k])
        assert stats[k] <= tol["fwd"], (k, stats[k])
    stats["out"] = float(np.abs(out_g - out_o).max())
    assert stats["out"] <= tol["out"], stats["out"]
    stats["C"] = float(np.abs(G["C"] - O["C"]).max())
    assert stats["C"] <= tol["out"], stats["C"]
    train = bool(sc.get("do_train", 1))
    if not train:
        return m, o, stats
    _check_grads(spec, G, O, tol, stats)
    st_g, st_o = m.state(), o.p
    # occupancy: proposals from the GPU's own compositing reproduce its grid word for word
    assert np.array_equal(st_g["occ_in"], p["occ_in"])
    if sc["occ_strength"] > 0.0:
        occ = p["occ_st"].copy()
        ora.occ_propose(o.cfg, rays, S, sc["rng_seed"], G["Ts"], G["DTs"], G["Tr"], G["T_final"], G["flags"],
                        p["occ_in"], occ)
        assert np.array_equal(st_g["occ_st"], occ)
        stats["occ_raised"] = int((occ != p["occ_st"]).sum())
        stats["occ_differ_own_tr"] = int((st_o["occ_st"] != st_g["occ_st"]).sum())
    else:
        assert np.array_equal(st_g["occ_st"], p["occ_st"])
    if not check_params:
        return m, o, stats
    x = (rays[:, None, :3] + G["Ts"].reshape(-1, S)[:, :, None] * rays[:, None, 4:7]).astype(np.float32)
    _check_params(spec, p, G, O, st_g, st_o, sc, tol, ora, o.cfg, x.reshape(-1, 3), stats)
    return m, o, stats


def _check_grads(spec, G, O, tol, stats):
    """Loss and encoding gradients of every sample; the summed weight and table gradients."""
    for k in ("dL_dsigma", "dL_dc", "dL_da0"):
        stats[k] = _maxrel(G[k], O[k])
        assert stats[k] <= tol["loss"], (k, stats[k])
    for wn in layer_shapes(spec):
        bn = BIASES[LAYERS.index(wn)]
        for k in (wn, bn):
            stats["g" + k] = _normrel(G["g" + k], O["g" + k])
            assert stats["g" + k] <= tol["grad"], (k, stats["g" + k])
    if int(spec.get("hash_opt", 0)) == 1:
        stats["g_table"] = _maxrel(G["g_table"], O["g_table"])
        assert stats["g_table"] <= tol["table"], stats["g_table"]


def _check_params(spec, p, G, O, st_g, st_o, sc, tol, ora, cfg, x, stats):
    """The updated parameters from state p: Adam on the MLP (colour layers at lr_t * color_rel_lr, as
    float32) and on the table, or the reference SGD on the table.  x [n, 3]: the step's sample positions."""
    f16 = spec.get("table_dtype", 0) in (1, "fp16")
    lr_t = np.float32(sc["lr_t"])
    for wn in layer_shapes(spec):
        bn = BIASES[LAYERS.index(wn)]
        lr = float(lr_t * np.float32(sc["color_rel_lr"])) if LAYERS.index(wn) >= 4 else float(lr_t)
        for k in (wn, bn):
            _check_adam(k, p[k], p["m" + k], p["v" + k], G["g" + k], O["g" + k], st_g, st_o, lr, sc, tol["grad"],
                        tol["undet_frac"], ora, stats)
    if int(spec.get("hash_opt", 0)) == 1:
        _check_adam("table", p["table"], p["m_table"], p["v_table"], G["g_table"], O["g_table"], st_g, st_o,
                    float(lr_t), sc, tol["table"], tol["undet_frac"], ora, stats, f16=f16)
        return
    # reference SGD: the update is linear in the gradient.  The restatement adds every (sample, corner)
    # contribution to the float table one at a time, as the reference's atomics do, rounding each time at the
    # entry's magnitude; the GPU adds each entry's exact sum once.  An entry with n contributions may so differ
    # by n/2 + 1 ulps beyond the gradient tolerance.
    d_g = st_g["table"].astype(np.float64) - p["table"]
    d_o = st_o["table"].astype(np.float64) - p["table"]
    big = np.maximum(np.abs(p["table"]), np.abs(st_o["table"])).astype(np.float32)
    ulp = np.spacing(big).astype(np.float64)
    err = np.abs(d_g - d_o)
    stats["table_sgd"] = float(err.max() / (np.abs(d_o).max() + 1e-30))
    if f16:  # both add each entry's summed update once, rounding to binary16: one ulp of binary16 apart
        lim = tol["table"] * np.abs(d_o).max() + np.spacing(big.astype(np.float16)).astype(np.float64)
    else:
        _, idx, _ = ora.hash_encode(cfg, p["table"], x, with_idx=True)
        F = int(spec["f_per_level"])
        n_per_entry = np.bincount((idx.ravel() // F).astype(np.int64), minlength=p["table"].size // F)
        n_contrib = np.repeat(n_per_entry, F).astype(np.float64)
        lim = tol["table"] * np.abs(d_o).max() + (0.5 * n_contrib + 2.0) * ulp
    assert (err <= lim).all(), stats["table_sgd"]


def compare_marched_step(spec, p, rays, tg, bits, mp, sc, gh, ora, flip_frac=0.01):
    """One marched training step (ffn_train_step_marched against ora_train_step_marched) from state p, checked
    as compare_step checks the resampled step.  The march is bit-exact (sample times, samples per ray), and so
    are the encodings; the restatement takes the GPU's ReLU branches, loss colours and samples composited per
    ray.  Rays whose termination differs from the restatement's own run are counted (at most flip_frac of the
    rays), and each stops where T lies within rounding of T_stop.  With occ_strength > 0 the proposals of the
    marched runs, restated from the GPU's own transmittances, must reproduce its occ_st word for word;
    otherwise both grids stay as they were."""
    prec = int(spec.get("mlp_precision", 0))
    tol = TOL[prec]
    m = gh.GpuModel(spec, p)
    out_g, used_g, G = m.train_step_marched(rays, tg, bits, mp, sc)
    mcfg = ora.march_cfg(mp.res, mp.dt, mp.max_steps, T_stop=mp.T_stop, sh_multiplier=mp.sh_multiplier)
    free = ora.OracleModel(spec, {k: v.copy() for k, v in p.items()})
    _, used_free, F = free.train_step_marched(rays, tg, bits, mcfg, sc)
    o = ora.OracleModel(spec, {k: v.copy() for k, v in p.items()})
    out_o, used_o, O = o.train_step_marched(rays, tg, bits, mcfg, sc, relu_in=G["relu"], C_in=G["C"],
                                            used_in=used_g)
    stats = {"samples": int(G["Ts"].size), "composited": int(used_g.sum())}
    assert np.array_equal(G["Ts"], O["Ts"])
    assert np.array_equal(used_o, used_g)
    assert np.array_equal(G["a0"].view(np.uint32), O["a0"].view(np.uint32))
    flips = np.flatnonzero(used_g != used_free)
    stats["termination_flips"] = int(flips.size)
    assert flips.size <= max(2, flip_frac * rays.shape[0]), flips.size
    assert mp.T_stop > 0.0 or flips.size == 0
    off = np.concatenate([[0], np.cumsum(G["n_march"])]).astype(np.int64)
    for r in flips:
        k = int(min(used_g[r], used_free[r]))  # the earlier stop: T after its last sample straddles T_stop
        T_after = F["Tr"][off[r] + k] if k < G["n_march"][r] else F["T_final"][r]
        # T is a product of up to max_steps factors, each carrying the forward tolerance of sigma
        assert abs(T_after / mp.T_stop - 1.0) <= 50.0 * tol["fwd"], (r, T_after)
    _check_relu(spec, G, O, tol, stats)
    for k in ("sigma", "rgb", "Tr", "T_final"):
        stats[k] = _maxrel(G[k], O[k])
        assert stats[k] <= tol["fwd"], (k, stats[k])
    stats["out"] = float(np.abs(out_g - out_o).max())
    assert stats["out"] <= tol["out"], stats["out"]
    stats["C"] = float(np.abs(G["C"] - O["C"]).max())
    assert stats["C"] <= tol["out"], stats["C"]
    _check_grads(spec, G, O, tol, stats)
    st_g, st_o = m.state(), o.p
    assert np.array_equal(st_g["occ_in"], p["occ_in"])
    if sc["occ_strength"] > 0.0:
        # the restatement's proposal pass over the marched runs, fed the GPU's own transmittances, reproduces
        # the GPU's grid word for word
        occ = p["occ_st"].copy()
        ora.occ_propose_marched(o.cfg, rays, G["n_march"], sc["rng_seed"], G["Ts"], G["Tr"], G["T_final"],
                                p["occ_in"], occ)
        assert np.array_equal(st_g["occ_st"], occ)
        stats["occ_raised"] = int((occ != p["occ_st"]).sum())
        stats["occ_differ_own_tr"] = int((st_o["occ_st"] != st_g["occ_st"]).sum())
    else:
        assert np.array_equal(st_g["occ_st"], p["occ_st"])
    _check_params(spec, p, G, O, st_g, st_o, sc, tol, ora, o.cfg, G["x"], stats)
    return m, o, stats
