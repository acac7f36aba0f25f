"""GPU parity of the fp16/bf16-MFMA MLP path (mlp_precision = fp16) against the
fp32 oracle, at the 1e-2 tolerance the north star sets for that path.

Reduced precision moves hidden pre-activations that lie within ~1e-3 of zero
to the other side of their ReLU for ~1-2% of the samples; those samples'
backward (dL/da0, and through it the table gradient) then differs by a
discrete step.  The per-sample checks bound how many samples may do so and by
how much; everything else is held to 1e-2."""
import numpy as np
import pytest

from common import (BIASES, LAYERS, default_scalars, layer_shapes, look_at_rays, random_params, spec_cfg0,
                    spec_ref, sphere_targets)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gh():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a visible GPU")
    import gpu_helpers
    return gpu_helpers


def _maxrel(a, b):
    return float(np.abs(a - b).max() / (np.abs(b).max() + 1e-30))


def _normrel(a, b):
    return float(np.linalg.norm((a - b).ravel()) / (np.linalg.norm(b.ravel()) + 1e-30))


def _per_sample(a, b, tol=1e-2, frac=0.03):
    a = a.reshape(a.shape[0], -1)
    b = b.reshape(b.shape[0], -1)
    err = np.abs(a - b).max(1) / (np.abs(b).max() + 1e-30)
    assert (err > tol).mean() < frac, (err > tol).mean()
    assert np.median(err) < 1e-3, np.median(err)


def _compare16(spec, p, rays, tg, S, sc, gh, ora):
    m = gh.GpuModel(spec, p)
    o = ora.OracleModel(spec, {k: v.copy() for k, v in p.items()})
    out_g, tg_ = m.train_step(rays, tg, S, sc, taps=True)
    out_o, to_ = o.train_step(rays, tg, S, sc, taps=True)
    # sampling and encoding do not depend on the MLP precision: still bit-exact
    assert np.array_equal(tg_["Ts"], to_["Ts"])
    assert np.array_equal(tg_["a0"].view(np.uint32), to_["a0"].view(np.uint32))
    # MLP outputs and the loss
    assert _maxrel(tg_["sigma"], to_["sigma"]) < 1e-2
    assert _maxrel(tg_["rgb"], to_["rgb"]) < 1e-2
    assert _maxrel(out_g, out_o) < 1e-2
    if not sc.get("do_train", 1):
        return
    assert _maxrel(tg_["dL_dsigma"], to_["dL_dsigma"]) < 1e-2
    assert _maxrel(tg_["dL_dc"], to_["dL_dc"]) < 1e-2
    _per_sample(tg_["dL_da0"], to_["dL_da0"])
    # weight gradients sum over the samples, the ReLU-flipped ones included (normwise 0.3-1.5e-2 measured
    # over seeds); the Adam-updated parameters below are held to 1e-2
    for wn in layer_shapes(spec):
        bn = BIASES[LAYERS.index(wn)]
        assert _normrel(tg_["g" + wn], to_["g" + wn]) < 2e-2, wn
        assert _normrel(tg_["g" + bn], to_["g" + bn]) < 2e-2, bn
    if "g_table" in to_:
        assert _normrel(tg_["g_table"], to_["g_table"]) < 3e-2
    # Adam after one step: where the gradient is well determined the update matches
    sg, so = m.state(), o.p
    for k in list(layer_shapes(spec)) + ["table"]:
        g = to_["g_table"] if k == "table" else to_["g" + k]
        sel = np.abs(g) > 1e-2 * np.abs(g).max()
        d_g = sg[k].astype(np.float64) - p[k]
        d_o = so[k].astype(np.float64) - p[k]
        err = np.abs(d_g[sel] - d_o[sel])
        lim = 1e-2 * np.abs(d_o[sel]) + 1e-5 * np.abs(d_o).max()
        assert (err <= lim).mean() > 0.99, (k, (err <= lim).mean())


@pytest.mark.parametrize("S", [64, 32, 16, 8, 1])
def test_train_step_fp16_cfg0(gh, ora, S):
    print(f"[case] fp16 train step cfg0 S={S}", flush=True)
    spec = spec_cfg0(hash_opt=1, mlp_precision=1)
    p = random_params(spec, seed=161)
    rays = look_at_rays(96 * 64 // S, spec, seed=162, miss_frac=0.1)
    _compare16(spec, p, rays, sphere_targets(rays, spec), S, default_scalars(), gh, ora)


def test_train_step_fp16_reference_shape(gh, ora):
    """L=16, F=4 (LF=64), ND=NC=2, reference SGD on the table."""
    print("[case] fp16 train step reference shape", flush=True)
    spec = spec_ref(hash_opt=0, mlp_precision=1)
    p = random_params(spec, seed=171, table_scale=0.05)
    rays = look_at_rays(64, spec, seed=172, miss_frac=0.1)
    m = gh.GpuModel(spec, p)
    o = ora.OracleModel(spec, {k: v.copy() for k, v in p.items()})
    sc = default_scalars()
    out_g, tg_ = m.train_step(rays, sphere_targets(rays, spec), 64, sc, taps=True)
    out_o, to_ = o.train_step(rays, sphere_targets(rays, spec), 64, sc, taps=True)
    assert _maxrel(tg_["sigma"], to_["sigma"]) < 1e-2
    assert _maxrel(out_g, out_o) < 1e-2
    _per_sample(tg_["dL_da0"], to_["dL_da0"])
    for wn in layer_shapes(spec):
        assert _normrel(tg_["g" + wn], to_["g" + wn]) < 2e-2, wn


def test_render_fp16(gh, ora):
    print("[case] fp16 render", flush=True)
    spec = spec_cfg0(hash_opt=1, mlp_precision=1)
    p = random_params(spec, seed=181)
    rays = look_at_rays(128, spec, seed=182, miss_frac=0.1)
    _compare16(spec, p, rays, sphere_targets(rays, spec), 64, default_scalars(do_train=0, occ_strength=0.0), gh,
               ora)
