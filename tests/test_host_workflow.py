"""CPU checks of the host workflow: the scene config, the BA-archive reader and
image geometry (the reference's tests/test_scene_workflow.py:1-80 restated on
this package, with PNGs written by the package's own codec), the schedules,
the loss log and the command line's checks.  No GPU needed."""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

import ffnerf_cli
import ffnerf_tools as ft
import png_io
import synthetic_scene as sc
import trainer
from scene_config import load_config
from sfm_data import area_resize, load_images, read_scene, scaled_intrinsics, scene_bounds


@pytest.fixture
def scene(tmp_path):
    for i in range(2):
        png_io.write_png(tmp_path / f"{i}.png", np.full((80, 40, 3), 80 + i, np.uint8))
    K = np.array([[40, 0, 10], [0, 40, 20], [0, 0, 1]], np.float32)
    poses = np.tile(np.eye(4), (2, 1, 1))
    poses[1, :3, 3] = [1, 2, 3]
    data = {"reconstruction": str(tmp_path / "scene.npz"), "images_dir": str(tmp_path), "sfm_max_side": 40,
            "max_side": 20}

    def save(**kw):
        np.savez(data["reconstruction"], K=K, img_paths=np.array(["old/place/0.png", "old/place/1.png"]), **kw)

    return dict(root=tmp_path, K=K, poses=poses, data=data, save=save)


def test_ba_w2c_and_relocated_images(scene):
    scene["save"](RT=np.linalg.inv(scene["poses"]), rt_dir=np.array(["w2c"]), active_cam_global=[8, 12])
    paths, poses, K, ids, points = read_scene(scene["data"])
    np.testing.assert_allclose(poses, scene["poses"], atol=1e-6)
    assert ids.tolist() == [8, 12]
    images, K2, wh = load_images(scene["data"], paths, K)
    assert images.shape == (2, 20, 10, 3)
    np.testing.assert_allclose(K2[:2], scene["K"][:2] / 2)
    np.testing.assert_allclose(images[1], (81 / 255.0), rtol=1e-6)


def test_stage2_filters_before_loading_images(scene):
    scene["save"](c2w=scene["poses"], posed=[True, True], keep_mask=[False, True],
                  X_track=[[1, 2, 3], [9, 9, 9]], has_X=[True, False])
    sel = scene["root"] / "selected"
    sel.mkdir()
    png_io.write_png(sel / "1.png", np.zeros((80, 40, 3), np.uint8))
    scene["data"]["images_dir"] = str(sel)
    paths, poses, K, ids, points = read_scene(scene["data"])
    assert ids.tolist() == [1]
    np.testing.assert_allclose(points, [[1, 2, 3]])
    assert len(paths) == 1


def test_object_arrays_are_refused_not_unpickled(scene):
    np.savez(scene["data"]["reconstruction"], K=scene["K"], c2w=scene["poses"],
             img_paths=np.array(["0.png", "1.png"], dtype=object))
    with pytest.raises(ValueError, match="unpickling"):
        read_scene(scene["data"])


def test_geometry_and_bounds(scene):
    K = scene["K"]
    np.testing.assert_allclose(scaled_intrinsics(K, (40, 80), (20, 40), 40), K)
    with pytest.raises(ValueError):
        scene_bounds({"box_min": [1, 0, 0], "box_max": [0, 1, 1]}, np.empty((0, 3)))
    lo, hi = scene_bounds({"box_min": None, "box_max": None}, np.array([[1, 2, 3]]))
    assert np.all(hi > lo)
    points = np.array([[0, 0, 0], [2, 4, 6], [1, 2, 3]], np.float32)
    q_lo, q_hi = np.percentile(points, [1, 99], axis=0)
    center = 0.5 * (q_lo + q_hi)
    radius = max(0.5 * np.linalg.norm(q_hi - q_lo), 0.01) * 1.5
    lo, hi = scene_bounds({"box_min": None, "box_max": None}, points)
    np.testing.assert_allclose((lo + hi) * 0.5, center, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose((hi - lo) * 0.5, np.full(3, radius), rtol=1e-6, atol=1e-6)


def test_review_rays_match_training_intrinsics(scene):
    images = np.zeros((2, 80, 40, 3), np.float32)
    u, v = np.array([0, 19, 39]), np.array([0, 29, 79])
    training, _ = ft.rays_targets_from_indices(np.ones(3, np.int32), u, v, images, scene["poses"], 40, 80,
                                               K=scene["K"])
    review = ft.rays_from_rt_indices(scene["poses"][1], u, v, 40, 80, K=scene["K"])
    np.testing.assert_allclose(training["o"], review["o"])
    np.testing.assert_allclose(training["d"], review["d"], atol=1e-7)


def test_config_paths_and_unknown_keys(tmp_path):
    path = tmp_path / "scene.json"
    path.write_text(json.dumps({"data": {"reconstruction": "scene.npz"}}))
    assert load_config(path)["data"]["reconstruction"] == str(tmp_path / "scene.npz")
    for bad in ({"training": {"stepz": 10}}, {"trainin": {}}, {"data": {"reconstruction": "x", "max_side": -1}},
                {"data": {"reconstruction": "x"}, "training": {"samples_per_ray": 128}},
                {"data": {"reconstruction": "x"}, "training": {"model_id": "a b"}},
                {"data": {"reconstruction": "x"}, "model": {"hash_opt": "rmsprop"}}):
        path.write_text(json.dumps(bad))
        with pytest.raises(ValueError):
            load_config(path)


def test_area_resize_is_a_box_filter():
    rng = np.random.default_rng(0)
    img = rng.random((12, 18, 3)).astype(np.float32)
    half = area_resize(img, (9, 6))
    np.testing.assert_allclose(half, img.reshape(6, 2, 9, 2, 3).mean(axis=(1, 3)), rtol=1e-6)
    odd = area_resize(img, (7, 5))  # non-integer factors: a convex combination, so constants stay constant
    np.testing.assert_allclose(area_resize(np.full((12, 18, 3), 0.3, np.float32), (7, 5)), 0.3, rtol=1e-6)
    assert odd.shape == (5, 7, 3) and np.all(odd >= img.min()) and np.all(odd <= img.max())
    np.testing.assert_allclose(odd.mean(axis=(0, 1)), img.mean(axis=(0, 1)), rtol=1e-5)


def test_schedules_closed_form():
    B, S, lr, lmd = 512, 64, 1e-4, 1e-4
    n = B * S
    for step in (0, 1, 1000, 50000):
        want = max(lr * np.sqrt(65536 / n) * np.exp(-lmd * np.sqrt(n / 65536) * step), 5e-6)
        assert trainer.lr_schedule(step, lr, lmd, B, S) == np.float32(want)
    assert trainer.lr_schedule(10 ** 9, lr, lmd, B, S) == np.float32(5e-6)
    assert [trainer.sh_multiplier(s) for s in (0, 3000, 3750, 4500, 9000)] == [0.0, 0.0, 0.5, 1.0, 1.0]
    assert [trainer.occ_multiplier(s) for s in (1500, 1501)] == [0.0, 1.0]
    assert [trainer.color_rel_lr(s) for s in (0, 1500, 2250, 3000)] == [0.15, 0.15, 0.15 + 0.85 * 0.5, 1.0]


def test_adam_lr_t_is_the_bias_correction():
    """lr_t folds Adam's bias corrections into the step size: p - lr_t m / (sqrt(v) + eps) with the raw moments
    equals p - lr m_hat / (sqrt(v_hat) + eps_hat) with m_hat = m / (1 - b1^t), v_hat = v / (1 - b2^t) and
    eps_hat = eps / sqrt(1 - b2^t) (Kingma & Ba, section 2).  Checked by running both forms in float64 on a
    gradient sequence; lr_t itself is float32, so the two agree to float32 rounding."""
    from types import SimpleNamespace
    stub = SimpleNamespace(spec=SimpleNamespace(beta1=0.9, beta2=0.99))
    b1, b2, lr, eps = float(np.float32(0.9)), float(np.float32(0.99)), 1e-2, 1e-15
    rng = np.random.default_rng(3)
    g = rng.normal(size=(40, 5)) * np.logspace(-6, 0, 5)
    p_raw = np.zeros(5)
    p_hat = np.zeros(5)
    m = np.zeros(5)
    v = np.zeros(5)
    for t in range(1, 41):
        m = b1 * m + (1 - b1) * g[t - 1]
        v = b2 * v + (1 - b2) * g[t - 1] ** 2
        lr_t = ft.Nerf.adam_lr_t(stub, lr, t)
        assert lr_t.dtype == np.float32
        p_raw -= float(lr_t) * m / (np.sqrt(v) + eps)
        c1, c2 = 1 - b1 ** t, 1 - b2 ** t
        p_hat -= lr * (m / c1) / (np.sqrt(v / c2) + eps / np.sqrt(c2))
        # each step differs by the float32 rounding of lr_t (6e-8 of a step of at most a few lr)
        np.testing.assert_allclose(p_raw, p_hat, rtol=0, atol=1e-6 * lr * t)
    # t = 1: sqrt(1 - b2) / (1 - b1) with the float32 betas; large t: the corrections vanish
    assert abs(float(ft.Nerf.adam_lr_t(stub, lr, 1)) - lr * np.sqrt(1 - b2) / (1 - b1)) < 1e-9
    assert abs(float(ft.Nerf.adam_lr_t(stub, lr, 10 ** 5)) - lr) < 1e-8


def test_occ_decay_q24():
    """The decay factor in 24-bit fixed point: no decay at strength 0, the plain decay at strength 1, linear in
    the strength between, rounded half to even, and clamped (a strength past 1 / (1 - decay) clears)."""
    one = 1 << 24
    assert ft.occ_decay_q24(0.0, 0.95) == one
    assert ft.occ_decay_q24(1.0, 1.0) == one
    assert ft.occ_decay_q24(1.0, 0.95) == 15938355  # 0.95 * 2^24 = 15938355.2
    assert ft.occ_decay_q24(0.5, 0.95) == 16357786  # 0.975 * 2^24 = 16357785.6
    assert ft.occ_decay_q24(1.0, 0.5) == one // 2
    assert ft.occ_decay_q24(1.0, 1 - 2.5 / one) == one - 2  # 2^24 - 2.5 rounds to the even neighbour
    assert ft.occ_decay_q24(1.0, 1 - 3.5 / one) == one - 4
    assert ft.occ_decay_q24(25.0, 0.95) == 0  # 1 - 25 * 0.05 < 0
    assert ft.occ_decay_q24(-1.0, 0.95) == one  # clamped above
    for s_ in np.linspace(0.0, 1.0, 11):
        assert abs(ft.occ_decay_q24(s_, 0.9) - (1 - 0.1 * s_) * one) <= 0.5


def test_loss_log_format(tmp_path):
    path, f = trainer.open_loss_log(tmp_path, "m1")
    trainer.write_loss_row(f, 1.5, 10, 1e-3, 0.25, 0.5, 0.75, [2], 3)
    f.close()
    lines = path.read_text().splitlines()
    assert path.name.startswith("m1_loss_") and path.suffix == ".csv"
    assert lines[0] == "wall_s,step,lr_f,mse,rmse_rgb,l2mean,inflight,batch_q"
    assert lines[1].split(",")[:3] == ["1.500000", "10", "1.000e-03"]
    out = np.array([[0.5, 0.5, 0.5, 0]], np.float32)
    tg = np.array([[0.0, 0.5, 1.0, 0]], np.float32)
    mse, rmse, l2 = trainer.batch_loss(out, tg)
    assert mse == pytest.approx(0.5 / 3) and l2 == pytest.approx(np.sqrt(0.5))
    assert trainer.psnr(out, tg) == pytest.approx(-10 * np.log10(0.5 / 3))


def _synthetic_config(tmp_path, **training):
    npz = sc.write_archive(tmp_path / "scene", "cfg0")
    cfg = {"data": {"reconstruction": str(npz), "sfm_max_side": 0, "max_side": 0},
           "scene": {"box_min": [0, 0, 0], "box_max": [1, 1, 1]},
           "training": dict({"directory": str(tmp_path / "run"), "model_id": "ball", "steps": 5, "period": 5,
                             "batch_rays": 256, "lr": 0.01, "lmd": 0.0}, **training),
           "model": {"n_levels": 8, "f_per_level": 2, "log2_T": [14] * 8, "base_res": 16.0,
                     "finest_res": 16.0 * 1.5 ** 7, "nd": 1, "nc": 2, "hash_opt": "adam", "init": "xavier",
                     "beta1": 0.9, "beta2": 0.99, "eps": 1e-15, "background": "black", "schedule": "constant"}}
    path = tmp_path / "scene.json"
    path.write_text(json.dumps(cfg))
    return path


def test_synthetic_archive_reads_back(tmp_path, capsys):
    path = _synthetic_config(tmp_path)
    cfg = load_config(path)
    paths, poses, K, ids, points = read_scene(cfg["data"])
    assert len(paths) == 8 and ids.tolist() == list(range(8))
    images, K2, (W, H) = load_images(cfg["data"], paths, K)
    assert (W, H) == (64, 64)
    cams = sc.cameras_for("cfg0")
    np.testing.assert_allclose(poses, cams.c2w)
    np.testing.assert_allclose(images[3], np.round(np.clip(sc.render_image(cams, 3), 0, 1) * 255) / 255,
                               atol=1e-6)
    assert ffnerf_cli.main(["inspect", "--config", str(path)]) == 0
    out = capsys.readouterr().out
    rows = dict(ffnerf_cli.scene_report(cfg))
    assert rows["registered cameras"] == 8 and rows["training image size"] == "64x64"
    assert rows["sparse points inside box"] == "100.0%"
    assert any(line.split() == ["registered", "cameras", "8"] for line in out.splitlines())


def test_cli_checks(tmp_path):
    path = _synthetic_config(tmp_path)
    for argv in (["train", "--config", str(path), "--steps", "0"],
                 ["train", "--config", str(path), "--model-id", "bad id"]):
        with pytest.raises(SystemExit):
            ffnerf_cli.main(argv)
    run = tmp_path / "run"
    run.mkdir()
    (run / "ball_weights_20260101.npz").write_bytes(b"")
    with pytest.raises(SystemExit):  # would overwrite checkpoints without --resume
        ffnerf_cli.main(["train", "--config", str(path)])
    out = tmp_path / "exists.png"
    out.write_bytes(b"")
    with pytest.raises(SystemExit):
        ffnerf_cli.main(["snapshot", "--config", str(path), "--output", str(out)])


def test_reference_checkpoint_layout_loads(tmp_path):
    """A checkpoint in the reference's own layout (no keys of this build: reference hash layout, F = 4,
    ND = NC = 2, int32 bit patterns) is read by Nerf.load_latest's parser into the reference shape, every
    value bit for bit (the GPU test steps it)."""
    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    import reference_checkpoint as rc
    path = rc.write(tmp_path, "refckpt", seed=3)
    data = np.load(path, allow_pickle=False)
    assert "level_log2_T" not in data.files and "m_table_i" not in data.files
    nerf = ft.Nerf.__new__(ft.Nerf)  # the parser alone: no device
    nerf.training_dir, nerf.spec, nerf.occ = tmp_path, ft.ModelSpec(), ft.OccParams()
    host = nerf.load_latest("refckpt", push=False)
    assert nerf.spec.log2_T == rc.LEVEL_LOG2 and nerf.spec.f_per_level == 4
    assert (nerf.spec.nd, nerf.spec.nc, nerf.spec.hash_opt) == (2, 2, "sgd")
    assert nerf.steps_trained == 1234 and nerf.occ.G_occ == rc.G_OCC
    assert np.array_equal(host["table"].view(np.int32), data["table_i"])
    for name in [str(x) for x in data["active_params"]]:
        for pre in ("", "m", "v"):
            assert np.array_equal(host[pre + name].reshape(-1).view(np.int32), data[pre + name + "_i"]), pre + name
    assert not host["m_table"].any() and not host["v_table"].any()
    assert np.array_equal(host["occ_in"], data["occ_grid_in_u32"])


def test_jpeg_archive_reads_back(tmp_path):
    """An archive that lists JPEGs (as most SfM archives do; the reference reads them with cv2.imread): the
    images decode through Pillow to the pixels Pillow itself decodes, and a JPEG whose EXIF orientation says
    "rotate" comes back upright, as cv2.imread returns it."""
    from PIL import Image
    from sfm_data import read_rgb
    rng = np.random.default_rng(5)
    arrs = [np.clip(rng.normal(120, 40, (48, 32, 3)), 0, 255).astype(np.uint8) for _ in range(2)]
    for i, a in enumerate(arrs):
        Image.fromarray(a).save(tmp_path / f"{i}.jpg", quality=95)
    ref = [np.asarray(Image.open(tmp_path / f"{i}.jpg").convert("RGB")) for i in range(2)]
    K = np.array([[40, 0, 16], [0, 40, 24], [0, 0, 1]], np.float32)
    data = {"reconstruction": str(tmp_path / "scene.npz"), "images_dir": str(tmp_path), "sfm_max_side": 0,
            "max_side": 0}
    np.savez(data["reconstruction"], K=K, img_paths=np.array(["0.jpg", "1.jpg"]), RT=np.tile(np.eye(4), (2, 1, 1)),
             rt_dir=np.array(["c2w"]))
    paths, _, _, _, _ = read_scene(data)
    images, _, (W, H) = load_images(data, paths, K)
    assert (W, H) == (32, 48)
    for i in range(2):
        np.testing.assert_array_equal(np.round(images[i] * 255).astype(np.uint8), ref[i])
    # EXIF orientation 6 (rotate 90 degrees clockwise to view): read back 32 x 48 -> 48 rows become columns
    exif = Image.Exif()
    exif[0x0112] = 6
    Image.fromarray(arrs[0]).save(tmp_path / "rot.jpg", quality=95, exif=exif)
    assert read_rgb(tmp_path / "rot.jpg").shape == (32, 48, 3)
    (tmp_path / "bad.jpg").write_bytes(b"not an image")
    with pytest.raises(Exception):
        read_rgb(tmp_path / "bad.jpg")


def test_preview_rays_are_block_centres(tmp_path):
    """The training previews' rays (run_ffnerf_OG.py:1160-1190): preview.width x preview.height divided by
    preview.downscale, one ray through each block's centre pixel of the configured view, with the intrinsics
    scaled from the training image size to the preview size; views outside the registered cameras refused."""
    cfg = load_config(_synthetic_config(tmp_path))
    paths, poses, K, _, _ = read_scene(cfg["data"])
    cfg["preview"].update(width=40, height=24, downscale=4, views=[1, 5])
    rays, W_ds, H_ds = trainer.preview_rays(cfg, poses, K, 64, 64)
    assert (W_ds, H_ds) == (10, 6) and len(rays) == 2 and rays[0].shape == (60, 8)
    K_prev = np.asarray(K, np.float32).copy()
    K_prev[0] *= 40 / 64
    K_prev[1] *= 24 / 64
    r = 1 * 10 + 3  # block (x 3, y 1): its centre pixel (14, 6)
    want = ft.rays_as_array(ft.rays_from_rt_indices(poses[5], [3 * 4 + 2], [1 * 4 + 2], 40, 24, K=K_prev))
    np.testing.assert_array_equal(rays[1][r], want[0])
    cfg["preview"]["views"] = [8]
    with pytest.raises(ValueError, match="preview.views"):
        trainer.preview_rays(cfg, poses, K, 64, 64)


@pytest.mark.parametrize("init", ["he", "xavier"])
def test_fresh_init_follows_the_reference(init):
    """R17, a fresh model (ffnerf_tools.py:836-895 of the reference): the table ~ U(+-1e-4) drawn first from
    the seeded generator, then the active weights in kernel-argument order (He: N(0, 2 / fan_in), output
    heads of <= 16 rows N(0, 0.01); Xavier: U(+-sqrt(6 / (fan_in + fan_out)))), the density head's bias
    bd_out[0] = -2 and, under He, bc_2 ~ N(-2, 0.05); zero moments, every occupancy nibble 14 (words
    0xEEEEEEEE).  The moments are checked against the distributions' closed forms with bounds a plausible
    mistake breaks (fan_out for fan_in: the 64 x 32 colour input layer tells them apart)."""
    spec = ft.ModelSpec(n_levels=16, f_per_level=4, nd=2, nc=3, init=init)
    occ = ft.OccParams(G_occ=32)
    occ.finalize()
    p = ft.init_params(spec, occ, np.random.default_rng(7))
    n_tab = spec.table_entries() * spec.f_per_level
    np.testing.assert_array_equal(p["table"], np.random.default_rng(7).uniform(-1e-4, 1e-4, n_tab).astype(np.float32))
    shapes = spec.layer_shapes()
    assert set(shapes) == {"Wd_in", "Wd_01", "Wd_out", "Wc_in", "Wc_01", "Wc_12", "Wc_out"}
    for wn, (rows, fan_in) in shapes.items():
        w = p[wn].astype(np.float64)
        assert w.shape == (rows, fan_in)
        n = w.size
        if init == "xavier":
            lim = np.sqrt(6.0 / (rows + fan_in))
            assert np.abs(w).max() <= lim and np.abs(w).max() > 0.9 * lim, wn
            var = lim * lim / 3.0
        else:
            var = 0.01 ** 2 if rows <= 16 else 2.0 / fan_in
        sd_var = var * np.sqrt(2.0 / n) * (1.0 if init == "he" else np.sqrt(0.4))  # sd of the sample variance
        assert abs(w.var() - var) < 5.0 * sd_var, (wn, w.var(), var)
        assert abs(w.mean()) < 5.0 * np.sqrt(var / n), wn
    for bn in ("bd_0", "bd_1", "bc_0", "bc_1", "bc_out"):
        assert not p[bn].any(), bn
    assert p["bd_out"][0] == np.float32(-2.0) and not p["bd_out"][1:].any()
    if init == "he":
        b = p["bc_2"].astype(np.float64)
        assert abs(b.mean() + 2.0) < 5 * 0.05 / 8 and 0.6 * 0.05 < b.std() < 1.4 * 0.05
    else:
        assert not p["bc_2"].any()
    for k, v in p.items():
        if k[0] in "mv" and k not in ("table",):
            assert not v.any(), k
    assert (p["occ_in"] == 0xEEEEEEEE).all() and (p["occ_st"] == 0xEEEEEEEE).all()
