"""Training loop of the host: schedules, pixel batches, loss log, checkpoints.

Counterpart of the reference's run_ffnerf_OG.train (run_ffnerf_OG.py:974-1577)
for the training step that this package implements on the GPU.  Kept:
  * the learning-rate, SH-ramp, occupancy-ramp and colour-learning-rate
    schedules (run_ffnerf_OG.py:49-62, 1355-1365),
  * the loss CSV (name <model_id>_loss_<stamp>.csv and its header,
    run_ffnerf_OG.py:328-341), written every `period` steps from the last
    batch's rendered colours,
  * graceful Ctrl+C, checkpoints through Nerf.save (time-throttled during the
    run, unconditional at the end) and resuming with load_id.
Pixels are drawn as the reference's producer draws them (model.pixel_sampler
"adaptive", the default): the image uniformly, 20 % of the rays uniformly
within it and the rest by rejection against per-image uint8 weight maps that
every loss report updates from the batch's per-ray colour errors
(run_ffnerf_OG.py:402-686; pixel_weights.py); "uniform" draws every pixel
uniformly over all images.  The images stay resident on the GPU and every
batch's rays and targets are produced there (ffn_make_batch_weighted,
ffn_make_batch), so no per-step host work or host-to-device copy remains.
Training previews are exported as the reference exports them
(run_ffnerf_OG.py:1160-1190, 1519-1545): the configured views rendered
forward-only at preview.width x preview.height divided by preview.downscale
(block centres), side by side in <model_id>_preview_<W>p_step<step>_multiview.png,
at the first step and every preview.image_seconds.  The preview server,
viewer and review UI are not part of this build.
"""
from __future__ import annotations

import ctypes as C
import signal
import time
from datetime import datetime
from pathlib import Path

import numpy as np

import ffn_lib as fl
import ffnerf_tools as ft
import pixel_weights as pw

T_MID = 1500
LR_FLOOR = 5e-6


def lr_schedule(step: int, lr: float, lmd: float, batch_rays: int, samples_per_ray: int) -> np.float32:
    """lr_f = max(lr sqrt(65536 / N) exp(-lmd sqrt(N / 65536) step), 5e-6), N = rays x samples."""
    n = batch_rays * samples_per_ray
    lmbda = lmd * np.sqrt(n / (1024 * 64))
    return np.float32(max(lr * np.sqrt((1024 * 64) / n) * np.exp(-lmbda * step), LR_FLOOR))


def sh_multiplier(step: int) -> float:
    return float(np.clip((step - 2 * T_MID) / T_MID, 0.0, 1.0))


def occ_multiplier(step: int) -> float:
    return float(step > T_MID)


def color_rel_lr(step: int) -> float:
    return 0.15 + 0.85 * min(1.0, max(0.0, (step - T_MID) / T_MID))


def open_loss_log(training_dir: Path, model_id: str):
    training_dir = Path(training_dir)
    training_dir.mkdir(parents=True, exist_ok=True)
    stamp = datetime.now().strftime("%Y%m%d-%H%M%S")
    ms = int((time.time() * 1000) % 1000)
    path = training_dir / f"{model_id}_loss_{stamp}-{ms:03d}.csv"
    f = open(path, "a", buffering=1, encoding="utf-8")
    f.write("wall_s,step,lr_f,mse,rmse_rgb,l2mean,inflight,batch_q\n")
    return path, f


def write_loss_row(f, wall_s, step, lr_f, mse, rmse, l2mean, inflight=(0,), batch_q=0):
    f.write(f"{wall_s:.6f},{step},{lr_f:.3e},{mse:.9e},{rmse:.9e},{l2mean:.9e},"
            f"{'|'.join(str(x) for x in inflight)},{batch_q}\n")


def batch_loss(out: np.ndarray, targets: np.ndarray):
    """(mse, rmse over RGB, mean per-ray L2) of rendered vs target colours."""
    d = out[:, :3].astype(np.float64) - targets[:, :3]
    mse = float(np.mean(d * d))
    return mse, float(np.sqrt(mse)), float(np.sqrt(np.mean(np.sum(d * d, axis=1))))


def psnr(out: np.ndarray, targets: np.ndarray) -> float:
    mse = float(np.mean((out[:, :3].astype(np.float64) - targets[:, :3]) ** 2))
    return float(-10.0 * np.log10(max(mse, 1e-20)))


class DeviceImages:
    """Training images, poses and intrinsics resident on the GPU, and the on-device batch generator."""

    def __init__(self, images: np.ndarray, c2w: np.ndarray, K: np.ndarray, device="cuda"):
        import torch
        n, h, w, _ = images.shape
        self.n, self.W, self.H = n, w, h
        self.images = torch.from_numpy(np.ascontiguousarray(images, np.float32)).to(device)
        self.c2w = torch.from_numpy(np.ascontiguousarray(c2w, np.float32).reshape(n, 16)).to(device)
        self.K = torch.from_numpy(np.ascontiguousarray(K, np.float32).reshape(9)).to(device)
        self.lib = fl.load()

    def make_batch(self, io: ft.RayBatch, seed: int, stream=None):
        fl.check(self.lib.ffn_make_batch(fl.ptr(self.images), self.n, self.W, self.H, fl.ptr(self.c2w),
                                         fl.ptr(self.K), io.num_rays, int(seed) & 0xFFFFFFFF, fl.ptr(io.rays_buf),
                                         fl.ptr(io.targets_buf), None, fl.stream_ptr(stream)), "ffn_make_batch")


def model_spec(cfg: dict) -> ft.ModelSpec:
    m = cfg["model"]
    L = int(m["n_levels"])
    log2_T = m["log2_T"] if m["log2_T"] is not None else None
    if log2_T is None:
        log2_T = list(ft.REF_LEVEL_LOG2) if L == 16 else [19] * L
    return ft.ModelSpec(n_levels=L, f_per_level=int(m["f_per_level"]), log2_T=[int(v) for v in log2_T],
                        res=ft.level_resolutions(L, float(m["base_res"]), finest=float(m["finest_res"])),
                        nd=int(m["nd"]), nc=int(m["nc"]), background=m["background"], hash_opt=m["hash_opt"],
                        mlp_precision=m["mlp_precision"], init=m["init"], beta1=float(m["beta1"]),
                        beta2=float(m["beta2"]), eps=float(m["eps"]))


def occ_params(cfg: dict, box_min, box_max) -> ft.OccParams:
    m, t = cfg["model"], cfg["training"]
    ext = float(np.max(np.asarray(box_max) - np.asarray(box_min)))
    S = int(t["samples_per_ray"])
    return ft.OccParams(G_occ=int(m["occ_G"]), box_min=np.asarray(box_min, np.float32),
                        box_max=np.asarray(box_max, np.float32), rho_min=1.0, rho_max=16.0,
                        dt_min=np.float32(ext / 8192), dt_max=np.float32(12.8 / S / 6 * ext),
                        t_near_clip=float(cfg["scene"]["near"]), t_far_clip=1.0e9, occ_update_strength0=1.0,
                        decay=float(m["occ_decay"]), maintenance_period=int(m["occ_period"]))


def preview_rays(cfg: dict, poses: np.ndarray, K: np.ndarray, W: int, H: int):
    """Rays of the preview views (run_ffnerf_OG.py:1160-1190): each registered camera of preview.views seen
    at preview.width x preview.height (K scaled to that size), one ray per block of preview.downscale^2
    pixels through the block's centre.  Returns ([rays [W_ds * H_ds, 8] per view], W_ds, H_ds)."""
    p = cfg["preview"]
    W_prev, H_prev, down = int(p["width"]), int(p["height"]), int(p["downscale"])
    views = p["views"]
    if any(type(i) is not int or i < 0 or i >= len(poses) for i in views):
        raise ValueError("preview.views must contain valid registered-camera indices")
    K_prev = np.asarray(K, np.float32).copy()
    K_prev[0] *= W_prev / W
    K_prev[1] *= H_prev / H
    W_ds, H_ds = W_prev // down, H_prev // down
    idx = np.clip(np.tile(np.arange(W_ds, dtype=np.int32), H_ds) * down + down // 2, 0, W_prev - 1)
    idy = np.clip(np.repeat(np.arange(H_ds, dtype=np.int32), W_ds) * down + down // 2, 0, H_prev - 1)
    rays = [ft.rays_as_array(ft.rays_from_rt_indices(poses[v], idx, idy, W_prev, H_prev, K=K_prev)) for v in views]
    return rays, W_ds, H_ds


def preview_jobs(cfg: dict, poses: np.ndarray, K: np.ndarray, W: int, H: int) -> list:
    """The preview views' rays resident on the GPU, one batch per view."""
    rays, W_ds, H_ds = preview_rays(cfg, poses, K, W, H)
    jobs = []
    for v, r in zip(cfg["preview"]["views"], rays):
        io = ft.RayBatch.init(W_ds * H_ds, int(cfg["preview"]["samples_per_ray"]))
        io.upload_rays(r)
        jobs.append(dict(view=v, io=io, W_ds=W_ds, H_ds=H_ds))
    return jobs


def write_preview(nerf: ft.Nerf, jobs: list, training_dir, model_id: str, step: int) -> Path:
    """Render the preview views forward-only and write them side by side as one 8-bit PNG
    (run_ffnerf_OG.py:1519-1545)."""
    import png_io
    imgs = []
    for job in jobs:
        out, _ = nerf.step(job["io"], lr_f=0.0, do_train=False, occ_update_strength=0.0, return_output=True)
        img = np.clip(out[:, :3].reshape(job["H_ds"], job["W_ds"], 3), 0.0, 1.0)
        imgs.append((img * 255).astype(np.uint8))
    path = Path(training_dir) / f"{model_id}_preview_{jobs[0]['W_ds']}p_step{step}_multiview.png"
    png_io.write_png(path, np.concatenate(imgs, axis=1))
    return path


_STOP = False


def _on_sigint(sig, frame):
    global _STOP
    _STOP = True
    print("\n[CTRL+C] Graceful shutdown requested...")


def train(cfg: dict, load_id: str | None = None, log=print, eval_every: int = 0, eval_rays: int = 4096) -> dict:
    """Train the configured scene for cfg['training']['steps'] more steps; returns a summary."""
    global _STOP
    _STOP = False
    import torch
    from sfm_data import load_images, read_scene, scene_bounds
    t = cfg["training"]
    B, S = int(t["batch_rays"]), int(t["samples_per_ray"])
    if S > ft.S_MAX or S & (S - 1):
        raise ValueError(f"samples_per_ray={S} must be a power of two <= {ft.S_MAX}")
    paths, poses, K_sfm, _, points = read_scene(cfg["data"])
    images, K, (W, H) = load_images(cfg["data"], paths, K_sfm)
    box_min, box_max = scene_bounds(cfg["scene"], points)
    log(f"Loaded {images.shape[0]} images {W}x{H}; scene box {box_min.tolist()} .. {box_max.tolist()}")
    spec = model_spec(cfg)
    occ = occ_params(cfg, box_min, box_max)
    nerf = ft.Nerf(t["directory"], t["model_id"], spec=spec, occ=occ, load_id=load_id, rng_seed=int(t["seed"]))
    dev = DeviceImages(images, poses, K)
    weights = pw.PixelWeights(images) if cfg["model"]["pixel_sampler"] == "adaptive" else None
    pixel_ids = torch.zeros(B, dtype=torch.int32, device="cuda") if weights is not None else None
    constant = cfg["model"]["schedule"] == "constant"
    ios = [ft.RayBatch.init(B, S) for _ in range(2)]
    rng = np.random.default_rng(int(t["seed"]))
    eval_io = None
    if eval_every > 0:
        im = rng.integers(0, images.shape[0], eval_rays)
        u, v = rng.integers(0, W, eval_rays), rng.integers(0, H, eval_rays)
        rays_e, tg_e = ft.rays_targets_from_indices(im, u, v, images, poses, W, H, K=K)
        eval_io = ft.RayBatch.init(eval_rays, S)
        eval_io.upload_rays(rays_e)
        eval_io.upload_targets(tg_e)
    jobs = preview_jobs(cfg, poses, K, W, H) if cfg["preview"]["views"] else []
    loss_path, loss_f = open_loss_log(t["directory"], t["model_id"])
    old = signal.signal(signal.SIGINT, _on_sigint)
    t0 = time.time()
    last_save = t0
    last_preview = None  # the first preview is written at the first step
    save_every = float(cfg["preview"]["save_seconds"])
    preview_every = float(cfg["preview"]["image_seconds"])
    history, evals, previews = [], [], []
    step0 = int(nerf.steps_trained)
    try:
        for k in range(int(t["steps"])):
            if _STOP:
                break
            step = step0 + k + 1
            io = ios[k & 1]
            if weights is not None:
                weights.make_batch(dev, io, seed=int(rng.integers(0, 2 ** 32)), pixel_ids=pixel_ids)
            else:
                dev.make_batch(io, seed=int(rng.integers(0, 2 ** 32)))
            if constant:
                lr_f, sh, cr, occ_s = np.float32(t["lr"]), 1.0, 1.0, float(occ.occ_update_strength0)
            else:
                lr_f = lr_schedule(step, float(t["lr"]), float(t["lmd"]), B, S)
                sh, cr = sh_multiplier(step), color_rel_lr(step)
                occ_s = float(occ.occ_update_strength0) * occ_multiplier(step)
            nerf.step(io, lr_f=float(lr_f), do_train=True, sh_multiplier=sh, color_MLP_rel_lr=cr,
                      occ_update_strength=occ_s)
            if step % int(t["period"]) == 0 or k == int(t["steps"]) - 1:
                out, _ = io.download_out()
                tg = io.targets_buf.detach().cpu().numpy()
                mse, rmse, l2 = batch_loss(out, tg)
                write_loss_row(loss_f, time.time() - t0, step, float(lr_f), mse, rmse, l2)
                if weights is not None:  # the reference's feedback of the reported batch's errors
                    weights.update(pixel_ids.cpu().numpy().view(np.uint32), pw.ray_errors(out, tg))
                    weights.upload()
                history.append((step, mse))
                log(f"[step {step}] lr_f={float(lr_f):.3e} mse={mse:.6e} rmse_rgb={rmse:.6e} l2mean={l2:.6e}")
            if eval_io is not None and (step % eval_every == 0):
                nerf.step(eval_io, lr_f=0.0, do_train=False, occ_update_strength=0.0, sh_multiplier=sh)
                out_e, _ = eval_io.download_out()
                evals.append((step, psnr(out_e, eval_io.targets_buf.cpu().numpy())))
            if time.time() - last_save > save_every:
                nerf.save(min_new_file_seconds=300)
                last_save = time.time()
            if jobs and (last_preview is None or time.time() - last_preview > preview_every):
                previews.append(write_preview(nerf, jobs, t["directory"], t["model_id"], step))
                log(f"[preview] saved {previews[-1]}")
                last_preview = time.time()
        torch.cuda.synchronize()
    finally:
        saved = nerf.save(min_new_file_seconds=0)
        loss_f.close()
        signal.signal(signal.SIGINT, old)
    log(f"Saved model -> {saved}")
    return dict(steps_trained=int(nerf.steps_trained), loss_log=str(loss_path), checkpoint=str(saved),
                history=history, evals=evals, previews=[str(p) for p in previews], nerf=nerf,
                pixel_weights=weights)
