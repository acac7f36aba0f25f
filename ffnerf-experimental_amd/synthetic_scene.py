"""The synthetic scene of the benchmark configurations, and its archive.

Scene: the unit cube [0,1]^3 holds a ball of radius 0.25 at (0.5, 0.5, 0.5)
with constant density sigma = 50 and colour equal to the position (RGB = xyz);
everything else is empty.  Targets are the exact volume rendering of a pixel
ray on a black background: along the chord [ta, tb] with x_a = o + ta d and
l = tb - ta,
    C = x_a (1 - e^{-sigma l}) + d (1 - e^{-sigma l} (1 + sigma l)) / sigma.

Cameras: pinhole (OpenCV axes: x right, y down, z forward) on a sphere of
radius 1.5 about the centre, directions uniform on the upper hemisphere from a
seed, looking at the centre with +Z up.  The archive is written in the
BA-reconstruction npz layout that sfm_data.read_scene reads
(img_paths, K, RT + rt_dir, X, active_cam_global).
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np

CENTER = np.array([0.5, 0.5, 0.5])
RADIUS = 0.25
SIGMA = 50.0

# (n_cameras, W, H, f) of the benchmark configurations
SHAPES = {
    "cfg0": (8, 64, 64, 51.2),
    "cfg1": (56, 450, 800, 640.0),
}


@dataclass
class Cameras:
    c2w: np.ndarray  # [n, 4, 4]
    K: np.ndarray    # [3, 3]
    W: int
    H: int


def look_at_c2w(pos, target, up=(0.0, 0.0, 1.0)):
    fwd = np.asarray(target, np.float64) - np.asarray(pos, np.float64)
    fwd /= np.linalg.norm(fwd)
    up = np.asarray(up, np.float64)
    if abs(np.dot(fwd, up)) > 0.999:
        up = np.array([0.0, 1.0, 0.0])
    right = np.cross(fwd, up)
    right /= np.linalg.norm(right)
    down = np.cross(fwd, right)
    m = np.eye(4)
    m[:3, 0], m[:3, 1], m[:3, 2], m[:3, 3] = right, down, fwd, pos
    return m


def hemisphere_cameras(n, W, H, f, seed=0, radius=1.5) -> Cameras:
    rng = np.random.default_rng(seed)
    v = rng.normal(size=(n, 3))
    v[:, 2] = np.abs(v[:, 2])
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    c2w = np.stack([look_at_c2w(CENTER + radius * d, CENTER) for d in v]).astype(np.float32)
    K = np.array([[f, 0, W / 2.0], [0, f, H / 2.0], [0, 0, 1]], np.float32)
    return Cameras(c2w=c2w, K=K, W=W, H=H)


def cameras_for(config: str, seed=0) -> Cameras:
    n, W, H, f = SHAPES["cfg1" if config in ("cfg1", "cfg2") else config]
    return hemisphere_cameras(n, W, H, f, seed=seed)


def pixel_rays(cams: Cameras, im_idx, u, v):
    """Rays as float32 [n, 8] = (o, 1, d, 0), same convention as the trainer."""
    im_idx, u, v = (np.asarray(a) for a in (im_idx, u, v))
    K = cams.K
    x = (u.astype(np.float32) + 0.5 - K[0, 2]) / K[0, 0]
    y = (v.astype(np.float32) + 0.5 - K[1, 2]) / K[1, 1]
    cam = np.stack([x, y, np.ones_like(x)], 1)
    R = cams.c2w[im_idx, :3, :3]
    d = np.einsum("nij,nj->ni", R, cam)
    d /= (np.linalg.norm(d, axis=1, keepdims=True) + 1e-12)
    rays = np.zeros((len(im_idx), 8), np.float32)
    rays[:, :3] = cams.c2w[im_idx, :3, 3]
    rays[:, 3] = 1.0
    rays[:, 4:7] = d
    return rays


def render(rays) -> np.ndarray:
    """Exact chord integral of the ball scene on black: float32 [n, 4]."""
    o, d = rays[:, :3].astype(np.float64), rays[:, 4:7].astype(np.float64)
    oc = o - CENTER
    b = np.sum(oc * d, 1)
    c = np.sum(oc * oc, 1) - RADIUS * RADIUS
    disc = b * b - c
    hit = disc > 0
    sq = np.sqrt(np.where(hit, disc, 0.0))
    ta = np.maximum(-b - sq, 0.0)
    tb = -b + sq
    ell = np.maximum(tb - ta, 0.0)
    xa = o + ta[:, None] * d
    e = np.exp(-SIGMA * ell)
    C = xa * (1 - e)[:, None] + d * ((1 - e * (1 + SIGMA * ell)) / SIGMA)[:, None]
    out = np.zeros((rays.shape[0], 4), np.float32)
    out[:, :3] = np.where(hit[:, None], C, 0.0)
    return out


def render_image(cams: Cameras, i: int) -> np.ndarray:
    v, u = np.mgrid[0:cams.H, 0:cams.W]
    rays = pixel_rays(cams, np.full(u.size, i), u.reshape(-1), v.reshape(-1))
    return render(rays)[:, :3].reshape(cams.H, cams.W, 3)


def uniform_batch(cams: Cameras, n, rng):
    """n pixels drawn uniformly over all images -> (rays [n,8], targets [n,4])."""
    im = rng.integers(0, cams.c2w.shape[0], n)
    u = rng.integers(0, cams.W, n)
    v = rng.integers(0, cams.H, n)
    rays = pixel_rays(cams, im, u, v)
    return rays, render(rays)


def sphere_surface_points(n=64, seed=1):
    rng = np.random.default_rng(seed)
    v = rng.normal(size=(n, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    return (CENTER + RADIUS * v).astype(np.float32)


def write_archive(out_dir, config="cfg0", seed=0) -> Path:
    """Render every camera to PNG and write the BA-format npz next to them."""
    import png_io
    out_dir = Path(out_dir)
    (out_dir / "images").mkdir(parents=True, exist_ok=True)
    cams = cameras_for(config, seed)
    paths = []
    for i in range(cams.c2w.shape[0]):
        img = np.clip(render_image(cams, i), 0, 1)
        p = out_dir / "images" / f"{i:04d}.png"
        png_io.write_png(p, np.round(img * 255).astype(np.uint8))
        paths.append(f"images/{i:04d}.png")
    npz = out_dir / "reconstruction.npz"
    np.savez(npz, img_paths=np.array(paths), K=cams.K, RT=cams.c2w, rt_dir=np.array(["c2w"]),
             X=sphere_surface_points(), active_cam_global=np.arange(len(paths), dtype=np.int32))
    return npz
