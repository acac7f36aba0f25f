"""Reading the BA / SfM-stage-2 reconstruction archives and their images.

Counterpart of the reference's sfm_data.py (read_scene, scene_bounds,
image_geometry, scaled_intrinsics, load_images; sfm_data.py:1-110), with the
same archive keys and validation:
  img_paths, K (shared 3x3), c2w or RT + rt_dir ('c2w' / 'w2c'), optional
  posed / keep_mask filters, X or X_track + has_X sparse points,
  active_cam_global camera ids.
Differences, both forced by this environment: archives are opened without
unpickling (np.load(allow_pickle=False)), so img_paths must be stored as a
string array rather than an object array; and images are read with the
package's PNG codec and resized with an area filter of its own instead of
OpenCV (8-bit PNG only).
"""
from __future__ import annotations

from pathlib import Path, PureWindowsPath

import numpy as np

import png_io


def _load_archive(path: Path) -> dict:
    try:
        with np.load(path, allow_pickle=False) as archive:
            return {k: archive[k] for k in archive.files}
    except ValueError as e:
        raise ValueError(f"{path}: arrays stored as Python objects are not read (no unpickling); "
                         f"store img_paths as a string array ({e})") from None


def read_scene(data: dict):
    """-> (image paths, c2w poses [n,4,4] float32, K [3,3], camera ids, finite sparse points [m,3])."""
    path = Path(data["reconstruction"])
    d = _load_archive(path)
    paths = d["img_paths"]
    n = len(paths)
    keep = np.ones(n, dtype=bool)
    for key in ("posed", "keep_mask"):
        if key in d:
            mask = np.asarray(d[key], dtype=bool)
            if mask.shape != (n,):
                raise ValueError(f"{key} must align with img_paths")
            keep &= mask
    if not keep.any():
        raise ValueError("No registered cameras in reconstruction")
    if "c2w" in d:
        poses = d["c2w"]
    else:
        poses = d["RT"]
        direction = str(np.asarray(d["rt_dir"]).reshape(-1)[0]).lower()
        if direction == "w2c":
            poses = np.linalg.inv(poses)
        elif direction != "c2w":
            raise ValueError(f"Unknown rt_dir: {direction}")
    if poses.shape != (n, 4, 4):
        raise ValueError("Camera transforms must align with img_paths and have shape (N,4,4)")
    poses = np.asarray(poses[keep], dtype=np.float32)
    if not np.isfinite(poses).all():
        raise ValueError("Non-finite camera transforms")
    K = np.asarray(d["K"], dtype=np.float32)
    if K.shape != (3, 3) or not np.isfinite(K).all() or K[0, 0] <= 0 or K[1, 1] <= 0:
        raise ValueError("Expected finite shared 3x3 intrinsics with positive focal lengths")
    resolved = []
    for stored in paths[keep]:
        if data.get("images_dir"):
            p = Path(data["images_dir"]) / PureWindowsPath(str(stored)).name
        else:
            p = Path(str(stored))
            if not p.is_absolute():
                p = path.parent / p
        if not p.is_file():
            raise FileNotFoundError(f"Image missing: {p}. Set data.images_dir to relocate images.")
        resolved.append(p)
    if "X" in d:
        points = np.asarray(d["X"], dtype=np.float32).reshape(-1, 3)
    elif "X_track" in d:
        points = np.asarray(d["X_track"], dtype=np.float32).reshape(-1, 3)
        if "has_X" in d:
            points = points[np.asarray(d["has_X"], dtype=bool)]
    else:
        points = np.empty((0, 3), np.float32)
    points = points[np.isfinite(points).all(axis=1)]
    ids = np.asarray(d.get("active_cam_global", np.arange(n)), dtype=np.int32)[keep]
    return resolved, poses, K, ids, points


def scene_bounds(scene: dict, points: np.ndarray):
    """Explicit box, or a cube around the sparse points: the sphere circumscribing their 1%/99%
    percentile box, radius enlarged by 3/2 (the reference's rule, sfm_data.py:66-84)."""
    lo, hi = scene["box_min"], scene["box_max"]
    if lo is None and hi is None:
        if not len(points):
            raise ValueError("No finite sparse points: set scene.box_min and scene.box_max")
        q_lo, q_hi = np.percentile(points, [1, 99], axis=0)
        center = 0.5 * (q_lo + q_hi)
        radius = 1.5 * max(0.5 * float(np.linalg.norm(q_hi - q_lo)), 0.01)
        lo, hi = center - radius, center + radius
    elif lo is None or hi is None:
        raise ValueError("Set both scene.box_min and scene.box_max, or leave both null")
    lo, hi = np.asarray(lo, dtype=np.float32), np.asarray(hi, dtype=np.float32)
    if lo.shape != (3,) or hi.shape != (3,) or not np.isfinite([lo, hi]).all() or not (hi > lo).all():
        raise ValueError("Scene bounds must be finite xyz vectors with box_max > box_min")
    return lo, hi


def read_rgb(path) -> np.ndarray:
    """uint8 [H, W, 3] RGB."""
    im = png_io.read_png(path)
    if im.shape[2] == 1:
        im = np.repeat(im, 3, axis=2)
    return im[:, :, :3]


def image_geometry(path, data: dict):
    """(image, training size (w, h)): the longer side is limited to data.max_side (0 = unlimited)."""
    try:
        im = read_rgb(path)
    except (ValueError, OSError) as e:
        raise ValueError(f"Cannot decode image: {path} ({e})") from None
    h, w = im.shape[:2]
    max_side = data["max_side"]
    scale = min(1.0, max_side / max(h, w)) if max_side > 0 else 1.0
    return im, (max(1, int(w * scale)), max(1, int(h * scale)))


def scaled_intrinsics(K, original_wh, target_wh, sfm_max_side):
    """K of the SfM images (their longer side limited to sfm_max_side with integer sizes) mapped to target."""
    w, h = original_wh
    s = min(1.0, sfm_max_side / max(w, h)) if sfm_max_side > 0 else 1.0
    sw, sh = max(1, int(w * s)), max(1, int(h * s))
    out = np.asarray(K, np.float32).copy()
    out[0] *= target_wh[0] / sw
    out[1] *= target_wh[1] / sh
    return out


def _area_matrix(n_in: int, n_out: int) -> np.ndarray:
    """Row i averages the source pixels under output pixel i, weighted by overlap (box filter)."""
    s = n_in / n_out
    m = np.zeros((n_out, n_in), np.float64)
    for i in range(n_out):
        a, b = i * s, (i + 1) * s
        j0, j1 = int(np.floor(a)), min(int(np.ceil(b)), n_in)
        for j in range(j0, j1):
            m[i, j] = min(b, j + 1) - max(a, j)
        m[i] /= m[i].sum()
    return m


def area_resize(img: np.ndarray, wh) -> np.ndarray:
    w, h = wh
    if img.shape[0] == h and img.shape[1] == w:
        return img.astype(np.float32)
    my = _area_matrix(img.shape[0], h)
    mx = _area_matrix(img.shape[1], w)
    x = img.astype(np.float64)
    out = np.einsum("ij,jkc->ikc", my, x)
    out = np.einsum("ij,kjc->kic", mx, out)
    return out.astype(np.float32)


def load_images(data: dict, paths, K):
    """-> (float32 RGB images [n, h, w, 3] in [0, 1], K for that size, (w, h))."""
    first, (w, h) = image_geometry(paths[0], data)
    h0, w0 = first.shape[:2]
    images = np.empty((len(paths), h, w, 3), dtype=np.float32)
    for i, path in enumerate(paths):
        im = first if i == 0 else read_rgb(path)
        if im.shape[:2] != (h0, w0):
            raise ValueError(f"Unreadable image or inconsistent image dimensions: {path}")
        images[i] = area_resize(im, (w, h)) / 255.0
    return images, scaled_intrinsics(K, (w0, h0), (w, h), data["sfm_max_side"]), (w, h)
