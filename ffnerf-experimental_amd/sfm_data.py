"""Reading the BA / SfM-stage-2 reconstruction archives and their images.

Counterpart of the reference's sfm_data.py (read_scene, scene_bounds,
image_geometry, scaled_intrinsics, load_images; sfm_data.py:1-110): the same
archive keys, filters and validation rules, organised here as one validator
per archive part feeding a Reconstruction record.  Keys:
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

from dataclasses import dataclass
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


@dataclass
class Reconstruction:
    """The registered cameras of a BA / SfM-stage-2 archive."""
    image_paths: list          # resolved image files, registered cameras only
    c2w: np.ndarray            # [n, 4, 4] float32 camera-to-world (OpenCV camera axes)
    K: np.ndarray              # [3, 3] float32 intrinsics shared by all cameras
    camera_ids: np.ndarray     # [n] int32 global camera ids
    points: np.ndarray         # [m, 3] float32 finite sparse points

    def as_tuple(self):
        return self.image_paths, self.c2w, self.K, self.camera_ids, self.points


def _registered(d: dict, n: int) -> np.ndarray:
    """Cameras kept by every filter the archive carries (posed, keep_mask)."""
    masks = []
    for key in ("posed", "keep_mask"):
        if key not in d:
            continue
        m = np.asarray(d[key], dtype=bool)
        if m.shape != (n,):
            raise ValueError(f"{key} must align with img_paths")
        masks.append(m)
    keep = np.logical_and.reduce(masks) if masks else np.ones(n, dtype=bool)
    if not keep.any():
        raise ValueError("No registered cameras in reconstruction")
    return keep


# RT arrays are stored in either direction; rt_dir names it
_TO_C2W = {"c2w": lambda m: m, "w2c": np.linalg.inv}


def _camera_to_world(d: dict, n: int) -> np.ndarray:
    if "c2w" in d:
        poses = d["c2w"]
    else:
        direction = str(np.asarray(d["rt_dir"]).reshape(-1)[0]).lower()
        if direction not in _TO_C2W:
            raise ValueError(f"Unknown rt_dir: {direction}")
        poses = _TO_C2W[direction](d["RT"])
    if np.shape(poses) != (n, 4, 4):
        raise ValueError("Camera transforms must align with img_paths and have shape (N,4,4)")
    return np.asarray(poses)


def _shared_intrinsics(d: dict) -> np.ndarray:
    K = np.asarray(d["K"], dtype=np.float32)
    ok = K.shape == (3, 3) and bool(np.isfinite(K).all()) and K[0, 0] > 0 and K[1, 1] > 0
    if not ok:
        raise ValueError("Expected finite shared 3x3 intrinsics with positive focal lengths")
    return K


def _locate_image(stored, archive_dir: Path, images_dir) -> Path:
    """An image named in the archive: relocated by file name into data.images_dir when that is set (stored
    Windows paths included), else taken as stored, relative to the archive."""
    if images_dir:
        found = Path(images_dir) / PureWindowsPath(str(stored)).name
    else:
        found = Path(str(stored))
        found = found if found.is_absolute() else archive_dir / found
    if not found.is_file():
        raise FileNotFoundError(f"Image missing: {found}. Set data.images_dir to relocate images.")
    return found


def _sparse_points(d: dict) -> np.ndarray:
    """X, or X_track filtered by has_X; rows with a non-finite coordinate dropped."""
    if "X" in d:
        pts = np.asarray(d["X"], dtype=np.float32).reshape(-1, 3)
    elif "X_track" in d:
        pts = np.asarray(d["X_track"], dtype=np.float32).reshape(-1, 3)
        if "has_X" in d:
            pts = pts[np.asarray(d["has_X"], dtype=bool)]
    else:
        pts = np.empty((0, 3), np.float32)
    return pts[np.isfinite(pts).all(axis=1)]


def open_reconstruction(data: dict) -> Reconstruction:
    archive = Path(data["reconstruction"])
    d = _load_archive(archive)
    stored = d["img_paths"]
    n = len(stored)
    keep = _registered(d, n)
    c2w = np.asarray(_camera_to_world(d, n)[keep], dtype=np.float32)
    if not np.isfinite(c2w).all():
        raise ValueError("Non-finite camera transforms")
    K = _shared_intrinsics(d)
    paths = [_locate_image(p, archive.parent, data.get("images_dir")) for p in stored[keep]]
    ids = np.asarray(d.get("active_cam_global", np.arange(n)), dtype=np.int32)[keep]
    return Reconstruction(paths, c2w, K, ids, _sparse_points(d))


def read_scene(data: dict):
    """-> (image paths, c2w poses [n,4,4] float32, K [3,3], camera ids, finite sparse points [m,3])."""
    return open_reconstruction(data).as_tuple()


def _check_box(lo, hi):
    lo, hi = np.asarray(lo, dtype=np.float32), np.asarray(hi, dtype=np.float32)
    valid = lo.shape == (3,) and hi.shape == (3,) and bool(np.isfinite(lo).all() and np.isfinite(hi).all())
    if not valid or not (hi > lo).all():
        raise ValueError("Scene bounds must be finite xyz vectors with box_max > box_min")
    return lo, hi


def _cube_around(points: np.ndarray):
    """A cube centred on the sparse points' 1 %/99 % percentile box, half-side 3/2 of the radius of the sphere
    through that box's corners (at least 0.015): room around the reconstruction without chasing outliers."""
    if not len(points):
        raise ValueError("No finite sparse points: set scene.box_min and scene.box_max")
    q = np.percentile(points, [1, 99], axis=0)
    half = 1.5 * max(0.5 * float(np.linalg.norm(q[1] - q[0])), 0.01)
    mid = q.mean(axis=0)
    return mid - half, mid + half


def scene_bounds(scene: dict, points: np.ndarray):
    """The scene box: scene.box_min/box_max when both are set, the cube around the sparse points when both
    are null (sfm_data.py:58-76 of the reference gives the same rule)."""
    lo, hi = scene["box_min"], scene["box_max"]
    given = (lo is not None, hi is not None)
    if given == (False, False):
        lo, hi = _cube_around(points)
    elif given != (True, True):
        raise ValueError("Set both scene.box_min and scene.box_max, or leave both null")
    return _check_box(lo, hi)


def fit_within(w: int, h: int, max_side) -> tuple:
    """Integer (w, h) with the longer side limited to max_side (0 = unlimited), never upscaled."""
    if max_side <= 0:
        return w, h
    s = min(1.0, max_side / max(w, h))
    return max(1, int(w * s)), max(1, int(h * s))


def read_rgb(path) -> np.ndarray:
    """uint8 [H, W, 3] RGB.  PNG through the package's own codec; any other format (the JPEGs most SfM
    archives list, which the reference reads with cv2.imread, sfm_data.py:80,105) through Pillow when it
    imports, upright by the file's EXIF orientation as cv2.imread leaves it."""
    with open(path, "rb") as f:
        is_png = f.read(8) == b"\x89PNG\r\n\x1a\n"
    if is_png:
        im = png_io.read_png(path)
    else:
        try:
            from PIL import Image, ImageOps
        except ImportError:
            raise ValueError("not a PNG, and Pillow (needed for other image formats) is not installed") from None
        with Image.open(path) as pim:
            im = np.asarray(ImageOps.exif_transpose(pim).convert("RGB"), dtype=np.uint8)
    if im.ndim == 2:
        im = im[:, :, None]
    if im.shape[2] == 1:
        im = np.repeat(im, 3, axis=2)
    return im[:, :, :3]


def image_geometry(path, data: dict):
    """(image, training size (w, h)): the image's size fit within data.max_side."""
    try:
        im = read_rgb(path)
    except (ValueError, OSError) as e:
        raise ValueError(f"Cannot decode image: {path} ({e})") from None
    return im, fit_within(im.shape[1], im.shape[0], data["max_side"])


def scaled_intrinsics(K, original_wh, target_wh, sfm_max_side):
    """The archive's K belongs to the images SfM saw: the originals fit within sfm_max_side (the same integer
    rule).  Rescale its focal and principal rows to the target size."""
    sfm_w, sfm_h = fit_within(original_wh[0], original_wh[1], sfm_max_side)
    return np.asarray(K, np.float32) * np.array([[target_wh[0] / sfm_w], [target_wh[1] / sfm_h], [1.0]],
                                                np.float32)


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
