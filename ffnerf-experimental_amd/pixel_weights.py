"""Error-weighted pixel sampling for the host trainer.

Counterpart of the reference's batch producer (run_ffnerf_OG.py:585-686) with
its per-image uint8 weight maps: foreground masks from the images
(run_ffnerf_OG.py:402-440), the map update from per-ray colour errors
(run_ffnerf_OG.py:459-488) and the rejection sampler (run_ffnerf_OG.py:490-516,
20 % uniform pixels).  The maps live on the host, where the update runs at the
loss-report period exactly as the reference's does (one EMA step per ray, in
batch order, rounded to uint8 after each), and are copied to the GPU after
each update; the sampler itself runs on the GPU (ffn_make_batch_weighted), so
no per-step host work remains.
"""
from __future__ import annotations

import numpy as np

import ffn_lib as fl

UNIFORM_FRAC = 0.2      # share of each batch drawn uniformly (run_ffnerf_OG.py:677)
MAX_TRIES = 4096        # proposals per weighted ray before the last one is kept
INIT_WEIGHT = 16        # initial map value (run_ffnerf_OG.py:596)


def foreground_masks(images: np.ndarray, tau: float = 8, dilate: int = 0) -> np.ndarray:
    """[n, H, W] bool: a pixel is foreground when its largest RGB channel exceeds tau (uint8 images) or
    tau / 255 (float images), then grown by a square of radius `dilate` (run_ffnerf_OG.py:402-440)."""
    rgb = images[..., :3]
    thr = np.uint8(tau) if rgb.dtype == np.uint8 else float(tau) / 255.0
    fg = rgb.max(axis=-1) > thr
    r = int(dilate)
    if r > 0:
        # square max filter as two separable passes (rows, then columns)
        grown = np.zeros_like(fg)
        n, H, W = fg.shape
        for d in range(-r, r + 1):
            lo, hi = max(0, d), min(W, W + d)
            grown[:, :, lo:hi] |= fg[:, :, lo - d:hi - d]
        fg = np.zeros_like(grown)
        for d in range(-r, r + 1):
            lo, hi = max(0, d), min(H, H + d)
            fg[:, lo:hi, :] |= grown[:, lo - d:hi - d, :]
    return fg


def target_weights(err: np.ndarray) -> np.ndarray:
    """Per-ray target weights in [1, 255]: the error over twice the batch median (plus 1e-6), clipped to
    [0, 8] and mapped linearly onto [1, 255], in float32 (run_ffnerf_OG.py:469-474)."""
    err = np.asarray(err, np.float32)
    med = float(np.median(err)) if err.size else 0.0
    knee = (med + 1e-6) * 2.0
    s = np.clip(err / knee, 0.0, 8.0)
    return (1.0 + 254.0 * (s / 8.0)).astype(np.float32)


class PixelWeights:
    """Per-image uint8 weight maps (host copy and device copy) and the GPU sampler that reads them."""

    def __init__(self, images: np.ndarray, ema: float = 0.05, bg_cap: int = 16, tau: float = 8, dilate: int = 0,
                 device: str | None = "cuda"):
        n, H, W = images.shape[:3]
        self.n, self.H, self.W = n, H, W
        self.ema, self.bg_cap = float(ema), int(bg_cap)
        self.maps = np.full((n, H, W), INIT_WEIGHT, np.uint8)
        self.fg = foreground_masks(images, tau, dilate)
        self._first = None  # [n H W] int32 scratch of update(): a pixel's first entry in the batch
        self.dev = None
        if device is not None:
            import torch
            self.dev = torch.from_numpy(self.maps).to(device)

    def update(self, pixel_ids: np.ndarray, err: np.ndarray) -> None:
        """One EMA step per ray towards its target weight (capped at bg_cap off the foreground), in batch
        order: a pixel drawn k times moves k steps, each rounded to an integer in [1, 255]
        (run_ffnerf_OG.py:459-488).  pixel_ids are flat indices over the n H W pixels."""
        ids = np.asarray(pixel_ids).astype(np.int64).ravel()
        if ids.size == 0:
            return
        w_t = target_weights(err).astype(np.float64)
        flat_maps = self.maps.reshape(-1)
        if self.bg_cap < 255:
            off = ~self.fg.reshape(-1)[ids]
            w_t[off] = np.minimum(w_t[off], float(self.bg_cap))
        if self._first is None:
            self._first = np.empty(flat_maps.size, np.int32)
        keep = 1.0 - self.ema
        rest = np.arange(ids.size)
        while rest.size:
            # the first remaining entry of every pixel (written last, so it wins), one EMA step for each,
            # then the same for the entries left: a pixel's draws apply in batch order
            p = ids[rest]
            self._first[p[::-1]] = rest[::-1]
            head = self._first[p] == rest
            sel, ph = rest[head], p[head]
            w_new = keep * flat_maps[ph].astype(np.float64) + self.ema * w_t[sel]
            flat_maps[ph] = np.clip(np.floor(w_new + 0.5), 1, 255).astype(np.uint8)
            rest = rest[~head]

    def upload(self) -> None:
        import torch
        self.dev.copy_(torch.from_numpy(self.maps))

    def make_batch(self, images, io, seed: int, pixel_ids=None, uniform_frac: float = UNIFORM_FRAC,
                   max_tries: int = MAX_TRIES, stream=None) -> None:
        """A batch of io.num_rays rays from the resident images (trainer.DeviceImages), the first
        floor(uniform_frac * num_rays) uniform within their image, the others weighted by the maps."""
        lib = images.lib
        n = io.num_rays
        fl.check(lib.ffn_make_batch_weighted(fl.ptr(images.images), images.n, images.W, images.H,
                                             fl.ptr(images.c2w), fl.ptr(images.K), fl.ptr(self.dev), n,
                                             int(np.floor(uniform_frac * n)), int(max_tries),
                                             int(seed) & 0xFFFFFFFF, fl.ptr(io.rays_buf), fl.ptr(io.targets_buf),
                                             fl.ptr(pixel_ids) if pixel_ids is not None else None,
                                             fl.stream_ptr(stream)), "ffn_make_batch_weighted")


def ray_errors(out: np.ndarray, targets: np.ndarray) -> np.ndarray:
    """Per-ray RMS colour error clipped to [0, 1], float32 (the reference's feedback,
    run_ffnerf_OG.py:1383)."""
    d = out[:, :3] - targets[:, :3]
    return np.clip(np.sqrt(np.mean(d * d, axis=1)).astype(np.float32), 0.0, 1.0)
