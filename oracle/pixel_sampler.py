"""CPU restatement of the error-weighted pixel sampler and of its weight-map
update (run_ffnerf_OG.py:459-516, 585-686) for the tests.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of
ffn_make_batch_weighted and of pixel_weights.PixelWeights.update.  The product
never imports it.

- ``draw_weighted`` follows ffn_make_batch_weighted's draw (include/ffnerf_hip.h)
  step by step with a vectorised lowbias32; its distribution is the
  reference's: the image uniform, a uniform share of rays, the rest accepted
  with probability (w + 1) / 256 per uniform proposal
  (run_ffnerf_OG.py:490-516: ``rng.integers(0, 256) <= w``).
- ``update_weights_loop`` is the reference's per-ray loop
  (run_ffnerf_OG.py:459-488): target weight from the error over twice the
  batch median, background pixels capped, one EMA step per ray in batch
  order, each rounded to an integer in [1, 255].
"""
from __future__ import annotations

import numpy as np

GOLDEN = 2654435769
PROPOSAL_MUL = 0x9E3779B9
ACCEPT_XOR = 0x5BD1E995


def lowbias32(x):
    """C. Wellons' lowbias32 (the reference's hash, ffnerf_OG.cl:296-300) on uint32 arrays."""
    x = np.asarray(x, np.uint64) & 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x ^= x >> 15
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    x ^= x >> 16
    return x.astype(np.uint64)


def draw_weighted(seed: int, num_rays: int, n: int, W: int, H: int, maps: np.ndarray, uniform_rays: int,
                  max_tries: int) -> np.ndarray:
    """Flat pixel index of every ray (over the n W H pixels), as ffn_make_batch_weighted draws it."""
    per = W * H
    r = np.arange(num_rays, dtype=np.uint64)
    h0 = lowbias32(np.uint64(seed & 0xFFFFFFFF) ^ ((r * np.uint64(GOLDEN)) & np.uint64(0xFFFFFFFF)))
    im = (h0 * np.uint64(n)) >> np.uint64(32)
    flat = maps.reshape(n, per)
    q = np.zeros(num_rays, np.uint64)
    pending = np.ones(num_rays, bool)
    for t in range(max_tries):
        idx = np.nonzero(pending)[0]
        if idx.size == 0:
            break
        ht = lowbias32(h0[idx] ^ np.uint64(((t + 1) * PROPOSAL_MUL) & 0xFFFFFFFF))
        q[idx] = (ht * np.uint64(per)) >> np.uint64(32)
        acc = (lowbias32(ht ^ np.uint64(ACCEPT_XOR)) & np.uint64(255)) <= flat[im[idx], q[idx]].astype(np.uint64)
        acc |= idx < uniform_rays
        pending[idx[acc]] = False
    return (im * np.uint64(per) + q).astype(np.int64)


def update_weights_loop(maps: np.ndarray, fg: np.ndarray, pixel_ids, err, ema: float = 0.05,
                        bg_cap: int = 16) -> None:
    """The reference's map update, one ray at a time (maps [n][H][W] uint8 updated in place)."""
    err = np.asarray(err, np.float32)
    med = float(np.median(err)) if err.size else 0.0
    scale = (med + 1e-6) * 2.0
    score = np.clip(err / scale, 0.0, 8.0)
    target = (1.0 + 254.0 * (score / 8.0)).astype(np.float32)
    n, H, W = maps.shape
    for k, p in enumerate(np.asarray(pixel_ids).ravel()):
        im, rem = divmod(int(p), W * H)
        y, x = divmod(rem, W)
        w_t = float(target[k])
        if not bool(fg[im, y, x]) and bg_cap < 255:
            w_t = min(w_t, float(bg_cap))
        w_new = (1.0 - ema) * float(maps[im, y, x]) + ema * w_t
        maps[im, y, x] = np.uint8(np.clip(int(w_new + 0.5), 1, 255))
