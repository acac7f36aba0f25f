"""The error-weighted pixel sampler of the trainer (run_ffnerf_OG.py:402-686):
the host weight-map update (pixel_weights.PixelWeights.update) against the
reference's one-ray-at-a-time loop restated in oracle/pixel_sampler.py and
against hand-computed values; the foreground masks against a library max
filter; and the restated draw (the checker of ffn_make_batch_weighted) against
the distribution the reference's rejection sampler has."""
import numpy as np
import pytest
from scipy import ndimage

import pixel_weights as pw
from oracle import pixel_sampler as ps


def _weights(n=3, H=5, W=7, seed=0):
    rng = np.random.default_rng(seed)
    images = rng.random((n, H, W, 3)).astype(np.float32) * 0.03  # dark: background at tau = 8 (0.0314)
    images[:, 1:4, 2:5, :] = 0.8                                # a bright block: foreground
    return pw.PixelWeights(images, device=None), images


def test_update_equals_the_reference_loop_with_repeated_pixels():
    w, _ = _weights()
    rng = np.random.default_rng(1)
    w.maps[:] = rng.integers(1, 256, w.maps.shape, dtype=np.uint8)
    ref = w.maps.copy()
    for rnd in range(5):
        ids = rng.integers(0, w.maps.size // 4, 400)  # a quarter of the pixels: many drawn several times
        err = rng.random(400).astype(np.float32)
        err[rng.random(400) < 0.1] = 0.0
        err[:3] = [1.0, 0.5, 0.0]
        w.update(ids, err)
        ps.update_weights_loop(ref, w.fg, ids, err, ema=w.ema, bg_cap=w.bg_cap)
        np.testing.assert_array_equal(w.maps, ref, err_msg=f"round {rnd}")
    assert np.bincount(ids).max() >= 3


def test_update_hand_computed():
    """Errors 0.1, 0.3, 0.2, 0.2 (median 0.2, knee 0.400002): scores 0.25, 0.75, 0.5, 0.5 (to 5e-6),
    targets 1 + 254 s / 8 = 8.937, 24.81, 16.87, 16.87.  With ema 1/2 from 16: the foreground pixel drawn
    first and last moves 16 -> floor(8 + 4.469 + 0.5) = 12 -> floor(6 + 8.437 + 0.5) = 14; the other
    foreground pixel to floor(8 + 8.437 + 0.5) = 16; the background pixel's target is capped at 16:
    floor(8 + 8 + 0.5) = 16.  A batch of one ray has its own error as the median: score 0.5, target 16.87,
    capped at 16 again on the background."""
    w, _ = _weights()
    w.ema = 0.5
    n, H, W = w.maps.shape
    fg0 = 0 * H * W + 2 * W + 3  # (image 0, y 2, x 3): inside the bright block
    fg1 = 1 * H * W + 1 * W + 2
    bg = 2 * H * W + 0 * W + 0
    assert w.fg.reshape(-1)[[fg0, fg1]].all() and not w.fg.reshape(-1)[bg]
    w.update(np.array([fg0, bg, fg1, fg0]), np.array([0.1, 0.3, 0.2, 0.2], np.float32))
    flat = w.maps.reshape(-1)
    assert (flat[fg0], flat[fg1], flat[bg]) == (14, 16, 16)
    w.update(np.array([bg]), np.array([1.0], np.float32))
    assert flat[bg] == 16
    untouched = np.ones(flat.size, bool)
    untouched[[fg0, fg1, bg]] = False
    assert (flat[untouched] == pw.INIT_WEIGHT).all()
    # one more step of fg0 alone (target 16.87): floor(7 + 8.437 + 0.5) = 15
    w.update(np.array([fg0]), np.array([0.5], np.float32))
    assert flat[fg0] == 15


def test_target_weights_closed_form():
    err = np.array([0.0, 0.05, 0.1, 0.2, 0.4, 10.0], np.float32)  # median 0.15
    t = pw.target_weights(err)
    s = np.minimum(err.astype(np.float64) / ((0.15 + 1e-6) * 2.0), 8.0)
    np.testing.assert_allclose(t, 1.0 + 254.0 * s / 8.0, rtol=2e-7)
    assert t[0] == 1.0 and t[-1] == 255.0 and t.dtype == np.float32


@pytest.mark.parametrize("dtype", [np.float32, np.uint8])
@pytest.mark.parametrize("dilate", [0, 1, 2])
def test_foreground_masks(dtype, dilate):
    rng = np.random.default_rng(2)
    img = rng.integers(0, 20, (2, 16, 12, 3)).astype(np.uint8)
    img[0, 5, 5, 1] = 200
    src = img.astype(np.float32) / 255.0 if dtype == np.float32 else img
    got = pw.foreground_masks(src, tau=8, dilate=dilate)
    base = img.max(axis=-1) > 8
    want = base if dilate == 0 else np.stack([ndimage.maximum_filter(b, size=2 * dilate + 1, mode="constant")
                                              for b in base])
    np.testing.assert_array_equal(got, want)


def test_draw_reduces_to_uniform_draws():
    """max_tries = 1, or every weight 255 (proposal 0 always accepted): every ray keeps proposal 0, the
    draw of a batch that is all uniform rays."""
    n, W, H = 3, 9, 7
    rng = np.random.default_rng(3)
    maps = rng.integers(0, 256, (n, H, W), dtype=np.uint8)
    uni = ps.draw_weighted(11, 5000, n, W, H, maps, 5000, 64)
    np.testing.assert_array_equal(ps.draw_weighted(11, 5000, n, W, H, maps, 1000, 1), uni)
    np.testing.assert_array_equal(ps.draw_weighted(11, 5000, n, W, H, np.full_like(maps, 255), 0, 64), uni)
    # the uniform draw covers images and pixels evenly
    cnt = np.bincount(ps.draw_weighted(5, 60000, n, W, H, maps, 60000, 1), minlength=n * W * H)
    assert abs(cnt.mean() - 60000 / (n * W * H)) < 1e-9 and cnt.std() < 4 * np.sqrt(cnt.mean())


def test_draw_follows_the_rejection_distribution():
    """Weighted rays land on pixel q of their (uniform) image with probability (w_q + 1) / sum(w + 1): the
    distribution of the reference's sampler, which accepts a uniform proposal when
    rng.integers(0, 256) <= w."""
    n, W, H = 2, 8, 4
    maps = np.zeros((n, H, W), np.uint8)
    maps[:, :, :4] = 255
    maps[:, 0, 4:] = 63
    num = 200000
    ids = ps.draw_weighted(7, num, n, W, H, maps, 0, 4096)
    im = ids // (W * H)
    assert abs(np.mean(im == 0) - 0.5) < 0.01
    p = (maps.astype(np.float64) + 1.0).reshape(n, -1)
    p /= p.sum(axis=1, keepdims=True)
    got = np.bincount(ids, minlength=n * W * H).reshape(n, -1) / np.bincount(im, minlength=n)[:, None]
    np.testing.assert_allclose(got, p, atol=4e-3)
    # the uniform share keeps the first uniform_rays rays uniform
    ids_u = ps.draw_weighted(7, num, n, W, H, maps, num // 5, 4096)
    np.testing.assert_array_equal(ids_u[num // 5:], ids[num // 5:])
    np.testing.assert_array_equal(ids_u[:num // 5], ps.draw_weighted(7, num, n, W, H, maps, num, 1)[:num // 5])
