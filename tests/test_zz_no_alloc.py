"""ffn_march_noalloc -- the march whose scan scratch lives in the library's
fixed device array instead of handle-owned allocations -- against ffn_march,
bit for bit, through the C ABI: three calls in a row on one handle, the first
at the largest ray count the array holds (FFN_MARCH_NOALLOC_MAX_RAYS), the
next ones with fewer rays (the array keeps the previous call's contents), and
a ray count beyond the array refused with an error before any launch."""
import ctypes as C

import numpy as np
import pytest

from common import look_at_rays, random_params, spec_cfg0

pytestmark = pytest.mark.gpu

SPEC = spec_cfg0(occ_G=16)


def _shell_bits(R, seed=0, frac=0.02):
    rng = np.random.default_rng(seed)
    c = (np.arange(R) + 0.5) / R
    z, y, x = np.meshgrid(c, c, c, indexing="ij")
    rad = np.sqrt((x - 0.5) ** 2 + (y - 0.5) ** 2 + (z - 0.5) ** 2)
    occ = (np.abs(rad - 0.3) <= 0.06) | (rng.random((R, R, R)) < frac)
    idx = np.nonzero(occ.reshape(-1))[0]
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits


def _march(lib, fn, h, rays_t, n, bits_t, mp, cap):
    import torch
    import ffn_lib as fl
    counts = torch.full((n,), -1, dtype=torch.int32, device="cuda")
    offsets = torch.full((n,), -1, dtype=torch.int32, device="cuda")
    samples = torch.full((cap, 4), -1.0, dtype=torch.float32, device="cuda")
    ids = torch.full((cap,), -1, dtype=torch.int32, device="cuda")
    total = torch.full((4,), -1, dtype=torch.int32, device="cuda")
    fl.check(getattr(lib, fn)(h, fl.ptr(rays_t), n, fl.ptr(bits_t), C.byref(mp), fl.ptr(counts), fl.ptr(offsets),
                              fl.ptr(samples), fl.ptr(ids), cap, fl.ptr(total), fl.stream_ptr()), fn)
    torch.cuda.synchronize()
    tot = int(total[0].item())
    return (counts.cpu().numpy(), offsets.cpu().numpy(), samples[:tot].cpu().numpy(), ids[:tot].cpu().numpy(), tot)


def test_march_noalloc_matches_march():
    import torch
    import ffn_lib as fl
    from gpu_helpers import GpuModel, to_dev
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    g = GpuModel(SPEC, random_params(SPEC, seed=1))
    lib, h = g.lib, g.h.h
    R = 64
    bits_t = to_dev(_shell_bits(R, seed=5))
    # the largest accepted call first (its offsets and tile sums fill the array exactly), then calls with fewer
    # rays on the array the previous one left behind
    for n, max_steps in ((fl.MARCH_NOALLOC_MAX_RAYS, 4), (6000, 300), (1700, 300)):
        print(f"[case] march_noalloc n={n} max_steps={max_steps}", flush=True)
        mp = fl.march_params(R, np.float32(np.sqrt(3.0) / 256), max_steps)
        rays_t = to_dev(look_at_rays(n, SPEC, seed=n).reshape(-1, 8))
        cap = n * max_steps
        ref = _march(lib, "ffn_march", h, rays_t, n, bits_t, mp, cap)
        got = _march(lib, "ffn_march_noalloc", h, rays_t, n, bits_t, mp, cap)
        assert ref[4] == got[4] and ref[4] > n
        for a, b in zip(ref[:4], got[:4]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # more rays than the array holds: refused on the host, nothing launched (the rays buffer is not read)
    rays_t = to_dev(look_at_rays(16, SPEC, seed=3).reshape(-1, 8))
    with pytest.raises(fl.FfnError, match="exceeds its scratch"):
        _march(lib, "ffn_march_noalloc", h, rays_t, fl.MARCH_NOALLOC_MAX_RAYS + 1, bits_t, mp, 16)
