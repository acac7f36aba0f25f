"""Error bounds of the MLP kernels' per-sample math helpers (ffn_device.h), each evaluated on the GPU
through the test probe tests/hip/libffn_probe_math.so and compared with a float64 numpy reference of the
same float32 input, over the argument range its call sites pass (the clamps in ffn_mlp.hip,
ffn_mlp16.hip, ffn_mlp_common.h and ffn_march.hip).

The activations follow ffnerf_OG.cl:214-253 (softplus of the density, sigmoid of the colour, their
derivatives) and the Charbonnier loss derivative; the kernels compute them with the hardware exp2, log2,
reciprocal and reciprocal square root instead of correctly rounded library calls, and these tests pin
the resulting relative errors.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

PROBE = Path(__file__).resolve().parent / "hip" / "libffn_probe_math.so"
P_EXP, P_SOFTPLUS, P_SOFTPLUS_PRIME, P_SIGMOID_SOFT, P_CHARBONNIER_PRIME, P_RCP = range(6)


def _load():
    # torch before the probe, so that the probe's dependency on libamdhip64.so.7 resolves to torch's HIP
    # runtime instead of mapping the system's as a second runtime in the process
    import torch  # noqa: F401
    if not PROBE.exists():
        pytest.fail(f"{PROBE} is not built (run __graft_entry__.build())")
    return C.CDLL(str(PROBE))


def test_probe_exports():
    assert hasattr(_load(), "ffn_probe_math")


def _eval(fn, x):
    import torch
    lib = _load()
    lib.ffn_probe_math.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int]
    xd = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()
    yd = torch.empty_like(xd)
    torch.cuda.synchronize()
    rc = lib.ffn_probe_math(fn, xd.data_ptr(), yd.data_ptr(), xd.numel())
    assert rc == 0, f"ffn_probe_math({fn}) returned {rc}"
    return yd.cpu().numpy()


def _rel(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref) / np.abs(ref)))


def _grid(lo, hi, n=1 << 20):
    return np.linspace(lo, hi, n, dtype=np.float32)


@pytest.mark.gpu
def test_fast_exp():
    # e^x as 2^(x log2 e): the rounding of x log2 e dominates, |x| <= 20 covers every call site
    x = _grid(-20.0, 20.0)
    rel = _rel(_eval(P_EXP, x), np.exp(x.astype(np.float64)))
    print(f"fast_exp rel {rel:.3e}")
    assert rel < 2e-6


@pytest.mark.gpu
def test_softplus():
    # density activation: softplus of the pre-activation clamped to [-10, 10]; wider arguments exercise the
    # small-u branch of the log1p correction and the large-x shortcut
    for lo, hi, tol in ((-10.0, 10.0, 1e-6), (-30.0, 30.0, 3e-6)):
        x = _grid(lo, hi)
        ref = np.logaddexp(0.0, x.astype(np.float64))
        rel = _rel(_eval(P_SOFTPLUS, x), ref)
        print(f"softplus [{lo}, {hi}] rel {rel:.3e}")
        assert rel < tol


@pytest.mark.gpu
def test_softplus_prime_and_sigmoid():
    # d softplus / dx = sigmoid(x) at pre-activations clamped to [-18, 18]; the colour activation is
    # sigmoid(x / 2) with x / 2 clamped to [-18, 18] inside the helper
    x = _grid(-18.0, 18.0)
    rel = _rel(_eval(P_SOFTPLUS_PRIME, x), 1.0 / (1.0 + np.exp(-x.astype(np.float64))))
    print(f"softplus' rel {rel:.3e}")
    assert rel < 2e-6
    x = _grid(-60.0, 60.0)
    h = np.clip(x.astype(np.float64) * 0.5, -18.0, 18.0)
    rel = _rel(_eval(P_SIGMOID_SOFT, x), 1.0 / (1.0 + np.exp(-h)))
    print(f"sigmoid_soft rel {rel:.3e}")
    assert rel < 2e-6


@pytest.mark.gpu
def test_charbonnier_prime_and_rcp():
    # d/dx sqrt(x^2 + eps^2) with eps = 1e-3, for colour residuals of either sign and any magnitude
    mag = np.logspace(-9, 2, 1 << 19, dtype=np.float64)
    x = np.concatenate([-mag[::-1], mag]).astype(np.float32)
    xd = x.astype(np.float64)
    rel = _rel(_eval(P_CHARBONNIER_PRIME, x), xd / np.sqrt(xd * xd + 1e-6))
    print(f"charbonnier' rel {rel:.3e}")
    assert rel < 5e-7
    x = np.logspace(-12, 12, 1 << 20, dtype=np.float64).astype(np.float32)
    rel = _rel(_eval(P_RCP, x), 1.0 / x.astype(np.float64))
    print(f"rcp rel {rel:.3e}")
    assert rel < 2.5e-7
