"""ctypes binding of libffnerf_hip.so (C ABI declared in include/ffnerf_hip.h).

The library is the only compute path: if it is missing or cannot be loaded,
every call raises.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libffnerf_hip.so"

MAX_LEVELS = 32
N_LAYERS = 9
LAYER_NAMES = ["Wd_in", "Wd_01", "Wd_12", "Wd_out", "Wc_in", "Wc_01", "Wc_12", "Wc_23", "Wc_out"]
BIAS_NAMES = ["bd_0", "bd_1", "bd_2", "bd_out", "bc_0", "bc_1", "bc_2", "bc_3", "bc_out"]

BG = {"black": 0, "white": 1, "random": 2}
HASH_OPT = {"sgd": 0, "adam": 1}
MLP_PRECISION = {"fp32": 0, "fp16": 1}
TABLE_DTYPE = {"fp32": 0, "fp16": 1}
SAMPLER = {"resample": 0, "march": 1}

EXPORTS = [
    "ffn_version", "ffn_last_error", "ffn_create", "ffn_destroy", "ffn_bind_params", "ffn_train_step",
    "ffn_occ_decay", "ffn_sample", "ffn_hash_encode_fwd", "ffn_hash_encode_bwd", "ffn_adam",
    "ffn_set_profiling", "ffn_stage_times", "ffn_occ_bitfield", "ffn_march", "ffn_render", "ffn_make_batch",
    "ffn_march_noalloc", "ffn_train_step_marched", "ffn_make_batch_weighted",
]
ABI_VERSION = 3  # FFN_ABI_VERSION of the header these structures and signatures follow
MARCH_NOALLOC_MAX_RAYS = 1 << 20
RELU_WORDS = 14  # ReLU-branch tap words per sample
STAGES = ["sample", "hash_fwd", "mlp", "hash_bwd", "mlp_adam", "table_adam"]

_vp = C.c_void_p
_fp = C.POINTER(C.c_float)


class FfnConfig(C.Structure):
    _fields_ = [
        ("n_levels", C.c_int32), ("f_per_level", C.c_int32),
        ("log2_T", C.c_uint32 * MAX_LEVELS), ("res", C.c_int32 * MAX_LEVELS),
        ("lvl_lr_scale", C.c_float * MAX_LEVELS),
        ("nd", C.c_int32), ("nc", C.c_int32), ("occ_G", C.c_int32),
        ("box_min", C.c_float * 3), ("box_max", C.c_float * 3),
        ("rho_min", C.c_float), ("rho_max", C.c_float), ("dt_min", C.c_float), ("dt_max", C.c_float),
        ("t_near", C.c_float), ("t_far", C.c_float),
        ("background", C.c_int32), ("hash_opt", C.c_int32), ("mlp_precision", C.c_int32),
        ("table_dtype", C.c_int32),
        ("sampler", C.c_int32), ("march_max_steps", C.c_int32), ("march_dt", C.c_float),
        ("march_T_stop", C.c_float), ("march_q_min", C.c_int32), ("reserved", C.c_int32 * 2),
    ]


class FfnParams(C.Structure):
    _fields_ = [
        ("W", _vp * N_LAYERS), ("b", _vp * N_LAYERS), ("mW", _vp * N_LAYERS), ("vW", _vp * N_LAYERS),
        ("mb", _vp * N_LAYERS), ("vb", _vp * N_LAYERS),
        ("table", _vp), ("m_table", _vp), ("v_table", _vp), ("occ_in", _vp), ("occ_st", _vp),
    ]


class FfnStepScalars(C.Structure):
    _fields_ = [
        ("lr", C.c_float), ("lr_t", C.c_float), ("color_rel_lr", C.c_float), ("sh_multiplier", C.c_float),
        ("occ_strength", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
        ("rng_seed", C.c_uint32), ("do_train", C.c_int32),
    ]


class FfnTaps(C.Structure):
    _fields_ = [
        ("Ts", _vp), ("DTs", _vp), ("flags", _vp), ("a0", _vp), ("sigma", _vp), ("rgb", _vp), ("Tr", _vp),
        ("dL_dsigma", _vp), ("dL_dc", _vp), ("dL_da0", _vp), ("gW", _vp * N_LAYERS), ("gb", _vp * N_LAYERS),
        ("g_table", _vp), ("T_final", _vp), ("relu", _vp), ("color", _vp),
    ]


class FfnMarchParams(C.Structure):
    _fields_ = [
        ("res", C.c_int32), ("dt", C.c_float), ("max_steps", C.c_uint32), ("T_stop", C.c_float),
        ("chunk", C.c_uint32), ("sh_multiplier", C.c_float), ("sample_capacity", C.c_uint32),
        ("flags", C.c_uint32),
    ]


RENDER_NO_WAIT = 1  # FFN_RENDER_NO_WAIT


def march_params(res, dt, max_steps, T_stop=1e-4, chunk=32, sh_multiplier=1.0, sample_capacity=0,
                 flags=0) -> FfnMarchParams:
    m = FfnMarchParams()
    m.res, m.dt, m.max_steps, m.T_stop, m.chunk, m.sh_multiplier = int(res), float(dt), int(max_steps), \
        float(T_stop), int(chunk), float(sh_multiplier)
    m.sample_capacity, m.flags = int(sample_capacity), int(flags)
    return m


class FfnError(RuntimeError):
    pass


_LIB = None


def load(path: Path | str | None = None) -> C.CDLL:
    """Load the HIP library (no fallback: raises if it is not built)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FfnError(f"{p} is not built; run __graft_entry__.build() (hipcc, gfx950)")
    # torch first: its wheel bundles a HIP runtime that its libraries name "libamdhip64.so", while this
    # library names the system's "libamdhip64.so.7".  Loaded first, this library would map the system runtime
    # and torch would then map its own as a second one, so that torch's device pointers and streams would
    # belong to another runtime than this library's launches.  With torch loaded, the soname
    # "libamdhip64.so.7" resolves to torch's copy and the process has one runtime.
    import torch  # noqa: F401
    lib = C.CDLL(str(p))
    lib.ffn_version.restype = C.c_int
    if lib.ffn_version() != ABI_VERSION:
        raise FfnError(f"{p} has ABI version {lib.ffn_version()}; this binding is written for {ABI_VERSION} "
                       "(rebuild the library or use the matching binding)")
    lib.ffn_last_error.restype = C.c_char_p
    lib.ffn_create.argtypes = [C.POINTER(FfnConfig), C.POINTER(_vp)]
    lib.ffn_destroy.argtypes = [_vp]
    lib.ffn_bind_params.argtypes = [_vp, C.POINTER(FfnParams)]
    lib.ffn_train_step.argtypes = [_vp, _vp, _vp, _vp, C.c_uint32, C.c_uint32, C.POINTER(FfnStepScalars),
                                   C.POINTER(FfnTaps), _vp]
    lib.ffn_occ_decay.argtypes = [_vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32, _vp]
    lib.ffn_sample.argtypes = [_vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int32, _vp, _vp, _vp, _vp]
    lib.ffn_hash_encode_fwd.argtypes = [_vp, _vp, C.c_int64, _vp, _vp, _vp]
    lib.ffn_hash_encode_bwd.argtypes = [_vp, _vp, _vp, C.c_int64, _vp, _vp]
    lib.ffn_adam.argtypes = [_vp, _vp, _vp, _vp, C.c_int64, C.c_float, C.c_float, C.c_float, C.c_float, C.c_int32,
                             _vp]
    lib.ffn_occ_bitfield.argtypes = [_vp, C.c_int32, C.c_uint32, _vp, _vp]
    lib.ffn_march.argtypes = [_vp, _vp, C.c_uint32, _vp, C.POINTER(FfnMarchParams), _vp, _vp, _vp, _vp, C.c_uint64,
                              _vp, _vp]
    lib.ffn_march_noalloc.argtypes = [_vp, _vp, C.c_uint32, _vp, C.POINTER(FfnMarchParams), _vp, _vp, _vp, _vp,
                                      C.c_uint64, _vp, _vp]
    lib.ffn_train_step_marched.argtypes = [_vp, _vp, _vp, _vp, C.c_uint32, _vp, C.POINTER(FfnMarchParams),
                                           C.POINTER(FfnStepScalars), C.POINTER(FfnTaps), _vp, _vp]
    lib.ffn_render.argtypes = [_vp, _vp, C.c_uint32, _vp, C.POINTER(FfnMarchParams), _vp, _vp, _vp]
    lib.ffn_make_batch.argtypes = [_vp, C.c_uint32, C.c_uint32, C.c_uint32, _vp, _vp, C.c_uint32, C.c_uint32, _vp,
                                   _vp, _vp, _vp]
    lib.ffn_make_batch_weighted.argtypes = [_vp, C.c_uint32, C.c_uint32, C.c_uint32, _vp, _vp, _vp, C.c_uint32,
                                            C.c_uint32, C.c_uint32, C.c_uint32, _vp, _vp, _vp, _vp]
    lib.ffn_set_profiling.argtypes = [_vp, C.c_int32]
    lib.ffn_stage_times.argtypes = [_vp, _fp, C.POINTER(C.c_int32), C.c_int32]
    for name in ("ffn_create", "ffn_destroy", "ffn_bind_params", "ffn_train_step", "ffn_occ_decay", "ffn_sample",
                 "ffn_hash_encode_fwd", "ffn_hash_encode_bwd", "ffn_adam", "ffn_set_profiling", "ffn_stage_times",
                 "ffn_occ_bitfield", "ffn_march", "ffn_render", "ffn_make_batch", "ffn_march_noalloc",
                 "ffn_train_step_marched", "ffn_make_batch_weighted"):
        getattr(lib, name).restype = C.c_int
    if path is None:
        _LIB = lib
    return lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = load().ffn_last_error()
        raise FfnError(f"{what or 'ffn call'} failed ({rc}): {msg.decode() if msg else ''}")


def ptr(t) -> int | None:
    """Raw device pointer of a torch tensor (None passes through)."""
    if t is None:
        return None
    if not t.is_contiguous():
        raise FfnError("tensor must be contiguous")
    return t.data_ptr()


def stream_ptr(stream=None) -> int | None:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def lvl_lr_scale(n_levels: int):
    """2^(-(float)l * 0.1f), the per-level SGD rate of ffnerf_OG.cl:2107-2108."""
    import numpy as np
    e = np.float32(0.1)
    return [float(np.float32(2.0 ** float(np.float32(-np.float32(l) * e)))) for l in range(n_levels)]


def make_config(spec: dict) -> FfnConfig:
    c = FfnConfig()
    L = int(spec["n_levels"])
    c.n_levels = L
    c.f_per_level = int(spec["f_per_level"])
    sc = lvl_lr_scale(L)
    for l in range(L):
        c.log2_T[l] = int(spec["log2_T"][l])
        c.res[l] = int(spec["res"][l])
        c.lvl_lr_scale[l] = sc[l]
    c.nd = int(spec["nd"])
    c.nc = int(spec["nc"])
    c.occ_G = int(spec["occ_G"])
    for i in range(3):
        c.box_min[i] = float(spec["box_min"][i])
        c.box_max[i] = float(spec["box_max"][i])
    for k in ("rho_min", "rho_max", "dt_min", "dt_max", "t_near", "t_far"):
        setattr(c, k, float(spec[k]))
    bg = spec.get("background", 0)
    c.background = BG[bg] if isinstance(bg, str) else int(bg)
    ho = spec.get("hash_opt", 0)
    c.hash_opt = HASH_OPT[ho] if isinstance(ho, str) else int(ho)
    mp = spec.get("mlp_precision", 0)
    c.mlp_precision = MLP_PRECISION[mp] if isinstance(mp, str) else int(mp)
    td = spec.get("table_dtype", 0)
    c.table_dtype = TABLE_DTYPE[td] if isinstance(td, str) else int(td)
    sm = spec.get("sampler", 0)
    c.sampler = SAMPLER[sm] if isinstance(sm, str) else int(sm)
    if c.sampler == SAMPLER["march"]:
        # defaults: the reference's inference predicate (nibble >= 3), a lattice step of the box diagonal over
        # max_steps, and the cfg4 stop
        c.march_max_steps = int(spec.get("march_max_steps", 1024))
        ext = max(float(spec["box_max"][i]) - float(spec["box_min"][i]) for i in range(3))
        c.march_dt = float(spec.get("march_dt") or (3.0 ** 0.5) * ext / c.march_max_steps)
        c.march_T_stop = float(spec.get("march_T_stop", 1e-4))
        c.march_q_min = int(spec.get("march_q_min", 4))
    return c


class Handle:
    """One ffn_create handle (owns the library's scratch for this configuration)."""

    def __init__(self, spec: dict):
        self.lib = load()
        self.spec = dict(spec)
        self.cfg = make_config(spec)
        h = _vp()
        check(self.lib.ffn_create(C.byref(self.cfg), C.byref(h)), "ffn_create")
        self.h = h
        self._keep = None

    def bind(self, params: FfnParams, keep=None):
        check(self.lib.ffn_bind_params(self.h, C.byref(params)), "ffn_bind_params")
        self._keep = keep

    def set_profiling(self, on: bool):
        check(self.lib.ffn_set_profiling(self.h, 1 if on else 0), "ffn_set_profiling")

    def stage_times(self, reset: bool = True) -> dict:
        """{stage: (total_ms, launches)} since the last reset (waits for the work)."""
        ms = (C.c_float * len(STAGES))()
        n = (C.c_int32 * len(STAGES))()
        check(self.lib.ffn_stage_times(self.h, ms, n, 1 if reset else 0), "ffn_stage_times")
        return {s: (float(ms[i]), int(n[i])) for i, s in enumerate(STAGES)}

    def close(self):
        if getattr(self, "h", None):
            self.lib.ffn_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
