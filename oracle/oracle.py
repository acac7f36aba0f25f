"""ctypes binding of the CPU oracle (oracle/ffnerf_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by the ``cpu_baseline`` leg of ``bench.py``, always as the checker or as
the timed CPU baseline.  The product (the HIP library and its Python host)
never imports this module.

Every function here restates the reference semantics of
``/root/reference/ffnerf_OG.cl``, ``weight_update.cl`` and
``decay_occ_grid_in-st.cl``; see the C file for the line-level citations.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

M = 64
D_OUT = 16
L_DIR = 16
C_IN = 32
C_OUT = 3
MAX_LEVELS = 32
LAYER_NAMES = ["Wd_in", "Wd_01", "Wd_12", "Wd_out", "Wc_in", "Wc_01", "Wc_12", "Wc_23", "Wc_out"]
BIAS_NAMES = ["bd_0", "bd_1", "bd_2", "bd_out", "bc_0", "bc_1", "bc_2", "bc_3", "bc_out"]

_fp = C.POINTER(C.c_float)
_up = C.POINTER(C.c_uint32)
_dp = C.POINTER(C.c_double)


class OraCfg(C.Structure):
    _fields_ = [
        ("n_levels", C.c_int32), ("f_per_level", C.c_int32),
        ("log2_T", C.c_uint32 * MAX_LEVELS), ("offset", C.c_uint32 * MAX_LEVELS),
        ("res", C.c_int32 * MAX_LEVELS), ("lvl_lr_scale", C.c_float * MAX_LEVELS),
        ("nd", C.c_int32), ("nc", C.c_int32), ("occ_G", C.c_int32),
        ("box_min", C.c_float * 3), ("box_max", C.c_float * 3),
        ("rho_min", C.c_float), ("rho_max", C.c_float), ("dt_min", C.c_float), ("dt_max", C.c_float),
        ("t_near", C.c_float), ("t_far", C.c_float),
        ("background", C.c_int32), ("hash_opt", C.c_int32), ("table_f16", C.c_int32),
    ]


class OraScalars(C.Structure):
    _fields_ = [
        ("lr", C.c_float), ("lr_t", C.c_float), ("color_rel_lr", C.c_float), ("sh_multiplier", C.c_float),
        ("occ_strength", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
        ("rng_seed", C.c_uint32), ("do_train", C.c_int32),
    ]


class OraParams(C.Structure):
    _fields_ = [
        ("W", _fp * 9), ("b", _fp * 9), ("mW", _fp * 9), ("vW", _fp * 9), ("mb", _fp * 9), ("vb", _fp * 9),
        ("table", _fp), ("m_table", _fp), ("v_table", _fp), ("occ_in", _up), ("occ_st", _up),
    ]


class OraDebug(C.Structure):
    _fields_ = [
        ("Ts", _fp), ("DTs", _fp), ("flags", _up), ("a0", _fp), ("sigma", _fp), ("rgb", _fp), ("Tr", _fp),
        ("T_final", _fp), ("dL_dsigma", _fp), ("dL_dc", _fp), ("dL_da0", _fp), ("gW", _fp * 9), ("gb", _fp * 9),
        ("g_table", _fp), ("relu_in", _up), ("relu_out", _up), ("preact", _fp), ("C_in", _fp), ("C_out", _fp),
    ]


RELU_WORDS = 14  # ReLU-branch words per sample: two per hidden layer (3 density, 4 colour)


class OraMarchCfg(C.Structure):
    _fields_ = [("res", C.c_int32), ("dt", C.c_float), ("max_steps", C.c_uint32), ("T_stop", C.c_float),
                ("sh_multiplier", C.c_float)]


def _build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


OMP_LIB_PATH = HERE / "liboracle_omp.so"


def load(path: Path = None) -> C.CDLL:
    """The checker build (one thread, fixed order), or with path=OMP_LIB_PATH the same restatement on every
    host core (the CPU baseline only)."""
    path = LIB_PATH if path is None else path
    if not path.exists():
        _build()
    lib = C.CDLL(str(path))
    lib.ora_set_threads.argtypes = [C.c_int]
    lib.ora_f32_to_f16_bits.restype = C.c_uint16
    lib.ora_f32_to_f16_bits.argtypes = [C.c_float]
    lib.ora_f16_bits_to_f32.restype = C.c_float
    lib.ora_f16_bits_to_f32.argtypes = [C.c_uint16]
    lib.ora_f16_round.restype = C.c_float
    lib.ora_f16_round.argtypes = [C.c_float]
    lib.ora_max_threads.restype = C.c_int
    lib.ora_hash_u32.restype = C.c_uint32
    lib.ora_hash_u32.argtypes = [C.c_uint32]
    lib.ora_xorshift32.restype = C.c_uint32
    lib.ora_xorshift32.argtypes = [C.c_uint32]
    lib.ora_rand01_first.restype = C.c_float
    lib.ora_rand01_first.argtypes = [C.c_uint32]
    lib.ora_det_powr.restype = C.c_float
    lib.ora_det_powr.argtypes = [C.c_float, C.c_float]
    lib.ora_det_log.restype = C.c_double
    lib.ora_det_log.argtypes = [C.c_double]
    lib.ora_det_exp.restype = C.c_double
    lib.ora_det_exp.argtypes = [C.c_double]
    lib.ora_ray_aabb.restype = C.c_int
    lib.ora_ray_aabb.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp]
    lib.ora_scan_excl_f.argtypes = [_fp, C.c_int]
    lib.ora_reduce_sum_f.restype = C.c_float
    lib.ora_reduce_sum_f.argtypes = [_fp, C.c_int]
    lib.ora_scan_excl_aff_rev.argtypes = [_fp, _fp, C.c_int, _fp, _fp]
    lib.ora_sample_ray.argtypes = [C.POINTER(OraCfg), _fp, C.c_uint32, C.c_int, C.c_uint32, _up, C.c_int, _fp, _fp,
                                   _up]
    lib.ora_hash_encode.argtypes = [C.POINTER(OraCfg), _fp, _fp, C.c_int64, _fp, _up, _fp]
    lib.ora_hash_backward.argtypes = [C.POINTER(OraCfg), _fp, _fp, C.c_int64, _dp]
    lib.ora_sh_encode.argtypes = [_fp, _fp]
    lib.ora_mlp_forward.argtypes = [C.POINTER(OraCfg), C.POINTER(OraParams), _fp, _fp, C.c_float, _fp, _fp, _fp]
    lib.ora_occ_propose_ray.argtypes = [C.POINTER(OraCfg), _fp, C.c_uint32, C.c_int, C.c_uint32, _fp, _fp, _fp,
                                        C.c_float, _up, _up, _up]
    lib.ora_occ_propose_batch.argtypes = [C.POINTER(OraCfg), _fp, C.c_int32, C.c_int, C.c_uint32, _fp, _fp, _fp,
                                          _fp, _up, _up, _up]
    lib.ora_occ_propose_marched_ray.argtypes = [C.POINTER(OraCfg), _fp, C.c_uint32, C.c_int, C.c_uint32, _fp, _fp,
                                                C.c_float, _up, _up]
    lib.ora_occ_propose_marched_batch.argtypes = [C.POINTER(OraCfg), _fp, C.c_int32, _up, C.c_uint32, _fp, _fp,
                                                  _fp, _up, _up]
    lib.ora_composite_ray.argtypes = [C.POINTER(OraCfg), C.c_uint32, C.c_int, C.c_uint32, C.c_int, _fp, _fp, _fp,
                                      _fp, _fp, _fp, _fp, _fp, _fp]
    lib.ora_adam.argtypes = [_fp, _fp, _fp, _fp, C.c_int64, C.c_float, C.c_float, C.c_float, C.c_float]
    lib.ora_occ_decay.argtypes = [_up, _up, C.c_uint32, C.c_uint32, C.c_uint32]
    lib.ora_train_step.restype = C.c_int
    lib.ora_train_step.argtypes = [C.POINTER(OraCfg), C.POINTER(OraParams), _fp, _fp, _fp, C.c_int32, C.c_int32,
                                   C.POINTER(OraScalars), C.POINTER(OraDebug)]
    lib.ora_occ_bitfield.argtypes = [_up, C.c_int32, C.c_uint32, _up]
    lib.ora_train_step_marched.restype = C.c_int
    lib.ora_train_step_marched.argtypes = [C.POINTER(OraCfg), C.POINTER(OraParams), C.POINTER(OraMarchCfg), _up, _fp,
                                           _fp, _fp, C.c_int32, C.POINTER(OraScalars), C.POINTER(OraDebug), _up, _up]
    lib.ora_composite_marched.restype = C.c_int
    lib.ora_composite_marched.argtypes = [_fp, _fp, C.c_int, C.c_float, C.c_float, _fp, _fp, _fp, C.c_int, C.c_float,
                                          _fp, _fp, _fp, _fp, _fp]
    lib.ora_march_ray.restype = C.c_int
    lib.ora_march_ray.argtypes = [C.POINTER(OraCfg), C.POINTER(OraMarchCfg), _up, _fp, _fp]
    lib.ora_render_ray.restype = C.c_int
    lib.ora_render_ray.argtypes = [C.POINTER(OraCfg), C.POINTER(OraParams), C.POINTER(OraMarchCfg), _up, _fp, _fp]
    return lib


_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def use_library(cdll: C.CDLL) -> None:
    """Route the wrappers below to another build of the restatement (the OpenMP baseline build)."""
    global _LIB
    _LIB = cdll


def fptr(a):
    if a is None:
        return C.cast(None, _fp)
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_fp)


def uptr(a):
    if a is None:
        return C.cast(None, _up)
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(_up)


# ---------------------------------------------------------------------------
# configuration


def level_offsets(log2_T):
    off, acc = [], 0
    for lt in log2_T:
        off.append(acc)
        acc += 1 << int(lt)
    return off, acc


def lvl_lr_scale(n_levels):
    # 2^(-(float)l * 0.1f) of ffnerf_OG.cl:2107-2108, evaluated once on the host
    e = np.float32(0.1)
    return [float(np.float32(2.0 ** float(np.float32(-np.float32(l) * e)))) for l in range(n_levels)]


def make_cfg(spec: dict) -> OraCfg:
    """spec keys: n_levels, f_per_level, log2_T (list), res (list), nd, nc, occ_G, box_min, box_max,
    rho_min, rho_max, dt_min, dt_max, t_near, t_far, background (0/1/2), hash_opt (0/1)."""
    c = OraCfg()
    L = int(spec["n_levels"])
    c.n_levels = L
    c.f_per_level = int(spec["f_per_level"])
    off, _ = level_offsets(spec["log2_T"])
    sc = lvl_lr_scale(L)
    for l in range(L):
        c.log2_T[l] = int(spec["log2_T"][l])
        c.offset[l] = off[l]
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
    c.background = int(spec.get("background", 0))
    c.hash_opt = int(spec.get("hash_opt", 0))
    td = spec.get("table_dtype", 0)
    c.table_f16 = 1 if td in (1, "fp16") else 0
    return c


def table_size(spec) -> int:
    _, n = level_offsets(spec["log2_T"])
    return n * int(spec["f_per_level"])


def layer_shapes(spec) -> dict:
    LF = int(spec["n_levels"]) * int(spec["f_per_level"])
    nd, nc = int(spec["nd"]), int(spec["nc"])
    shp = {"Wd_in": (M, LF), "Wd_out": (D_OUT, M), "Wc_in": (M, C_IN), "Wc_out": (C_OUT, M)}
    if nd >= 2:
        shp["Wd_01"] = (M, M)
    if nd >= 3:
        shp["Wd_12"] = (M, M)
    if nc >= 2:
        shp["Wc_01"] = (M, M)
    if nc >= 3:
        shp["Wc_12"] = (M, M)
    if nc >= 4:
        shp["Wc_23"] = (M, M)
    return shp


# ---------------------------------------------------------------------------
# thin wrappers


def hash_u32(x: int) -> int:
    return int(lib().ora_hash_u32(int(x) & 0xFFFFFFFF))


def det_powr(x: float, y: float) -> float:
    return float(lib().ora_det_powr(x, y))


def sample_ray(cfg: OraCfg, ray: np.ndarray, ray_id: int, S: int, seed: int, occ_in: np.ndarray, do_train=True):
    Ts = np.zeros(S, np.float32)
    DTs = np.zeros(S, np.float32)
    flags = np.zeros(2, np.uint32)
    ray = np.ascontiguousarray(ray, np.float32).reshape(8)
    lib().ora_sample_ray(C.byref(cfg), fptr(ray), ray_id, S, seed & 0xFFFFFFFF, uptr(occ_in), int(bool(do_train)),
                         fptr(Ts), fptr(DTs), uptr(flags))
    return Ts, DTs, flags


def hash_encode(cfg: OraCfg, table: np.ndarray, x: np.ndarray, with_idx=False):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 3)
    n = x.shape[0]
    LF = cfg.n_levels * cfg.f_per_level
    a0 = np.zeros((n, LF), np.float32)
    idx = np.zeros((n, cfg.n_levels, 8), np.uint32) if with_idx else None
    w = np.zeros((n, cfg.n_levels, 8), np.float32) if with_idx else None
    lib().ora_hash_encode(C.byref(cfg), fptr(table), fptr(x), n, fptr(a0), uptr(idx), fptr(w))
    return (a0, idx, w) if with_idx else a0


def hash_backward(cfg: OraCfg, x: np.ndarray, g: np.ndarray, table_n: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 3)
    g = np.ascontiguousarray(g, np.float32)
    grad = np.zeros(table_n, np.float64)
    lib().ora_hash_backward(C.byref(cfg), fptr(x), fptr(g), x.shape[0], grad.ctypes.data_as(_dp))
    return grad


def occ_propose(cfg: OraCfg, rays, S: int, seed: int, Ts, DTs, Tr, T_final, flags, occ_in, occ_st):
    """The proposal pass over a batch from given compositing results; raises occ_st in place."""
    rays = np.ascontiguousarray(rays, np.float32).reshape(-1, 8)
    n = rays.shape[0]
    arrs = [np.ascontiguousarray(a, np.float32).reshape(-1) for a in (Ts, DTs, Tr, T_final)]
    fl = np.ascontiguousarray(flags, np.uint32).reshape(-1)
    assert arrs[0].size == n * S and arrs[3].size == n and fl.size == 2 * n
    lib().ora_occ_propose_batch(C.byref(cfg), fptr(rays), n, S, seed & 0xFFFFFFFF, *[fptr(a) for a in arrs],
                                uptr(fl), uptr(np.ascontiguousarray(occ_in, np.uint32).reshape(-1)), uptr(occ_st))


def occ_propose_marched(cfg: OraCfg, rays, counts, seed: int, Ts, Tr, T_final, occ_in, occ_st):
    """The proposal pass over marched rays (counts samples each, Ts / Tr in march order) from given compositing
    results; raises occ_st in place."""
    rays = np.ascontiguousarray(rays, np.float32).reshape(-1, 8)
    n = rays.shape[0]
    cnt = np.ascontiguousarray(counts, np.uint32).reshape(-1)
    arrs = [np.ascontiguousarray(a, np.float32).reshape(-1) for a in (Ts, Tr, T_final)]
    assert cnt.size == n and arrs[0].size == arrs[1].size == int(cnt.sum()) and arrs[2].size == n
    lib().ora_occ_propose_marched_batch(C.byref(cfg), fptr(rays), n, uptr(cnt), seed & 0xFFFFFFFF,
                                        *[fptr(a) for a in arrs], uptr(np.ascontiguousarray(occ_in, np.uint32)
                                                                       .reshape(-1)), uptr(occ_st))


def occ_decay(occ_in: np.ndarray, occ_st: np.ndarray, decay_q24: int, seed: int):
    lib().ora_occ_decay(uptr(occ_in), uptr(occ_st), occ_in.size, decay_q24, seed & 0xFFFFFFFF)


def adam(p, m, v, g, lr_t, beta1, beta2, eps):
    lib().ora_adam(fptr(p), fptr(m), fptr(v), fptr(g), p.size, lr_t, beta1, beta2, eps)


def march_cfg(res, dt, max_steps, T_stop=0.0, sh_multiplier=1.0) -> OraMarchCfg:
    m = OraMarchCfg()
    m.res, m.dt, m.max_steps, m.T_stop, m.sh_multiplier = int(res), float(dt), int(max_steps), float(T_stop), \
        float(sh_multiplier)
    return m


def occ_bitfield(occ: np.ndarray, G: int, q_min: int) -> np.ndarray:
    R = 2 * G
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    lib().ora_occ_bitfield(uptr(np.ascontiguousarray(occ, np.uint32)), G, q_min, uptr(bits))
    return bits


def composite_marched(sigma, rgb, dt, T_stop, bg, target, regu, C_force=None, used_force=-1):
    """One marched ray's compositing and backward: (used, Tr, dL/dsigma, dL/dc, Cf, T_end)."""
    sigma = np.ascontiguousarray(sigma, np.float32)
    rgb = np.ascontiguousarray(rgb, np.float32).reshape(-1, 3)
    n = sigma.size
    Tr, dLds = np.zeros(n, np.float32), np.zeros(n, np.float32)
    dLdc, Cf, T = np.zeros((n, 3), np.float32), np.zeros(3, np.float32), np.zeros(1, np.float32)
    cf = None if C_force is None else np.ascontiguousarray(C_force, np.float32)
    used = lib().ora_composite_marched(fptr(sigma), fptr(rgb), n, dt, T_stop, fptr(np.asarray(bg, np.float32)),
                                       fptr(np.asarray(target, np.float32)), fptr(cf), used_force, regu, fptr(Tr),
                                       fptr(dLds), fptr(dLdc), fptr(Cf), fptr(T))
    return used, Tr, dLds, dLdc, Cf, float(T[0])


def march_ray(cfg: OraCfg, m: OraMarchCfg, bits: np.ndarray, ray: np.ndarray) -> np.ndarray:
    ray = np.ascontiguousarray(ray, np.float32).reshape(8)
    t = np.zeros(max(1, m.max_steps), np.float32)
    n = lib().ora_march_ray(C.byref(cfg), C.byref(m), uptr(bits), fptr(ray), fptr(t))
    return t[:n].copy()


class OracleModel:
    """All state of one model on the CPU (float32 arrays), mirroring the device layout."""

    def __init__(self, spec: dict, params: dict):
        self.spec = dict(spec)
        self.cfg = make_cfg(spec)
        self.p = {k: np.ascontiguousarray(v) for k, v in params.items()}

    def _params(self) -> OraParams:
        P = OraParams()
        for i, (wn, bn) in enumerate(zip(LAYER_NAMES, BIAS_NAMES)):
            if wn in self.p:
                P.W[i] = fptr(self.p[wn])
                P.b[i] = fptr(self.p[bn])
                P.mW[i] = fptr(self.p["m" + wn])
                P.vW[i] = fptr(self.p["v" + wn])
                P.mb[i] = fptr(self.p["m" + bn])
                P.vb[i] = fptr(self.p["v" + bn])
        P.table = fptr(self.p["table"])
        P.m_table = fptr(self.p.get("m_table"))
        P.v_table = fptr(self.p.get("v_table"))
        P.occ_in = uptr(self.p["occ_in"])
        P.occ_st = uptr(self.p["occ_st"])
        return P

    def render(self, rays, bits, m: OraMarchCfg):
        """Early-terminated forward render of every ray: (out [N,4] = rgb + T_final, samples used [N])."""
        rays = np.ascontiguousarray(rays, np.float32).reshape(-1, 8)
        out = np.zeros((rays.shape[0], 4), np.float32)
        used = np.zeros(rays.shape[0], np.int32)
        P = self._params()
        for r in range(rays.shape[0]):
            o = out[r]
            used[r] = lib().ora_render_ray(C.byref(self.cfg), C.byref(P), C.byref(m), uptr(bits),
                                           fptr(rays[r].copy()), o.ctypes.data_as(_fp))
        return out, used

    def train_step_marched(self, rays, targets, bits, m: OraMarchCfg, scalars: dict, relu_in=None, C_in=None,
                           used_in=None):
        """One training step over marched samples (ora_train_step_marched).  Returns (out [N,4], n_used [N],
        taps) with the taps indexed by sample in march order.  relu_in / C_in / used_in (optional): another
        implementation's ReLU branches [n][14], loss colours [N][4] and samples composited per ray [N]."""
        rays = np.ascontiguousarray(rays, np.float32).reshape(-1, 8)
        targets = np.ascontiguousarray(targets, np.float32).reshape(-1, 4)
        bits = np.ascontiguousarray(bits, np.uint32)
        N = rays.shape[0]
        n = int(sum(march_ray(self.cfg, m, bits, r).size for r in rays))
        LF = self.cfg.n_levels * self.cfg.f_per_level
        t = dict(Ts=np.zeros(n, np.float32), a0=np.zeros((n, LF), np.float32), sigma=np.zeros(n, np.float32),
                 rgb=np.zeros((n, 3), np.float32), Tr=np.zeros(n, np.float32), T_final=np.zeros(N, np.float32),
                 dL_dsigma=np.zeros(n, np.float32), dL_dc=np.zeros((n, 3), np.float32),
                 dL_da0=np.zeros((n, LF), np.float32), relu_out=np.zeros((n, RELU_WORDS), np.uint32),
                 preact=np.zeros((n, 7, M), np.float32), C=np.zeros((N, 4), np.float32))
        dbg = OraDebug()
        for k, v in t.items():
            key = {"relu_out": "relu_out", "C": "C_out"}.get(k, k)
            setattr(dbg, key, uptr(v) if v.dtype == np.uint32 else fptr(v))
        for i, wn in enumerate(LAYER_NAMES):
            if wn in self.p:
                t["g" + wn] = np.zeros_like(self.p[wn])
                t["g" + BIAS_NAMES[i]] = np.zeros_like(self.p[BIAS_NAMES[i]])
                dbg.gW[i] = fptr(t["g" + wn])
                dbg.gb[i] = fptr(t["g" + BIAS_NAMES[i]])
        if self.cfg.hash_opt == 1:
            t["g_table"] = np.zeros_like(self.p["table"])
            dbg.g_table = fptr(t["g_table"])
        keep = []
        if relu_in is not None:
            keep.append(np.ascontiguousarray(relu_in, np.uint32).reshape(n, RELU_WORDS))
            dbg.relu_in = uptr(keep[-1])
        if C_in is not None:
            keep.append(np.ascontiguousarray(C_in, np.float32).reshape(N, 4))
            dbg.C_in = fptr(keep[-1])
        ui = None if used_in is None else np.ascontiguousarray(used_in, np.uint32).reshape(N)
        sc = OraScalars()
        for k in ("lr", "lr_t", "color_rel_lr", "sh_multiplier", "occ_strength", "beta1", "beta2", "eps"):
            setattr(sc, k, float(scalars[k]))
        sc.rng_seed = int(scalars["rng_seed"]) & 0xFFFFFFFF
        sc.do_train = 1
        out = np.zeros((N, 4), np.float32)
        used = np.zeros(N, np.uint32)
        P = self._params()
        rc = lib().ora_train_step_marched(C.byref(self.cfg), C.byref(P), C.byref(m), uptr(bits), fptr(rays),
                                          fptr(targets), fptr(out), N, C.byref(sc), C.byref(dbg), uptr(ui),
                                          uptr(used))
        if rc != 0:
            raise RuntimeError(f"ora_train_step_marched failed: {rc}")
        return out, used, t

    def train_step(self, rays, targets, S, scalars: dict, taps=False, relu_in=None, C_in=None):
        """One step of the restatement.  relu_in ([N*S][14] u32, optional): take every hidden unit's ReLU
        branch from these words (another implementation's decisions) instead of the sign of its
        pre-activation; the taps then also hold the restatement's own signs (relu_out) and the
        pre-activations (preact [N*S][7][64]).  C_in ([N][4], optional): evaluate the photometric loss
        gradient at these composited colours; the taps hold the restatement's own colours (C)."""
        rays = np.ascontiguousarray(rays, np.float32).reshape(-1, 8)
        targets = np.ascontiguousarray(targets, np.float32).reshape(-1, 4)
        N = rays.shape[0]
        out = np.zeros((N, 4), np.float32)
        sc = OraScalars()
        for k in ("lr", "lr_t", "color_rel_lr", "sh_multiplier", "occ_strength", "beta1", "beta2", "eps"):
            setattr(sc, k, float(scalars[k]))
        sc.rng_seed = int(scalars["rng_seed"]) & 0xFFFFFFFF
        sc.do_train = int(bool(scalars.get("do_train", 1)))
        dbg = OraDebug()
        t = None
        if taps:
            LF = self.cfg.n_levels * self.cfg.f_per_level
            t = dict(Ts=np.zeros(N * S, np.float32), DTs=np.zeros(N * S, np.float32),
                     flags=np.zeros(N * 2, np.uint32), a0=np.zeros((N * S, LF), np.float32),
                     sigma=np.zeros(N * S, np.float32), rgb=np.zeros((N * S, 3), np.float32),
                     Tr=np.zeros(N * S, np.float32), T_final=np.zeros(N, np.float32),
                     dL_dsigma=np.zeros(N * S, np.float32), dL_dc=np.zeros((N * S, 3), np.float32),
                     dL_da0=np.zeros((N * S, LF), np.float32))
            for k, v in t.items():
                setattr(dbg, k, uptr(v) if v.dtype == np.uint32 else fptr(v))
            for i, wn in enumerate(LAYER_NAMES):
                if wn in self.p:
                    t["g" + wn] = np.zeros_like(self.p[wn])
                    t["g" + BIAS_NAMES[i]] = np.zeros_like(self.p[BIAS_NAMES[i]])
                    dbg.gW[i] = fptr(t["g" + wn])
                    dbg.gb[i] = fptr(t["g" + BIAS_NAMES[i]])
            if self.cfg.hash_opt == 1:
                t["g_table"] = np.zeros_like(self.p["table"])
                dbg.g_table = fptr(t["g_table"])
            t["C"] = np.zeros((N, 4), np.float32)
            dbg.C_out = fptr(t["C"])
            t["relu_out"] = np.zeros((N * S, RELU_WORDS), np.uint32)
            t["preact"] = np.zeros((N * S, 7, M), np.float32)
            dbg.relu_out = uptr(t["relu_out"])
            dbg.preact = fptr(t["preact"])
        if relu_in is not None:
            assert taps, "relu_in needs taps=True"
            relu_in = np.ascontiguousarray(relu_in, np.uint32).reshape(N * S, RELU_WORDS)
            dbg.relu_in = uptr(relu_in)
        if C_in is not None:
            assert taps, "C_in needs taps=True"
            C_in = np.ascontiguousarray(C_in, np.float32).reshape(N, 4)
            dbg.C_in = fptr(C_in)
        P = self._params()
        rc = lib().ora_train_step(C.byref(self.cfg), C.byref(P), fptr(rays), fptr(targets), fptr(out), N, S,
                                  C.byref(sc), C.byref(dbg) if taps else None)
        if rc != 0:
            raise RuntimeError(f"ora_train_step failed: {rc}")
        return out, t
