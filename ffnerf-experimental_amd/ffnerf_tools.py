"""Host-side model container of the MI355X build: the counterpart of the
reference's ``ffnerf_tools.py`` (Nerf, RayBatch, OccParams, ray generation,
checkpoint npz layout), driving libffnerf_hip.so through ctypes instead of
PyOpenCL programs.  PyTorch-ROCm tensors are used only as device buffers.

Reference interface mirrored here (file:line in /root/reference):
  rays_targets_from_indices  ffnerf_tools.py:175-234
  rays_from_rt_indices       ffnerf_tools.py:237-272
  RayBatch                   ffnerf_tools.py:281-395
  OccParams                  ffnerf_tools.py:398-424
  Nerf.step                  ffnerf_tools.py:1357-1544
  Nerf.save / load_latest    ffnerf_tools.py:989-1189
"""
from __future__ import annotations

import ctypes as C
import shutil
import time
from dataclasses import dataclass, field
from datetime import datetime
from pathlib import Path
from typing import Optional

import numpy as np

import ffn_lib as fl

# ---------------------------------------------------------------------------
# constants of the reference (ffnerf_tools.py:23-69); the hash-grid and MLP
# shapes are runtime parameters here (ModelSpec), these are their defaults.
M = 64
D_OUT = 16
L_DIR = 16
C_IN = D_OUT + L_DIR
C_OUT = 3
S_MAX = 64
NDMAX, NCMAX = 3, 4
SIGMA_BIAS = -2.0
OCC_U_STR = 1
DECAY = 0.9
RHO_MIN_DEF = 1.0
RHO_MAX_DEF = 64.0
OCC_INIT_DENSITY = 0xEEEEEEEE
OCC_MAINTENANCE_PERIOD = 32
ADAM_BETA1 = np.float32(0.9)
ADAM_BETA2 = np.float32(0.999)
ADAM_EPS = np.float32(1e-6)

# reference hash layout (ffnerf_OG.cl:161-200)
REF_LEVEL_LOG2 = [13, 13, 13, 13, 15, 15, 15, 15, 17, 17, 17, 17, 18, 18, 19, 19]

ray_dtype = np.dtype([("o", np.float32, 4), ("d", np.float32, 4)], align=True)
if ray_dtype.itemsize != 32:
    raise RuntimeError(f"Unexpected Ray dtype size: {ray_dtype.itemsize} (expected 32)")


def default_ray_dtype() -> np.dtype:
    return ray_dtype


# ---------------------------------------------------------------------------
# rays


def camera_directions(u, v, W, H, K=None) -> np.ndarray:
    """Camera-frame directions [n, 3] float32 through the centres of pixels (u, v), OpenCV axes (x right,
    y down, z forward).  K: shared [3, 3], per-pixel [n, 3, 3], or None for the reference's focal-free
    fallback, (u + 1/2 - W/2, v + 1/2 - H/2, sqrt(W H))."""
    uc = np.asarray(u, np.float32).reshape(-1) + np.float32(0.5)
    vc = np.asarray(v, np.float32).reshape(-1) + np.float32(0.5)
    if K is None:
        return np.stack([uc - W / 2.0, vc - H / 2.0, np.full(uc.shape, np.sqrt(H * W), np.float32)], axis=1)
    K = np.asarray(K, np.float32)
    fx, fy, cx, cy = K[..., 0, 0], K[..., 1, 1], K[..., 0, 2], K[..., 1, 2]
    return np.stack([(uc - cx) / fx, (vc - cy) / fy, np.ones(uc.shape, np.float32)], axis=1)


def world_rays(c2w, dirs_cam: np.ndarray) -> np.ndarray:
    """Rays (ray_dtype) from camera-to-world transforms ([4, 4] shared or [n, 4, 4]) and camera-frame
    directions: origin = the camera centre (w = 1), direction = R d normalised with +1e-12 (w = 0)."""
    c2w = np.asarray(c2w, np.float32)
    R, t = c2w[..., :3, :3], c2w[..., :3, 3]
    d = np.einsum("...ij,...j->...i", R, dirs_cam, dtype=np.float32)
    d /= np.linalg.norm(d, axis=1, keepdims=True) + np.float32(1e-12)
    rays = np.zeros(dirs_cam.shape[0], dtype=ray_dtype)
    rays["o"][:, :3] = t
    rays["o"][:, 3] = 1.0
    rays["d"][:, :3] = d
    return rays


def rays_targets_from_indices(im_idx, u_idx, v_idx, Ims, c2w_all, W, H, K=None):
    """Training rays and targets for pixels (u, v) of images im_idx (ffnerf_tools.py:175-234 of the
    reference): Ims [N, H, W, 3] (float in [0, 1], or 8-bit), c2w_all [N, 4, 4], K [3, 3], [N, 3, 3] or
    None.  Targets are {rgb, 0}."""
    im = np.asarray(im_idx, np.int32).reshape(-1)
    u = np.asarray(u_idx, np.int32).reshape(-1)
    v = np.asarray(v_idx, np.int32).reshape(-1)
    assert Ims.ndim == 4 and Ims.shape[1:3] == (H, W), (Ims.shape, H, W)
    assert len(c2w_all) == len(Ims)
    K_pix = None if K is None else (K if np.ndim(K) == 2 else np.asarray(K)[im])
    rays = world_rays(np.asarray(c2w_all)[im], camera_directions(u, v, W, H, K_pix))
    targets = np.zeros((im.size, 4), np.float32)
    rgb = Ims[im, v, u, :3]
    targets[:, :3] = rgb if rgb.dtype == np.float32 else rgb.astype(np.float32) / 255.0
    return rays, targets


def rays_from_rt_indices(RT, idx, idy, W, H, K=None):
    """Rays of pixels (idx, idy) of one camera RT [4, 4] (camera-to-world), as the training rays are made
    (ffnerf_tools.py:237-272 of the reference)."""
    RT = np.asarray(RT, np.float32)
    if RT.shape != (4, 4):
        raise ValueError(f"RT must be shape (4,4), got {RT.shape}")
    u = np.asarray(idx, np.int32).reshape(-1)
    v = np.asarray(idy, np.int32).reshape(-1)
    if u.size != v.size:
        raise ValueError("idx and idy must have the same length.")
    return world_rays(RT, camera_directions(u, v, W, H, K))


def rays_as_array(rays) -> np.ndarray:
    """Structured ray array -> contiguous float32 [n, 8]."""
    rays = np.asarray(rays)
    if rays.dtype.names:
        out = np.empty((rays.shape[0], 8), np.float32)
        out[:, :4] = rays["o"]
        out[:, 4:] = rays["d"]
        return out
    return np.ascontiguousarray(rays, np.float32).reshape(-1, 8)


# ---------------------------------------------------------------------------
# model description


def level_resolutions(n_levels: int, base: float = 16.0, finest: float | None = None,
                      growth: float | None = None) -> list[int]:
    """Per-level grid resolution R_l = max(2, rint(base * b^l)), evaluated once
    on the host in float64 (the reference evaluates pow on the device,
    ffnerf_OG.cl:1308-1311).  Either the finest resolution or the growth b."""
    out = []
    for l in range(n_levels):
        if growth is not None:
            r = base * growth ** l
        else:
            t = 0.0 if n_levels == 1 else l / (n_levels - 1)
            r = base * (finest / base) ** t
        out.append(max(2, int(np.rint(r))))
    return out


@dataclass
class ModelSpec:
    """Every compile-time knob of the reference kernels as a value."""
    n_levels: int = 16
    f_per_level: int = 4
    log2_T: list = field(default_factory=lambda: list(REF_LEVEL_LOG2))
    res: list = field(default_factory=lambda: level_resolutions(16, 16.0, 1024.0))
    nd: int = 2
    nc: int = 2
    background: str = "black"   # training background: black | white | random
    hash_opt: str = "sgd"       # sgd (reference, in-step) | adam
    mlp_precision: str = "fp32"
    table_dtype: str = "fp32"   # fp32 (reference) | fp16: the table's storage; its Adam state stays fp32
    sampler: str = "resample"   # resample (reference) | march: step() samples by the bitfield march
    march_max_steps: int = 1024
    march_dt: float | None = None   # default: the box's largest extent times sqrt(3) / march_max_steps
    march_T_stop: float = 1e-4
    march_q_min: int = 4            # cells with occupancy level q >= q_min (the inference predicate)
    init: str = "he"            # he (reference) | xavier
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-6

    @property
    def lf(self) -> int:
        return self.n_levels * self.f_per_level

    def table_entries(self) -> int:
        return int(sum(1 << int(t) for t in self.log2_T[: self.n_levels]))

    def layer_shapes(self) -> dict:
        shp = {"Wd_in": (M, self.lf), "Wd_out": (D_OUT, M), "Wc_in": (M, C_IN), "Wc_out": (C_OUT, M)}
        if self.nd >= 2:
            shp["Wd_01"] = (M, M)
        if self.nd >= 3:
            shp["Wd_12"] = (M, M)
        if self.nc >= 2:
            shp["Wc_01"] = (M, M)
        if self.nc >= 3:
            shp["Wc_12"] = (M, M)
        if self.nc >= 4:
            shp["Wc_23"] = (M, M)
        return shp


@dataclass
class OccParams:
    G_occ: int = 32
    box_min: np.ndarray = None
    box_max: np.ndarray = None
    rho_min: np.float32 = np.float32(RHO_MIN_DEF)
    rho_max: np.float32 = np.float32(RHO_MAX_DEF)
    dt_min: np.float32 = np.float32(4e-3)
    dt_max: np.float32 = np.float32(0.8)
    t_near_clip: np.float32 = np.float32(0.3)
    t_far_clip: np.float32 = np.float32(1e9)
    occ_update_strength0: np.float32 = np.float32(OCC_U_STR)
    decay: float = DECAY
    maintenance_period: int = OCC_MAINTENANCE_PERIOD

    def finalize(self):
        if self.box_min is None:
            self.box_min = np.array([-3.0, -3.0, -3.0], dtype=np.float32)
        if self.box_max is None:
            self.box_max = np.array([+3.0, +3.0, +3.0], dtype=np.float32)
        self.box_min = np.asarray(self.box_min, dtype=np.float32).reshape(3)
        self.box_max = np.asarray(self.box_max, dtype=np.float32).reshape(3)
        self.t_near_clip = np.float32(self.t_near_clip)
        self.t_far_clip = np.float32(self.t_far_clip)
        if not np.isfinite(self.t_near_clip) or self.t_near_clip < 0:
            raise ValueError("t_near_clip must be finite and nonnegative")
        if not np.isfinite(self.t_far_clip) or self.t_far_clip <= self.t_near_clip:
            raise ValueError("t_far_clip must be finite and greater than t_near_clip")
        if int(self.G_occ) < 1:
            raise ValueError("G_occ must be positive")
        return self


def spec_dict(spec: ModelSpec, occ: OccParams) -> dict:
    """Flat description shared by the library config (and the test oracle)."""
    return dict(
        n_levels=spec.n_levels, f_per_level=spec.f_per_level, log2_T=list(spec.log2_T[: spec.n_levels]),
        res=list(spec.res[: spec.n_levels]), nd=spec.nd, nc=spec.nc, occ_G=int(occ.G_occ),
        box_min=[float(v) for v in occ.box_min], box_max=[float(v) for v in occ.box_max],
        rho_min=float(occ.rho_min), rho_max=float(occ.rho_max), dt_min=float(occ.dt_min),
        dt_max=float(occ.dt_max), t_near=float(occ.t_near_clip), t_far=float(occ.t_far_clip),
        background=fl.BG[spec.background], hash_opt=fl.HASH_OPT[spec.hash_opt],
        mlp_precision=fl.MLP_PRECISION[spec.mlp_precision], table_dtype=fl.TABLE_DTYPE[spec.table_dtype],
        sampler=fl.SAMPLER[spec.sampler], march_max_steps=int(spec.march_max_steps), march_dt=spec.march_dt,
        march_T_stop=float(spec.march_T_stop), march_q_min=int(spec.march_q_min),
    )


def occ_decay_q24(strength: float, decay: float) -> int:
    """The occupancy decay factor 1 - strength (1 - decay) in 24-bit fixed point, rounded half to even and
    clamped to [0, 2^24] (ffnerf_tools.py:1453-1457): 2^24 leaves every level as it is, 0 clears it."""
    d = 1 - float(strength) * (1 - float(decay))
    return max(0, min(int(round(d * (1 << 24))), 1 << 24))


def init_params(spec: ModelSpec, occ: OccParams, rng: np.random.Generator) -> dict:
    """Fresh parameters (float32 numpy), draw order of Nerf._init_fresh
    (ffnerf_tools.py:836-895): table, then weights, then biases."""
    shapes = spec.layer_shapes()
    p = {}
    n_tab = spec.table_entries() * spec.f_per_level
    p["table"] = rng.uniform(-1e-4, 1e-4, size=n_tab).astype(np.float32)
    if spec.table_dtype == "fp16":  # the values a binary16 table holds (round to nearest even)
        p["table"] = p["table"].astype(np.float16).astype(np.float32)
    for wn in fl.LAYER_NAMES:
        if wn not in shapes:
            continue
        sh = shapes[wn]
        if spec.init == "xavier":
            lim = np.sqrt(6.0 / (sh[0] + sh[1]))
            p[wn] = rng.uniform(-lim, lim, size=sh).astype(np.float32)
        elif sh[0] <= 16:
            p[wn] = rng.normal(0.0, 0.01, size=sh).astype(np.float32)
        else:
            p[wn] = rng.normal(0.0, np.sqrt(2.0 / sh[1]), size=sh).astype(np.float32)
    for wn, bn in zip(fl.LAYER_NAMES, fl.BIAS_NAMES):
        if wn not in shapes:
            continue
        b = np.zeros(shapes[wn][0], np.float32)
        if bn == "bd_out":
            b[0] = SIGMA_BIAS
        if bn == "bc_2" and spec.init != "xavier":
            b = rng.normal(-2.0, 0.05, size=b.shape).astype(np.float32)
        p[bn] = b
    for wn, bn in zip(fl.LAYER_NAMES, fl.BIAS_NAMES):
        if wn not in shapes:
            continue
        for pre in ("m", "v"):
            p[pre + wn] = np.zeros_like(p[wn])
            p[pre + bn] = np.zeros_like(p[bn])
    p["m_table"] = np.zeros_like(p["table"])
    p["v_table"] = np.zeros_like(p["table"])
    n_occ = int(occ.G_occ) ** 3
    p["occ_in"] = np.full(n_occ, OCC_INIT_DENSITY, np.uint32)
    p["occ_st"] = np.full(n_occ, OCC_INIT_DENSITY, np.uint32)
    return p


# ---------------------------------------------------------------------------
# device buffers


def _torch():
    import torch
    return torch


def _dev_tensor(arr: np.ndarray, device):
    torch = _torch()
    if arr.dtype == np.uint32:
        t = torch.from_numpy(arr.view(np.int32).copy())
    else:
        t = torch.from_numpy(np.ascontiguousarray(arr))
    return t.to(device)


def _to_numpy(t, dtype=None) -> np.ndarray:
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


@dataclass
class RayBatch:
    """Per-batch rays/targets/output device buffers (ffnerf_tools.py:281-395)."""
    num_rays: int
    samples_per_ray: int
    device: str = "cuda"
    rays_buf: object = None     # torch float32 [n, 8]
    targets_buf: object = None  # torch float32 [n, 4]
    out_buf: object = None      # torch float32 [n, 4]
    ev_last: object = None

    def __post_init__(self):
        self.num_rays = int(self.num_rays)
        self.samples_per_ray = int(self.samples_per_ray)
        if self.num_rays <= 0 or self.samples_per_ray <= 0:
            raise ValueError("num_rays and samples_per_ray must be > 0")

    @property
    def B_total(self) -> int:
        return self.num_rays * self.samples_per_ray

    @classmethod
    def init(cls, num_rays: int, samples_per_ray: int, device="cuda", **_ignored) -> "RayBatch":
        torch = _torch()
        rb = cls(num_rays=num_rays, samples_per_ray=samples_per_ray, device=device)
        rb.rays_buf = torch.zeros((rb.num_rays, 8), dtype=torch.float32, device=device)
        rb.targets_buf = torch.zeros((rb.num_rays, 4), dtype=torch.float32, device=device)
        rb.out_buf = torch.zeros((rb.num_rays, 4), dtype=torch.float32, device=device)
        return rb

    def upload_rays(self, rays, wait: bool = False):
        arr = rays_as_array(rays)
        if arr.shape != (self.num_rays, 8):
            raise ValueError(f"rays must be shape ({self.num_rays},), got {np.asarray(rays).shape}")
        self.rays_buf.copy_(_torch().from_numpy(arr), non_blocking=False)
        return self._event(wait)

    def upload_targets(self, targets, wait: bool = False):
        targets = np.asarray(targets, dtype=np.float32)
        if targets.shape != (self.num_rays, 4):
            raise ValueError(f"targets must be shape ({self.num_rays},4), got {targets.shape}")
        self.targets_buf.copy_(_torch().from_numpy(np.ascontiguousarray(targets)))
        return self._event(wait)

    def download_out(self, out: Optional[np.ndarray] = None, wait: bool = True, wait_for=None):
        res = self.out_buf.detach().cpu().numpy()
        if out is not None:
            out[...] = res
            res = out
        return res, self._event(True)

    def _event(self, wait: bool):
        torch = _torch()
        ev = torch.cuda.Event()
        ev.record()
        if wait:
            ev.synchronize()
        return ev


# ---------------------------------------------------------------------------


class Nerf:
    """Model container: device parameters, Adam state, occupancy grids; step()
    enqueues one fused training step (or a forward-only render) through
    ffn_train_step, then the occupancy maintenance pass when it is due."""

    def __init__(self, training_dir, model_id: str, spec: ModelSpec | None = None, occ: OccParams | None = None,
                 load_id: str | None = None, rng_seed: int = 777, device: str = "cuda"):
        self.training_dir = Path(training_dir)
        self.training_dir.mkdir(parents=True, exist_ok=True)
        self.model_id = model_id
        self.spec = spec or ModelSpec()
        self.occ = (occ or OccParams()).finalize()
        self.device = device
        self.rng = np.random.default_rng(int(rng_seed))
        self.steps_trained = 0
        self.transfer_fmt = "fp32"
        self.handle = None
        self.t = {}
        if load_id:
            host = self.load_latest(load_id, push=False)
        else:
            host = init_params(self.spec, self.occ, self.rng)
        self._upload(host)

    # -- state -----------------------------------------------------------
    @property
    def ND(self):
        return self.spec.nd

    @property
    def NC(self):
        return self.spec.nc

    def _upload(self, host: dict):
        f16 = self.spec.table_dtype == "fp16"
        self.t = {k: _dev_tensor(v.astype(np.float16) if (k == "table" and f16) else v, self.device)
                  for k, v in host.items()}
        self._rebind()

    def _rebind(self):
        if self.handle is not None:
            self.handle.close()
        self.handle = fl.Handle(spec_dict(self.spec, self.occ))
        P = fl.FfnParams()
        for i, (wn, bn) in enumerate(zip(fl.LAYER_NAMES, fl.BIAS_NAMES)):
            if wn in self.t:
                P.W[i] = fl.ptr(self.t[wn])
                P.b[i] = fl.ptr(self.t[bn])
                P.mW[i] = fl.ptr(self.t["m" + wn])
                P.vW[i] = fl.ptr(self.t["v" + wn])
                P.mb[i] = fl.ptr(self.t["m" + bn])
                P.vb[i] = fl.ptr(self.t["v" + bn])
        P.table = fl.ptr(self.t["table"])
        P.m_table = fl.ptr(self.t["m_table"])
        P.v_table = fl.ptr(self.t["v_table"])
        P.occ_in = fl.ptr(self.t["occ_in"])
        P.occ_st = fl.ptr(self.t["occ_st"])
        self.handle.bind(P, keep=self.t)

    def host_state(self) -> dict:
        _torch().cuda.synchronize()
        out = {}
        for k, v in self.t.items():
            out[k] = _to_numpy(v, np.uint32 if k.startswith("occ_") else None).copy()
        out["table"] = out["table"].astype(np.float32)  # a binary16 table widens exactly
        return out

    def setup_buffers(self, num_rays: int, samples_per_ray: int, do_train=None):
        """Scratch is sized by the library on the first step of a shape."""
        self.num_rays = int(num_rays)
        self.samples_per_ray = int(samples_per_ray)

    def _get_rng_u32(self) -> np.uint32:
        return np.uint32(self.rng.integers(0, 2 ** 32, dtype=np.uint32))

    def adam_lr_t(self, lr_f: float, t: int) -> np.float32:
        """lr_t = lr_f sqrt(1 - b2^t) / (1 - b1^t) in float32 (ffnerf_tools.py:1479-1482)."""
        b1 = np.float32(self.spec.beta1)
        b2 = np.float32(self.spec.beta2)
        b1t = b1 ** np.float32(t)
        b2t = b2 ** np.float32(t)
        return np.float32(np.float32(lr_f) * np.sqrt(np.float32(1.0) - b2t) / (np.float32(1.0) - b1t))

    # -- the step ----------------------------------------------------------
    def step(self, io: RayBatch, lr_f: float, do_train: bool, return_output: bool = False,
             sh_multiplier: float = 1.0, color_MLP_rel_lr: float = 1.0, occ_update_strength: float | None = None,
             rng_u32: np.uint32 | None = None, wait: bool = False, taps: fl.FfnTaps | None = None, stream=None,
             **_launch_geometry):
        if io.samples_per_ray > S_MAX or (io.samples_per_ray & (io.samples_per_ray - 1)):
            raise ValueError(f"samples_per_ray={io.samples_per_ray} must be a power of two <= {S_MAX}")
        if occ_update_strength is None:
            occ_update_strength = float(self.occ.occ_update_strength0 if do_train else 0.0)
        if rng_u32 is None:
            rng_u32 = self._get_rng_u32()
        if do_train:
            self.steps_trained = int(self.steps_trained) + 1
        sc = fl.FfnStepScalars()
        sc.lr = float(np.float32(lr_f))
        sc.lr_t = float(self.adam_lr_t(lr_f, self.steps_trained)) if do_train else 0.0
        sc.color_rel_lr = float(color_MLP_rel_lr)
        sc.sh_multiplier = float(sh_multiplier)
        sc.occ_strength = float(occ_update_strength)
        sc.beta1, sc.beta2, sc.eps = float(self.spec.beta1), float(self.spec.beta2), float(self.spec.eps)
        sc.rng_seed = int(rng_u32) & 0xFFFFFFFF
        sc.do_train = 1 if do_train else 0
        sp = fl.stream_ptr(stream)
        lib = self.handle.lib
        fl.check(lib.ffn_train_step(self.handle.h, fl.ptr(io.rays_buf), fl.ptr(io.targets_buf), fl.ptr(io.out_buf),
                                    io.num_rays, io.samples_per_ray, C.byref(sc),
                                    C.byref(taps) if taps is not None else None, sp), "ffn_train_step")
        # the occupancy maintenance of ffnerf_tools.py:1424-1476; with the march sampler the proposals of the
        # marched runs and this decay keep the grid, so the next steps' bitfield, following the density
        if (do_train and float(occ_update_strength) > 0.0
                and self.steps_trained % int(self.occ.maintenance_period) == 0):
            decay_q24 = occ_decay_q24(occ_update_strength, self.occ.decay)
            n_words = int(self.occ.G_occ) ** 3
            fl.check(lib.ffn_occ_decay(fl.ptr(self.t["occ_in"]), fl.ptr(self.t["occ_st"]), n_words, decay_q24,
                                       int(rng_u32) & 0xFFFFFFFF, sp), "ffn_occ_decay")
        torch = _torch()
        ev = torch.cuda.Event()
        ev.record()
        io.ev_last = ev
        if return_output:
            out, _ = io.download_out(wait=True)
            return out, ev
        if wait:
            ev.synchronize()
        return None, ev

    # -- forward render with the DDA marcher (no counterpart in the reference) --
    def occupancy_bitfield(self, q_min: int = 4, out=None):
        """Bitfield of the (2G)^3 occupancy subcells with q >= q_min (q = nibble + 1).  The default keeps
        the subcells the reference's inference sampler gives non-zero weight (q_infer > 0, i.e. nibble >= 3,
        ffnerf_OG.cl:1116)."""
        torch = _torch()
        G = int(self.occ.G_occ)
        R = 2 * G
        if out is None:
            out = torch.zeros((R ** 3 + 31) // 32, dtype=torch.int32, device=self.device)
        fl.check(self.handle.lib.ffn_occ_bitfield(fl.ptr(self.t["occ_in"]), G, int(q_min), fl.ptr(out),
                                                  fl.stream_ptr()), "ffn_occ_bitfield")
        return out

    def step_marched(self, io: RayBatch, lr_f: float, bits, res: int, dt: float, max_steps: int = 1024,
                     T_stop: float = 1e-4, sh_multiplier: float = 1.0, color_MLP_rel_lr: float = 1.0,
                     rng_u32: np.uint32 | None = None, n_samples=None, taps: fl.FfnTaps | None = None, stream=None,
                     sample_capacity: int = 0):
        """A training step whose samples come from the bitfield march instead of the resampler (the step of
        ffnerf_tools.py:1446-1530 with ffn_train_step_marched): io's rays and targets, the same learning-rate
        schedule and Adam counter as step().  The occupancy grid is not updated (the bitfield is an input);
        n_samples (optional, device [num_rays]) gets the samples composited per ray.  With sample_capacity 0 it
        waits on the stream once inside, after the march's count; with sample_capacity C > 0 it does not wait
        and trains the rays whose samples fit into the first C slots of the march order (the later rays are
        dropped: no samples, background colour)."""
        if rng_u32 is None:
            rng_u32 = self._get_rng_u32()
        self.steps_trained = int(self.steps_trained) + 1
        sc = fl.FfnStepScalars()
        sc.lr = float(np.float32(lr_f))
        sc.lr_t = float(self.adam_lr_t(lr_f, self.steps_trained))
        sc.color_rel_lr = float(color_MLP_rel_lr)
        sc.sh_multiplier = float(sh_multiplier)
        sc.occ_strength = 0.0
        sc.beta1, sc.beta2, sc.eps = float(self.spec.beta1), float(self.spec.beta2), float(self.spec.eps)
        sc.rng_seed = int(rng_u32) & 0xFFFFFFFF
        sc.do_train = 1
        mp = fl.march_params(res, dt, max_steps, T_stop=T_stop, sh_multiplier=sh_multiplier,
                             sample_capacity=sample_capacity)
        fl.check(self.handle.lib.ffn_train_step_marched(
            self.handle.h, fl.ptr(io.rays_buf), fl.ptr(io.targets_buf), fl.ptr(io.out_buf), io.num_rays,
            fl.ptr(bits), C.byref(mp), C.byref(sc), C.byref(taps) if taps is not None else None, fl.ptr(n_samples),
            fl.stream_ptr(stream)), "ffn_train_step_marched")
        torch = _torch()
        ev = torch.cuda.Event()
        ev.record()
        io.ev_last = ev
        return ev

    def render_marched(self, io: RayBatch, bits, res: int, dt: float, max_steps: int = 1024, T_stop: float = 1e-4,
                       chunk: int = 32, sh_multiplier: float = 1.0, n_samples=None, stream=None,
                       no_wait: bool = False):
        """Forward-only render of io's rays: bitfield DDA march, MLPs, front-to-back compositing stopped at
        T < T_stop.  io.out_buf gets {r, g, b, T_final} per ray (black background).  no_wait: every round is
        enqueued and sized on the device (no wait on the stream; the same results)."""
        mp = fl.march_params(res, dt, max_steps, T_stop=T_stop, chunk=chunk, sh_multiplier=sh_multiplier,
                             flags=fl.RENDER_NO_WAIT if no_wait else 0)
        fl.check(self.handle.lib.ffn_render(self.handle.h, fl.ptr(io.rays_buf), io.num_rays, fl.ptr(bits),
                                            C.byref(mp), fl.ptr(io.out_buf), fl.ptr(n_samples),
                                            fl.stream_ptr(stream)), "ffn_render")
        torch = _torch()
        ev = torch.cuda.Event()
        ev.record()
        io.ev_last = ev
        return ev

    # -- checkpoints (npz layout of ffnerf_tools.py:989-1189) --------------
    def _checkpoint_payload(self) -> dict:
        """The npz contents: the reference's keys and int32 bit-pattern storage (ffnerf_tools.py:989-1086),
        plus this build's per-level layout, options and the table's Adam state."""
        st = self.host_state()
        bits = lambda a: np.ascontiguousarray(a, np.float32).view(np.int32).reshape(-1)
        sp, oc = self.spec, self.occ
        payload = dict(
            timestamp=datetime.now().strftime("%Y%m%d-%H%M%S"), model_id=self.model_id,
            steps_trained=np.int32(self.steps_trained), transfer_fmt=np.array(self.transfer_fmt),
            ND=np.int32(sp.nd), NC=np.int32(sp.nc), table_i=bits(st["table"]),
            table_size_entries=np.int32(sp.table_entries()), table_f_per_level=np.int32(sp.f_per_level),
            occ_grid_in_u32=st["occ_in"].astype(np.uint32), occ_grid_st_u32=st["occ_st"].astype(np.uint32),
            G_occ=np.int32(oc.G_occ), box_min=np.asarray(oc.box_min, np.float32),
            box_max=np.asarray(oc.box_max, np.float32),
            level_log2_T=np.asarray(sp.log2_T[: sp.n_levels], np.int32),
            level_res=np.asarray(sp.res[: sp.n_levels], np.int32), n_levels=np.int32(sp.n_levels),
            hash_opt=np.array(sp.hash_opt), table_dtype=np.array(sp.table_dtype), background=np.array(sp.background),
            init=np.array(sp.init), adam_beta1=np.float32(sp.beta1), adam_beta2=np.float32(sp.beta2),
            adam_eps=np.float32(sp.eps), m_table_i=bits(st["m_table"]), v_table_i=bits(st["v_table"]),
        )
        for k in ("rho_min", "rho_max", "dt_min", "dt_max", "t_near_clip", "t_far_clip"):
            payload[k] = np.float32(getattr(oc, k))
        shapes = sp.layer_shapes()
        names = sorted(list(shapes) + [fl.BIAS_NAMES[fl.LAYER_NAMES.index(wn)] for wn in shapes])
        payload["active_params"] = np.array(names, dtype="U32")
        for name in names:
            for pre in ("", "m", "v"):
                payload[f"{pre}{name}_i"] = bits(st[pre + name])
        return payload

    def _checkpoint_targets(self, min_new_file_seconds: float) -> list:
        """Files one save writes.  `<id>_weights_latest.npz` always; a new `<id>_weights_<timestamp>.npz`
        besides it unless the latest file is younger than min_new_file_seconds (so frequent saves refresh
        one file while a history of snapshots accumulates at that spacing)."""
        d = self.training_dir
        d.mkdir(parents=True, exist_ok=True)
        latest = d / f"{self.model_id}_weights_latest.npz"
        try:
            age = time.time() - latest.stat().st_mtime
        except OSError:  # no latest file yet (or unreadable): start a new snapshot
            age = float("inf")
        if age < float(min_new_file_seconds):
            return [latest]
        return [d / f"{self.model_id}_weights_{datetime.now().strftime('%Y%m%d-%H%M%S')}.npz", latest]

    def save(self, min_new_file_seconds: int = 300) -> Path:
        """Write a checkpoint; returns the file named for this save (the new snapshot, or the latest file)."""
        targets = self._checkpoint_targets(min_new_file_seconds)
        np.savez_compressed(targets[0], **self._checkpoint_payload())
        for extra in targets[1:]:
            shutil.copyfile(targets[0], extra)
        return targets[0]

    def load_latest(self, load_id: str, push: bool = True) -> dict:
        td = self.training_dir
        pats = sorted(td.glob(f"{load_id}_weights_*.npz"))
        path = max(pats, key=lambda p: p.stat().st_mtime_ns) if pats else None
        if path is None:
            raise FileNotFoundError(f"No saved model found for id='{load_id}' in {td.resolve()}")
        data = np.load(path, allow_pickle=False)
        i2f = lambda a: np.asarray(a, np.int32).reshape(-1).view(np.float32).copy()
        nd, nc = int(data["ND"]), int(data["NC"])
        f = int(data["table_f_per_level"])
        if "level_log2_T" in data.files:
            log2_T = [int(v) for v in data["level_log2_T"]]
            res = [int(v) for v in data["level_res"]]
        else:  # a checkpoint of the reference: its compiled-in hash layout
            log2_T = list(REF_LEVEL_LOG2)
            res = level_resolutions(16, 16.0, 1024.0)
        self.spec = ModelSpec(
            n_levels=len(log2_T), f_per_level=f, log2_T=log2_T, res=res, nd=nd, nc=nc,
            background=str(data["background"]) if "background" in data.files else self.spec.background,
            hash_opt=str(data["hash_opt"]) if "hash_opt" in data.files else "sgd",
            mlp_precision=self.spec.mlp_precision,
            table_dtype=str(data["table_dtype"]) if "table_dtype" in data.files else "fp32",
            init=str(data["init"]) if "init" in data.files else "he",
            beta1=float(data["adam_beta1"]) if "adam_beta1" in data.files else self.spec.beta1,
            beta2=float(data["adam_beta2"]) if "adam_beta2" in data.files else self.spec.beta2,
            eps=float(data["adam_eps"]) if "adam_eps" in data.files else self.spec.eps,
        )
        self.transfer_fmt = str(data["transfer_fmt"].item())
        self.occ = OccParams(
            G_occ=int(data["G_occ"]), box_min=np.asarray(data["box_min"], np.float32),
            box_max=np.asarray(data["box_max"], np.float32), rho_min=np.float32(data["rho_min"]),
            rho_max=np.float32(data["rho_max"]), dt_min=np.float32(data["dt_min"]),
            dt_max=np.float32(data["dt_max"]), t_near_clip=np.float32(data["t_near_clip"]),
            t_far_clip=np.float32(data["t_far_clip"]), occ_update_strength0=self.occ.occ_update_strength0,
            decay=self.occ.decay, maintenance_period=self.occ.maintenance_period,
        ).finalize()
        self.steps_trained = int(data["steps_trained"]) if "steps_trained" in data.files else 0
        host = {"table": i2f(data["table_i"])}
        shapes = self.spec.layer_shapes()
        for name in [str(x) for x in data["active_params"].tolist()]:
            host[name] = i2f(data[name + "_i"])
            host["m" + name] = i2f(data["m" + name + "_i"])
            host["v" + name] = i2f(data["v" + name + "_i"])
        for wn in shapes:
            host[wn] = host[wn].reshape(shapes[wn])
            for pre in ("m", "v"):
                host[pre + wn] = host[pre + wn].reshape(shapes[wn])
        n_tab = host["table"].size
        host["m_table"] = i2f(data["m_table_i"]) if "m_table_i" in data.files else np.zeros(n_tab, np.float32)
        host["v_table"] = i2f(data["v_table_i"]) if "v_table_i" in data.files else np.zeros(n_tab, np.float32)
        host["occ_in"] = np.asarray(data["occ_grid_in_u32"], np.uint32).reshape(-1).copy()
        host["occ_st"] = np.asarray(data["occ_grid_st_u32"], np.uint32).reshape(-1).copy()
        if push:
            self._upload(host)
        return host

    def sync_params_from_device(self) -> dict:
        return self.host_state()
