"""Drive libffnerf_hip.so through its C ABI from the tests (torch tensors as
device buffers), with the same spec/parameter dictionaries the oracle takes."""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

import ffn_lib as fl

DEV = "cuda"


def to_dev(a: np.ndarray):
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32).copy()).to(DEV)
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def to_np(t, dtype=None):
    a = t.detach().cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def table_f16(spec) -> bool:
    return spec.get("table_dtype", 0) in (1, "fp16")


class GpuModel:
    """With an fp16 table (spec table_dtype), params["table"] holds binary16 values as float32: it is uploaded
    as float16 (exactly) and state() widens it back."""

    def __init__(self, spec: dict, params: dict):
        self.spec = dict(spec)
        self.h = fl.Handle(spec)
        self.f16 = table_f16(spec)
        self.t = {k: to_dev(v.astype(np.float16) if (k == "table" and self.f16) else v) for k, v in params.items()}
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
        self.h.bind(P, keep=self.t)
        self.lib = self.h.lib

    def state(self) -> dict:
        torch.cuda.synchronize()
        out = {k: to_np(v, np.uint32 if k.startswith("occ_") else None).copy() for k, v in self.t.items()}
        out["table"] = out["table"].astype(np.float32)
        return out

    def train_step(self, rays, targets, S, scalars: dict, taps=False):
        rays_t = to_dev(np.ascontiguousarray(rays, np.float32).reshape(-1, 8))
        tg_t = to_dev(np.ascontiguousarray(targets, np.float32).reshape(-1, 4))
        N = rays_t.shape[0]
        out = torch.zeros((N, 4), dtype=torch.float32, device=DEV)
        sc = fl.FfnStepScalars()
        for k in ("lr", "lr_t", "color_rel_lr", "sh_multiplier", "occ_strength", "beta1", "beta2", "eps"):
            setattr(sc, k, float(scalars[k]))
        sc.rng_seed = int(scalars["rng_seed"]) & 0xFFFFFFFF
        sc.do_train = int(bool(scalars.get("do_train", 1)))
        tp = None
        td = None
        if taps:
            LF = self.spec["n_levels"] * self.spec["f_per_level"]
            z = lambda *s: torch.zeros(s, dtype=torch.float32, device=DEV)
            td = dict(Ts=z(N * S), DTs=z(N * S), flags=torch.zeros(N * 2, dtype=torch.int32, device=DEV),
                      a0=z(N * S, LF), sigma=z(N * S), rgb=z(N * S, 3), Tr=z(N * S), T_final=z(N), dL_dsigma=z(N * S),
                      dL_dc=z(N * S, 3), dL_da0=z(N * S, LF),
                      relu=torch.zeros((N * S, fl.RELU_WORDS), dtype=torch.int32, device=DEV), C=z(N, 4))
            tp = fl.FfnTaps()
            for k, v in td.items():
                setattr(tp, "color" if k == "C" else k, fl.ptr(v))
            for i, wn in enumerate(fl.LAYER_NAMES):
                if wn in self.t:
                    bn = fl.BIAS_NAMES[i]
                    td["g" + wn] = torch.zeros_like(self.t[wn])
                    td["g" + bn] = torch.zeros_like(self.t[bn])
                    tp.gW[i] = fl.ptr(td["g" + wn])
                    tp.gb[i] = fl.ptr(td["g" + bn])
            if self.spec.get("hash_opt", 0) == 1:
                td["g_table"] = torch.zeros(self.t["table"].shape, dtype=torch.float32, device=DEV)
                tp.g_table = fl.ptr(td["g_table"])
        fl.check(self.lib.ffn_train_step(self.h.h, fl.ptr(rays_t), fl.ptr(tg_t), fl.ptr(out), N, S, C.byref(sc),
                                         C.byref(tp) if tp is not None else None, fl.stream_ptr()), "ffn_train_step")
        torch.cuda.synchronize()
        res = None
        if taps:
            res = {k: to_np(v) for k, v in td.items()}
            res["flags"] = res["flags"].view(np.uint32)
            res["relu"] = res["relu"].view(np.uint32)
        return to_np(out), res

    def sample(self, rays, S, seed, do_train=1):
        rays_t = to_dev(np.ascontiguousarray(rays, np.float32).reshape(-1, 8))
        N = rays_t.shape[0]
        Ts = torch.zeros(N * S, dtype=torch.float32, device=DEV)
        DTs = torch.zeros(N * S, dtype=torch.float32, device=DEV)
        flags = torch.zeros(N * 2, dtype=torch.int32, device=DEV)
        fl.check(self.lib.ffn_sample(self.h.h, fl.ptr(rays_t), N, S, seed & 0xFFFFFFFF, do_train, fl.ptr(Ts),
                                     fl.ptr(DTs), fl.ptr(flags), fl.stream_ptr()), "ffn_sample")
        torch.cuda.synchronize()
        return to_np(Ts).reshape(N, S), to_np(DTs).reshape(N, S), to_np(flags, np.uint32).reshape(N, 2)

    def encode(self, x, with_idx=False):
        x_t = to_dev(np.ascontiguousarray(x, np.float32).reshape(-1, 3))
        n = x_t.shape[0]
        LF = self.spec["n_levels"] * self.spec["f_per_level"]
        a0 = torch.zeros((n, LF), dtype=torch.float32, device=DEV)
        idx = torch.zeros((n, self.spec["n_levels"], 8), dtype=torch.int32, device=DEV) if with_idx else None
        fl.check(self.lib.ffn_hash_encode_fwd(self.h.h, fl.ptr(x_t), n, fl.ptr(a0), fl.ptr(idx), fl.stream_ptr()),
                 "ffn_hash_encode_fwd")
        torch.cuda.synchronize()
        return (to_np(a0), to_np(idx, np.uint32)) if with_idx else to_np(a0)

    def encode_bwd(self, x, g, table_n):
        x_t = to_dev(np.ascontiguousarray(x, np.float32).reshape(-1, 3))
        g_t = to_dev(np.ascontiguousarray(g, np.float32))
        grad = torch.zeros(table_n, dtype=torch.float16 if self.f16 else torch.float32, device=DEV)
        fl.check(self.lib.ffn_hash_encode_bwd(self.h.h, fl.ptr(x_t), fl.ptr(g_t), x_t.shape[0], fl.ptr(grad),
                                              fl.stream_ptr()), "ffn_hash_encode_bwd")
        torch.cuda.synchronize()
        return to_np(grad).astype(np.float32)

    def bitfield(self, occ: np.ndarray, G: int, q_min: int) -> np.ndarray:
        occ_t = to_dev(np.ascontiguousarray(occ, np.uint32))
        R = 2 * G
        bits = torch.zeros((R ** 3 + 31) // 32, dtype=torch.int32, device=DEV)
        fl.check(self.lib.ffn_occ_bitfield(fl.ptr(occ_t), G, q_min, fl.ptr(bits), fl.stream_ptr()),
                 "ffn_occ_bitfield")
        torch.cuda.synchronize()
        return to_np(bits, np.uint32)

    def march(self, rays, bits, mp, capacity=None):
        rays_t = to_dev(np.ascontiguousarray(rays, np.float32).reshape(-1, 8))
        bits_t = to_dev(np.ascontiguousarray(bits, np.uint32))
        N = rays_t.shape[0]
        cap = N * mp.max_steps if capacity is None else capacity
        counts = torch.zeros(N, dtype=torch.int32, device=DEV)
        offsets = torch.zeros(N, dtype=torch.int32, device=DEV)
        samples = torch.zeros((max(cap, 1), 4), dtype=torch.float32, device=DEV)
        ids = torch.zeros(max(cap, 1), dtype=torch.int32, device=DEV)
        total = torch.zeros(4, dtype=torch.int32, device=DEV)
        fl.check(self.lib.ffn_march(self.h.h, fl.ptr(rays_t), N, fl.ptr(bits_t), C.byref(mp), fl.ptr(counts),
                                    fl.ptr(offsets), fl.ptr(samples), fl.ptr(ids), cap, fl.ptr(total),
                                    fl.stream_ptr()), "ffn_march")
        torch.cuda.synchronize()
        return (to_np(counts, np.uint32), to_np(offsets, np.uint32), to_np(samples), to_np(ids, np.uint32),
                int(to_np(total, np.uint32)[0]))

    def render(self, rays, bits, mp):
        rays_t = to_dev(np.ascontiguousarray(rays, np.float32).reshape(-1, 8))
        bits_t = to_dev(np.ascontiguousarray(bits, np.uint32))
        N = rays_t.shape[0]
        out = torch.zeros((N, 4), dtype=torch.float32, device=DEV)
        used = torch.zeros(N, dtype=torch.int32, device=DEV)
        fl.check(self.lib.ffn_render(self.h.h, fl.ptr(rays_t), N, fl.ptr(bits_t), C.byref(mp), fl.ptr(out),
                                     fl.ptr(used), fl.stream_ptr()), "ffn_render")
        torch.cuda.synchronize()
        return to_np(out), to_np(used)

    def step_marched_plain(self, rays, targets, bits, mp, scalars: dict):
        """ffn_train_step_marched without taps (so that mp.sample_capacity may be set): (out [N,4], n_used [N])."""
        rays_t = to_dev(np.ascontiguousarray(rays, np.float32).reshape(-1, 8))
        tg_t = to_dev(np.ascontiguousarray(targets, np.float32).reshape(-1, 4))
        bits_t = to_dev(np.ascontiguousarray(bits, np.uint32))
        N = rays_t.shape[0]
        out = torch.zeros((N, 4), dtype=torch.float32, device=DEV)
        used = torch.zeros(N, dtype=torch.int32, device=DEV)
        sc = fl.FfnStepScalars()
        for k in ("lr", "lr_t", "color_rel_lr", "sh_multiplier", "occ_strength", "beta1", "beta2", "eps"):
            setattr(sc, k, float(scalars[k]))
        sc.rng_seed = int(scalars["rng_seed"]) & 0xFFFFFFFF
        sc.do_train = 1
        fl.check(self.lib.ffn_train_step_marched(self.h.h, fl.ptr(rays_t), fl.ptr(tg_t), fl.ptr(out), N,
                                                 fl.ptr(bits_t), C.byref(mp), C.byref(sc), None, fl.ptr(used),
                                                 fl.stream_ptr()), "ffn_train_step_marched")
        torch.cuda.synchronize()
        return to_np(out), to_np(used, np.uint32)

    def train_step_marched(self, rays, targets, bits, mp, scalars: dict):
        """ffn_train_step_marched with every tap.  The step's samples (and so the taps' length) come from an
        ffn_march of the same rays first, which also gives the sample times (Ts), positions (x) and samples
        marched per ray (n_march).  Returns (out [N,4], n_used [N], taps)."""
        counts, _, smp, _, n = self.march(rays, bits, mp)
        rays_t = to_dev(np.ascontiguousarray(rays, np.float32).reshape(-1, 8))
        tg_t = to_dev(np.ascontiguousarray(targets, np.float32).reshape(-1, 4))
        bits_t = to_dev(np.ascontiguousarray(bits, np.uint32))
        N = rays_t.shape[0]
        out = torch.zeros((N, 4), dtype=torch.float32, device=DEV)
        used = torch.zeros(N, dtype=torch.int32, device=DEV)
        sc = fl.FfnStepScalars()
        for k in ("lr", "lr_t", "color_rel_lr", "sh_multiplier", "occ_strength", "beta1", "beta2", "eps"):
            setattr(sc, k, float(scalars[k]))
        sc.rng_seed = int(scalars["rng_seed"]) & 0xFFFFFFFF
        sc.do_train = 1
        LF = self.spec["n_levels"] * self.spec["f_per_level"]
        nz = max(n, 1)
        z = lambda *s: torch.zeros(s, dtype=torch.float32, device=DEV)
        td = dict(a0=z(nz, LF), sigma=z(nz), rgb=z(nz, 3), Tr=z(nz), T_final=z(N), dL_dsigma=z(nz), dL_dc=z(nz, 3),
                  dL_da0=z(nz, LF), relu=torch.zeros((nz, fl.RELU_WORDS), dtype=torch.int32, device=DEV), C=z(N, 4))
        tp = fl.FfnTaps()
        for k, v in td.items():
            setattr(tp, "color" if k == "C" else k, fl.ptr(v))
        for i, wn in enumerate(fl.LAYER_NAMES):
            if wn in self.t:
                bn = fl.BIAS_NAMES[i]
                td["g" + wn] = torch.zeros_like(self.t[wn])
                td["g" + bn] = torch.zeros_like(self.t[bn])
                tp.gW[i] = fl.ptr(td["g" + wn])
                tp.gb[i] = fl.ptr(td["g" + bn])
        if self.spec.get("hash_opt", 0) == 1:
            td["g_table"] = torch.zeros(self.t["table"].shape, dtype=torch.float32, device=DEV)
            tp.g_table = fl.ptr(td["g_table"])
        fl.check(self.lib.ffn_train_step_marched(self.h.h, fl.ptr(rays_t), fl.ptr(tg_t), fl.ptr(out), N,
                                                 fl.ptr(bits_t), C.byref(mp), C.byref(sc), C.byref(tp), fl.ptr(used),
                                                 fl.stream_ptr()), "ffn_train_step_marched")
        torch.cuda.synchronize()
        res = {k: to_np(v) for k, v in td.items()}
        res["relu"] = res["relu"].view(np.uint32)
        for k in ("a0", "sigma", "rgb", "Tr", "dL_dsigma", "dL_dc", "dL_da0", "relu"):
            res[k] = res[k][:n]
        res["Ts"] = smp[:n, 3].copy()
        res["x"] = smp[:n, :3].copy()
        res["n_march"] = counts.astype(np.int64)
        return to_np(out), to_np(used, np.uint32), res
