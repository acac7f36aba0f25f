"""Writes a checkpoint in the reference's npz layout (ffnerf_tools.py:989-1086
of the reference, read as text; nothing of the reference is imported): the
keys its Nerf.save writes and nothing else -- int32 bit patterns of float32
values, the reference's compiled-in hash layout (16 levels, F = 4,
2,260,992 entries), ND = NC = 2, and only the active layers, each with its m
and v.  The file is made at test time (about 40 MB uncompressed), so no
binary is committed; `write` is deterministic for a seed.

    python tests/golden/reference_checkpoint.py OUT_DIR MODEL_ID
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

LEVEL_LOG2 = [13, 13, 13, 13, 15, 15, 15, 15, 17, 17, 17, 17, 18, 18, 19, 19]  # ffnerf_OG.cl:179-200
F = 4
M, D_OUT, C_IN, C_OUT = 64, 16, 32, 3
SHAPES = {  # ND = NC = 2: density LF -> 64 -> 64 -> 16, colour 32 -> 64 -> 64 -> 3, weights [out][in]
    "Wd_in": (M, 16 * F), "Wd_01": (M, M), "Wd_out": (D_OUT, M),
    "Wc_in": (M, C_IN), "Wc_01": (M, M), "Wc_out": (C_OUT, M),
}
BIASES = {"bd_0": M, "bd_1": M, "bd_out": D_OUT, "bc_0": M, "bc_1": M, "bc_out": C_OUT}
G_OCC = 32


def _bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.int32)


def payload(seed: int = 0, steps_trained: int = 1234) -> dict:
    rng = np.random.default_rng(seed)
    entries = sum(1 << t for t in LEVEL_LOG2)
    p = dict(
        timestamp="20260101-000000", model_id="refckpt", steps_trained=np.int32(steps_trained),
        transfer_fmt=np.array("fp32"), ND=np.int32(2), NC=np.int32(2),
        table_i=_bits(rng.uniform(-0.05, 0.05, entries * F)), table_size_entries=np.int32(entries),
        table_f_per_level=np.int32(F),
        occ_grid_in_u32=np.full(G_OCC ** 3, 0xEEEEEEEE, np.uint32),
        occ_grid_st_u32=np.full(G_OCC ** 3, 0xEEEEEEEE, np.uint32),
        G_occ=np.int32(G_OCC), box_min=np.full(3, -3.0, np.float32), box_max=np.full(3, 3.0, np.float32),
        rho_min=np.float32(1.0), rho_max=np.float32(64.0), dt_min=np.float32(6.0 / 8192),
        dt_max=np.float32(0.2), t_near_clip=np.float32(0.3), t_far_clip=np.float32(1e9),
    )
    names = sorted(list(SHAPES) + list(BIASES))
    p["active_params"] = np.array(names, dtype="U32")
    for name in names:
        shape = SHAPES.get(name, (BIASES.get(name),))
        fan_in = shape[1] if len(shape) == 2 else 1
        val = rng.normal(0.0, np.sqrt(2.0 / fan_in), shape) if len(shape) == 2 else rng.normal(0.0, 0.1, shape)
        p[name + "_i"] = _bits(val)
        p["m" + name + "_i"] = _bits(rng.normal(0.0, 1e-3, shape))
        p["v" + name + "_i"] = _bits(np.abs(rng.normal(0.0, 1e-6, shape)))
    return p


def write(out_dir, model_id: str, seed: int = 0) -> Path:
    """<out_dir>/<model_id>_weights_latest.npz in the reference's layout."""
    out = Path(out_dir) / f"{model_id}_weights_latest.npz"
    p = payload(seed)
    p["model_id"] = model_id
    np.savez_compressed(out, **p)
    return out


if __name__ == "__main__":
    print(write(sys.argv[1], sys.argv[2]))
