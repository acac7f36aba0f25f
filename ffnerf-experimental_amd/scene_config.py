"""Scene configuration: one JSON file per scene, paths relative to the file.

The schema and validation rules are those of the reference (scene_config.py:1-76):
the same sections and keys with the same defaults, unknown sections or keys are
errors, path keys are resolved against the JSON file's directory, and the same
range checks apply.  This build adds one optional section, "model", for the
knobs the reference compiles into its kernels or hard-wires in its trainer
(hash-grid shape, table optimizer, MLP precision, learning-rate schedule,
pixel sampler); a reference config, which has no such section, loads
unchanged.
"""
from __future__ import annotations

import copy
import json
from pathlib import Path

ROOT = Path(__file__).resolve().parent

MODEL_ID_CHARS = set("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789_.-")

DEFAULTS = {
    "data": {"reconstruction": "", "images_dir": "", "sfm_max_side": 1600, "max_side": 800},
    "scene": {"box_min": None, "box_max": None, "near": 0.3},
    "training": {"directory": "../training/test_dataset", "model_id": "test_dataset",
                 "steps": 10000, "period": 100, "batch_rays": 512,
                 "samples_per_ray": 64, "lr": 0.0001, "lmd": 0.0001, "seed": 777},
    "preview": {"enabled": True, "host": "127.0.0.1", "port": 8080,
                "width": 360, "height": 640, "downscale": 5,
                "samples_per_ray": 64, "views": [0, 1, 2],
                "save_seconds": 120, "image_seconds": 30},
    "viewer": {"width": 540, "height": 960, "block_size": 12,
               "samples_per_ray": 64, "camera": 0, "move_speed": 1.0},
    # additions of this build (see the module docstring)
    "model": {"n_levels": 16, "f_per_level": 4, "log2_T": None, "base_res": 16.0, "finest_res": 1024.0,
              "nd": 2, "nc": 2, "hash_opt": "sgd", "mlp_precision": "fp32", "init": "he",
              "beta1": 0.9, "beta2": 0.999, "eps": 1e-6, "occ_G": 32, "occ_decay": 0.9,
              "occ_period": 32, "background": "random", "schedule": "reference", "pixel_sampler": "adaptive"},
}

PATH_KEYS = [("data", "reconstruction"), ("data", "images_dir"), ("training", "directory")]


def _positive_int(cfg, section, key):
    v = cfg[section][key]
    if type(v) is not int or v <= 0:
        raise ValueError(f"{section}.{key} must be a positive integer")


def _positive_finite(cfg, section, key):
    v = cfg[section][key]
    if not (isinstance(v, (int, float)) and 0 < v < float("inf")):
        raise ValueError(f"{section}.{key} must be positive and finite")


def load_config(path) -> dict:
    path = Path(path).resolve()
    raw = json.loads(path.read_text(encoding="utf-8-sig"))
    if not isinstance(raw, dict):
        raise ValueError("Config must be a JSON object")
    cfg = copy.deepcopy(DEFAULTS)
    for section, values in raw.items():
        if section not in cfg or not isinstance(values, dict):
            raise ValueError(f"Unknown or invalid config section: {section}")
        for key, value in values.items():
            if key not in cfg[section]:
                raise ValueError(f"Unknown config key: {section}.{key}")
            cfg[section][key] = value
    for section, key in PATH_KEYS:
        if cfg[section][key]:
            cfg[section][key] = str((path.parent / cfg[section][key]).resolve())
    validate(cfg)
    return cfg


def validate(cfg: dict) -> None:
    if not cfg["data"]["reconstruction"]:
        raise ValueError("data.reconstruction is required")
    for key in ("steps", "period", "batch_rays", "samples_per_ray"):
        _positive_int(cfg, "training", key)
    for key in ("width", "height", "downscale", "samples_per_ray", "port"):
        _positive_int(cfg, "preview", key)
    for key in ("width", "height", "block_size", "samples_per_ray"):
        _positive_int(cfg, "viewer", key)
    for section in ("training", "preview", "viewer"):
        if cfg[section]["samples_per_ray"] > 64:
            raise ValueError(f"{section}.samples_per_ray must be <= 64")
    for key in ("sfm_max_side", "max_side"):
        v = cfg["data"][key]
        if type(v) is not int or v < 0:
            raise ValueError(f"data.{key} must be a nonnegative integer (0 disables resizing)")
    cam = cfg["viewer"]["camera"]
    if type(cam) is not int or cam < 0:
        raise ValueError("viewer.camera must be a nonnegative integer")
    if type(cfg["preview"]["enabled"]) is not bool:
        raise ValueError("preview.enabled must be true or false")
    if not isinstance(cfg["preview"]["views"], list):
        raise ValueError("preview.views must be a list of registered-camera indices")
    for section, key in (("scene", "near"), ("training", "lmd")):
        v = cfg[section][key]
        if not (isinstance(v, (int, float)) and 0 <= v < float("inf")):
            raise ValueError(f"{section}.{key} must be nonnegative and finite")
    if cfg["preview"]["port"] > 65535:
        raise ValueError("preview.port must be <= 65535")
    v, p, t = cfg["viewer"], cfg["preview"], cfg["training"]
    if v["width"] % v["block_size"] or v["height"] % v["block_size"]:
        raise ValueError("Viewer width and height must be multiples of block_size")
    if p["downscale"] > min(p["width"], p["height"]):
        raise ValueError("Preview downscale exceeds image dimensions")
    if not t["model_id"] or any(ch not in MODEL_ID_CHARS for ch in t["model_id"]):
        raise ValueError("model_id may contain only letters, digits, _, . and -")
    _positive_finite(cfg, "training", "lr")
    _positive_finite(cfg, "preview", "save_seconds")
    _positive_finite(cfg, "preview", "image_seconds")
    _positive_finite(cfg, "viewer", "move_speed")
    m = cfg["model"]
    if m["hash_opt"] not in ("sgd", "adam"):
        raise ValueError("model.hash_opt must be 'sgd' or 'adam'")
    if m["mlp_precision"] not in ("fp32", "fp16"):
        raise ValueError("model.mlp_precision must be 'fp32' or 'fp16'")
    if m["background"] not in ("black", "white", "random"):
        raise ValueError("model.background must be 'black', 'white' or 'random'")
    if m["schedule"] not in ("reference", "constant"):
        raise ValueError("model.schedule must be 'reference' or 'constant'")
    if m["init"] not in ("he", "xavier"):
        raise ValueError("model.init must be 'he' or 'xavier'")
    if m["pixel_sampler"] not in ("adaptive", "uniform"):
        raise ValueError("model.pixel_sampler must be 'adaptive' or 'uniform'")
    for key in ("n_levels", "f_per_level", "nd", "nc", "occ_G", "occ_period"):
        _positive_int(cfg, "model", key)
    if m["log2_T"] is not None and (not isinstance(m["log2_T"], list) or len(m["log2_T"]) != m["n_levels"]):
        raise ValueError("model.log2_T must be null or a list with one entry per level")
