"""Command line of the workflow: inspect, train and snapshot one configured scene.

Counterpart of the reference's ffnerf_cli.py (ffnerf_cli.py:1-86): the same
commands, flags and checks -- --config, --steps (positive), --model-id
(restricted characters), --resume, --no-web, --output (must not exist); train
refuses to overwrite existing checkpoints of a model id unless --resume is
given and writes the resolved config next to them.  `snapshot` renders one
training view with the trained model (forward-only step) to a PNG; the
interactive `review` viewer is not part of this build.
"""
from __future__ import annotations

import argparse
import json
import sys
from datetime import datetime
from pathlib import Path

HERE = Path(__file__).resolve().parent
if str(HERE) not in sys.path:
    sys.path.insert(0, str(HERE))

import numpy as np

from scene_config import MODEL_ID_CHARS, load_config
from sfm_data import image_geometry, read_scene, scaled_intrinsics, scene_bounds


def inspect(cfg) -> None:
    paths, poses, K, indices, points = read_scene(cfg["data"])
    lo, hi = scene_bounds(cfg["scene"], points)
    first, wh = image_geometry(paths[0], cfg["data"])
    h, w = first.shape[:2]
    for path in paths[1:]:
        image, _ = image_geometry(path, cfg["data"])
        if image.shape[:2] != (h, w):
            raise ValueError(f"Inconsistent image dimensions: {path}")
    print(f"Registered cameras: {len(paths)}; finite sparse points: {len(points)}")
    print(f"Original images: {w}x{h}; training images: {wh[0]}x{wh[1]}")
    print(f"Training RGB memory: {len(paths) * wh[0] * wh[1] * 12 / 1024 ** 3:.2f} GiB")
    print("Camera IDs:", indices.tolist())
    print("Training K:\n", scaled_intrinsics(K, (w, h), wh, cfg["data"]["sfm_max_side"]))
    print("Scene bounds:", json.dumps({"box_min": lo.tolist(), "box_max": hi.tolist()}))
    if len(points):
        inside = np.all((points >= lo) & (points <= hi), axis=1).mean()
        print(f"Sparse points inside box: {inside:.1%}")
    print("Camera position range:", poses[:, :3, 3].min(axis=0), poses[:, :3, 3].max(axis=0))


def snapshot(cfg, output: Path, view: int = 0) -> Path:
    """Render registered camera `view` with the latest checkpoint of the model id."""
    import ffnerf_tools as ft
    import png_io
    import trainer
    from sfm_data import load_images
    t = cfg["training"]
    paths, poses, K_sfm, _, points = read_scene(cfg["data"])
    images, K, (W, H) = load_images(cfg["data"], paths[: view + 1], K_sfm)
    lo, hi = scene_bounds(cfg["scene"], points)
    nerf = ft.Nerf(t["directory"], t["model_id"], spec=trainer.model_spec(cfg),
                   occ=trainer.occ_params(cfg, lo, hi), load_id=t["model_id"])
    v, u = np.mgrid[0:H, 0:W]
    rays = ft.rays_from_rt_indices(poses[view], u.reshape(-1), v.reshape(-1), W, H, K=K)
    S = int(cfg["viewer"]["samples_per_ray"])
    out = np.zeros((W * H, 4), np.float32)
    chunk = 1 << 16
    io = ft.RayBatch.init(chunk, S)
    arr = ft.rays_as_array(rays)
    for s0 in range(0, W * H, chunk):
        n = min(chunk, W * H - s0)
        block = np.zeros((chunk, 8), np.float32)
        block[:n] = arr[s0:s0 + n]
        io.upload_rays(block)
        nerf.step(io, lr_f=0.0, do_train=False, occ_update_strength=0.0)
        res, _ = io.download_out()
        out[s0:s0 + n] = res[:n]
    img = np.clip(out[:, :3].reshape(H, W, 3), 0.0, 1.0)
    png_io.write_png(output, np.round(img * 255).astype(np.uint8))
    return output


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("command", choices=["inspect", "train", "snapshot"])
    parser.add_argument("--config", required=True, type=Path)
    parser.add_argument("--steps", type=int, help="Override the number of additional training steps")
    parser.add_argument("--model-id", help="Override output/review model ID")
    parser.add_argument("--resume", metavar="MODEL_ID", help="Continue weights and optimizer state from this ID")
    parser.add_argument("--no-web", action="store_true", help="Accepted for compatibility (no preview server)")
    parser.add_argument("--output", type=Path, help="Snapshot PNG path (must not already exist)")
    parser.add_argument("--view", type=int, default=0, help="Snapshot: registered camera index")
    args = parser.parse_args(argv)
    cfg = load_config(args.config)
    if args.steps is not None:
        if args.steps <= 0:
            parser.error("--steps must be positive")
        cfg["training"]["steps"] = args.steps
    if args.model_id:
        if any(ch not in MODEL_ID_CHARS for ch in args.model_id):
            parser.error("Invalid --model-id")
        cfg["training"]["model_id"] = args.model_id
    if args.no_web:
        cfg["preview"]["enabled"] = False
    if args.command == "inspect":
        inspect(cfg)
        return 0
    t = cfg["training"]
    directory = Path(t["directory"])
    if args.command == "snapshot":
        output = args.output or directory / (
            t["model_id"] + "_snapshot_" + datetime.now().strftime("%Y%m%d-%H%M%S-%f") + ".png")
        if output.exists():
            parser.error(f"Snapshot already exists: {output}")
        print(f"Snapshot -> {snapshot(cfg, output, args.view)}")
        return 0
    if not args.resume and list(directory.glob(f"{t['model_id']}_weights_*.npz")):
        parser.error("Checkpoints already exist for this model ID. Use --resume or choose a new --model-id.")
    _, _, _, _, points = read_scene(cfg["data"])
    lo, hi = scene_bounds(cfg["scene"], points)
    cfg["scene"].update(box_min=lo.tolist(), box_max=hi.tolist())
    directory.mkdir(parents=True, exist_ok=True)
    stamp = datetime.now().strftime("%Y%m%d-%H%M%S-%f")
    manifest = directory / f"{t['model_id']}_config_{stamp}.json"
    manifest.write_text(json.dumps(cfg, indent=2) + "\n", encoding="utf-8")
    print(f"Resolved run config: {manifest}")
    import trainer
    res = trainer.train(cfg, load_id=args.resume)
    print(f"steps_trained={res['steps_trained']} loss log {res['loss_log']}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
