"""Command line of the workflow: inspect, train and snapshot one configured scene.

Counterpart of the reference's ffnerf_cli.py (ffnerf_cli.py:1-86): the same
commands, flags and checks -- --config, --steps (positive), --model-id
(restricted characters), --resume, --no-web, --output (must not exist); train
refuses to overwrite existing checkpoints of a model id unless --resume is
given and writes the resolved config next to them.  Here each command is a
handler in a table; `inspect` prints a report of the scene as aligned rows;
`snapshot` renders one training view with the trained model (forward-only
step) to a PNG.  The interactive `review` viewer is not part of this build.
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
from sfm_data import image_geometry, open_reconstruction, read_scene, scaled_intrinsics, scene_bounds


def scene_report(cfg) -> list:
    """(label, value) rows describing the configured scene: cameras, image sizes, the training images'
    memory, the intrinsics at the training size, the scene box and how much of the sparse cloud it holds,
    and the range of camera positions.  Every image must decode to one common size."""
    rec = open_reconstruction(cfg["data"])
    sizes = {}
    for path in rec.image_paths:
        img, train_wh = image_geometry(path, cfg["data"])
        sizes.setdefault(img.shape[:2], path)
        if len(sizes) > 1:
            raise ValueError(f"Inconsistent image dimensions: {path}")
    (h, w), = sizes.keys()
    lo, hi = scene_bounds(cfg["scene"], rec.points)
    centres = rec.c2w[:, :3, 3]
    rows = [
        ("registered cameras", len(rec.image_paths)),
        ("finite sparse points", len(rec.points)),
        ("camera ids", rec.camera_ids.tolist()),
        ("original image size", f"{w}x{h}"),
        ("training image size", f"{train_wh[0]}x{train_wh[1]}"),
        ("training RGB memory", f"{len(rec.image_paths) * train_wh[0] * train_wh[1] * 12 / 2 ** 30:.2f} GiB"),
        ("training K", scaled_intrinsics(rec.K, (w, h), train_wh, cfg["data"]["sfm_max_side"]).tolist()),
        ("scene box", json.dumps({"box_min": lo.tolist(), "box_max": hi.tolist()})),
    ]
    if len(rec.points):
        rows.append(("sparse points inside box", f"{np.all((rec.points >= lo) & (rec.points <= hi), axis=1).mean():.1%}"))
    rows.append(("camera positions", f"{centres.min(axis=0).tolist()} .. {centres.max(axis=0).tolist()}"))
    return rows


def inspect(cfg) -> None:
    rows = scene_report(cfg)
    width = max(len(k) for k, _ in rows)
    for k, v in rows:
        print(f"{k:<{width}}  {v}")


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


def _parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("command", choices=sorted(COMMANDS))
    p.add_argument("--config", required=True, type=Path)
    p.add_argument("--steps", type=int, help="Override the number of additional training steps")
    p.add_argument("--model-id", help="Override output/review model ID")
    p.add_argument("--resume", metavar="MODEL_ID", help="Continue weights and optimizer state from this ID")
    p.add_argument("--no-web", action="store_true", help="Accepted for compatibility (no preview server)")
    p.add_argument("--output", type=Path, help="Snapshot PNG path (must not already exist)")
    p.add_argument("--view", type=int, default=0, help="Snapshot: registered camera index")
    return p


class UsageError(Exception):
    pass


def _overrides(cfg, args) -> None:
    """Command-line values over the config file (validated like the file's own)."""
    if args.steps is not None:
        if args.steps <= 0:
            raise UsageError("--steps must be positive")
        cfg["training"]["steps"] = args.steps
    if args.model_id:
        if not set(args.model_id) <= set(MODEL_ID_CHARS):
            raise UsageError("Invalid --model-id")
        cfg["training"]["model_id"] = args.model_id
    if args.no_web:
        cfg["preview"]["enabled"] = False


def _stamp() -> str:
    return datetime.now().strftime("%Y%m%d-%H%M%S-%f")


def cmd_inspect(cfg, args) -> None:
    inspect(cfg)


def cmd_snapshot(cfg, args) -> None:
    t = cfg["training"]
    out = args.output or Path(t["directory"]) / f"{t['model_id']}_snapshot_{_stamp()}.png"
    if out.exists():
        raise UsageError(f"Snapshot already exists: {out}")
    print(f"Snapshot -> {snapshot(cfg, out, args.view)}")


def cmd_train(cfg, args) -> None:
    """A new model id must not have checkpoints yet (unless resuming); the scene box is resolved once and
    the resolved config is written beside the checkpoints before training starts."""
    t = cfg["training"]
    run_dir = Path(t["directory"])
    if args.resume is None and any(run_dir.glob(f"{t['model_id']}_weights_*.npz")):
        raise UsageError("Checkpoints already exist for this model ID. Use --resume or choose a new --model-id.")
    lo, hi = scene_bounds(cfg["scene"], open_reconstruction(cfg["data"]).points)
    cfg["scene"]["box_min"], cfg["scene"]["box_max"] = lo.tolist(), hi.tolist()
    run_dir.mkdir(parents=True, exist_ok=True)
    manifest = run_dir / f"{t['model_id']}_config_{_stamp()}.json"
    manifest.write_text(json.dumps(cfg, indent=2) + "\n", encoding="utf-8")
    print(f"Resolved run config: {manifest}")
    import trainer
    res = trainer.train(cfg, load_id=args.resume)
    print(f"steps_trained={res['steps_trained']} loss log {res['loss_log']}")


COMMANDS = {"inspect": cmd_inspect, "train": cmd_train, "snapshot": cmd_snapshot}


def main(argv=None) -> int:
    parser = _parser()
    args = parser.parse_args(argv)
    cfg = load_config(args.config)
    try:
        _overrides(cfg, args)
        COMMANDS[args.command](cfg, args)
    except UsageError as e:
        parser.error(str(e))
    return 0


if __name__ == "__main__":
    sys.exit(main())
