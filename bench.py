"""Benchmark of the fused NeRF training step on one MI355X.

Workload (the GPU-saturating batch): 2^18 rays x 64
samples per step (16.8M samples), hash grid 16 levels x 2 features, T = 2^19
per level, resolutions 16 -> 2048; density MLP 32->64->16, colour MLP
32->64->64->3, Xavier init; Adam (lr 1e-2, betas 0.9/0.99, eps 1e-15) on the
MLP and the table; 128^3 occupancy (64^3 words) with proposals every step and
decay 0.95 every 16 steps.  Rays and targets come from the synthetic ball scene
(56 cameras, 450x800, f=640) and are resident in HBM before timing starts.

One step = sampler + hash encode + fused MLP/compositing/backward + hash
scatter + Adam (MLP and table) [+ occupancy decay].  Prints one JSON line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "ffnerf-experimental_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
FP16_PEAK_TFLOPS = 2500.0


def cfg2_spec(mlp="fp32"):
    import ffnerf_tools as ft
    L = 16
    spec = ft.ModelSpec(n_levels=L, f_per_level=2, log2_T=[19] * L,
                        res=ft.level_resolutions(L, 16.0, finest=2048.0), nd=1, nc=2, background="black",
                        hash_opt="adam", mlp_precision=mlp, init="xavier", beta1=0.9, beta2=0.99, eps=1e-15)
    S = 64
    occ = ft.OccParams(G_occ=64, box_min=np.zeros(3, np.float32), box_max=np.ones(3, np.float32),
                       rho_min=1.0, rho_max=16.0, dt_min=np.float32(1.0 / 8192), dt_max=np.float32(12.8 / S / 6),
                       t_near_clip=0.3, t_far_clip=1e9, occ_update_strength0=1.0, decay=0.95,
                       maintenance_period=16)
    return spec, occ, S


def algorithmic(spec):
    L, F = spec.n_levels, spec.f_per_level
    LF = L * F
    s_tab = 2 if spec.table_dtype == "fp16" else 4  # bytes per table (and table-gradient) value
    fwd_b = L * 8 * F * s_tab + 12 + LF * 4        # corner gathers + xyz + features out
    bwd_b = 2 * L * 8 * F * s_tab + 12 + LF * 4    # atomic read-modify-write + xyz + upstream grad
    macs = LF * 64 + 64 * 16 + 32 * 64 + (spec.nc - 1) * 64 * 64 + 64 * 3 + (spec.nd - 1) * 64 * 64
    mlp_flops = 6 * macs                           # fwd + dX + dW
    adam_b = 28                                    # per parameter: r p,g,m,v; w p,m,v
    return fwd_b, bwd_b, mlp_flops, adam_b


STAGE_KERNELS = {"mlp": ("void ffn::k_mlp<",), "hash_fwd": ("void ffn::k_hash_fwd<",),
                 "hash_bwd": ("void ffn::k_bin_emit<", "void ffn::k_bin_reduce<")}


def recorded_traffic(stage, mlp):
    """HBM-side bytes of one launch of `stage` from the committed PMC summary
    (FETCH_SIZE and WRITE_SIZE runs, each scaled by what the counter reads for
    a plain copy of known size), with the launch duration measured there."""
    f = ROOT / "profiles" / f"pmc_traffic_cfg2_{mlp}.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text())
    ks = d["kernels"]
    kernels = dict(STAGE_KERNELS, mlp=("void ffn::k_mlp16<",) if mlp == "fp16" else STAGE_KERNELS["mlp"])
    ref = [v for n, v in ks.items() if n.startswith(kernels["mlp"][0])]
    if not ref:
        return None
    steps = ref[0]["dispatches"]
    fetch = write = ns = 0.0
    for n, v in ks.items():
        if n.startswith(kernels[stage]):
            per_step = v["dispatches"] / steps
            fetch += v["fetch_bytes"] * per_step
            write += v["write_bytes"] * per_step
            ns += v["avg_ns"] * per_step
    if ns == 0.0:
        return None
    return dict(bytes=fetch + write, fetch=fetch, write=write, profiled_ms=ns * 1e-6,
                source=f"profiles/{f.name}")


def active_fractions(nerf, pool, S):
    """(fraction of 64-sample tiles holding at least one active sample, fraction of active samples) of the
    resident batches: active = dt > 0 (the ray meets the box), from the library's own sampler on the same
    rays."""
    import torch
    import ffn_lib as fl
    lib = nerf.handle.lib
    tot = act = n_smp = n_act = 0
    for i, io in enumerate(pool):
        n = io.num_rays
        Ts = torch.zeros(n * S, dtype=torch.float32, device="cuda")
        DTs = torch.zeros(n * S, dtype=torch.float32, device="cuda")
        flags = torch.zeros(2 * n, dtype=torch.int32, device="cuda")
        fl.check(lib.ffn_sample(nerf.handle.h, fl.ptr(io.rays_buf), n, S, 1234 + i, 1, fl.ptr(Ts), fl.ptr(DTs),
                                fl.ptr(flags), fl.stream_ptr()), "ffn_sample")
        d = DTs.cpu().numpy()
        n_smp += d.size
        n_act += int(np.count_nonzero(d > 0))
        d = np.pad(d, (0, (-d.size) % 64)).reshape(-1, 64)
        tot += d.shape[0]
        act += int(np.count_nonzero((d > 0).any(axis=1)))
    return act / max(tot, 1), n_act / max(n_smp, 1)


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, warmup=3, reps=10):
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_baseline(points=1 << 18, points_one_core=1 << 16):
    """The C restatement of the reference step (oracle/, its OpenMP build) on the host: whole training steps of
    512 rays x 64 samples at the cfg0 and cfg1 model shapes (3 warm-ups, then the median of 10), and the cfg3
    hash encode/scatter on uniform points (2^18 on all cores, 2^16 on one; 1 warm-up, the median of 5), each on
    all available cores and on one."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle import oracle as ora
    import ffnerf_tools as ft
    import synthetic_scene as sc
    lib = ora.load(ora.OMP_LIB_PATH)
    ora.use_library(lib)
    cores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    S, n_rays = 64, 512
    res = {}
    for name, cams_for, L, log2T, finest, G in (("cfg0", "cfg0", 8, 14, None, 32), ("cfg1", "cfg1", 16, 19, 2048.0, 64)):
        res_l = ft.level_resolutions(L, 16.0, growth=1.5) if finest is None else \
            ft.level_resolutions(L, 16.0, finest=finest)
        spec = ft.ModelSpec(n_levels=L, f_per_level=2, log2_T=[log2T] * L, res=res_l, nd=1, nc=2,
                            background="black", hash_opt="adam", init="xavier", beta1=0.9, beta2=0.99, eps=1e-15)
        occ = ft.OccParams(G_occ=G, box_min=np.zeros(3, np.float32), box_max=np.ones(3, np.float32), rho_min=1.0,
                           rho_max=16.0, dt_min=np.float32(1.0 / 8192), dt_max=np.float32(12.8 / S / 6),
                           t_near_clip=0.3, t_far_clip=1e9, occ_update_strength0=1.0, decay=0.95,
                           maintenance_period=16)
        rng = np.random.default_rng(0)
        p = ft.init_params(spec, occ, rng)
        model = ora.OracleModel(ft.spec_dict(spec, occ), {k: v.reshape(spec.layer_shapes()[k])
                                                         if k in spec.layer_shapes() else v for k, v in p.items()})
        rays, tg = sc.uniform_batch(sc.cameras_for(cams_for), n_rays, rng)
        scal = dict(lr=1e-2, lr_t=1e-2, color_rel_lr=1.0, sh_multiplier=1.0, occ_strength=1.0, beta1=0.9,
                    beta2=0.99, eps=1e-15, rng_seed=1, do_train=1)
        for n in (cores, 1):
            lib.ora_set_threads(n)
            t = _median_time(lambda: model.train_step(rays, tg, S, scal))
            res[(name, n)] = dict(samples_per_s=n_rays * S / t, ms_per_step=t * 1e3, threads=n)
    # cfg3 subset: L16 F2 T2^22 fp32 table, uniform points
    L = 16
    spec3 = dict(n_levels=L, f_per_level=2, log2_T=[22] * L, res=ft.level_resolutions(L, 16.0, finest=2048.0), nd=1,
                 nc=2, occ_G=64, box_min=[0.0] * 3, box_max=[1.0] * 3, rho_min=1.0, rho_max=16.0, dt_min=1e-4,
                 dt_max=0.03, t_near=0.3, t_far=1e9)
    cfg3 = ora.make_cfg(spec3)
    rng = np.random.default_rng(1)
    tab = rng.uniform(-1e-4, 1e-4, L * (1 << 22) * 2).astype(np.float32)
    x_all = rng.random((points, 3), dtype=np.float32)
    g_all = rng.standard_normal((points, 2 * L), dtype=np.float32)
    fwd_b, bwd_b = L * 8 * 2 * 4 + 12 + 2 * L * 4, 2 * L * 8 * 2 * 4 + 12 + 2 * L * 4
    grad = np.zeros(tab.size, np.float64)
    for n, npts in ((cores, points), (1, points_one_core)):
        lib.ora_set_threads(n)
        x, g = x_all[:npts], g_all[:npts]
        tf = _median_time(lambda: ora.hash_encode(cfg3, tab, x), warmup=1, reps=5)
        bwd = lambda: lib.ora_hash_backward(C.byref(cfg3), ora.fptr(x), ora.fptr(g), npts,
                                            grad.ctypes.data_as(ora._dp))  # accumulates: the rate is the same
        tb = _median_time(bwd, warmup=1, reps=5)
        res[("cfg3", n)] = dict(points=npts, fwd_points_per_s=npts / tf, bwd_points_per_s=npts / tb,
                                fwd_GBps=fwd_b * npts / tf / 1e9, bwd_GBps=bwd_b * npts / tb / 1e9, threads=n)
    lib.ora_set_threads(cores)
    head = res[("cfg1", cores)]
    return dict(value=head["samples_per_s"], unit="samples/s", cores=cores, kind="port",
                label=f"C restatement of ffnerf_OG.cl semantics (oracle/, OpenMP), {cores} cores",
                cpu_model=_cpu_model(), nproc=os.cpu_count(),
                sample=f"training steps of {n_rays} rays x {S} samples at the cfg1 model shape (L16 F2 T2^19, Adam "
                       f"on table and MLPs), 3 warm-ups then the median of 10, {cores} threads",
                one_core=res[("cfg1", 1)], cfg0={"all_cores": res[("cfg0", cores)], "one_core": res[("cfg0", 1)]},
                cfg3_subset={"table": "L16 F2 T2^22 fp32, uniform points",
                             "all_cores": res[("cfg3", cores)], "one_core": res[("cfg3", 1)]})


def profiled_pass(nerf, one, first, steps):
    """Run `steps` more steps with the library's stage events on; returns (per-stage (total ms, launches),
    ms per step of this pass)."""
    import torch
    nerf.handle.set_profiling(True)
    nerf.handle.stage_times(reset=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        one(first + i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    stages = nerf.handle.stage_times(reset=True)
    nerf.handle.set_profiling(False)
    return stages, (t1 - t0) * 1e3 / steps


def _timed(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def run_cfg3(args):
    """hash-encoding microbench, 2^24 points, L16 F2 T=2^22, forward gather and backward
    scatter-add, fp32 and fp16 tables (the gradient table in the table's type), uniform and shell point
    distributions.  One JSON line per (table type, distribution)."""
    import torch
    import ffn_lib as fl
    import ffnerf_tools as ft
    L, n = 16, int(args.points)
    LF = 2 * L
    _, occ, _ = cfg2_spec()
    rng = np.random.default_rng(1)
    pts = {}
    pts["uniform"] = rng.random((n, 3), dtype=np.float32)
    k = n // 10
    v = rng.normal(size=(n - k, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    r = rng.uniform(0.24, 0.26, (n - k, 1))
    x = np.concatenate([0.5 + v * r, rng.random((k, 3))]).astype(np.float32)
    pts["shell"] = x[rng.permutation(n)]
    tab_np = rng.uniform(-1e-4, 1e-4, L * (1 << 22) * 2).astype(np.float32)
    lines = []
    for dtype in args.table_dtypes.split(","):
        tdt = torch.float16 if dtype == "fp16" else torch.float32
        spec = ft.ModelSpec(n_levels=L, f_per_level=2, log2_T=[22] * L,
                            res=ft.level_resolutions(L, 16.0, finest=2048.0), nd=1, nc=2, background="black",
                            hash_opt="adam", init="xavier", table_dtype=dtype)
        h = fl.Handle(ft.spec_dict(spec, occ))
        table = torch.from_numpy(tab_np).cuda().to(tdt)
        occ_t = torch.zeros(64 ** 3, dtype=torch.int32, device="cuda")
        P = fl.FfnParams()
        dummies = {}
        for i, (wn, bn) in enumerate(zip(fl.LAYER_NAMES, fl.BIAS_NAMES)):
            if wn in spec.layer_shapes():
                for kk in ("W", "b", "mW", "vW", "mb", "vb"):
                    dummies[kk + str(i)] = torch.zeros(4096, device="cuda")
                    getattr(P, kk)[i] = fl.ptr(dummies[kk + str(i)])
        mv = torch.zeros(tab_np.size, dtype=torch.float32, device="cuda")
        P.table, P.m_table, P.v_table, P.occ_in, P.occ_st = fl.ptr(table), fl.ptr(mv), fl.ptr(mv), \
            fl.ptr(occ_t), fl.ptr(occ_t)
        h.bind(P, keep=dict(dummies, table=table, occ=occ_t, mv=mv))
        fwd_b, bwd_b, _, _ = algorithmic(spec)
        for dist in ("uniform", "shell"):
            xt = torch.from_numpy(np.ascontiguousarray(pts[dist])).cuda()
            a0 = torch.empty((n, LF), dtype=torch.float32, device="cuda")
            g = torch.randn((n, LF), dtype=torch.float32, device="cuda",
                            generator=torch.Generator("cuda").manual_seed(1))
            grad = torch.zeros(tab_np.size, dtype=tdt, device="cuda")
            sp = fl.stream_ptr()
            fwd = lambda: fl.check(h.lib.ffn_hash_encode_fwd(h.h, fl.ptr(xt), n, fl.ptr(a0), None, sp))
            bwd = lambda: fl.check(h.lib.ffn_hash_encode_bwd(h.h, fl.ptr(xt), fl.ptr(g), n, fl.ptr(grad), sp))
            t_f = _timed(fwd, args.steps, args.warmup)
            t_b = _timed(bwd, args.steps, args.warmup)
            line = {"metric": "hash-grid gather/scatter HBM GB/s (algorithmic bytes)", "workload": f"cfg3-{dist}-{dtype}",
                    "value": (fwd_b + bwd_b) * n / ((t_f + t_b) * 1e-3) / 1e9, "unit": "GB/s", "n_gpus": 1,
                    "higher_is_better": True, "dtype": dtype, "data": "synthetic",
                    "config": {"workload": f"BASELINE configs[3] ({dist}): 2^{int(np.log2(n))} points, L16 F2 "
                                           f"T2^22 {dtype} table (and gradient table), res 16->2048", "points": n},
                    "fwd": {"ms": t_f, "points_per_s": n / (t_f * 1e-3), "GBps": fwd_b * n / (t_f * 1e-3) / 1e9,
                            "frac": fwd_b * n / (t_f * 1e-3) / 1e9 / HBM_PEAK_GBS, "bytes_per_point": fwd_b},
                    "bwd": {"ms": t_b, "points_per_s": n / (t_b * 1e-3), "GBps": bwd_b * n / (t_b * 1e-3) / 1e9,
                            "frac": bwd_b * n / (t_b * 1e-3) / 1e9 / HBM_PEAK_GBS, "bytes_per_point": bwd_b}}
            print(json.dumps(line), flush=True)
            lines.append(line)
            del xt, a0, g, grad
        h.close()
        del table, mv
    return lines


def shell_bitfield(R, seed=4, radius=0.3, thickness=0.02, noise=0.007):
    """BASELINE configs[4] bitfield: the cells whose centre lies in a shell around the box centre, plus seeded
    isolated cells (R^3 bits, x fastest, 32 per word)."""
    rng = np.random.default_rng(seed)
    c = (np.arange(R, dtype=np.float32) + 0.5) / R
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    set_cells = 0
    for z in range(R):  # slab by slab to bound host memory
        yy, xx = np.meshgrid(c, c, indexing="ij")
        rad = np.sqrt((xx - 0.5) ** 2 + (yy - 0.5) ** 2 + (c[z] - 0.5) ** 2)
        occ = (np.abs(rad - radius) <= 0.5 * thickness) | (rng.random((R, R)) < noise)
        idx = np.nonzero(occ.reshape(-1))[0].astype(np.int64) + z * R * R
        set_cells += idx.size
        np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits, set_cells / R ** 3


def ball_bitfield(R, radius=0.25):
    """The synthetic scene's ball as an R^3 bitfield: the cells whose centre lies within radius plus one cell
    diagonal of the box centre."""
    c = (np.arange(R, dtype=np.float32) + 0.5) / R
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    lim = radius + np.sqrt(3.0) / R
    for z in range(R):
        yy, xx = np.meshgrid(c, c, indexing="ij")
        occ = (xx - 0.5) ** 2 + (yy - 0.5) ** 2 + (c[z] - 0.5) ** 2 <= lim * lim
        idx = np.nonzero(occ.reshape(-1))[0].astype(np.int64) + z * R * R
        np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits


def run_marched_train(args, pool_rays, pool_tg, mlp="fp32"):
    """The training step fed by the march (ffn_train_step_marched): the cfg2 model and batches (2^18 rays of
    the ball scene per step), a 256^3 bitfield of the ball's cells, dt = sqrt(3)/1024, at most 1024 samples
    per ray, compositing stopped at T < 1e-4.  Returns the measurement as a dict."""
    import tempfile
    import torch
    import ffnerf_tools as ft
    spec, occ, _ = cfg2_spec(mlp)
    nerf = ft.Nerf(tempfile.mkdtemp(prefix="ffn_benchm_"), "benchm", spec=spec, occ=occ, rng_seed=0)
    R, max_steps = 256, 1024
    dt = float(np.float32(np.sqrt(3.0) / max_steps))
    bits = torch.from_numpy(ball_bitfield(R).view(np.int32)).cuda()
    n_rays = pool_rays[0].shape[0]
    pool = []
    for rays, tg in zip(pool_rays, pool_tg):
        io = ft.RayBatch.init(n_rays, 1)
        io.upload_rays(rays)
        io.upload_targets(tg)
        pool.append(io)
    used = torch.zeros(n_rays, dtype=torch.int32, device="cuda")
    # samples marched per step (the MLP's work): one march of each batch
    import ctypes as C
    import ffn_lib as fl
    mp = fl.march_params(R, dt, max_steps)
    counts = torch.zeros(n_rays, dtype=torch.int32, device="cuda")
    offs = torch.zeros(n_rays, dtype=torch.int32, device="cuda")
    total = torch.zeros(4, dtype=torch.int32, device="cuda")
    marched = []
    for io in pool:
        fl.check(nerf.handle.lib.ffn_march(nerf.handle.h, fl.ptr(io.rays_buf), n_rays, fl.ptr(bits), C.byref(mp),
                                           fl.ptr(counts), fl.ptr(offs), None, None, 0, fl.ptr(total),
                                           fl.stream_ptr()))
        torch.cuda.synchronize()
        marched.append(int(total[0].item()))
    # the step without a host wait: a sample capacity above every batch's total (so no ray is dropped)
    cap = (int(1.125 * max(marched)) + 4095) // 4096 * 4096
    one = lambda i, c=0: nerf.step_marched(pool[i % len(pool)], 1e-2, bits, R, dt, max_steps=max_steps,
                                           T_stop=1e-4, n_samples=used, sample_capacity=c)
    steps = max(1, args.steps // 2)
    for i in range(args.warmup):
        one(i)
    nerf.handle.set_profiling(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        one(args.warmup + i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    composited = int(used.sum().item())  # of the last step
    stages, ms_prof = profiled_pass(nerf, one, args.warmup + steps, steps)
    avg = {("march" if k == "sample" else k): (v[0] / v[1] if v[1] else 0.0) for k, v in stages.items()}
    one(0, cap)  # the capacity's buffers
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for i in range(steps):
        one(args.warmup + i, cap)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / steps
    n_avg = float(np.mean(marched))
    fwd_b, bwd_b, mlp_flops, _ = algorithmic(spec)
    del nerf
    return {"ms_per_step": ms, "rays": n_rays, "samples_marched_avg": n_avg, "samples_composited_last": composited,
            "value": n_avg / (ms * 1e-3), "unit": "marched samples/s",
            "rays_per_s": n_rays / (ms * 1e-3), "steps": steps, "profiled_ms_per_step": ms_prof,
            "no_wait": {"ms_per_step": (t3 - t2) * 1e3 / steps, "sample_capacity": cap},
            "stages_ms_avg": {k: round(v, 4) for k, v in avg.items()},
            "hash_grid_gbs": (fwd_b + bwd_b) * n_avg / ((avg["hash_fwd"] + avg["hash_bwd"]) * 1e-3) / 1e9,
            "config": "cfg2 model and ray batches (ball scene), 256^3 bitfield of the ball (r 0.25 + one cell "
                      "diagonal), dt sqrt(3)/1024, <= 1024 samples/ray, T_stop 1e-4; stage 'march' = one walk into "
                      "per-ray slots, scan, host wait, pack; 'mlp' = forward, compositing, backward"}


def run_cfg4(args):
    """256^3 bitfield (~3% set, shell), 2^20 rays, <= 1024 steps/ray, early termination at
    T < 1e-4, cfg1 MLPs (forward render); and Adam over 16 x 2^22 x 2 table params with sparse gradients."""
    import ctypes as C
    import tempfile
    import torch
    import ffn_lib as fl
    import ffnerf_tools as ft
    import synthetic_scene as sc
    spec, occ, _ = cfg2_spec("fp32")
    nerf = ft.Nerf(tempfile.mkdtemp(prefix="ffn_bench4_"), "bench4", spec=spec, occ=occ, rng_seed=0)
    R, n_rays, max_steps = 256, int(args.rays4), 1024
    dt = float(np.float32(np.sqrt(3.0) / max_steps))
    bits_np, frac = shell_bitfield(R)
    bits = torch.from_numpy(bits_np.view(np.int32)).cuda()
    rng = np.random.default_rng(5)
    rays, _ = sc.uniform_batch(sc.cameras_for("cfg1"), n_rays, rng)
    io = ft.RayBatch.init(n_rays, 1)
    io.upload_rays(rays)
    used = torch.zeros(n_rays, dtype=torch.int32, device="cuda")
    chunk = int(args.chunk)
    render = lambda: nerf.render_marched(io, bits, R, dt, max_steps=max_steps, T_stop=1e-4, chunk=chunk,
                                         n_samples=used)
    t_r = _timed(render, max(1, args.steps // 3), 1)
    n_smp = int(used.sum().item())
    out_wait = io.out_buf.clone()
    render_nw = lambda: nerf.render_marched(io, bits, R, dt, max_steps=max_steps, T_stop=1e-4, chunk=chunk,
                                            n_samples=used, no_wait=True)
    t_rnw = _timed(render_nw, max(1, args.steps // 3), 1)
    same_nw = bool(torch.equal(io.out_buf, out_wait)) and int(used.sum().item()) == n_smp
    # march + compaction alone (full march, no termination)
    lib, h = nerf.handle.lib, nerf.handle.h
    mp = fl.march_params(R, dt, max_steps)
    counts = torch.zeros(n_rays, dtype=torch.int32, device="cuda")
    offs = torch.zeros(n_rays, dtype=torch.int32, device="cuda")
    total = torch.zeros(4, dtype=torch.int32, device="cuda")
    fl.check(lib.ffn_march(h, fl.ptr(io.rays_buf), n_rays, fl.ptr(bits), C.byref(mp), fl.ptr(counts), fl.ptr(offs),
                           None, None, 0, fl.ptr(total), fl.stream_ptr()))
    torch.cuda.synchronize()
    cap = int(total[0].item())
    smp = torch.empty((max(cap, 1), 4), dtype=torch.float32, device="cuda")
    ids = torch.empty(max(cap, 1), dtype=torch.int32, device="cuda")
    march = lambda: fl.check(lib.ffn_march(h, fl.ptr(io.rays_buf), n_rays, fl.ptr(bits), C.byref(mp), fl.ptr(counts),
                                           fl.ptr(offs), fl.ptr(smp), fl.ptr(ids), cap, fl.ptr(total),
                                           fl.stream_ptr()))
    t_m = _timed(march, args.steps, args.warmup)
    march_bytes = n_rays * (32 + 8) + cap * (16 + 4)
    # Adam over the cfg4 table with sparse gradients (5% of the rows non-zero, N(0, 1e-3))
    n_par = 16 * (1 << 22) * 2
    p = torch.empty(n_par, dtype=torch.float32, device="cuda").uniform_(-1e-4, 1e-4)
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    g = torch.zeros(n_par // 2, 2, dtype=torch.float32, device="cuda")
    rows = torch.rand(n_par // 2, device="cuda") < 0.05
    g[rows] = torch.randn(int(rows.sum().item()), 2, device="cuda") * 1e-3
    g = g.reshape(-1)
    adam = lambda: fl.check(lib.ffn_adam(fl.ptr(p), fl.ptr(m), fl.ptr(v), fl.ptr(g), n_par, 1e-3, 0.9, 0.99, 1e-15, 0,
                                         fl.stream_ptr()))
    t_a = _timed(adam, args.steps, args.warmup)
    line = {"metric": "forward render rays/s with DDA march + early termination (cfg4)", "workload": "cfg4",
            "value": n_rays / (t_r * 1e-3), "unit": "rays/s", "n_gpus": 1, "higher_is_better": True,
            "dtype": "fp32", "data": "synthetic",
            "config": {"workload": "BASELINE configs[4]: 256^3 bitfield shell r=0.3 t=0.02 + seeded cells, "
                                   "2^20 rays, <=1024 steps/ray, T_stop 1e-4, cfg1 MLPs; Adam over 16x2^22x2 params, "
                                   "5% rows N(0,1e-3)", "rays": n_rays, "bits_set_frac": frac, "chunk": chunk},
            "render": {"ms": t_r, "samples": n_smp, "samples_per_s": n_smp / (t_r * 1e-3)},
            "render_no_wait": {"ms": t_rnw, "equal_to_waiting": same_nw,
                               "rounds": (max_steps + chunk - 1) // chunk},
            "march": {"ms": t_m, "samples": cap, "GBps": march_bytes / (t_m * 1e-3) / 1e9,
                      "frac": march_bytes / (t_m * 1e-3) / 1e9 / HBM_PEAK_GBS,
                      "bytes": "40 B/ray (ray + offset, count) + 20 B/sample (xyz t + ray id)"},
            "adam": {"ms": t_a, "params": n_par, "GBps": 28 * n_par / (t_a * 1e-3) / 1e9,
                     "frac": 28 * n_par / (t_a * 1e-3) / 1e9 / HBM_PEAK_GBS}}
    if not args.no_marched_train:
        del nerf, io
        cams = sc.cameras_for("cfg2")
        rng2 = np.random.default_rng(123)
        pr, pt = [], []
        for _ in range(4):
            r_, t_ = sc.uniform_batch(cams, 1 << 18, rng2)
            pr.append(r_)
            pt.append(t_)
        print("[bench] marched training step", flush=True)
        line["train_marched"] = run_marched_train(args, pr, pt)
        print("[bench] marched training step, fp16 MLP", flush=True)
        m16 = run_marched_train(args, pr, pt, mlp="fp16")
        line["train_marched"]["fp16_mlp_path"] = {k: m16[k] for k in ("ms_per_step", "value", "unit",
                                                                       "stages_ms_avg")}
    print(json.dumps(line), flush=True)
    return line


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--mlp", default="fp32", choices=["fp32", "fp16"])
    ap.add_argument("--rays", type=int, default=1 << 18)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fp16-line", action="store_true", help="skip the fp16-MLP path measurement")
    ap.add_argument("--workload", default="cfg2", choices=["cfg2", "cfg3", "cfg4"],
                    help="cfg2 (default): the training step; cfg3: hash microbench; cfg4: marched render + Adam")
    ap.add_argument("--points", type=int, default=1 << 24, help="cfg3 points")
    ap.add_argument("--table-dtypes", default="fp32,fp16", help="cfg3 table types")
    ap.add_argument("--rays4", type=int, default=1 << 20, help="cfg4 rays")
    ap.add_argument("--chunk", type=int, default=64, help="cfg4 samples per ray per render round")
    ap.add_argument("--no-marched-train", action="store_true", help="cfg4: skip the marched training step")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run one plain device copy of this size (a known-traffic kernel for PMC scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested): this build runs the step on a "
              f"single GPU; sharding rays over GPUs with all-reduced table and MLP gradients is not built.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import ffnerf_tools as ft
    import synthetic_scene as sc

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] calibration copy: {args.copy_calibration_mib} MiB read + {args.copy_calibration_mib} MiB "
              f"written by one copy kernel", flush=True)
        del src, dst

    if args.workload == "cfg3":
        run_cfg3(args)
        return
    if args.workload == "cfg4":
        run_cfg4(args)
        return

    spec, occ, S = cfg2_spec(args.mlp)
    n_rays = int(args.rays)
    import tempfile
    nerf = ft.Nerf(tempfile.mkdtemp(prefix="ffn_bench_"), "bench", spec=spec, occ=occ, rng_seed=0)
    print(f"[bench] cfg2 model built: table {spec.table_entries() * spec.f_per_level / 1e6:.1f}M params", flush=True)
    cams = sc.cameras_for("cfg2")
    rng = np.random.default_rng(123)
    pool = []
    for _ in range(4):
        rays, tg = sc.uniform_batch(cams, n_rays, rng)
        io = ft.RayBatch.init(n_rays, S)
        io.upload_rays(rays)
        io.upload_targets(tg)
        pool.append(io)
    torch.cuda.synchronize()
    print(f"[bench] {len(pool)} ray batches of {n_rays} resident; warm-up {args.warmup}", flush=True)

    def one(i):
        nerf.step(pool[i % len(pool)], lr_f=1e-2, do_train=True, occ_update_strength=1.0, sh_multiplier=1.0,
                  color_MLP_rel_lr=1.0)

    for i in range(args.warmup):
        one(i)
    # the timed region: K steps, nothing else on the stream (stage timing off)
    nerf.handle.set_profiling(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        one(args.warmup + i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    print(f"[bench] timed {args.steps} steps in {t1 - t0:.3f} s", flush=True)
    # a second pass of the same steps with the library's stage events on the step's stream: the per-kernel
    # durations the rooflines use
    stages, ms_prof = profiled_pass(nerf, one, args.warmup + args.steps, args.steps)

    N = n_rays * S
    ms_step = (t1 - t0) * 1e3 / args.steps
    value = N * args.steps / (t1 - t0)
    fwd_b, bwd_b, mlp_flops, adam_b = algorithmic(spec)
    avg = {k: (v[0] / v[1] if v[1] else 0.0) for k, v in stages.items()}
    per = {
        "hash_fwd": ("hbm", fwd_b * N / (avg["hash_fwd"] * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", fwd_b * N),
        "hash_bwd": ("hbm", bwd_b * N / (avg["hash_bwd"] * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", bwd_b * N),
        "mlp": ("mfma", mlp_flops * N / (avg["mlp"] * 1e-3) / 1e12,
                FP16_PEAK_TFLOPS if args.mlp == "fp16" else FP32_PEAK_TFLOPS, "TFLOP/s", mlp_flops * N),
    }
    # the MLP kernels skip 64-sample tiles whose samples are all inactive (rays that miss the box); count
    # the tiles with an active sample on the resident batches to state the rate over the computed tiles
    act, act_smp = active_fractions(nerf, pool, S)
    dominant = max(per, key=lambda k: avg[k])
    bound, ach, peak, unit, alg = per[dominant]
    hash_gbs = (fwd_b + bwd_b) * N / ((avg["hash_fwd"] + avg["hash_bwd"]) * 1e-3) / 1e9
    tr = recorded_traffic(dominant, args.mlp) if n_rays == 1 << 18 else None
    line = {
        "metric": "train samples/sec (fwd+bwd+Adam) per step; hash-grid gather/scatter HBM GB/s",
        "value": value, "unit": "samples/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32" if args.mlp == "fp32" else "fp16-mfma/fp32", "data": "synthetic",
        "config": {"workload": "BASELINE configs[2]: 2^18 rays x 64 samples/step, hash L16 F2 T2^19 16->2048 fp32, "
                               "MLP 32-64-16 / 32-64-64-3, Adam table+MLP, occupancy 128^3, decay 0.95 every 16",
                   "global_batch": n_rays, "samples_per_ray": S, "samples_per_step": N, "mlp": args.mlp},
        "hash_grid_gbs": hash_gbs,
        "roofline": {"kernel": dominant, "bound": bound, "achieved": ach, "peak": peak, "unit": unit,
                     "frac": ach / peak, "algorithmic_per_launch": alg,
                     "traffic": tr["bytes"] if tr else None,
                     "traffic_detail": tr},
        "stages_ms_avg": {k: round(v, 4) for k, v in avg.items()},
        "stage_rooflines": {k: {"achieved": v[1], "unit": v[3], "frac": v[1] / v[2]} for k, v in per.items()},
        "active_samples": {"frac": act_smp, "value": value * act_smp, "unit": "samples/s",
                           "note": "samples whose ray meets the box (dt > 0); value counts every sample of the "
                                   "batch, as the reference's fixed S samples per ray do"},
        "profiled_pass": {"ms_per_step": ms_prof, "steps": args.steps,
                          "note": "stage durations come from this second pass, with HIP events recorded around "
                                  "each stage on the step's stream; ms_per_step above is timed without them"},
        "mlp_active_tiles": {"frac": act, "achieved_over_computed_tiles": per["mlp"][1] * act,
                             "frac_of_peak_over_computed_tiles": per["mlp"][1] * act / per["mlp"][2],
                             "note": "the MLP kernels skip 64-sample tiles whose samples are all inactive "
                                     "(rays that miss the box: every gradient of such a tile is zero); "
                                     "roofline.achieved counts all samples, as the per-sample work unit does"},
    }
    if args.mlp == "fp32" and not args.no_fp16_line:
        # the same step with the fp16/bf16-MFMA MLP (BASELINE reports both paths), same resident batches
        spec16, _, _ = cfg2_spec("fp16")
        nerf16 = ft.Nerf(tempfile.mkdtemp(prefix="ffn_bench16_"), "bench16", spec=spec16, occ=occ, rng_seed=0)
        def one16(i):
            nerf16.step(pool[i % len(pool)], lr_f=1e-2, do_train=True, occ_update_strength=1.0)

        for i in range(args.warmup):
            one16(i)
        nerf16.handle.set_profiling(False)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        for i in range(args.steps):
            one16(args.warmup + i)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        st16, _ = profiled_pass(nerf16, one16, args.warmup + args.steps, args.steps)
        avg16 = {k: (v[0] / v[1] if v[1] else 0.0) for k, v in st16.items()}
        line["fp16_mlp_path"] = {
            "value": N * args.steps / (t3 - t2), "unit": "samples/s", "ms_per_step": (t3 - t2) * 1e3 / args.steps,
            "dtype": "fp16/bf16-mfma, fp32 accumulate", "stages_ms_avg": {k: round(v, 4) for k, v in avg16.items()},
            "mlp_tflops": mlp_flops * N / (avg16["mlp"] * 1e-3) / 1e12,
            "mlp_frac_of_fp16_peak": mlp_flops * N / (avg16["mlp"] * 1e-3) / 1e12 / FP16_PEAK_TFLOPS}
        print(f"[bench] fp16-MLP path: {(t3 - t2) * 1e3 / args.steps:.2f} ms/step", flush=True)
        del nerf16
    if not args.no_cpu_baseline and int(os.environ.get("RANK", "0")) == 0:
        print("[bench] timing the CPU oracle on a bounded sample", flush=True)
        line["cpu_baseline"] = cpu_baseline()
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))


if __name__ == "__main__":
    main()
