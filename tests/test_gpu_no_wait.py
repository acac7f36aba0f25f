"""The marched paths without host waits: ffn_train_step_marched with a sample capacity and ffn_render with
FFN_RENDER_NO_WAIT size every launch from counts read on the device (no wait on the stream, so a caller can
capture them in a graph).  Each is checked bit for bit against the waiting path on the same inputs, which
test_gpu_marched_train.py, test_gpu_march.py and test_gpu_configs.py check against the oracle:

- a capacity of at least the march's total gives the waiting step's state, colours and samples used exactly
  (the MLP's persistent blocks take the same tiles and the partial gradients are summed in the same order;
  the scatter's fixed-point sums do not depend on its launch plan);
- a smaller capacity trains the rays whose samples all fit and drops the rest: the state equals the waiting
  step's on those rays alone, and the dropped rays get no samples and the background;
- the render's rounds after the last ray stops are empty launches: colours and samples used as the waiting
  render, which stops after the first round without samples.
"""
import numpy as np
import pytest

from common import cfg4_shell_bitfield, default_scalars, look_at_rays, random_params, spec_cfg0, spec_cfg1, sphere_targets

pytestmark = pytest.mark.gpu

R = 32
DT = np.float32(np.sqrt(3.0) / 128)


@pytest.fixture(scope="module")
def gh():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a visible GPU")
    import gpu_helpers
    return gpu_helpers


def shell_bits(R, seed=0, frac=0.02):
    rng = np.random.default_rng(seed)
    c = (np.arange(R) + 0.5) / R
    z, y, x = np.meshgrid(c, c, c, indexing="ij")
    rad = np.sqrt((x - 0.5) ** 2 + (y - 0.5) ** 2 + (z - 0.5) ** 2)
    occ = (np.abs(rad - 0.3) <= 0.08) | (rng.random((R, R, R)) < frac)
    idx = np.nonzero(occ.reshape(-1))[0]
    bits = np.zeros((R ** 3 + 31) // 32, np.uint32)
    np.bitwise_or.at(bits, idx >> 5, (np.uint32(1) << (idx & 31).astype(np.uint32)))
    return bits


def assert_same_state(a, b):
    assert sorted(a) == sorted(b)
    for k in a:
        np.testing.assert_array_equal(np.ascontiguousarray(a[k]).view(np.uint32),
                                      np.ascontiguousarray(b[k]).view(np.uint32), err_msg=k)


def _spec(shape, mlp):
    if shape == "cfg0":
        return spec_cfg0(occ_G=R // 2, hash_opt=1, mlp_precision=mlp, background=1)
    return spec_cfg1(occ_G=R // 2, hash_opt=1, mlp_precision=mlp, background=1)


@pytest.mark.parametrize("mlp", [0, 1])
@pytest.mark.parametrize("shape", ["cfg0", "cfg1"])
def test_marched_step_capacity_equals_waiting(gh, mlp, shape):
    """Two marched steps with proposals from one state, waiting and with a capacity of exactly the march's
    total and of num_rays * max_steps: identical state, occupancy grids, colours and samples used."""
    import ffn_lib as fl
    print(f"[case] marched step capacity >= total shape={shape} mlp_precision={mlp}", flush=True)
    spec = _spec(shape, mlp)
    p = random_params(spec, seed=61)
    p["bd_out"][0] = 8.0
    rays = look_at_rays(384, spec, seed=62, miss_frac=0.1)
    tg = sphere_targets(rays, spec)
    bits = shell_bits(R, seed=63, frac=0.2)
    max_steps = 128
    total = gh.GpuModel(spec, p).march(rays, bits, fl.march_params(R, DT, max_steps))[4]
    assert total > 2000
    runs = {}
    for cap in (0, total, rays.shape[0] * max_steps):
        m = gh.GpuModel(spec, p)
        outs = []
        for step in range(2):
            sc = default_scalars(rng_seed=600 + step, occ_strength=1.0)
            mp = fl.march_params(R, DT, max_steps, T_stop=1e-2, sample_capacity=cap)
            outs.append(m.step_marched_plain(rays, tg, bits, mp, sc))
        runs[cap] = (m.state(), outs)
    st0, outs0 = runs[0]
    for cap in runs:
        st, outs = runs[cap]
        assert_same_state(st, st0)
        for (o, u), (o0, u0) in zip(outs, outs0):
            np.testing.assert_array_equal(o.view(np.uint32), o0.view(np.uint32))
            np.testing.assert_array_equal(u, u0)
    assert not np.array_equal(st0["occ_st"], p["occ_st"])  # the proposals raised some words


@pytest.mark.parametrize("mlp,budget", [(0, "8192"), (1, "8192"), (0, "0")])
def test_marched_step_capacity_drops_the_later_rays(gh, monkeypatch, mlp, budget):
    """A capacity below the total: the rays whose samples all fit into the first `cap` slots of the march
    order are trained exactly as a waiting step on those rays alone; every later ray gets no sample and the
    (white) background.  With FFN_MARCH_SLOT_BUDGET_MB=0 the march walks twice (count, then emit into the
    scanned slots, where a dropped ray's first samples may land past the kept count, unread)."""
    import ffn_lib as fl
    print(f"[case] marched step capacity < total mlp_precision={mlp} slot budget {budget}", flush=True)
    monkeypatch.setenv("FFN_MARCH_SLOT_BUDGET_MB", budget)
    spec = _spec("cfg0", mlp)
    p = random_params(spec, seed=71)
    p["bd_out"][0] = 8.0
    rays = look_at_rays(384, spec, seed=72, miss_frac=0.1)
    tg = sphere_targets(rays, spec)
    bits = shell_bits(R, seed=73, frac=0.2)
    max_steps = 128
    counts, _, _, _, total = gh.GpuModel(spec, p).march(rays, bits, fl.march_params(R, DT, max_steps))
    ends = np.cumsum(counts.astype(np.int64))
    cap = int(total * 0.55)
    K = int(np.count_nonzero(ends <= cap))
    assert np.all(ends[:K] <= cap) and 50 < K < rays.shape[0] - 50, K
    sc = default_scalars(rng_seed=700, occ_strength=1.0)
    m = gh.GpuModel(spec, p)
    out, used = m.step_marched_plain(rays, tg, bits, fl.march_params(R, DT, max_steps, T_stop=1e-2,
                                                                       sample_capacity=cap), sc)
    m0 = gh.GpuModel(spec, p)
    out0, used0 = m0.step_marched_plain(rays[:K], tg[:K], bits, fl.march_params(R, DT, max_steps, T_stop=1e-2), sc)
    assert_same_state(m.state(), m0.state())
    np.testing.assert_array_equal(out[:K].view(np.uint32), out0.view(np.uint32))
    np.testing.assert_array_equal(used[:K], used0)
    assert not used[K:].any()
    np.testing.assert_array_equal(out[K:], np.tile(np.float32([1.0, 1.0, 1.0, 4.0]), (rays.shape[0] - K, 1)))


def test_marched_step_capacity_checks(gh):
    """taps need the waiting step; a capacity above num_rays * max_steps is refused."""
    import ctypes as C
    import ffn_lib as fl
    import torch
    spec = _spec("cfg0", 0)
    m = gh.GpuModel(spec, random_params(spec, seed=81))
    rays = look_at_rays(16, spec, seed=82)
    with pytest.raises(fl.FfnError, match="sample_capacity"):
        m.step_marched_plain(rays, sphere_targets(rays, spec), shell_bits(R), fl.march_params(
            R, DT, 8, sample_capacity=16 * 8 + 1), default_scalars())
    rays_t = gh.to_dev(rays.reshape(-1, 8))
    tg_t = gh.to_dev(sphere_targets(rays, spec).reshape(-1, 4))
    bits_t = gh.to_dev(shell_bits(R))
    out = torch.zeros((16, 4), dtype=torch.float32, device="cuda")
    sc = fl.FfnStepScalars()
    sc.lr, sc.lr_t, sc.beta1, sc.beta2, sc.eps, sc.do_train = 1e-2, 1e-2, 0.9, 0.99, 1e-15, 1
    tp = fl.FfnTaps()
    mp = fl.march_params(R, DT, 8, sample_capacity=64)
    rc = m.lib.ffn_train_step_marched(m.h.h, fl.ptr(rays_t), fl.ptr(tg_t), fl.ptr(out), 16, fl.ptr(bits_t),
                                      C.byref(mp), C.byref(sc), C.byref(tp), None, fl.stream_ptr())
    assert rc != 0 and b"taps" in fl.load().ffn_last_error()
    # the capacity belongs to the marched step; flags other than FFN_RENDER_NO_WAIT are refused everywhere
    for bad, what in ((fl.march_params(R, DT, 8, sample_capacity=64), "sample_capacity"),
                      (fl.march_params(R, DT, 8, flags=2), "flags")):
        with pytest.raises(fl.FfnError, match=what):
            m.render(rays, shell_bits(R), bad)
        with pytest.raises(fl.FfnError, match=what):
            m.march(rays, shell_bits(R), bad)
    with pytest.raises(fl.FfnError, match="flags"):
        m.step_marched_plain(rays, sphere_targets(rays, spec), shell_bits(R), fl.march_params(R, DT, 8, flags=2),
                             default_scalars())


@pytest.mark.parametrize("chunk,budget", [(16, "8192"), (512, "8192"), (16, "0")])
def test_render_no_wait_equals_waiting(gh, monkeypatch, chunk, budget):
    """cfg0 model: the no-wait render (every round enqueued, empty ones gated off on the device) against the
    waiting render, twice on one handle (the gate of the first round is opened again by every call); with
    FFN_MARCH_SLOT_BUDGET_MB=0 each round walks twice (count, emit), both walks gated."""
    import ffn_lib as fl
    print(f"[case] render no-wait chunk={chunk} slot budget {budget}", flush=True)
    monkeypatch.setenv("FFN_MARCH_SLOT_BUDGET_MB", budget)
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=91)
    p["bd_out"][0] = 6.0
    g = gh.GpuModel(spec, p)
    bits = shell_bits(R, seed=92, frac=0.05)
    rays = look_at_rays(700, spec, seed=93, miss_frac=0.05)
    out, used = g.render(rays, bits, fl.march_params(R, DT, 512, T_stop=1e-2, chunk=chunk))
    for _ in range(2):
        out2, used2 = g.render(rays, bits, fl.march_params(R, DT, 512, T_stop=1e-2, chunk=chunk,
                                                           flags=fl.RENDER_NO_WAIT))
        np.testing.assert_array_equal(out2.view(np.uint32), out.view(np.uint32))
        np.testing.assert_array_equal(used2, used)
    assert used.sum() > 2000


@pytest.mark.parametrize("mlp", [0, 1])
def test_render_no_wait_cfg4(gh, mlp):
    """configs[4]'s field and step (256^3 shell, dt = sqrt(3)/1024, <= 1024 steps, chunk 64, T_stop 1e-4) with
    the config-1 MLPs over 2^18 camera and centre-aimed rays: the no-wait render equals the waiting one."""
    import ffn_lib as fl
    import synthetic_scene as scn
    print(f"[case] cfg4 render no-wait mlp_precision={mlp}", flush=True)
    spec = spec_cfg1(hash_opt=1, mlp_precision=mlp)
    p = random_params(spec, seed=95)
    p["bd_out"][0] = 8.0
    g = gh.GpuModel(spec, p)
    bits, _ = cfg4_shell_bitfield(256)
    n = 1 << 18
    cam, _ = scn.uniform_batch(scn.cameras_for("cfg1"), n // 2, np.random.default_rng(96))
    rays = np.concatenate([cam, look_at_rays(n // 2, spec, seed=97, miss_frac=0.05)])
    dt = np.float32(np.sqrt(3.0) / 1024)
    out, used = g.render(rays, bits, fl.march_params(256, dt, 1024, T_stop=1e-4, chunk=64))
    out2, used2 = g.render(rays, bits, fl.march_params(256, dt, 1024, T_stop=1e-4, chunk=64,
                                                       flags=fl.RENDER_NO_WAIT))
    print(f"samples used {int(used.sum())}", flush=True)
    assert used.sum() > n
    np.testing.assert_array_equal(out2.view(np.uint32), out.view(np.uint32))
    np.testing.assert_array_equal(used2, used)


def _scalars_struct(fl, sc):
    s = fl.FfnStepScalars()
    for k in ("lr", "lr_t", "color_rel_lr", "sh_multiplier", "occ_strength", "beta1", "beta2", "eps"):
        setattr(s, k, float(sc[k]))
    s.rng_seed = int(sc["rng_seed"]) & 0xFFFFFFFF
    s.do_train = 1
    return s


@pytest.mark.parametrize("mlp", [0, 1])
def test_marched_step_with_capacity_replays_from_a_graph(gh, mlp):
    """What the capacity is for: the marched step captured once in a HIP graph (torch.cuda.CUDAGraph) and
    replayed three times, with eager work and synchronisations between the replays, leaves after every replay
    the state, colours and samples used of the same number of eager steps (bit for bit).  A warm-up call
    sizes the handle's buffers first, so the captured call allocates nothing."""
    import ctypes as C
    import ffn_lib as fl
    import torch
    print(f"[case] marched step graph replay mlp_precision={mlp}", flush=True)
    spec = _spec("cfg0", mlp)
    p = random_params(spec, seed=111)
    p["bd_out"][0] = 8.0
    rays = look_at_rays(256, spec, seed=112, miss_frac=0.1)
    tg = sphere_targets(rays, spec)
    bits = shell_bits(R, seed=113, frac=0.2)
    max_steps = 128
    total = gh.GpuModel(spec, p).march(rays, bits, fl.march_params(R, DT, max_steps))[4]
    mp = fl.march_params(R, DT, max_steps, T_stop=1e-2, sample_capacity=total + 4096)
    sc = default_scalars(rng_seed=1100, occ_strength=1.0)
    eager = gh.GpuModel(spec, p)
    m = gh.GpuModel(spec, p)
    N = rays.shape[0]
    rays_t = gh.to_dev(rays.reshape(-1, 8))
    tg_t = gh.to_dev(tg.reshape(-1, 4))
    bits_t = gh.to_dev(bits)
    out = torch.zeros((N, 4), dtype=torch.float32, device="cuda")
    used = torch.zeros(N, dtype=torch.int32, device="cuda")
    scs = _scalars_struct(fl, sc)
    s = torch.cuda.Stream()

    def call():
        fl.check(m.lib.ffn_train_step_marched(m.h.h, fl.ptr(rays_t), fl.ptr(tg_t), fl.ptr(out), N, fl.ptr(bits_t),
                                              C.byref(mp), C.byref(scs), None, fl.ptr(used), fl.stream_ptr()),
                 "ffn_train_step_marched")

    with torch.cuda.stream(s):
        call()  # warm-up: the handle's buffers
    torch.cuda.synchronize()
    eo, eu = eager.step_marched_plain(rays, tg, bits, mp, sc)
    assert_same_state(m.state(), eager.state())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        call()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        eo, eu = eager.step_marched_plain(rays, tg, bits, mp, sc)
        assert_same_state(m.state(), eager.state())
        np.testing.assert_array_equal(gh.to_np(out).view(np.uint32), eo.view(np.uint32))
        np.testing.assert_array_equal(gh.to_np(used, np.uint32), eu)
        torch.zeros(1 << 20, device="cuda").add_(1.0)  # eager work between the replays


def test_render_no_wait_replays_from_a_graph(gh):
    """The no-wait render captured once and replayed three times on changing inputs (the rays' buffer is
    refilled between replays) gives each time the waiting render's image of those rays."""
    import ctypes as C
    import ffn_lib as fl
    import torch
    print("[case] render no-wait graph replay", flush=True)
    spec = spec_cfg0(hash_opt=1)
    p = random_params(spec, seed=121)
    p["bd_out"][0] = 6.0
    g = gh.GpuModel(spec, p)
    ref = gh.GpuModel(spec, p)
    bits = shell_bits(R, seed=122, frac=0.05)
    N = 600
    mp = fl.march_params(R, DT, 512, T_stop=1e-2, chunk=32, flags=fl.RENDER_NO_WAIT)
    mp_wait = fl.march_params(R, DT, 512, T_stop=1e-2, chunk=32)
    rays_t = gh.to_dev(look_at_rays(N, spec, seed=123, miss_frac=0.05).reshape(-1, 8))
    bits_t = gh.to_dev(bits)
    out = torch.zeros((N, 4), dtype=torch.float32, device="cuda")
    used = torch.zeros(N, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()

    def call():
        fl.check(g.lib.ffn_render(g.h.h, fl.ptr(rays_t), N, fl.ptr(bits_t), C.byref(mp), fl.ptr(out),
                                  fl.ptr(used), fl.stream_ptr()), "ffn_render")

    with torch.cuda.stream(s):
        call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        call()
    for rep in range(3):
        rays = look_at_rays(N, spec, seed=130 + rep, miss_frac=0.05)
        rays_t.copy_(gh.to_dev(rays.reshape(-1, 8)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        o_ref, u_ref = ref.render(rays, bits, mp_wait)
        np.testing.assert_array_equal(gh.to_np(out).view(np.uint32), o_ref.view(np.uint32))
        np.testing.assert_array_equal(gh.to_np(used), u_ref)
        assert u_ref.sum() > 1000
