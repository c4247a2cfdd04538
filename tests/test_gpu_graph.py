"""The step's second segment as a captured hipGraph (the executor default) against the same step
launched directly (sxh_exec_set_graph(e, 0)): with the learning rates at zero every step sees the
same parameters, so renders, losses and counts must agree bit for bit on every replay. The poses
change the intersection count between replays (the graph reads it on the device), include one with
no intersection at all and one that grows the intersection buffers past their initial capacity
(the executor captures again with the new buffers); direct work of the other executor and
parameter downloads run between the replays. With learning rates on, the parameters after a few
steps agree to the raster backward's atomic-order tolerance."""
import math

import numpy as np
import pytest

import scene
import splatx_hip as sh

pytestmark = pytest.mark.gpu

INITIAL_CAPACITY = (1 << 16) + (1 << 15)  # the executor's intersection buffers at creation


def rel_l2(a, e):
    a = np.asarray(a, np.float64).ravel()
    e = np.asarray(e, np.float64).ravel()
    return float(np.sqrt(((a - e) ** 2).sum()) / max(np.sqrt((e * e).sum()), 1e-30))


def roty(deg):
    a = math.radians(deg)
    v = scene.identity_view()
    v[0, 0], v[0, 2], v[2, 0], v[2, 2] = math.cos(a), math.sin(a), -math.sin(a), math.cos(a)
    return v


def poses():
    """Turned away by 30 degrees first (about 60 % of the splats in view, under the initial capacity),
    then no intersection at all, then facing the scene (over the capacity: the buffers grow; with
    AABB tiles already at the second pose)."""
    rng = np.random.Generator(np.random.PCG64(11))
    away = scene.identity_view()
    away[2, 3] = -20.0  # every mean behind the camera
    return [roty(30), scene.jittered_view(rng) @ roty(30), away, roty(28), scene.identity_view(),
            scene.jittered_view(rng), roty(30)]


def make_pair(gpu, sc, isect):
    out = []
    for graph in (True, False):
        ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2, isect_mode=isect)
        ex.set_graph(graph)
        ex.upload_params(*scene.copy_state(sc), sc.n)
        out.append(ex)
    return out


@pytest.mark.parametrize("isect", [sh.SXH_ISECT_ACCUTILE, sh.SXH_ISECT_AABB])
def test_graph_replays_match_direct_launches(gpu, isect):
    sc = scene.make_scene(n=60000, sh_degree=3, width=256, height=192, fx=200.0, seed=5,
                          log_scale_mu=math.log(0.03))
    eg, ed = make_pair(gpu, sc, isect)
    counts = []
    for k, vm in enumerate(poses()):
        kw = dict(scene.step_kwargs(sc), viewmat=vm, lr=[0.0] * 6)
        print(f"graph replay {k} isect_mode {isect}", flush=True)
        rg = eg.step(want_render=True, gt_rgb=sc.gt, **kw)
        rd = ed.step(want_render=True, gt_rgb=sc.gt, **kw)
        assert rg["n_isects"] == rd["n_isects"] and rg["n_visible"] == rd["n_visible"], k
        assert np.float32(rg["loss"]).view(np.uint32) == np.float32(rd["loss"]).view(np.uint32), (k, rg, rd)
        assert np.array_equal(rg["render_colors"].view(np.uint32), rd["render_colors"].view(np.uint32)), k
        # forward only (the second executable graph) between training replays
        fg = eg.step(want_render=True, forward_only=True, **kw)
        assert np.array_equal(fg["render_colors"].view(np.uint32), rd["render_colors"].view(np.uint32)), k
        counts.append(rg["n_isects"])
        if k == 3:  # eager work between replays
            p, m, v = scene.copy_state(sc)
            eg.download_params(p, m, v, sc.n)
            assert np.array_equal(p[0], sc.params[0])
    assert counts[2] == 0 and min(c for i, c in enumerate(counts) if i != 2) > 0, counts
    # the buffers grew after graphs had been captured and replayed: captured again
    assert counts[0] <= INITIAL_CAPACITY < max(counts), counts
    assert len(set(counts)) >= 4, counts
    eg.close()
    ed.close()


def test_graph_training_steps_match_direct_launches(gpu):
    sc = scene.make_scene(n=8000, sh_degree=3, width=160, height=128, fx=140.0, seed=9)
    eg, ed = make_pair(gpu, sc, sh.SXH_ISECT_ACCUTILE)
    rng = np.random.Generator(np.random.PCG64(3))
    for it in range(4):
        vm = scene.jittered_view(rng)
        kw = dict(scene.step_kwargs(sc), viewmat=vm)
        extra = dict(opacity_reg_w=0.01 / sc.n, inject_noise=True, noise_seed=7, noise_offset=it, noise_scale=0.2)
        print(f"graph training step {it}", flush=True)
        rg = eg.step(gt_rgb=sc.gt, **kw, **extra)
        rd = ed.step(gt_rgb=sc.gt, **kw, **extra)
        assert rg["n_isects"] == rd["n_isects"], it
        assert abs(rg["loss"] - rd["loss"]) <= 1e-6 + 1e-4 * abs(rd["loss"]), (it, rg["loss"], rd["loss"])
    a, b = scene.copy_state(sc), scene.copy_state(sc)
    eg.download_params(*a, sc.n)
    ed.download_params(*b, sc.n)
    for grp in range(3):
        for x, y in zip(a[grp], b[grp]):
            if y.size:
                assert rel_l2(x, y) <= 1e-4, (grp, rel_l2(x, y))
    eg.close()
    ed.close()


def test_steps_returning_at_the_loss_match_fully_synced_steps(gpu):
    """A step without a render read-back returns once its loss is read back, while its parameter update
    may still run; the next step's preprocess is ordered after it on the executor's stream. Five such
    steps back to back must leave exactly the parameters, losses and counts of five steps that each
    wait for the whole stream (a render read-back forces that)."""
    sc = scene.make_scene(n=8000, sh_degree=3, width=160, height=128, fx=140.0, seed=13)
    execs = []
    for _ in range(2):
        ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2,
                                          isect_mode=sh.SXH_ISECT_ACCUTILE)
        ex.upload_params(*scene.copy_state(sc), sc.n)
        execs.append(ex)
    early, synced = execs
    rng = np.random.Generator(np.random.PCG64(5))
    views = [scene.jittered_view(rng) for _ in range(5)]
    out_e, out_s = [], []
    for it, vm in enumerate(views):
        kw = dict(scene.step_kwargs(sc), viewmat=vm, inject_noise=True, noise_seed=3, noise_offset=it,
                  noise_scale=0.1)
        print(f"early-return step {it}", flush=True)
        out_e.append(early.step(gt_rgb=sc.gt, **kw))
        out_s.append(synced.step(want_render=True, gt_rgb=sc.gt, **kw))
    early.sync()
    for it, (a, b) in enumerate(zip(out_e, out_s)):
        assert a["n_isects"] == b["n_isects"], it
        assert np.float32(a["loss"]).view(np.uint32) == np.float32(b["loss"]).view(np.uint32), (it, a, b)
    pa, pb = scene.copy_state(sc), scene.copy_state(sc)
    early.download_params(*pa, sc.n)
    synced.download_params(*pb, sc.n)
    for grp in range(3):
        for x, y in zip(pa[grp], pb[grp]):
            assert np.array_equal(np.asarray(x).view(np.uint32), np.asarray(y).view(np.uint32)), grp
    early.close()
    synced.close()


def test_gather_long_ranges_inline_match_queued(gpu, oracle):
    """The gather reduces a Gaussian's entries past 64 tiles either queued (a wave each, in a second
    launch) or inline (the gather's own waves, after its short ranges), chosen from the count of such
    ranges the previous step reported (its predecessor's: 0 before any): the first step of an executor
    queues them, the next one reduces them inline. Both must give the same sums: with b1 = 0 the first moment after a step is
    exactly its gradient, and with frozen parameters (learning rates 0) and the same pose the two
    steps' gradients must agree bit for bit. Large splats in a 512x384 image give ranges past 64."""
    sc = scene.make_scene(n=3000, sh_degree=1, width=512, height=384, fx=400.0, seed=21,
                          log_scale_mu=math.log(0.12))
    p = sc.params
    proj = oracle.projection_fused_fwd(
        means=p[0].reshape(-1, 3), quats=p[1].reshape(-1, 4), scales=np.exp(p[2].reshape(-1, 3)),
        opacities=(1.0 / (1.0 + np.exp(-p[3].reshape(-1)))).astype(np.float32),
        viewmats=sc.viewmat[None].astype(np.float32), Ks=sc.K[None].astype(np.float32), width=sc.width,
        height=sc.height)
    it = oracle.isect_tiles(means2d=proj["means2d"], radii=proj["radii"], depths=proj["depths"], I=1, N=sc.n,
                            tile_width=(sc.width + 15) // 16, tile_height=(sc.height + 15) // 16)
    n_long = int((np.asarray(it["tiles_per_gauss"]) > 64).sum())
    assert 0 < n_long <= 1024, n_long  # some long ranges, few enough for the inline path
    ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2, b1=0.0,
                                      isect_mode=sh.SXH_ISECT_AABB)
    ex.upload_params(*scene.copy_state(sc), sc.n)
    kw = dict(scene.step_kwargs(sc), lr=[0.0] * 6)
    grads = []
    for k in range(2):
        print(f"long-range gather step {k}", flush=True)
        ex.step(gt_rgb=sc.gt, **kw)
        pp, mm, vv = scene.copy_state(sc)
        ex.download_params(pp, mm, vv, sc.n)
        grads.append([np.asarray(x).copy() for x in mm])
        assert all(np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))
                   for a, b in zip(pp, sc.params))  # frozen
    for a, b in zip(*grads):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert any(np.abs(a).max() > 0 for a in grads[0])
    ex.close()
