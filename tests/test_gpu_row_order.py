"""The executor may keep the live rows in HBM along a Morton curve over their means (so that the rows
a camera culls fill whole waves, which the parameter update skips), with maps to the caller's rows.
Every result must be the caller's-order result bit for bit: an executor forced into spatial order
(SXH_ROW_ORDER_SPATIAL) and one kept in the caller's order (SXH_ROW_ORDER_ORIGINAL) must return the
same losses and renders and, downloaded, the same parameters and moments, through steps with learning
rates on, the MCMC position noise (drawn by original row), equal depths (the stable sorts' ties go by
original row; index first, the per-tile depth sort puts them in that order), both intersection orders, a change of the row count, uploads, checkpoints, PLY exports
and refines in between (each restores the caller's order; the next steps sort again)."""
import math

import numpy as np
import pytest

import inputs
import scene
import splatx_hip as sh

pytestmark = pytest.mark.gpu


def roty(deg):
    a = math.radians(deg)
    v = scene.identity_view()
    v[0, 0], v[0, 2], v[2, 0], v[2, 2] = math.cos(a), math.sin(a), -math.sin(a), math.cos(a)
    return v


def same_state(a, b):
    return all(np.array_equal(np.asarray(x).view(np.uint32), np.asarray(y).view(np.uint32))
               for ga, gb in zip(a, b) for x, y in zip(ga, gb))


def make(gpu, sc, order, isect_order=sh.SXH_ISECT_ORDER_AUTO, antialiased=False):
    ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2,
                                      isect_mode=sh.SXH_ISECT_ACCUTILE, antialiased=antialiased)
    ex.set_row_order(order)
    ex.set_isect_order(isect_order)
    ex.upload_params(*scene.copy_state(sc), sc.n)
    return ex


@pytest.mark.parametrize("isect_order", [sh.SXH_ISECT_ORDER_INDEX_FIRST, sh.SXH_ISECT_ORDER_DEPTH_FIRST])
def test_spatial_order_matches_original(gpu, isect_order):
    # a tenth of the means at one depth: ties in every tile's depth order
    sc = scene.make_scene(n=30000, sh_degree=3, width=256, height=192, fx=220.0, seed=41,
                          log_scale_mu=math.log(0.04), tie_frac=0.1)
    noise = dict(inject_noise=True, noise_seed=9, noise_offset=5, noise_scale=0.01)
    runs = []
    for order in (sh.SXH_ROW_ORDER_ORIGINAL, sh.SXH_ROW_ORDER_SPATIAL):
        print(f"row order {order}, isect order {isect_order}", flush=True)
        ex = make(gpu, sc, order, isect_order, antialiased=True)
        out = []
        for k, a in enumerate((0.0, 4.0, -3.0, 2.0, 1.0)):
            kw = dict(scene.step_kwargs(sc), viewmat=roty(a), gt_rgb=sc.gt, **(noise if k % 2 else {}))
            r = ex.step(want_render=True, **kw)
            out.append((r["loss"], r["n_isects"], r["n_visible"], r["render_colors"].copy()))
        state = scene.copy_state(sc)
        ex.download_params(*state, sc.n)
        ex.close()
        runs.append((out, state))
    (oa, sa), (ob, sb) = runs
    for k, (x, y) in enumerate(zip(oa, ob)):
        assert x[:3] == y[:3], (k, x[:3], y[:3])
        assert np.array_equal(x[3].view(np.uint32), y[3].view(np.uint32)), k
    assert same_state(sa, sb)
    assert not same_state(sa, scene.copy_state(sc))


# index first, tiles of every size: ~16 k-entry tiles (the per-tile sort's global-scratch path) with a
# fifth of the depths equal, one shared depth in large and in small tiles (the sort's all-equal case)
TIE_CASES = {
    "big_tiles_ties": (dict(n=20000, sh_degree=0, tie_frac=0.2, xy=0.6, log_scale_mu=math.log(0.1)), (64, 64, 60.0)),
    "one_depth_big": (dict(n=20000, sh_degree=0, tie_frac=1.0, xy=0.6, log_scale_mu=math.log(0.1)), (64, 64, 60.0)),
    "one_depth_small": (dict(n=3000, sh_degree=0, tie_frac=1.0), (96, 64, 90.0)),
}


@pytest.mark.parametrize("case", list(TIE_CASES))
def test_spatial_order_index_first_ties(gpu, case):
    """Index first, the visible rows are emitted in the internal (spatial) order: the per-tile depth sort
    orders equal depths by original row, so the lists, renders (a forward-only one among them) and updates
    match the caller's order."""
    skw, (w, h, fx) = TIE_CASES[case]
    skw = dict(skw)
    n, deg = skw.pop("n"), skw.pop("sh_degree")
    sc = scene.make_scene(n=n, sh_degree=deg, width=w, height=h, fx=fx, seed=44, **skw)
    runs = []
    for order in (sh.SXH_ROW_ORDER_ORIGINAL, sh.SXH_ROW_ORDER_SPATIAL):
        print(f"{case}, row order {order}", flush=True)
        ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2,
                                          isect_mode=sh.SXH_ISECT_AABB)
        ex.set_row_order(order)
        ex.set_isect_order(sh.SXH_ISECT_ORDER_INDEX_FIRST)
        ex.upload_params(*scene.copy_state(sc), sc.n)
        out = []
        for a in (0.0, 1.5, -1.0):
            r = ex.step(want_render=True, **dict(scene.step_kwargs(sc), viewmat=roty(a), gt_rgb=sc.gt))
            out.append((r["loss"], r["n_isects"], r["render_colors"].copy()))
        # a forward-only render in between (the rows stay in spatial order; the pending update applied)
        r = ex.step(want_render=True, forward_only=True, **dict(scene.step_kwargs(sc), viewmat=roty(0.5)))
        out.append((0.0, r["n_isects"], r["render_colors"].copy()))
        r = ex.step(want_render=True, **dict(scene.step_kwargs(sc), viewmat=roty(2.0), gt_rgb=sc.gt))
        out.append((r["loss"], r["n_isects"], r["render_colors"].copy()))
        state = scene.copy_state(sc)
        ex.download_params(*state, sc.n)
        ex.close()
        runs.append((out, state))
    (oa, sa), (ob, sb) = runs
    for k, (x, y) in enumerate(zip(oa, ob)):
        assert x[:2] == y[:2] and x[1] > 0, (case, k, x[:2], y[:2])
        assert np.array_equal(x[2].view(np.uint32), y[2].view(np.uint32)), (case, k)
    assert same_state(sa, sb), case


def test_spatial_order_capacity_growth(gpu):
    """Index first in spatial order through steps that overflow the intersection buffers (the step runs
    again on grown buffers) and a step without any intersection: the same results as in the caller's
    order."""
    sc = scene.make_scene(n=60000, sh_degree=1, width=256, height=192, fx=200.0, seed=45,
                          log_scale_mu=math.log(0.03), tie_frac=0.05)
    away = scene.identity_view()
    away[2, 3] = -20.0  # every mean behind the camera
    views = [roty(30), away, roty(28), scene.identity_view(), roty(-5), roty(10)]
    runs = []
    for order in (sh.SXH_ROW_ORDER_ORIGINAL, sh.SXH_ROW_ORDER_SPATIAL):
        print(f"capacity growth, row order {order}", flush=True)
        ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2,
                                          isect_mode=sh.SXH_ISECT_ACCUTILE)
        ex.set_row_order(order)
        ex.set_isect_order(sh.SXH_ISECT_ORDER_INDEX_FIRST)
        ex.upload_params(*scene.copy_state(sc), sc.n)
        out = []
        for vm in views:
            r = ex.step(want_render=True, **dict(scene.step_kwargs(sc), viewmat=vm, gt_rgb=sc.gt))
            out.append((r["loss"], r["n_isects"], r["render_colors"].copy()))
        state = scene.copy_state(sc)
        ex.download_params(*state, sc.n)
        ex.close()
        runs.append((out, state))
    (oa, sa), (ob, sb) = runs
    assert oa[1][1] == 0 and max(x[1] for x in oa) > (1 << 16) + (1 << 15)  # none, and past the first capacity
    for k, (x, y) in enumerate(zip(oa, ob)):
        assert x[:2] == y[:2], (k, x[:2], y[:2])
        assert np.array_equal(x[2].view(np.uint32), y[2].view(np.uint32)), k
    assert same_state(sa, sb)


def test_spatial_order_config3_steps(gpu):
    """The headline workload (N = 1M, 1297x840, SH3, AccuTile, SSIM 0.2, jittered poses): five training
    steps with the executor's default row order (spatial from the third step on, index first from the
    second) and five in the caller's order give the same losses, counts, last render and arena, bit for
    bit."""
    sc, cfg = scene.config_scene(3)
    rng = np.random.Generator(np.random.PCG64(7))
    gt = rng.uniform(0.0, 1.0, (sc.height, sc.width, 3)).astype(np.float32)
    views = [scene.jittered_view(rng) for _ in range(5)]
    runs = []
    for order in (sh.SXH_ROW_ORDER_ORIGINAL, sh.SXH_ROW_ORDER_SPATIAL_AUTO):
        print(f"config 3, row order {order}", flush=True)
        ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=cfg["ssim"],
                                          isect_mode=sh.SXH_ISECT_ACCUTILE)
        ex.set_row_order(order)
        ex.upload_params(*scene.copy_state(sc), sc.n)
        out = []
        for k, vm in enumerate(views):
            r = ex.step(want_render=k == len(views) - 1, gt_rgb=gt, **dict(scene.step_kwargs(sc), viewmat=vm))
            out.append((r["loss"], r["n_isects"], r["n_visible"]))
        render = r["render_colors"].copy()
        state = scene.copy_state(sc)
        ex.download_params(*state, sc.n)
        ex.close()
        runs.append((out, render, state))
    (oa, ra, sa), (ob, rb, sb) = runs
    assert oa == ob, (oa, ob)
    assert np.array_equal(ra.view(np.uint32), rb.view(np.uint32))
    assert same_state(sa, sb)


def test_spatial_order_through_exchanges(gpu, tmp_path):
    """Uploads, downloads, a checkpoint and a PLY export between steps (each restores the caller's
    order), a step over fewer rows, then steps again in spatial order."""
    sc = scene.make_scene(n=30000, sh_degree=1, width=256, height=192, fx=220.0, seed=42,
                          log_scale_mu=math.log(0.04))
    cfg = sh.CkptConfig.make(sh_degree=sc.sh_degree, total_iters=100)
    res = []
    for order in (sh.SXH_ROW_ORDER_ORIGINAL, sh.SXH_ROW_ORDER_SPATIAL):
        print(f"exchanges, row order {order}", flush=True)
        ex = make(gpu, sc, order)
        losses = []
        kw = dict(scene.step_kwargs(sc), gt_rgb=sc.gt)
        for a in (0.0, 2.0):
            losses.append(ex.step(**dict(kw, viewmat=roty(a)))["loss"])
        ckpt = tmp_path / f"c{order}.sxck"
        ply = tmp_path / f"p{order}.ply"
        ex.save_checkpoint(cfg, 2, sc.n, str(ckpt))
        ex.export_ply(sc.n, str(ply))
        state = scene.copy_state(sc)
        ex.download_params(*state, sc.n)
        ex.upload_params(*state, sc.n)
        losses.append(ex.step(**dict(kw, viewmat=roty(1.0), count=sc.n - 7000))["loss"])
        for a in (-1.0, 3.0, 0.5):
            losses.append(ex.step(**dict(kw, viewmat=roty(a)))["loss"])
        final = scene.copy_state(sc)
        ex.download_params(*final, sc.n)
        ex.close()
        res.append((losses, ckpt.read_bytes(), ply.read_bytes(), final))
    (la, ca, pa, fa), (lb, cb, pb, fb) = res
    assert la == lb, (la, lb)
    assert ca == cb and pa == pb
    assert same_state(fa, fb)


def test_spatial_order_with_refine(gpu, oracle):
    """Steps in spatial order, then an MCMC refine (which runs in the caller's order), then steps again:
    the same lists, counts and arena as in the caller's order."""
    n, cap, deg = 30000, 36000, 1
    p, m, v = inputs.make_cloud(n, cap, deg, 13, -1.0, 3.0)
    sc = scene.make_scene(n=n, sh_degree=deg, width=256, height=192, fx=220.0, seed=43)
    binoms = oracle.make_binoms_lut(51)
    res = []
    for order in (sh.SXH_ROW_ORDER_ORIGINAL, sh.SXH_ROW_ORDER_SPATIAL):
        print(f"refine, row order {order}", flush=True)
        ex = gpu.make_train_step_executor(arena_rows=cap, sh_degree=deg, ssim_weight=0.2,
                                          isect_mode=sh.SXH_ISECT_ACCUTILE)
        ex.set_row_order(order)
        ex.upload_params([x.copy() for x in p], [x.copy() for x in m], [x.copy() for x in v], cap)
        kw = dict(scene.step_kwargs(sc), gt_rgb=sc.gt, count=n)
        losses = [ex.step(**dict(kw, viewmat=roty(a)))["loss"] for a in (0.0, 2.0, -1.0)]
        rng = gpu.mt64_seed(5)
        r = ex.mcmc_refine(n, cap, rng, binoms, want_lists=True)
        cnt = r["count"]
        losses += [ex.step(**dict(kw, viewmat=roty(a), count=cnt))["loss"] for a in (1.0, -2.0, 0.5)]
        state = [np.zeros_like(x) for x in p], [np.zeros_like(x) for x in m], [np.zeros_like(x) for x in v]
        ex.download_params(*state, cap)
        ex.close()
        res.append((losses, r, state))
    (la, ra, sa), (lb, rb, sb) = res
    assert la == lb, (la, lb)
    for key in ("count", "n_relocated", "n_added"):
        assert ra[key] == rb[key], key
    for key in ("relocated_dead", "relocation_src", "added_src"):
        assert np.array_equal(ra[key], rb[key]), key
    assert same_state(sa, sb)
