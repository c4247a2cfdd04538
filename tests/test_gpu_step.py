"""The resident executor (sxh_exec_*) against the CPU oracle's host-path step (the reference's
resident-vs-host contrast, TrainerTests.cpp:1720-1746): n_isects exact, the render bit-exact (the
whole forward is bit-identical), |dloss| <= 1e-6 + 1e-4 |loss|, parameters after the steps within
rel_l2 1e-4 (atomic accumulation order in raster backward)."""
import numpy as np
import pytest

import oracle_py
import scene
import splatx_hip as sh

pytestmark = pytest.mark.gpu


def rel_l2(a, e):
    a = np.asarray(a, np.float64).ravel()
    e = np.asarray(e, np.float64).ravel()
    den = np.sqrt((e * e).sum())
    return float(np.sqrt(((a - e) ** 2).sum()) / max(den, 1e-30))


CASES = {
    "l1_sh0_aabb": dict(sh_degree=0, ssim=0.0, isect=sh.SXH_ISECT_AABB),
    "ssim_sh3_accutile": dict(sh_degree=3, ssim=0.2, isect=sh.SXH_ISECT_ACCUTILE),
    "ssim_sh3_deg1": dict(sh_degree=3, ssim=0.2, isect=sh.SXH_ISECT_ACCUTILE, degrees=1),
    "antialiased": dict(sh_degree=2, ssim=0.2, isect=sh.SXH_ISECT_ACCUTILE, aa=True),
    "reg_and_noise": dict(sh_degree=1, ssim=0.2, isect=sh.SXH_ISECT_ACCUTILE, reg=True, noise=True),
}


def run_pair(gpu, case, steps=3, n=6000, w=128, h=96):
    c = CASES[case]
    sc = scene.make_scene(n=n, sh_degree=c["sh_degree"], width=w, height=h, fx=110.0, seed=7)
    orc = oracle_py.Oracle(libm=False)
    ex = gpu.make_train_step_executor(arena_rows=n + 17, sh_degree=c["sh_degree"], ssim_weight=c["ssim"],
                                      antialiased=c.get("aa", False), isect_mode=c["isect"])
    gp, gm, gv = scene.copy_state(sc)
    # the arena is larger than count: upload all rows once (zero tail), like Trainer::resident_upload
    pad = lambda a: np.concatenate([a, np.zeros((17,) + a.shape[1:], a.dtype)])
    ex.upload_params([pad(x) for x in gp], [pad(x) for x in gm], [pad(x) for x in gv], n + 17)
    op, om, ov = scene.copy_state(sc)
    results = []
    for it in range(steps):
        kw = scene.step_kwargs(sc, c.get("degrees"))
        extra = {}
        if c.get("reg"):
            extra.update(opacity_reg_w=0.01 / n, scale_reg_w=0.01 / (3 * n))
        if c.get("noise"):
            extra.update(inject_noise=True, noise_seed=42, noise_offset=it, noise_scale=0.3)
        rg = ex.step(want_render=True, gt_rgb=sc.gt, **kw, **extra)
        ro = orc.train_step(op, om, ov, n, c["sh_degree"], sc.viewmat, sc.K, w, h, sc.gt, kw["degrees_to_use"],
                            kw["lr"], ssim_weight=c["ssim"], antialiased=c.get("aa", False), isect_mode=c["isect"],
                            **extra)
        results.append((rg, ro))
    ex.download_params(gp, gm, gv, n)
    ex.close()
    return results, (gp, gm, gv), (op, om, ov)


@pytest.mark.parametrize("case", list(CASES))
def test_step_matches_oracle(gpu, case):
    results, g, o = run_pair(gpu, case)
    for it, (rg, ro) in enumerate(results):
        assert rg["n_isects"] == ro["n_isects"] > 0, (it, rg["n_isects"], ro["n_isects"])
        assert rg["n_visible"] == ro["n_visible"]
        assert abs(rg["loss"] - ro["loss"]) <= 1e-6 + 1e-4 * abs(ro["loss"]), (it, rg["loss"], ro["loss"])
        if it == 0:
            assert np.array_equal(rg["render_colors"].view(np.uint32), ro["render_colors"].view(np.uint32))
        else:
            assert rel_l2(rg["render_colors"], ro["render_colors"]) <= 1e-5
    for grp in range(6):
        for a, b in zip((g[0][grp], g[1][grp], g[2][grp]), (o[0][grp], o[1][grp], o[2][grp])):
            if b.size:
                assert rel_l2(a, b) <= 1e-4, (case, grp, rel_l2(a, b))


def test_forward_only_render_and_gt_cache(gpu):
    n, w, h = 5000, 100, 80
    sc = scene.make_scene(n=n, sh_degree=3, width=w, height=h, fx=90.0, seed=3)
    ex = gpu.make_train_step_executor(arena_rows=n, sh_degree=3, ssim_weight=0.2)
    p, m, v = scene.copy_state(sc)
    ex.upload_params(p, m, v, n)
    kw = scene.step_kwargs(sc)
    r = ex.step(want_render=True, forward_only=True, **kw)
    ro = oracle_py.Oracle().train_step(*scene.copy_state(sc), n, 3, sc.viewmat, sc.K, w, h, None, 3, kw["lr"],
                                       forward_only=True)
    assert np.array_equal(r["render_colors"], ro["render_colors"]) and r["loss"] == 0.0
    # GT cache path == host GT path
    ex.set_gt_cache(np.stack([sc.gt, sc.gt * 0.5]))
    ex.render_to_gt_cache(1, **kw)
    ex2 = gpu.make_train_step_executor(arena_rows=n, sh_degree=3, ssim_weight=0.2)
    ex2.upload_params(p, m, v, n)
    a = ex.step(gt_index=0, **kw)
    b = ex2.step(gt_rgb=sc.gt, **kw)
    assert a["loss"] == b["loss"] and a["n_isects"] == b["n_isects"]
    c = ex.step(gt_index=1, **kw)  # a target rendered from (nearly) the same params
    assert c["loss"] < a["loss"]
    ex.close()
    ex2.close()


def test_upload_download_roundtrip_and_errors(gpu):
    n = 1000
    sc = scene.make_scene(n=n, sh_degree=2, width=64, height=64, fx=60.0, seed=5)
    ex = gpu.make_train_step_executor(arena_rows=n, sh_degree=2)
    p, m, v = scene.copy_state(sc)
    r = np.random.default_rng(0)
    m = [r.standard_normal(x.shape).astype(np.float32) for x in m]
    ex.upload_params(p, m, v, n)
    q = [np.zeros_like(x) for x in p]
    qm = [np.zeros_like(x) for x in p]
    qv = [np.zeros_like(x) for x in p]
    ex.download_params(q, qm, qv, n)
    for a, b in zip(p + m + v, q + qm + qv):
        assert np.array_equal(a, b)
    kw = scene.step_kwargs(sc)
    with pytest.raises(sh.SxInvalidArgument):
        ex.step(gt_rgb=sc.gt, **dict(kw, count=n + 1))
    with pytest.raises(sh.SxInvalidArgument):
        ex.step(**kw)  # no GT
    with pytest.raises(sh.SxInvalidArgument):
        gpu.make_train_step_executor(arena_rows=10, sh_degree=4)
    ex.close()


def test_full_size_forward_matches_oracle(gpu):
    """Config 3 scale (N = 1M, 1297x840, SH3, AccuTile): the forward is bit-identical to the oracle's."""
    sc, cfg = scene.config_scene(3)
    ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=3, ssim_weight=0.2)
    p, m, v = scene.copy_state(sc)
    ex.upload_params(p, m, v, sc.n)
    kw = scene.step_kwargs(sc)
    r = ex.step(want_render=True, forward_only=True, **kw)
    ro = oracle_py.Oracle().train_step(p, m, v, sc.n, 3, sc.viewmat, sc.K, sc.width, sc.height, None, 3, kw["lr"],
                                       forward_only=True)
    assert r["n_isects"] == ro["n_isects"] and r["n_visible"] == ro["n_visible"]
    assert np.array_equal(r["render_colors"], ro["render_colors"])
    ex.close()


@pytest.mark.parametrize("isect", [sh.SXH_ISECT_ACCUTILE, sh.SXH_ISECT_AABB])
def test_large_splats_forward_matches_oracle(gpu, isect):
    """Splats covering up to thousands of tiles, both sweep orientations and more than 64 tile lines
    (the emit's line queue, whose chunks of 64 lines then split one Gaussian's lines and mix
    Gaussians): n_isects exact, the render bit-identical."""
    sc = scene.make_scene(n=400, sh_degree=1, width=1100, height=1060, fx=500.0, seed=11, xy=2.0, z=(2.0, 5.0),
                          log_scale_mu=np.log(0.4), log_scale_sd=0.8)
    ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=1, ssim_weight=0.0, isect_mode=isect)
    p, m, v = scene.copy_state(sc)
    ex.upload_params(p, m, v, sc.n)
    kw = scene.step_kwargs(sc)
    r = ex.step(want_render=True, forward_only=True, **kw)
    ro = oracle_py.Oracle().train_step(p, m, v, sc.n, 1, sc.viewmat, sc.K, sc.width, sc.height, None, 1, kw["lr"],
                                       forward_only=True, isect_mode=isect)
    assert r["n_isects"] == ro["n_isects"] > 100 * sc.n
    assert np.array_equal(r["render_colors"].view(np.uint32), ro["render_colors"].view(np.uint32))
    ex.close()
