"""The step's two intersection orders (sxh_exec_set_isect_order): depth first (Gaussians sorted by
depth, tile ids emitted in that order, a stable tile sort) and index first (tile ids emitted in index
order, a stable tile sort, then each tile's list sorted by depth in LDS, or through global scratch
for tiles of more than 2048 entries) must give the same per-tile (depth, index) lists, hence
bit-identical renders, losses and parameters over several training steps. The depth-first path is
held to the CPU oracle in test_gpu_step.py; the first index-first step is checked against it here
too. Cases cover both intersection modes, antialiasing, tied depths (the stable tie order), a
single shared depth (the sort's all-equal exit) and tiles of up to ~16 k entries (the scratch
path, several chunks of 2048)."""
import numpy as np
import pytest

import oracle_py
import scene
import splatx_hip as sh

pytestmark = pytest.mark.gpu

CASES = {
    # name: scene kwargs, image (w, h, fx), executor kwargs
    "accutile_sh3": (dict(n=6000, sh_degree=3), (128, 96, 110.0), dict(isect_mode=sh.SXH_ISECT_ACCUTILE)),
    "aabb_sh0": (dict(n=6000, sh_degree=0), (128, 96, 110.0), dict(isect_mode=sh.SXH_ISECT_AABB)),
    "antialiased_ties": (dict(n=6000, sh_degree=1, tie_frac=0.3), (128, 96, 110.0),
                         dict(isect_mode=sh.SXH_ISECT_ACCUTILE, antialiased=True)),
    "one_depth": (dict(n=3000, sh_degree=0, tie_frac=1.0), (96, 64, 90.0), dict(isect_mode=sh.SXH_ISECT_AABB)),
    # 16 tiles: the 4 central ones hold ~16 k entries each (the scratch path, 8 chunks), the rest ~1 k
    "big_tiles_ties": (dict(n=20000, sh_degree=0, tie_frac=0.2, xy=0.6, log_scale_mu=np.log(0.1)), (64, 64, 60.0),
                       dict(isect_mode=sh.SXH_ISECT_AABB)),
    # 24 tiles: 4 of ~7 k entries (4 chunks), the rest under 4096 (LDS or 2 chunks)
    "mixed_tiles": (dict(n=12000, sh_degree=0, xy=1.0, log_scale_mu=np.log(0.1)), (96, 64, 80.0),
                    dict(isect_mode=sh.SXH_ISECT_AABB)),
}


def run_mode(gpu, sc, ex_kw, mode, steps, ssim=0.2):
    ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=ssim, **ex_kw)
    ex.set_isect_order(mode)
    gp, gm, gv = scene.copy_state(sc)
    ex.upload_params(gp, gm, gv, sc.n)
    out = []
    for it in range(steps):
        kw = scene.step_kwargs(sc)
        r = ex.step(want_render=True, gt_rgb=sc.gt, **kw)
        out.append((r["n_isects"], r["loss"], r["render_colors"].copy()))
    ex.download_params(gp, gm, gv, sc.n)
    ex.close()
    return out, (gp, gm, gv)


def make(case):
    skw, (w, h, fx), ex_kw = CASES[case]
    skw = dict(skw)
    n = skw.pop("n")
    deg = skw.pop("sh_degree")
    return scene.make_scene(n=n, sh_degree=deg, width=w, height=h, fx=fx, seed=11, **skw), ex_kw


@pytest.mark.parametrize("case", list(CASES))
def test_index_first_matches_depth_first_bitwise(gpu, case):
    sc, ex_kw = make(case)
    a, pa = run_mode(gpu, sc, ex_kw, sh.SXH_ISECT_ORDER_DEPTH_FIRST, steps=3)
    b, pb = run_mode(gpu, sc, ex_kw, sh.SXH_ISECT_ORDER_INDEX_FIRST, steps=3)
    for it, ((na, la, ra), (nb, lb, rb)) in enumerate(zip(a, b)):
        assert na == nb > 0, (case, it)
        assert np.array_equal(ra.view(np.uint32), rb.view(np.uint32)), (case, it)
        assert np.float32(la).view(np.uint32) == np.float32(lb).view(np.uint32), (case, it, la, lb)
    for k in range(3):
        for grp in range(6):
            x, y = pa[k][grp], pb[k][grp]
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), (case, k, grp)


def test_index_first_first_step_matches_oracle(gpu):
    sc, ex_kw = make("antialiased_ties")
    ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2, **ex_kw)
    ex.set_isect_order(sh.SXH_ISECT_ORDER_INDEX_FIRST)
    gp, gm, gv = scene.copy_state(sc)
    ex.upload_params(gp, gm, gv, sc.n)
    kw = scene.step_kwargs(sc)
    rg = ex.step(want_render=True, gt_rgb=sc.gt, **kw)
    ex.close()
    op, om, ov = scene.copy_state(sc)
    ro = oracle_py.Oracle(libm=False).train_step(op, om, ov, sc.n, sc.sh_degree, sc.viewmat, sc.K, sc.width,
                                                 sc.height, sc.gt, kw["degrees_to_use"], kw["lr"], ssim_weight=0.2,
                                                 antialiased=True, isect_mode=ex_kw["isect_mode"])
    assert rg["n_isects"] == ro["n_isects"]
    assert np.array_equal(rg["render_colors"].view(np.uint32), ro["render_colors"].view(np.uint32))


def test_auto_order_switches_to_index_first_and_back(gpu):
    """AUTO: the first step runs depth first (no tile statistics yet), later steps index first while the
    largest tile stays within 4096 entries; the renders equal those of a forced depth-first run."""
    sc, ex_kw = make("accutile_sh3")
    a, _ = run_mode(gpu, sc, ex_kw, sh.SXH_ISECT_ORDER_AUTO, steps=3)
    b, _ = run_mode(gpu, sc, ex_kw, sh.SXH_ISECT_ORDER_DEPTH_FIRST, steps=3)
    for (na, la, ra), (nb, lb, rb) in zip(a, b):
        assert na == nb and np.array_equal(ra.view(np.uint32), rb.view(np.uint32))


def test_set_isect_order_rejects_unknown_mode(gpu):
    ex = gpu.make_train_step_executor(arena_rows=16, sh_degree=0, ssim_weight=0.0)
    with pytest.raises(sh.SxInvalidArgument):
        ex.set_isect_order(3)
    ex.close()
