"""Executors created after others were destroyed report their own step's words.

The step's read-back block (mapped pinned memory) is tagged with sequence numbers that every executor
starts from 1. The runtime may hand a new executor the pinned block of a destroyed one; with that
block's old contents, the first step's waits would end on the old tag and return the old executor's
intersection count and loss (and, past the capacity, skip its own re-run). The block is zeroed at
allocation. Here executors over two different scenes are created and destroyed in turn, with and
without the graph, and the first step of each must report the oracle's count and loss of its own
scene, and a render identical to the oracle's."""
import math

import numpy as np
import pytest

import oracle_py
import scene
import splatx_hip as sh

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("graph", [True, False])
def test_first_step_of_each_new_executor_reports_its_own_words(gpu, graph):
    scenes = [scene.make_scene(n=12000, sh_degree=1, width=128, height=96, fx=110.0, seed=21,
                               log_scale_mu=math.log(0.03)),
              scene.make_scene(n=30000, sh_degree=1, width=160, height=112, fx=150.0, seed=22,
                               log_scale_mu=math.log(0.04))]
    orc = oracle_py.Oracle(libm=False)
    expect = []
    for sc in scenes:
        p, m, v = scene.copy_state(sc)
        ro = orc.train_step(p, m, v, sc.n, sc.sh_degree, sc.viewmat, sc.K, sc.width, sc.height, sc.gt,
                            sc.sh_degree, list(sc.lr), ssim_weight=0.2)
        expect.append(ro)
    assert expect[0]["n_isects"] != expect[1]["n_isects"]
    for cycle in range(6):
        k = cycle % 2
        sc = scenes[k]
        ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2,
                                          isect_mode=sh.SXH_ISECT_ACCUTILE)
        ex.set_graph(graph)
        ex.upload_params(*scene.copy_state(sc), sc.n)
        # the first cycle's render read-back waits for the stream; later ones return at the loss word
        r = ex.step(want_render=cycle < 2, gt_rgb=sc.gt, **scene.step_kwargs(sc))
        ex.close()
        print(f"cycle {cycle} scene {k}: n_isects {r['n_isects']} / {expect[k]['n_isects']}, "
              f"loss {r['loss']:.7f} / {expect[k]['loss']:.7f}", flush=True)
        assert r["n_isects"] == expect[k]["n_isects"], cycle
        assert r["n_visible"] == expect[k]["n_visible"], cycle
        assert abs(r["loss"] - expect[k]["loss"]) <= 1e-6 + 1e-4 * abs(expect[k]["loss"]), cycle
        if r["render_colors"] is not None:
            assert np.array_equal(r["render_colors"].view(np.uint32),
                                  expect[k]["render_colors"].view(np.uint32)), cycle
