"""A training step whose tile sort reports failure leaves the arena as it was.

The sort's error word is the one way a sort signals that its result is unusable; the reference throws
before any result of a failed command buffer is used (MetalBackend.cpp:1579-1584). Here the step's
postprocess reads that word and returns before touching the parameters or the moments, and the host
reports SXH_ERR_RUNTIME after sync 2. The executor's test switch (environment
SXH_DEBUG_FORCE_SORT_ERROR=1 when it is created) sets the word with a kernel right after the tile sort,
so every kernel of the step still runs to its end. Checked for both intersection orders, with the graph
and with direct launches: the step raises, and the downloaded parameters and both moments are bit for
bit the uploaded ones."""
import math
import os

import numpy as np
import pytest

import scene
import splatx_hip as sh

pytestmark = pytest.mark.gpu


def make_executor(gpu, sc, force_error):
    old = os.environ.get("SXH_DEBUG_FORCE_SORT_ERROR")
    os.environ["SXH_DEBUG_FORCE_SORT_ERROR"] = "1" if force_error else "0"
    try:
        return gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2,
                                            isect_mode=sh.SXH_ISECT_ACCUTILE)
    finally:
        if old is None:
            del os.environ["SXH_DEBUG_FORCE_SORT_ERROR"]
        else:
            os.environ["SXH_DEBUG_FORCE_SORT_ERROR"] = old


@pytest.mark.parametrize("order", [sh.SXH_ISECT_ORDER_INDEX_FIRST, sh.SXH_ISECT_ORDER_DEPTH_FIRST])
@pytest.mark.parametrize("graph", [True, False])
def test_sort_error_leaves_arena_unchanged(gpu, order, graph):
    sc = scene.make_scene(n=20000, sh_degree=3, width=160, height=128, fx=140.0, seed=9,
                          log_scale_mu=math.log(0.03))
    p, m, v = scene.copy_state(sc)
    # nonzero moments, so that an update of any of them would show
    rng = np.random.Generator(np.random.PCG64(3))
    for g in range(6):
        m[g][...] = rng.normal(0.0, 1e-3, m[g].shape).astype(np.float32)
        v[g][...] = rng.uniform(0.0, 1e-4, v[g].shape).astype(np.float32)
    kw = scene.step_kwargs(sc)

    ok = make_executor(gpu, sc, False)
    ok.set_isect_order(order)
    ok.set_graph(graph)
    ok.upload_params(p, m, v, sc.n)
    r = ok.step(gt_rgb=sc.gt, **kw)
    assert r["n_isects"] > 1000
    moved = [np.zeros_like(x) for x in p]
    ok.download_params(moved, [np.zeros_like(x) for x in m], [np.zeros_like(x) for x in v], sc.n)
    assert any(not np.array_equal(moved[g], p[g]) for g in range(6))  # a good step moves the parameters
    ok.close()

    bad = make_executor(gpu, sc, True)
    bad.set_isect_order(order)
    bad.set_graph(graph)
    bad.upload_params(p, m, v, sc.n)
    for it in range(2):  # the executor stays usable after the error, and the second failure is the same
        try:
            r = bad.step(gt_rgb=sc.gt, **kw)
            raised = f"no error (n_isects {r['n_isects']}, loss {r['loss']})"
        except sh.SxRuntimeError as e:
            raised = str(e)
        print(f"forced sort error, step {it}: {raised}", flush=True)
        assert "radix sort" in raised, (it, raised)
    gp, gm, gv = ([np.zeros_like(x) for x in grp] for grp in (p, m, v))
    bad.download_params(gp, gm, gv, sc.n)
    for g in range(6):
        for a, b in ((gp[g], p[g]), (gm[g], m[g]), (gv[g], v[g])):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), g
    bad.close()
