"""A training step's parameter update is deferred: the next training step's preprocess applies it row
by row in the same pass over the arena, and anything else that reads or writes the arena (a download,
a forward-only render, a refine, a checkpoint, a sync, a step over another row count) applies it first.
So the arena after a sequence of steps must not depend on when the updates were applied: an executor
that flushes after every step (downloads, forward-only renders and syncs between the steps) and one
whose updates all ride on the next step must agree bit for bit, moments included, with learning rates
on, with the MCMC position noise, and across a change of the row count."""
import math

import numpy as np
import pytest

import scene
import splatx_hip as sh

pytestmark = pytest.mark.gpu


def roty(deg):
    a = math.radians(deg)
    v = scene.identity_view()
    v[0, 0], v[0, 2], v[2, 0], v[2, 2] = math.cos(a), math.sin(a), -math.sin(a), math.cos(a)
    return v


def same_state(a, b):
    for grp_a, grp_b in zip(a, b):
        for x, y in zip(grp_a, grp_b):
            if not np.array_equal(np.asarray(x).view(np.uint32), np.asarray(y).view(np.uint32)):
                return False
    return True


def run(gpu, sc, steps, flush_between, isect=sh.SXH_ISECT_ACCUTILE):
    """steps: a list of (viewmat, count, extra step kwargs). Returns the losses and the final state."""
    ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree, ssim_weight=0.2, isect_mode=isect)
    ex.upload_params(*scene.copy_state(sc), sc.n)
    losses = []
    for k, (view, count, extra) in enumerate(steps):
        print(f"deferred-update step {k} (flush between: {flush_between})", flush=True)
        kw = dict(scene.step_kwargs(sc), viewmat=view, count=count, gt_rgb=sc.gt, **extra)
        losses.append(ex.step(**kw)["loss"])
        if flush_between:
            p, m, v = scene.copy_state(sc)
            ex.download_params(p, m, v, sc.n)  # applies the update
            fwd = dict(kw, forward_only=True)
            fwd.pop("gt_rgb")
            ex.step(want_render=True, **fwd)  # a forward-only step: sees the updated arena
            ex.sync()
    state = scene.copy_state(sc)
    ex.download_params(*state, sc.n)
    ex.close()
    return losses, state


@pytest.mark.parametrize("noise", [False, True])
def test_deferred_update_matches_flushed(gpu, noise):
    sc = scene.make_scene(n=20000, sh_degree=3, width=256, height=192, fx=220.0, seed=31,
                          log_scale_mu=math.log(0.04))
    extra = dict(inject_noise=True, noise_seed=7, noise_offset=3, noise_scale=0.01) if noise else {}
    steps = [(roty(a), sc.n, extra) for a in (0.0, 3.0, -2.0, 1.0)]
    la, sa = run(gpu, sc, steps, flush_between=True)
    lb, sb = run(gpu, sc, steps, flush_between=False)
    assert la == lb, (la, lb)
    assert same_state(sa, sb)
    assert not same_state(sa, scene.copy_state(sc))  # the steps did update the arena


def test_deferred_update_row_count_change(gpu):
    """A step over fewer rows than the pending update's applies that update first (the rows past the new
    count keep it), then runs its own over its rows."""
    sc = scene.make_scene(n=20000, sh_degree=1, width=256, height=192, fx=220.0, seed=32,
                          log_scale_mu=math.log(0.04))
    steps = [(roty(0.0), sc.n, {}), (roty(2.0), sc.n - 5000, {}), (roty(-1.0), sc.n - 5000, {}),
             (roty(1.0), sc.n, {})]
    la, sa = run(gpu, sc, steps, flush_between=True, isect=sh.SXH_ISECT_AABB)
    lb, sb = run(gpu, sc, steps, flush_between=False, isect=sh.SXH_ISECT_AABB)
    assert la == lb, (la, lb)
    assert same_state(sa, sb)
