"""MCMC refine on the device (sxh_exec_mcmc_refine) against the CPU oracle, bit for bit.

The oracle's refine is pinned to the reference's own Trainer in test_mcmc_refine.py. Here the
device path (the arena in HBM, kernels of k_mcmc.hip) must reproduce it exactly: every parameter
and Adam moment of the whole arena, the index lists, the count and the mt19937_64 state, over
consecutive refines; the noise tail; the reference's known answers; the error paths (which must
leave the arena untouched); and config 4 at full size (3M live rows in a 4M arena).

The two sequential primitives get their own exactness tests: the multinomial's running f64 sum
(a parallel scan that must equal the left-to-right loop, including rounding ties and binade
crossings) and the mt19937_64 stream from any engine position.
"""
import numpy as np
import pytest

import inputs
import oracle_py
import scene
import splatx_hip as sh
from inputs import make_cloud

pytestmark = pytest.mark.gpu

F = np.float32
KMAX = 51


def same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.fixture(scope="module")
def binoms(oracle):
    return oracle.make_binoms_lut(KMAX)


def _weights_cases():
    r = np.random.default_rng(0)
    c = {}
    c["uniform_100k"] = r.random(100_000).astype(F)
    logit = r.normal(-1.0, 3.0, 1_000_000).astype(F)
    c["sigmoid_1M"] = (1.0 / (1.0 + np.exp(-logit.astype(np.float64)))).astype(F)
    # exact half-ulp ties: after 1.0 each 2^-53 is a tie (stays at 1.0, even); odd multiples of
    # 2^-53 alternate the parity; 3*2^-53 rounds to 2*2^-53 or 4*2^-53 by parity
    t = [1.0] + [2.0 ** -53] * 20000 + [3 * 2.0 ** -53] * 20000 + [2.0 ** -52 + 2.0 ** -53] * 5000 + [0.75] * 7
    t += [2.0 ** -53, 2.0 ** -52] * 9000
    c["ties"] = np.array(t, F)
    c["leading_zeros"] = np.concatenate([np.zeros(20000, F), r.random(30000).astype(F)])
    c["all_zero"] = np.zeros(9000, F)
    den = r.integers(1, 2 ** 23, 40000).astype(np.uint32).view(F)  # float denormals
    c["denormals_then_large"] = np.concatenate([den, r.random(20000).astype(F), den])
    c["wide_range"] = (10.0 ** r.uniform(-30, 0, 200_000)).astype(F)
    c["doubling"] = (2.0 ** np.arange(0, 100)).astype(F)  # every element crosses a binade
    for n in (1, 7, 8191, 8192, 8193, 16385):
        c[f"n{n}"] = r.random(n).astype(F)
    return c


WEIGHTS = _weights_cases()


@pytest.mark.parametrize("name", list(WEIGHTS))
def test_running_sum_bit_exact(gpu, oracle, name):
    w = WEIGHTS[name]
    print(f"running sum case {name} n={w.size}", flush=True)
    a = gpu.running_sum_f64(w)
    b = oracle.running_sum_f64(w)
    assert same(a, b), (name, int(np.argmax(a != b)))


def test_running_sum_rejects_nan(gpu):
    w = np.ones(100, F)
    w[57] = np.nan
    with pytest.raises(sh.SxInvalidArgument):
        gpu.running_sum_f64(w)


@pytest.mark.parametrize("pre,n", [(0, 1), (0, 311), (0, 312), (0, 313), (5, 1000), (311, 2), (312, 5000),
                                   (100, 200_000)])
def test_mt64_stream_matches_std(gpu, oracle, pre, n):
    st_o = oracle.mt64_seed(42)
    if pre:
        oracle.mt64_draw(st_o, pre)
    st_g = st_o.copy()
    want = oracle.mt64_draw(st_o, n)
    got = gpu.mt64_draw(st_g, n)
    assert np.array_equal(got, want)
    assert st_g.equals(st_o)


def make_exec(gpu, cap, deg):
    return gpu.make_train_step_executor(arena_rows=cap, sh_degree=deg, ssim_weight=0.2)


def download_all(ex, cap, deg):
    dims = scene.group_dims(deg)
    p = [np.zeros((cap, d), F) for d in dims]
    m = [np.zeros((cap, d), F) for d in dims]
    v = [np.zeros((cap, d), F) for d in dims]
    ex.download_params(p, m, v, cap)
    return p, m, v


def assert_arena_equal(dev, orc, what=""):
    for k, name in enumerate(("params", "exp_avg", "exp_avg_sq")):
        for g in range(6):
            if dev[k][g].size:
                assert same(dev[k][g], orc[k][g]), (what, name, g, int(np.argmax(
                    (dev[k][g] != orc[k][g]).any(axis=1))))


CASES = [dict(n=300, cap=400, deg=1, seed=1, refines=3),
         dict(n=2000, cap=2100, deg=3, seed=2, refines=2),
         dict(n=1500, cap=1500, deg=0, seed=3, refines=2),
         dict(n=500, cap=1000, deg=2, seed=4, refines=4, mu=2.0, sd=0.5),
         dict(n=400, cap=900, deg=3, seed=5, refines=3, mu=-6.0, sd=1.0),
         dict(n=60_000, cap=80_000, deg=3, seed=6, refines=3)]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"n{c['n']}-cap{c['cap']}-deg{c['deg']}-s{c['seed']}")
def test_refine_matches_oracle(gpu, oracle, binoms, case):
    n, cap, deg = case["n"], case["cap"], case["deg"]
    print(f"refine case {case}", flush=True)
    p, m, v = make_cloud(n, cap, deg, case["seed"], case.get("mu", -1.0), case.get("sd", 3.0))
    ex = make_exec(gpu, cap, deg)
    ex.upload_params(p, m, v, cap)
    rng_o = oracle.mt64_seed(42)
    rng_g = gpu.mt64_seed(42)
    cnt_o = cnt_g = n
    for k in range(case["refines"]):
        ro = oracle.mcmc_refine(p, m, v, cnt_o, cap, deg, rng_o, binoms)
        rg = ex.mcmc_refine(cnt_g, cap, rng_g, binoms, want_lists=True)
        for key in ("count", "n_relocated", "n_added"):
            assert rg[key] == ro[key], (k, key)
        for key in ("relocated_dead", "relocation_src", "added_src"):
            assert np.array_equal(rg[key], ro[key]), (k, key)
        assert rng_g.equals(rng_o), k
        cnt_o, cnt_g = ro["count"], rg["count"]
    assert_arena_equal(download_all(ex, cap, deg), (p, m, v), "final")
    ex.close()


def test_refine_with_noise_matches_oracle(gpu, oracle, binoms):
    n, cap, deg = 5000, 6000, 3
    p, m, v = make_cloud(n, cap, deg, 11)
    ex = make_exec(gpu, cap, deg)
    ex.upload_params(p, m, v, cap)
    rng_o, rng_g = oracle.mt64_seed(7), gpu.mt64_seed(7)
    seed, offset, scale = 42, 1234, 0.3
    rg = ex.mcmc_refine(n, cap, rng_g, binoms, inject_noise=True, noise_seed=seed, noise_offset=offset,
                        noise_scale=scale)
    ro = oracle.mcmc_refine(p, m, v, n, cap, deg, rng_o, binoms)
    cnt = ro["count"]
    assert rg["count"] == cnt
    noise = oracle.rng_normal_f32(seed, offset, cnt * 3).reshape(cnt, 3)
    means = p[0][:cnt].copy()
    oracle.mcmc_perturb_positions(means, p[1][:cnt], p[2][:cnt], p[3][:cnt, 0], noise, scale)
    p[0][:cnt] = means
    assert_arena_equal(download_all(ex, cap, deg), (p, m, v), "noise")
    ex.close()


def test_refine_known_answers(gpu, binoms):
    """McmcStrategyTests.cpp:68-162 on the device: one alive row feeds the three dead ones; the
    sources' moments are zeroed, the dead rows' are not."""
    op = np.array([0.9, 0.001, 0.004, 0.002], F)
    p, m, v = make_cloud(4, 4, 1, 8, moments=False)
    p[3][:, 0] = np.log(op / (1 - op))
    for g in range(6):
        m[g][:] = 7.0
        v[g][:] = 3.0
    ex = make_exec(gpu, 4, 1)
    ex.upload_params(p, m, v, 4)
    r = ex.mcmc_refine(4, 4, gpu.mt64_seed(42), binoms, want_lists=True)
    assert list(r["relocated_dead"]) == [1, 2, 3] and list(r["relocation_src"]) == [0, 0, 0]
    dp, dm, dv = download_all(ex, 4, 1)
    for g in range(6):
        for i in (1, 2, 3):
            assert same(dp[g][i], dp[g][0])
        assert np.all(dm[g][0] == 0) and np.all(dv[g][0] == 0)
        assert np.all(dm[g][1:] == 7.0) and np.all(dv[g][1:] == 3.0)
    ex.close()


def test_refine_growth_trajectory(gpu, binoms):
    """McmcStrategyTests.cpp:218-243: 16 -> 17 -> 18 -> 19 -> 20 -> 21 -> 23 -> 24 -> 24 under cap 24."""
    p, m, v = make_cloud(16, 24, 1, 10, moments=False)
    p[3][:16, 0] = 0.0
    ex = make_exec(gpu, 24, 1)
    ex.upload_params(p, m, v, 24)
    rng = gpu.mt64_seed(42)
    count = 16
    for want in (17, 18, 19, 20, 21, 23, 24, 24, 24):
        r = ex.mcmc_refine(count, 24, rng, binoms)
        assert r["count"] == want and r["n_added"] == want - count
        count = want
    ex.close()


def test_refine_errors_leave_arena_untouched(gpu, binoms):
    n, cap, deg = 1000, 1200, 1
    p, m, v = make_cloud(n, cap, deg, 12)
    ex = make_exec(gpu, cap, deg)
    ex.upload_params(p, m, v, cap)
    before = download_all(ex, cap, deg)
    # a NaN logit: the multinomial rejects its weights (Trainer.cpp:1205-1206)
    bad = [x.copy() for x in p]
    bad[3][17, 0] = np.nan
    ex.upload_params(bad, m, v, cap)
    rng = gpu.mt64_seed(42)
    st0 = rng.copy()
    with pytest.raises(sh.SxInvalidArgument):
        ex.mcmc_refine(n, cap, rng, binoms)
    assert rng.equals(st0)
    after = download_all(ex, cap, deg)
    assert_arena_equal(after, (bad, m, v), "nan")
    # lists that do not fit: capacity error before anything moves
    ex.upload_params(p, m, v, cap)
    with pytest.raises(sh.SxCapacityError):
        ex.mcmc_refine(n, cap, rng, binoms, want_lists=True, capacity=3)
    assert rng.equals(st0)
    assert_arena_equal(download_all(ex, cap, deg), before, "capacity")
    # argument checks
    for kw in (dict(count=0, cap_max=cap), dict(count=n, cap_max=cap + 1), dict(count=n, cap_max=n - 1)):
        with pytest.raises(sh.SxInvalidArgument):
            ex.mcmc_refine(kw["count"], kw["cap_max"], rng, binoms)
    with pytest.raises(sh.SxInvalidArgument):
        ex.mcmc_refine(n, cap, rng, binoms, min_opacity=0.0)
    ex.close()


def test_step_after_device_refine_equals_step_after_host_refine(gpu, oracle, binoms):
    """The resident step consumes the refined arena exactly as if the host had refined and uploaded
    it (the reference's path): same intersections, same render, bit for bit."""
    sc = scene.make_scene(n=20_000, sh_degree=2, width=160, height=120, fx=150.0, seed=3)
    cap = 24_000
    dims = scene.group_dims(2)
    p = [np.zeros((cap, d), F) for d in dims]
    for g in range(6):
        p[g][:sc.n] = sc.params[g].reshape(sc.n, -1)
    p[3][:sc.n, 0] = np.random.default_rng(4).normal(-1.0, 3.0, sc.n)
    m = [np.zeros_like(x) for x in p]
    v = [np.zeros_like(x) for x in p]
    a, b = make_exec(gpu, cap, 2), make_exec(gpu, cap, 2)
    a.upload_params(p, m, v, cap)
    ra = a.mcmc_refine(sc.n, cap, gpu.mt64_seed(9), binoms)
    ro = oracle.mcmc_refine(p, m, v, sc.n, cap, 2, oracle.mt64_seed(9), binoms)
    assert ra["count"] == ro["count"]
    b.upload_params(p, m, v, cap)
    kw = dict(scene.step_kwargs(sc), count=ra["count"])
    outs = []
    for ex in (a, b):
        ex.set_gt_cache(sc.gt[None])
        outs.append(ex.step(want_render=True, gt_index=0, **kw))
    assert outs[0]["n_isects"] == outs[1]["n_isects"]
    assert same(outs[0]["render_colors"], outs[1]["render_colors"])
    assert outs[0]["loss"] == outs[1]["loss"]
    a.close()
    b.close()


def rel_l2(a, e):
    a = np.asarray(a, np.float64).ravel()
    e = np.asarray(e, np.float64).ravel()
    return float(np.sqrt(((a - e) ** 2).sum()) / max(np.sqrt((e * e).sum()), 1e-30))


def test_config4_full_size_refine(gpu, oracle, binoms):
    """Config 4: 3M live rows in a 4M arena, SH3, ~5% dead; one device
    refine against the oracle over the whole arena, then the training step that follows a refine in the
    reference's resident loop (Trainer.cpp:916-969: opacity and scale regularisation 1e-2 over the new
    count, MCMC noise with the step) against the oracle's step on the oracle's refined arena, under the
    resident-vs-host gates (TrainerTests.cpp:1720-1746): n_isects exact, the render bit-exact, the loss
    within 1e-6 + 1e-4 |loss|, parameters and both moments within rel_l2 1e-4, and the rows past the
    count untouched on both sides."""
    sc, cfg = scene.config_scene(4, seed=0)
    cap, n, deg = cfg["cap_max"], sc.n, sc.sh_degree
    dims = scene.group_dims(deg)
    p = [np.zeros((cap, d), F) for d in dims]
    for g in range(6):
        p[g][:n] = sc.params[g].reshape(n, -1)
    m = [np.zeros_like(x) for x in p]
    v = [np.zeros_like(x) for x in p]
    print("config 4: upload", flush=True)
    ex = gpu.make_train_step_executor(arena_rows=cap, sh_degree=deg, ssim_weight=cfg["ssim"],
                                      isect_mode=sh.SXH_ISECT_ACCUTILE)
    ex.upload_params(p, m, v, cap)
    rng_g, rng_o = gpu.mt64_seed(42), oracle.mt64_seed(42)
    print("config 4: device refine", flush=True)
    rg = ex.mcmc_refine(n, cap, rng_g, binoms, want_lists=True)
    print(f"config 4: relocated {rg['n_relocated']} added {rg['n_added']}; oracle refine", flush=True)
    ro = oracle.mcmc_refine(p, m, v, n, cap, deg, rng_o, binoms)
    assert 0.03 * n < rg["n_relocated"] < 0.08 * n
    assert rg["count"] == ro["count"] == (21 * n + 19) // 20
    for key in ("relocated_dead", "relocation_src", "added_src"):
        assert np.array_equal(rg[key], ro[key]), key
    assert rng_g.equals(rng_o)
    assert_arena_equal(download_all(ex, cap, deg), (p, m, v), "config4")

    # the target: the second seeded scene (seed 1) rendered from the same camera
    tsc, _ = scene.config_scene(4, seed=1)
    tex = gpu.make_train_step_executor(arena_rows=tsc.n, sh_degree=deg, ssim_weight=cfg["ssim"],
                                       isect_mode=sh.SXH_ISECT_ACCUTILE)
    tex.upload_params(*scene.copy_state(tsc), tsc.n)
    target = tex.step(want_render=True, forward_only=True, **scene.step_kwargs(tsc))["render_colors"]
    tex.close()
    count = rg["count"]
    it = 501  # a step past a refine: noise with the step (offset = the iteration)
    step_kw = dict(opacity_reg_w=float(F(cfg["opacity_reg"]) / F(count)),
                   scale_reg_w=float(F(cfg["scale_reg"]) / F(count * 3)), inject_noise=True, noise_seed=42,
                   noise_offset=it, noise_scale=float(F(scene.LR_MEANS) * F(5e5)))
    print("config 4: GPU step", flush=True)
    out = ex.step(want_render=True, gt_rgb=target, **dict(scene.step_kwargs(sc), count=count), **step_kw)
    gs = download_all(ex, cap, deg)
    ex.close()
    print("config 4: oracle step", flush=True)
    start_p = [x.copy() for x in p]
    ro2 = oracle.train_step(p, m, v, count, deg, sc.viewmat, sc.K, sc.width, sc.height, target, deg, list(sc.lr),
                            ssim_weight=cfg["ssim"], isect_mode=sh.SXH_ISECT_ACCUTILE, **step_kw)
    print(f"config 4: n_isects {out['n_isects']} / {ro2['n_isects']}, loss {out['loss']:.7f} / {ro2['loss']:.7f}",
          flush=True)
    assert out["n_isects"] == ro2["n_isects"] and out["n_isects"] > 1_000_000
    assert out["n_visible"] == ro2["n_visible"]
    assert abs(out["loss"] - ro2["loss"]) <= 1e-6 + 1e-4 * abs(ro2["loss"]), (out["loss"], ro2["loss"])
    assert np.array_equal(out["render_colors"].view(np.uint32), ro2["render_colors"].view(np.uint32))
    names = ("means", "quats", "scales", "opacities", "sh0", "shN")
    for g in range(6):
        for kind, a, b in zip(("param", "exp_avg", "exp_avg_sq"), (gs[0][g], gs[1][g], gs[2][g]),
                              (p[g], m[g], v[g])):
            d = rel_l2(a[:count], b[:count])
            print(f"  {names[g]} {kind}: rel_l2 {d:.2e}", flush=True)
            assert d <= 1e-4, (names[g], kind, d)
            assert same(a[count:], b[count:]), (names[g], kind)  # rows past the count: untouched
        assert not np.array_equal(gs[0][g][:count], start_p[g][:count]), names[g]
