"""The reference's own Trainer on this backend: the drop-in boundary end to end.

oracle/_ref/libsx_ref_hip.so is Sources/SplatXCore/Trainer.cpp (+ CpuKernels.cpp, Math.cpp) built
in place from the reference tree with splatx-metal_amd/host/hip_kernel_backend.cpp, the C++
splatx::KernelBackend adapter over the C ABI. Nothing in the Trainer is changed: it calls the
backend as it calls the Metal one. The checks are the reference's own contrast gates between its
host round-trip path (17 per-op virtuals) and its device-resident path (make_train_step_executor),
TrainerTests.cpp:1716-1747: equal n_isects every step, loss |d| <= 1e-6 + 1e-4 |loss|, the first
render within rel_l2 1e-5, every parameter group within rel_l2 1e-4 after the steps. The MCMC run
drives Trainer::step_resident's refine steps (download, host refine, re-upload) through the
executor. Skipped where the reference tree was absent when oracle/_ref was built.
"""
import numpy as np
import pytest

import oracle_py
import scene

pytestmark = pytest.mark.gpu

LR = [2e-3, 5e-3, 2e-2, 5e-2, 2e-2, 2e-2 / 20]  # means, quats, scales, opacities, sh0, shN


@pytest.fixture(scope="module")
def ref_hip():
    if not oracle_py.ReferenceTrainerOnHip.available():
        pytest.skip("oracle/_ref/libsx_ref_hip.so not built (reference tree absent)")
    return oracle_py.ReferenceTrainerOnHip()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("deg,aa", [(0, False), (1, False), (3, True)])
def test_reference_trainer_host_vs_resident_on_hip(ref_hip, deg, aa):
    sc = scene.make_scene(n=6000, sh_degree=deg, width=128, height=96, fx=110.0, seed=5)
    gt = np.full((sc.height, sc.width, 3), 0.35, np.float32)
    kw = dict(params=sc.params, count=sc.n, sh_degree=deg, viewmat=sc.viewmat, K=sc.K, width=sc.width,
              height=sc.height, gt=gt, steps=5, lr=LR, total_iters=100, ssim_weight=0.2, opacity_reg=0.01,
              scale_reg=0.01, antialiased=aa)
    print(f"reference Trainer on hip: deg={deg} aa={aa}", flush=True)
    h = ref_hip.run(resident=False, **kw)
    r = ref_hip.run(resident=True, **kw)
    assert np.all(h["n_isects"] > 0)
    assert np.array_equal(h["n_isects"], r["n_isects"])
    assert np.all(np.abs(h["losses"].astype(np.float64) - r["losses"]) <= 1e-6 + 1e-4 * np.abs(h["losses"]))
    assert rel_l2(r["render0"], h["render0"]) <= 1e-5
    for g in range(6):
        if h["params"][g].size:
            assert rel_l2(r["params"][g], h["params"][g]) <= 1e-4, g
    assert h["losses"][-1] < h["losses"][0]


def test_reference_trainer_mcmc_resident_on_hip(ref_hip):
    """MCMC on: refine every 2nd step from step 2 (Trainer::mcmc_refine_due), cap 7000 over 6000
    live rows; the resident path reclaims and re-uploads the arena around each refine."""
    sc = scene.make_scene(n=6000, sh_degree=1, width=128, height=96, fx=110.0, seed=6)
    logit = np.random.default_rng(7).normal(-1.0, 3.0, sc.n).astype(np.float32)
    params = list(sc.params)
    params[3] = logit
    gt = np.full((sc.height, sc.width, 3), 0.35, np.float32)
    kw = dict(params=params, count=sc.n, sh_degree=1, viewmat=sc.viewmat, K=sc.K, width=sc.width,
              height=sc.height, gt=gt, steps=8, lr=LR, total_iters=100, ssim_weight=0.2, opacity_reg=0.01,
              scale_reg=0.01, mcmc=True, cap_max=7000, seed=42, refine_start_ratio=0.01, refine_stop_ratio=0.9,
              refine_every_ratio=0.02)
    h = ref_hip.run(resident=False, **kw)
    r = ref_hip.run(resident=True, **kw)
    assert h["n_refined"] == r["n_refined"] >= 3
    assert h["count"] == r["count"] > sc.n
    assert np.all(np.isfinite(r["losses"])) and np.all(r["n_isects"] > 0)
    # the first steps precede any refine: the two paths agree there as in the contrast test
    assert r["n_isects"][0] == h["n_isects"][0]
    assert abs(float(h["losses"][0]) - float(r["losses"][0])) <= 1e-6 + 1e-4 * abs(float(h["losses"][0]))


def test_adapter_hip_mcmc_refine_matches_oracle(ref_hip, oracle):
    """splatx::hip_mcmc_refine (the C++ adapter's device refine, std::mt19937_64 exchanged through
    its text form) over three refines equals the oracle's refine chain bit for bit."""
    from inputs import make_cloud
    n, cap, deg = 3000, 3400, 2
    p, m, v = make_cloud(n, cap, deg, 21)
    binoms = oracle.make_binoms_lut(51)
    dp, dm, dv = [x.copy() for x in p], [x.copy() for x in m], [x.copy() for x in v]
    got = ref_hip.adapter_refine(dp, dm, dv, n, cap, deg, seed=42, n_refine=3, binoms=binoms)
    rng = oracle.mt64_seed(42)
    count = n
    for k in range(3):
        res = oracle.mcmc_refine(p, m, v, count, cap, deg, rng, binoms)
        count = res["count"]
        assert got["counts"][k] == count
    for key in ("relocated_dead", "relocation_src", "added_src"):
        assert np.array_equal(got[key], res[key]), key
    assert got["rng"].equals(rng)
    for a, b in ((dp, p), (dm, m), (dv, v)):
        for g in range(6):
            assert np.array_equal(a[g].view(np.uint32), b[g].view(np.uint32)), g
