"""MCMC refine (Trainer::mcmc_refine, Sources/SplatXCore/Trainer.cpp:1273-1435) — CPU side.

The oracle's restatement (oracle/sx_oracle.cpp sxo_mcmc_refine) is pinned three ways:
- against the reference's own Trainer on the reference CPU backend (oracle/_ref), bit for bit on
  every parameter, every Adam moment, the index lists, the counts and the mt19937_64 state, over
  several consecutive refines (skipped where the reference tree is absent);
- by the known answers of the reference's McmcStrategyTests.cpp (:68-216): one alive row feeds
  every dead row with ratio 4, Adam surgery on the sources only (relocate) and on the new rows
  only (add), the growth trajectory 16 -> 17 -> ... -> 24 under cap_max 24;
- by the std::mt19937_64 seeding recurrence and the product library's host seeding helper.
"""
import numpy as np
import pytest

import oracle_py
import splatx_hip as sh
from inputs import make_cloud

F = np.float32
KMAX = 51


def same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.fixture(scope="module")
def binoms(oracle):
    return oracle.make_binoms_lut(KMAX)


def test_mt64_seed_matches_std(oracle):
    lib = sh.load_library()
    for seed in (0, 1, 42, 2**63 + 12345):
        a = oracle.mt64_seed(seed)
        st = sh.MtState()
        f = lib.sxh_mt64_seed
        f.restype, f.argtypes = sh.C.c_int32, [sh.C.c_uint64, sh.C.POINTER(sh.MtState)]
        assert f(seed, sh.C.byref(st)) == sh.SXH_OK
        assert st.equals(a) and st.p == 312
    # the first output of std::mt19937_64 with its default seed is the standard's check value
    # (C++ [rand.predef]: the 10000th output is 9981545732273789042); here: the 10000th draw
    st = oracle.mt64_seed(5489)
    d = oracle.mt64_draw(st, 10000)
    assert int(d[-1]) == 9981545732273789042
    assert st.p == 10000 - 32 * 312  # 32 twists, 16 words into the 33rd buffer


CASES = [dict(n=300, cap=400, deg=1, seed=1, refines=3),
         dict(n=2000, cap=2100, deg=3, seed=2, refines=2),           # hits the cap on the 2nd add
         dict(n=1500, cap=1500, deg=0, seed=3, refines=2),           # at cap: relocate only
         dict(n=500, cap=1000, deg=2, seed=4, refines=4, mu=2.0, sd=0.5),   # no dead: add only
         dict(n=400, cap=900, deg=3, seed=5, refines=3, mu=-6.0, sd=1.0)]   # mostly dead, heavy duplicates


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"n{c['n']}-cap{c['cap']}-deg{c['deg']}-s{c['seed']}")
def test_oracle_refine_matches_reference_trainer(reference, oracle_libm, binoms, case):
    n, cap, deg = case["n"], case["cap"], case["deg"]
    p, m, v = make_cloud(n, cap, deg, case["seed"], case.get("mu", -1.0), case.get("sd", 3.0))
    ref = reference.trainer_mcmc_refine([x[:n] for x in p], m, v, n, cap, deg, seed=42, n_refine=case["refines"])
    rng = oracle_libm.mt64_seed(42)
    count = n
    for k in range(case["refines"]):
        res = oracle_libm.mcmc_refine(p, m, v, count, cap, deg, rng, binoms)
        count = res["count"]
        assert count == ref["counts"][k]
        assert res["n_relocated"] == ref["n_relocated"][k] and res["n_added"] == ref["n_added"][k]
    assert np.array_equal(res["relocated_dead"], ref["relocated_dead"])
    assert np.array_equal(res["relocation_src"], ref["relocation_src"])
    assert np.array_equal(res["added_src"], ref["added_src"])
    for g in range(6):
        assert same(p[g], ref["params"][g]), g
        assert same(m[g], ref["exp_avg"][g]), g
        assert same(v[g], ref["exp_avg_sq"][g]), g
    assert rng.equals(ref["rng"])
    assert ref["n_relocated"].sum() + ref["n_added"].sum() > 0


def test_relocation_single_alive_feeds_all_dead(any_oracle, binoms):
    """McmcStrategyTests.cpp:68-126: one alive (0.9) and three dead rows; the sources are all 0,
    ratio = 4, the Eq.9 values land on source and dead rows alike, the other params are copied."""
    o = any_oracle
    op = np.array([0.9, 0.001, 0.004, 0.002], F)
    cap = 4
    p, m, v = make_cloud(4, cap, 1, 7, moments=False)
    p[3][:, 0] = np.log(op / (1 - op))
    before = [x.copy() for x in p]
    rng = o.mt64_seed(42)
    res = o.mcmc_refine(p, m, v, 4, cap, 1, rng, binoms)
    assert list(res["relocated_dead"]) == [1, 2, 3] and list(res["relocation_src"]) == [0, 0, 0]
    assert res["n_added"] == 0 and res["count"] == 4
    expect_op, expect_sc = o.mcmc_relocation(np.array([0.9], F), np.exp(before[2][:1]).astype(F),
                                             np.array([4], np.int32), binoms)
    sig = 1 / (1 + np.exp(-p[3][:, 0].astype(np.float64)))
    assert np.allclose(sig, expect_op[0], rtol=1e-5)
    for i in (1, 2, 3):
        for g in range(6):
            assert same(p[g][i], p[g][0])
    for g in (0, 1, 4, 5):
        assert same(p[g][0], before[g][0])  # untouched source columns
    assert np.allclose(p[2][0], np.log(expect_sc[0]), rtol=1e-6, atol=1e-6)


def test_adam_surgery_relocate_sources_only(any_oracle, binoms):
    """McmcStrategyTests.cpp:134-162: relocate zeroes the sources' moments, not the dead rows'."""
    o = any_oracle
    op = np.array([0.9, 0.001, 0.004, 0.002], F)
    p, m, v = make_cloud(4, 4, 1, 8, moments=False)
    p[3][:, 0] = np.log(op / (1 - op))
    for g in range(6):
        m[g][:] = 7.0
        v[g][:] = 3.0
    o.mcmc_refine(p, m, v, 4, 4, 1, o.mt64_seed(42), binoms)
    for g in range(6):
        assert np.all(m[g][0] == 0) and np.all(v[g][0] == 0)
        assert np.all(m[g][1:] == 7.0) and np.all(v[g][1:] == 3.0)


def test_add_zeroes_new_rows_not_sources(any_oracle, binoms):
    """McmcStrategyTests.cpp:164-216: no dead rows, growth 2 -> 3; the new row copies its source
    after Eq.9 (ratio 2); the source's moments stay, the new row's are zero."""
    o = any_oracle
    p, m, v = make_cloud(2, 3, 1, 9, moments=False)
    p[3][:2, 0] = np.log(np.array([0.5, 0.6], F) / np.array([0.5, 0.4], F))
    for g in range(6):
        m[g][:] = 7.0
        v[g][:] = 3.0
    snap = [x.copy() for x in p]
    res = o.mcmc_refine(p, m, v, 2, 3, 1, o.mt64_seed(42), binoms)
    assert res["n_relocated"] == 0 and res["n_added"] == 1 and res["count"] == 3
    s = int(res["added_src"][0])
    assert s in (0, 1)
    o_s = 1 / (1 + np.exp(-snap[3][s, 0].astype(np.float64)))
    sig = 1 / (1 + np.exp(-p[3][s, 0].astype(np.float64)))
    assert abs(sig - (1 - np.sqrt(1 - o_s))) < 1e-5
    for g in range(6):
        assert same(p[g][2], p[g][s])
    for g in (0, 1, 4, 5):
        assert same(p[g][2], snap[g][s])
    for g in range(6):
        assert np.all(m[g][:2] == 7.0) and np.all(v[g][:2] == 3.0)
        assert np.all(m[g][2] == 0) and np.all(v[g][2] == 0)


def test_growth_trajectory_capped(any_oracle, binoms):
    """McmcStrategyTests.cpp:218-243: ceil(21N/20) growth, 16 -> ... -> 24 under cap 24."""
    o = any_oracle
    p, m, v = make_cloud(16, 24, 1, 10, moments=False)
    p[3][:16, 0] = 0.0  # sigmoid = 0.5, nobody dead
    rng = o.mt64_seed(42)
    count = 16
    for want in (17, 18, 19, 20, 21, 23, 24, 24, 24):
        res = o.mcmc_refine(p, m, v, count, 24, 1, rng, binoms)
        assert res["count"] == want and res["n_added"] == want - count
        count = want


def test_running_sum_pin():
    """The oracle's running sum is numpy's sequential cumsum in float64 (np.cumsum accumulates
    left to right for 1-D input)."""
    o = oracle_py.Oracle(libm=False)
    w = np.random.default_rng(3).random(100_000).astype(F) * F(0.01)
    assert np.array_equal(o.running_sum_f64(w), np.cumsum(w.astype(np.float64)))
