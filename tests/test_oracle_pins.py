"""Pins for the oracle functions that no golden fixture covers fully.

- the fused training step (sxo_train_step) against a numpy composition of the per-op oracle
  functions (each pinned by goldens and by the reference's own CPU code) with the step glue written
  here from Trainer.cpp:716-832 (forward) and :971-1131 (step): activations, AA opacity, SH post-op
  and relu mask, L1 + SSIM loss and gradient, gradient chains, regularisers, Adam, MCMC noise;
- SH backward for degrees 0-4 (the sh_k16 golden has degree 3 only): v_coeffs by linearity of the
  forward in the coefficients, v_dirs by central differences and by tangency to the unit sphere;
- AccuTile: every tile holding a pixel centre where alpha >= 1/255 is emitted (brute force in
  float64), and the AccuTile set is a subset of the AABB set;
- scan / sort / offsets against numpy brute force.
"""
import numpy as np
import pytest

import inputs
import scene

F = np.float32


# ---------------------------------------------------------------- full step composition ----------
def adam_np(p, g, m, v, valid, lr, b1=F(0.9), b2=F(0.999), eps=F(1e-15)):
    """CpuKernels.cpp:127-144 in float32: no bias correction, eps outside the sqrt, invalid rows skipped."""
    p, m, v = p.copy(), m.copy(), v.copy()
    sel = valid.astype(bool)
    g = g[sel]
    mm = b1 * m[sel] + (F(1) - b1) * g
    vv = b2 * v[sel] + (F(1) - b2) * g * g
    p[sel] = p[sel] + (-F(lr)) * mm / (np.sqrt(vv) + eps)
    m[sel], v[sel] = mm, vv
    return p, m, v


def compose_step(orc, p, m, v, vm, K, W, H, gt, sh_degree, deg, lr, lam, aa, accutile, reg_o, reg_s,
                 noise=None):
    n = p[0].shape[0]
    means, quats, logs, logit, sh0, shN = p
    # activations (Trainer.cpp:438-460): scales = exp(log s), opacity = 1 / (1 + exp(-logit))
    s_lin = orc.expf(logs)
    opac = F(1) / (F(1) + orc.expf(-logit))
    proj = orc.projection_fused_fwd(means=means, quats=quats, scales=s_lin, opacities=opac, viewmats=vm[None],
                                    Ks=K[None], width=W, height=H, calc_compensations=aa)
    radii = proj["radii"][0]
    valid = ((radii[:, 0] > 0) & (radii[:, 1] > 0)).astype(np.uint8)
    comp = proj["compensations"][0] if aa else None
    op_used = opac * comp if aa else opac
    # dirs = means - campos, campos = -R^T t (Trainer.cpp:752-757)
    campos = np.array([-(vm[0, i] * vm[0, 3] + vm[1, i] * vm[1, 3] + vm[2, i] * vm[2, 3]) for i in range(3)], F)
    dirs = means - campos
    kt = (sh_degree + 1) ** 2
    coeffs = np.concatenate([sh0[:, None, :], shN.reshape(n, kt - 1, 3)], axis=1)
    pre = orc.sh_fwd(dirs, coeffs, deg, masks=valid) + F(0.5)
    relu = pre > 0
    colors = np.maximum(pre, F(0))
    tw, th = (W + 15) // 16, (H + 15) // 16
    ik = dict(means2d=proj["means2d"], radii=proj["radii"], depths=proj["depths"], I=1, N=n, tile_width=tw,
              tile_height=th)
    if accutile:
        ik.update(conics=proj["conics"], opacities=op_used[None])
    it = orc.isect_tiles(**ik)
    ks, vs = orc.sort_isect(it["isect_ids"], it["flatten_ids"], 32 + it["tile_n_bits"] + it["image_n_bits"])
    off = orc.isect_offset_encode(ks, 1, tw, th)
    rk = dict(means2d=proj["means2d"], conics=proj["conics"], colors=colors[None], opacities=op_used[None],
              isect_offsets=off, flatten_ids=vs, I=1, N=n, n_isects=it["n_isects"], width=W, height=H,
              tile_width=tw, tile_height=th)
    rf = orc.rasterize_fwd(**rk)
    render = rf["render_colors"][0]
    # L1 (Trainer.cpp:330-345): f64 sum of |d|, gradient sign(d) / n
    d = render - gt
    n_el = d.size
    l1 = F(np.abs(d.astype(np.float64)).sum() / n_el)
    g1 = F(1) / F(n_el)
    v_render = np.where(d > 0, g1, np.where(d < 0, -g1, F(0))).astype(F)
    loss = l1
    if lam > 0:
        so = orc.ssim_fwd(render[None], gt[None], need_coeffs=True)
        v_ds = orc.ssim_bwd(render[None], gt[None], so["coeff_mu"], so["coeff_sigma"], so["coeff_cross"],
                            v_loss=lam)[0]
        v_render = F(1 - lam) * v_render + v_ds
        loss = F(1 - lam) * l1 + F(lam) * (F(1) - F(so["ssim"]))
    rg = orc.rasterize_bwd(rf["render_alphas"], rf["last_ids"], v_render[None], np.zeros((1, H, W, 1), F), **rk)
    v_colors = np.where(relu, rg["v_colors"], F(0))
    sg = orc.sh_bwd(dirs, coeffs, deg, v_colors, masks=valid, compute_v_dirs=True)
    v_op = rg["v_opacities"].copy()
    v_comp = None
    if aa:  # Trainer.cpp:526-536
        v_comp = v_op * opac
        v_op = v_op * comp
    pg = orc.projection_fused_bwd(radii=proj["radii"], conics=proj["conics"], v_means2d=rg["v_means2d"][None],
                                  v_depths=np.zeros((1, n), F), v_conics=rg["v_conics"][None],
                                  compensations=proj["compensations"] if aa else None,
                                  v_compensations=v_comp[None] if aa else None, means=means, quats=quats,
                                  scales=s_lin, viewmats=vm[None], Ks=K[None], width=W, height=H,
                                  calc_compensations=aa)
    v_means = pg["v_means"] + sg["v_dirs"]
    v_logs = pg["v_scales"] * s_lin
    v_logit = v_op * (opac * (F(1) - opac))
    if reg_o > 0:
        v_logit = v_logit + F(reg_o) * opac * (F(1) - opac)
    if reg_s > 0:
        v_logs = v_logs + F(reg_s) * s_lin
    grads = [v_means, pg["v_quats"], v_logs, v_logit, sg["v_coeffs"][:, 0, :],
             sg["v_coeffs"][:, 1:, :].reshape(n, -1)]
    out = [adam_np(p[g], grads[g], m[g], v[g], valid, lr[g]) for g in range(6)]
    np_, nm, nv = [o[0] for o in out], [o[1] for o in out], [o[2] for o in out]
    if noise is not None:  # resident noise tail: normals (seed, offset) over 3N, then perturb
        seed, offset, scale = noise
        z = orc.rng_normal_f32(seed, offset, 3 * n).reshape(n, 3)
        orc.mcmc_perturb_positions(np_[0], np_[1], np_[2], np_[3], z, scale)
    return dict(params=np_, m=nm, v=nv, loss=loss, n_isects=it["n_isects"], render=render)


STEP_CASES = [
    dict(id="accutile-ssim", aa=False, accutile=True, lam=0.2),
    dict(id="aabb-l1", aa=False, accutile=False, lam=0.0),
    dict(id="aa-reg-noise", aa=True, accutile=True, lam=0.2, reg=True, noise=True),
    dict(id="deg1-of-2", aa=False, accutile=True, lam=0.2, deg=1),
]


@pytest.mark.parametrize("case", STEP_CASES, ids=lambda c: c["id"])
def test_train_step_matches_per_op_composition(oracle, case):
    sh_degree = 2
    deg = case.get("deg", sh_degree)
    sc = scene.make_scene(n=1500, sh_degree=sh_degree, width=72, height=56, fx=70.0, seed=3)
    r = np.random.Generator(np.random.PCG64(5))
    gt = r.uniform(0, 1, (sc.height, sc.width, 3)).astype(F)
    vm = scene.jittered_view(r, 4.0, 0.1)
    lr = [1e-2, 1e-2, 1e-2, 5e-2, 1e-2, 1e-3]
    reg_o = 1e-2 / sc.n if case.get("reg") else 0.0
    reg_s = 1e-2 / (3 * sc.n) if case.get("reg") else 0.0
    noise = (7, 3, 0.05) if case.get("noise") else None
    p0 = [a.copy() for a in sc.params]
    m0 = [r.normal(0, 1e-3, a.shape).astype(F) for a in p0]
    v0 = [r.uniform(0, 1e-5, a.shape).astype(F) for a in p0]
    exp = compose_step(oracle, p0, m0, v0, vm, sc.K, sc.width, sc.height, gt, sh_degree, deg, lr, case["lam"],
                       case["aa"], case["accutile"], reg_o, reg_s, noise)
    p, m, v = [a.copy() for a in p0], [a.copy() for a in m0], [a.copy() for a in v0]
    got = oracle.train_step(p, m, v, sc.n, sh_degree, vm, sc.K, sc.width, sc.height, gt, deg, lr,
                            opacity_reg_w=reg_o, scale_reg_w=reg_s, ssim_weight=case["lam"],
                            antialiased=case["aa"],
                            isect_mode=0 if case["accutile"] else 1, inject_noise=noise is not None,
                            noise_seed=noise[0] if noise else 0, noise_offset=noise[1] if noise else 0,
                            noise_scale=noise[2] if noise else 0.0)
    assert got["n_isects"] == exp["n_isects"] > 1000
    np.testing.assert_array_equal(got["render_colors"], exp["render"])
    assert got["loss"] == pytest.approx(float(exp["loss"]), rel=1e-6)
    for g in range(6):
        changed = np.abs(exp["params"][g] - p0[g]).max()
        assert changed > 0, f"group {g} not updated"
        np.testing.assert_allclose(p[g], exp["params"][g], rtol=1e-5, atol=1e-7, err_msg=f"params {g}")
        np.testing.assert_allclose(m[g], exp["m"][g], rtol=1e-4, atol=1e-9, err_msg=f"exp_avg {g}")
        np.testing.assert_allclose(v[g], exp["v"][g], rtol=1e-4, atol=1e-12, err_msg=f"exp_avg_sq {g}")


# ---------------------------------------------------------------- SH backward, degrees 0-4 -------
@pytest.mark.parametrize("deg", [0, 1, 2, 3, 4])
def test_sh_bwd_linearity_fd_and_tangency(oracle, deg):
    r = inputs.rng(100 + deg)
    n, K = 64, 25 if deg == 4 else 16
    nb = (deg + 1) ** 2
    dirs = r.standard_normal((n, 3)).astype(F)
    coeffs = r.normal(0, 0.5, (n, K, 3)).astype(F)
    vcol = r.standard_normal((n, 3)).astype(F)
    out = oracle.sh_bwd(dirs, coeffs, deg, vcol, compute_v_dirs=True)
    # colors = sum_k Y_k(dir) c_k is linear in c: d colors / d c_k = Y_k(dir), read off sh_fwd with a one-hot c
    for k in range(K):
        onehot = np.zeros_like(coeffs)
        onehot[:, k, :] = 1.0
        Yk = oracle.sh_fwd(dirs, onehot, deg)[:, 0]
        want = Yk[:, None] * vcol if k < nb else np.zeros_like(vcol)
        np.testing.assert_allclose(out["v_coeffs"][:, k, :], want, rtol=1e-5, atol=1e-6, err_msg=f"k={k}")
    # v_dirs: central differences of L = <v_colors, sh_fwd(dirs)>, Richardson-extrapolated (error O(h^4))
    def central(a, rel):
        h = rel * np.linalg.norm(dirs.astype(np.float64), axis=1)  # step relative to |dir|
        dp, dm = dirs.astype(np.float64).copy(), dirs.astype(np.float64).copy()
        dp[:, a] += h
        dm[:, a] -= h
        lp = (oracle.sh_fwd(dp.astype(F), coeffs, deg).astype(np.float64) * vcol).sum(1)
        lm = (oracle.sh_fwd(dm.astype(F), coeffs, deg).astype(np.float64) * vcol).sum(1)
        return (lp - lm) / (dp[:, a] - dm[:, a])

    fd = np.stack([(4 * central(a, 5e-3) - central(a, 1e-2)) / 3 for a in range(3)], axis=1)
    vd = out["v_dirs"].astype(np.float64)
    if deg == 0:
        assert np.all(vd == 0)
        return
    err = np.linalg.norm(vd - fd) / np.linalg.norm(fd)
    assert err < 2e-3, err
    # SH is evaluated at dir/|dir|: the gradient is orthogonal to dir
    cos = np.abs((vd * dirs).sum(1)) / (np.linalg.norm(vd, axis=1) * np.linalg.norm(dirs, axis=1) + 1e-30)
    assert cos.max() < 1e-4


def test_sh_bwd_planted_error_is_caught(oracle):
    """The linearity check above fails for a plausible mistake: a transposed (coefficient, channel) index."""
    r = inputs.rng(7)
    dirs = r.standard_normal((16, 3)).astype(F)
    coeffs = r.normal(0, 0.5, (16, 16, 3)).astype(F)
    vcol = r.standard_normal((16, 3)).astype(F)
    good = oracle.sh_bwd(dirs, coeffs, 3, vcol)["v_coeffs"]
    bad = good[:, :, ::-1]  # channels swapped
    onehot = np.zeros_like(coeffs)
    onehot[:, 5, :] = 1.0
    Y5 = oracle.sh_fwd(dirs, onehot, 3)[:, 0]
    assert not np.allclose(bad[:, 5, :], Y5[:, None] * vcol, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- AccuTile coverage --------------
def test_accutile_covers_every_significant_pixel(oracle):
    W, H = 160, 120
    kw, p, pk = inputs.isect_kwargs(oracle, n=1500, seed=8, accutile=True, width=W, height=H, with_proj=True)
    tw, th = kw["tile_width"], kw["tile_height"]
    acc = oracle.isect_tiles(**kw)
    aabb = oracle.isect_tiles(**{k: v for k, v in kw.items() if k not in ("conics", "opacities")})
    tb = acc["tile_n_bits"]
    tmask = np.uint64((1 << tb) - 1)

    def sets(it):
        tiles = ((it["isect_ids"] >> np.uint64(32)) & tmask).astype(np.int64)
        return {(int(g), int(t)) for g, t in zip(it["flatten_ids"], tiles)}

    s_acc, s_aabb = sets(acc), sets(aabb)
    assert s_acc <= s_aabb and len(s_acc) < len(s_aabb)
    # brute force: pixel centres where opacity * exp(-sigma) >= 1/255 (float64)
    ys, xs = np.mgrid[0:H, 0:W]
    cx, cy = xs.ravel() + 0.5, ys.ravel() + 0.5
    tile_of = (ys.ravel() // 16) * tw + xs.ravel() // 16
    radii = p["radii"][0]
    m2, con = p["means2d"][0].astype(np.float64), p["conics"][0].astype(np.float64)
    op = pk["opacities"].astype(np.float64)
    checked = 0
    for g in np.nonzero((radii[:, 0] > 0) & (radii[:, 1] > 0))[0]:
        dx, dy = m2[g, 0] - cx, m2[g, 1] - cy
        sigma = 0.5 * (con[g, 0] * dx * dx + con[g, 2] * dy * dy) + con[g, 1] * dx * dy
        hit = op[g] * np.exp(-sigma) >= (1.0 / 255.0) * (1 + 1e-6)
        for t in np.unique(tile_of[hit]):
            assert (int(g), int(t)) in s_acc, (g, t)
            checked += 1
    assert checked > 1000


# ---------------------------------------------------------------- scan / sort / offsets ----------
def test_scan_sort_offsets_brute_force(oracle):
    r = inputs.rng(9)
    x = r.integers(0, 40, 100_003).astype(np.int32)
    np.testing.assert_array_equal(oracle.prefix_scan_i64(x), np.cumsum(x, dtype=np.int64))
    for bits in (45, 64):
        keys, vals = inputs.sort_inputs(50_000, bits, seed=bits)
        ks, vs = oracle.sort_isect(keys, vals, bits)
        ek, ev = inputs.stable_sort_ref(keys, vals)
        np.testing.assert_array_equal(ks, ek)
        np.testing.assert_array_equal(vs, ev)
    tw, th, I = 9, 7, 2
    nt = tw * th
    tiles = np.sort(r.integers(0, I * nt, 5000)).astype(np.uint64)
    keys = (tiles // np.uint64(nt)) << np.uint64(32 + 6) | (tiles % np.uint64(nt)) << np.uint64(32)
    off = oracle.isect_offset_encode(keys, I, tw, th)
    np.testing.assert_array_equal(off, np.searchsorted(tiles, np.arange(I * nt), side="left"))
    np.testing.assert_array_equal(oracle.isect_offset_encode(keys[:0], I, tw, th, n_isects=0), np.zeros(I * nt))


def test_sort_counting_passes_brute_force(oracle):
    """The oracle's sort (a counting pass on the top 16 significant bits, then 8-bit LSD counting passes
    inside each run of equal top bits) against numpy's stable argsort where the passes matter most: few
    key bits with heavy ties, keys whose low or middle bytes are all equal (passes skipped), long runs of
    equal top bits whose low bits need two passes, a key width that is not a multiple of 8, one key, and
    keys in descending order. A pass that dropped stability, used the wrong digit, split the bits at the
    wrong place or skipped a needed byte would reorder equal keys or leave keys unsorted."""
    r = inputs.rng(21)
    cases = {
        "13 bits, heavy ties": r.integers(0, 1 << 13, 40_000).astype(np.uint64),
        "1 bit": r.integers(0, 2, 5_000).astype(np.uint64),
        "45 bits, low 32 bits equal": (r.integers(0, 1 << 13, 30_000).astype(np.uint64) << np.uint64(32)) | np.uint64(7),
        "40 bits, middle bytes equal": (r.integers(0, 256, 20_000).astype(np.uint64) << np.uint64(32))
        | np.uint64(0x00ABCD00) | r.integers(0, 256, 20_000).astype(np.uint64),
        "30 bits, 4 runs of top bits": (r.integers(0, 4, 30_000).astype(np.uint64) << np.uint64(14))
        | r.integers(0, 1 << 14, 30_000).astype(np.uint64),
        "one key": np.array([5], np.uint64),
        "descending 17 bits": np.arange(70_000, 0, -1).astype(np.uint64),
    }
    widths = {"13 bits, heavy ties": 13, "1 bit": 1, "45 bits, low 32 bits equal": 45,
              "40 bits, middle bytes equal": 40, "30 bits, 4 runs of top bits": 30, "one key": 3, "descending 17 bits": 17}
    for name, keys in cases.items():
        vals = r.integers(-2**31, 2**31 - 1, keys.size).astype(np.int32)
        ks, vs = oracle.sort_isect(keys, vals, widths[name])
        ek, ev = inputs.stable_sort_ref(keys, vals)
        np.testing.assert_array_equal(ks, ek, err_msg=name)
        np.testing.assert_array_equal(vs, ev, err_msg=name)


# ---------------------------------------------------------------- projection bwd, covars path ----
def covars_fd_case(oracle, aa):
    """Projection backward on the covariance path (6-triu input), with the directional-free reference:
    central differences of L = <v_conics, conics> (+ <v_comp, compensations> when antialiased) in each
    triu entry, Richardson-extrapolated. An off-diagonal entry c_ij (i < j) sits at (i, j) and (j, i)
    of the symmetric matrix, so dL/dc_ij is the sum of both positions' derivatives
    (ProjectionEWA.metal:475-480)."""
    kw = inputs.proj_kwargs(n=96, seed=91, covars=True, aa=aa, znear=1.5)
    r = inputs.rng(92)
    fwd = oracle.projection_fused_fwd(**kw)
    n = kw["covars"].shape[0]
    v_conics = r.standard_normal((1, n, 3)).astype(F)
    v_comp = r.standard_normal((1, n)).astype(F) if aa else None
    bwd = oracle.projection_fused_bwd(radii=fwd["radii"], conics=fwd["conics"], compensations=fwd["compensations"],
                                      v_means2d=np.zeros((1, n, 2), F), v_depths=np.zeros((1, n), F),
                                      v_conics=v_conics, v_compensations=v_comp, **kw)
    cov0 = kw["covars"].astype(np.float64)
    keep = (fwd["radii"][0] > 0).all(axis=1)

    def loss(cov):
        o = oracle.projection_fused_fwd(**dict(kw, covars=cov.astype(F)))
        l = (o["conics"][0].astype(np.float64) * v_conics[0]).sum(1)
        if aa:
            l = l + o["compensations"][0].astype(np.float64) * v_comp[0]
        return l, (o["radii"][0] > 0).all(axis=1)

    def central(k, rel):
        h = rel * np.abs(cov0[:, [0, 3, 5]]).max(axis=1)  # step relative to the covariance's scale
        cp, cm = cov0.copy(), cov0.copy()
        cp[:, k] += h
        cm[:, k] -= h
        lp, vp = loss(cp)
        lm, vm_ = loss(cm)
        steps = cp[:, k].astype(F).astype(np.float64) - cm[:, k].astype(F).astype(np.float64)
        return (lp - lm) / steps, vp & vm_

    fd = np.zeros((n, 6))
    for k in range(6):
        a, va = central(k, 2e-3)
        b, vb = central(k, 4e-3)
        fd[:, k] = (4 * a - b) / 3
        keep &= va & vb
    assert keep.sum() > 40
    return bwd["v_covars"].astype(np.float64)[keep], fd[keep]


@pytest.mark.parametrize("aa", [False, True])
def test_projection_bwd_covars_central_differences(oracle, aa):
    got, fd = covars_fd_case(oracle, aa)
    err = np.linalg.norm(got - fd) / np.linalg.norm(fd)
    assert err < 1e-3, err
    # the off-diagonal entries carry a real share of the gradient (the check below is not vacuous)
    assert np.linalg.norm(fd[:, [1, 2, 4]]) > 0.1 * np.linalg.norm(fd)


def test_projection_bwd_covars_planted_error_is_caught(oracle):
    """A plausible mistake, one of the symmetric off-diagonal contributions not summed (any one of the
    c01, c02, c12 entries halved), fails the central-difference check above."""
    got, fd = covars_fd_case(oracle, False)
    for k in (1, 2, 4):
        bad = got.copy()
        bad[:, k] *= 0.5
        err = np.linalg.norm(bad - fd) / np.linalg.norm(fd)
        assert err > 1e-2, (k, err)
