"""Golden-fixture checks shared by the oracle tests (CPU) and the gfx950 backend tests (GPU).

Each check drives an `Ops`-like object (oracle_py.Oracle, oracle_py.Reference, or
splatx_hip.Backend) with the inputs of one committed fixture (tests/golden/fixtures, copied from
the reference's fixtures/) and compares against the stored outputs with the tolerances from that
fixture's meta.json, following the reference tests cited per function.
"""
from __future__ import annotations

import numpy as np

import sxt


def valid_mask(radii):
    r = np.asarray(radii).reshape(-1, 2)
    return ((r[:, 0] > 0) & (r[:, 1] > 0)).astype(np.uint8)


# AdamTests.cpp — *_out ignores valid, *_out_masked honours it (masked rows bit-identical).
def check_adam(ops):
    d = "adam_basic"
    m = sxt.meta(d)
    for masked in (False, True):
        p, ea, es = sxt.fx(d, "param").copy(), sxt.fx(d, "exp_avg").copy(), sxt.fx(d, "exp_avg_sq").copy()
        valid = sxt.fx(d, "valid") if masked else None
        ops.fused_adam(p, sxt.fx(d, "grad"), ea, es, valid, m["N"], m["lr"], m["b1"], m["b2"], m["eps"])
        sfx = "_out_masked" if masked else "_out"
        sxt.assert_all_close(p, sxt.fx(d, "param" + sfx), m, "param" + sfx)
        sxt.assert_all_close(ea, sxt.fx(d, "exp_avg" + sfx), m, "exp_avg" + sfx)
        sxt.assert_all_close(es, sxt.fx(d, "exp_avg_sq" + sfx), m, "exp_avg_sq" + sfx)
        if masked:
            inv = sxt.fx(d, "valid") == 0
            assert inv.any()
            for name, arr in (("param", p), ("exp_avg", ea), ("exp_avg_sq", es)):
                assert np.array_equal(arr[inv].view(np.uint32), sxt.fx(d, name)[inv].view(np.uint32))


def _proj_kw(d, use_covars=False, with_opacities=False):
    m = sxt.meta(d)
    kw = dict(means=sxt.fx(d, "means"), viewmats=sxt.fx(d, "viewmats"), Ks=sxt.fx(d, "Ks"),
              width=int(m["width"]), height=int(m["height"]), eps2d=m["eps2d"], near_plane=m["near_plane"],
              far_plane=m["far_plane"], radius_clip=m["radius_clip"], camera_model=int(m["camera_model"]),
              calc_compensations=bool(m["calc_compensations"]))
    if use_covars:
        kw["covars"] = sxt.fx(d, "covars_triu")
    else:
        kw["quats"], kw["scales"] = sxt.fx(d, "quats"), sxt.fx(d, "scales")
    if with_opacities:
        kw["opacities"] = sxt.fx(d, "opacities")
    return kw, m


# ProjectionMetalTests.cpp:56-94, :98-141 — radii exact, others masked allclose.
def check_projection_fwd(ops):
    for d, cov in (("proj_fused_qs/c1", False), ("proj_fused_qs/c2", False), ("proj_fully_fused", True)):
        kw, m = _proj_kw(d, use_covars=cov)
        out = ops.projection_fused_fwd(**kw)
        g_radii = sxt.fx(d, "radii")
        assert np.array_equal(out["radii"], g_radii.reshape(out["radii"].shape)), d + " radii"
        v = valid_mask(g_radii)
        assert 0 < v.sum() < v.size
        sxt.assert_all_close(out["means2d"], sxt.fx(d, "means2d"), m, "means2d", v)
        sxt.assert_all_close(out["depths"], sxt.fx(d, "depths"), m, "depths", v)
        sxt.assert_all_close(out["conics"], sxt.fx(d, "conics"), m, "conics", v)
        sxt.assert_all_close(out["compensations"], sxt.fx(d, "compensations"), m, "compensations", v)


# ProjectionMetalTests.cpp:300-420 — golden fwd outputs injected, autograd goldens compared.
def check_projection_bwd(ops):
    for d in ("proj_fused_qs/c1", "proj_fused_qs/c2"):
        kw, m = _proj_kw(d)
        inject = bool(m["bwd_inject_v_compensations"])
        g = ops.projection_fused_bwd(
            radii=sxt.fx(d, "radii"), conics=sxt.fx(d, "conics"), v_means2d=sxt.fx(d, "v_means2d"),
            v_depths=sxt.fx(d, "v_depths"), v_conics=sxt.fx(d, "v_conics"),
            compensations=sxt.fx(d, "compensations") if inject else None,
            v_compensations=sxt.fx(d, "v_compensations") if inject else None, viewmats_grad=True, **kw)
        sxt.assert_all_close(g["v_means"], sxt.fx(d, "v_means"), m, "v_means")
        sxt.assert_all_close(g["v_quats"], sxt.fx(d, "v_quats"), m, "v_quats")
        sxt.assert_all_close(g["v_scales"], sxt.fx(d, "v_scales"), m, "v_scales")
        sxt.assert_all_close(g["v_viewmats"], sxt.fx(d, "v_viewmats"), m, "v_viewmats")


# ShTests.cpp:74-130 (fwd deg 0..4, masked slots excluded) and :132-180 (bwd deg 3).
def check_sh(ops):
    d = "sh_k16"
    m = sxt.meta(d)
    B, N = m["B"], m["N"]
    dirs, coeffs, masks = sxt.fx(d, "dirs").reshape(-1, 3), sxt.fx(d, "coeffs"), sxt.fx(d, "masks").ravel()
    for deg in range(4):
        col = ops.sh_fwd(dirs, coeffs, deg, masks=masks, B=B)
        sxt.assert_all_close(col, sxt.fx(d, f"colors_deg{deg}"), m, f"colors_deg{deg}", masks)
    d25 = "sh_k25"
    m25 = sxt.meta(d25)
    col = ops.sh_fwd(sxt.fx(d25, "dirs").reshape(-1, 3), sxt.fx(d25, "coeffs"), 4, masks=None, B=1)
    sxt.assert_all_close(col, sxt.fx(d25, "colors_deg4"), m25, "colors_deg4")
    g = ops.sh_bwd(dirs, coeffs, int(m["degrees_to_use_bwd"]), sxt.fx(d, "v_colors").reshape(-1, 3),
                   masks=masks, B=B, compute_v_dirs=True)
    sxt.assert_all_close(g["v_coeffs"], sxt.fx(d, "v_coeffs"), m, "v_coeffs")
    sxt.assert_all_close(g["v_dirs"], sxt.fx(d, "v_dirs"), m, "v_dirs")
    v_means = g["v_dirs"].reshape(B, N, 3).sum(axis=0)
    sxt.assert_all_close(v_means, sxt.fx(d, "v_means"), m, "v_means")


def _isect_inputs(d, accu):
    m = sxt.meta(d)
    kw = dict(means2d=sxt.fx(d, "means2d"), radii=sxt.fx(d, "radii"), depths=sxt.fx(d, "depths"),
              I=int(m["I"]), N=int(m["N"]), tile_width=int(m["tile_width"]),
              tile_height=int(m["tile_height"]), tile_size=int(m["tile_size"]))
    if accu:
        kw["conics"], kw["opacities"] = sxt.fx(d, "conics"), sxt.fx(d, "opacities")
    return kw, m


# IsectTests.cpp:100-160 (AABB, exact), :200-330 (AccuTile, exact), sort + offsets chain :527-574.
def check_isect_sort_offsets(ops):
    for d, accu in (("isect_std", False), ("isect_ties", False), ("isect_accutile", True)):
        kw, m = _isect_inputs(d, accu)
        out = ops.isect_tiles(**kw)
        assert out["n_isects"] == m["n_isects"], d
        assert out["tile_n_bits"] == m["tile_n_bits"] and out["image_n_bits"] == m["image_n_bits"]
        assert np.array_equal(out["tiles_per_gauss"], sxt.fx(d, "tiles_per_gauss").ravel()), d
        ids = sxt.u64_from_lohi(sxt.fx(d, "isect_ids_lo"), sxt.fx(d, "isect_ids_hi"))
        assert np.array_equal(out["isect_ids"], ids), d + " isect_ids"
        assert np.array_equal(out["flatten_ids"], sxt.fx(d, "flatten_ids")), d + " flatten_ids"
        if accu:
            continue
        bits = 32 + out["tile_n_bits"] + out["image_n_bits"]
        ks, vs = ops.sort_isect(out["isect_ids"], out["flatten_ids"], bits)
        assert np.array_equal(ks, sxt.u64_from_lohi(sxt.fx(d, "isect_ids_sorted_lo"), sxt.fx(d, "isect_ids_sorted_hi")))
        assert np.array_equal(vs, sxt.fx(d, "flatten_ids_sorted")), d + " sorted values"
        off = ops.isect_offset_encode(ks, m["I"], m["tile_width"], m["tile_height"])
        assert np.array_equal(off, sxt.fx(d, "offsets").ravel()), d + " offsets"


def _raster_kw(d):
    m = sxt.meta(d)
    kw = dict(means2d=sxt.fx(d, "means2d"), conics=sxt.fx(d, "conics"), colors=sxt.fx(d, "colors"),
              opacities=sxt.fx(d, "opacities"), isect_offsets=sxt.fx(d, "isect_offsets"),
              flatten_ids=sxt.fx(d, "flatten_ids"), I=int(m["I"]), N=int(m["N"]), n_isects=int(m["n_isects"]),
              width=int(m["width"]), height=int(m["height"]), tile_width=int(m["tile_width"]),
              tile_height=int(m["tile_height"]))
    if sxt.has(d, "backgrounds"):
        kw["backgrounds"] = sxt.fx(d, "backgrounds")
    return kw, m


RASTER_FIXTURES = ("raster_small/nobg", "raster_small/bg", "raster_std", "raster_dense")


# RasterTests.cpp:120-140 — colors/alphas toleranced, last_ids exact.
def check_raster_fwd(ops):
    for d in RASTER_FIXTURES:
        kw, m = _raster_kw(d)
        out = ops.rasterize_fwd(**kw)
        sxt.assert_all_close(out["render_colors"], sxt.fx(d, "render_colors"), m, "render_colors")
        sxt.assert_all_close(out["render_alphas"], sxt.fx(d, "render_alphas"), m, "render_alphas")
        assert np.array_equal(out["last_ids"], sxt.fx(d, "last_ids")), d + " last_ids"


# RasterTests.cpp:96-106, :262-290 — golden fwd outputs injected, autograd goldens compared.
def check_raster_bwd(ops):
    for d in RASTER_FIXTURES:
        kw, m = _raster_kw(d)
        g = ops.rasterize_bwd(render_alphas=sxt.fx(d, "render_alphas"), last_ids=sxt.fx(d, "last_ids"),
                              v_render_colors=sxt.fx(d, "v_render_colors"),
                              v_render_alphas=sxt.fx(d, "v_render_alphas"), **kw)
        for t in ("v_means2d", "v_conics", "v_colors", "v_opacities"):
            sxt.assert_all_close(g[t], sxt.fx(d, t), m, t)


# SsimTests.cpp — map/scalar toleranced, v_img1 autograd golden with v_loss = 1.
def check_ssim(ops):
    d = "ssim_basic"
    m = sxt.meta(d)
    img1, img2 = sxt.fx(d, "img1"), sxt.fx(d, "img2")
    out = ops.ssim_fwd(img1, img2, need_coeffs=True)
    sxt.assert_all_close(out["ssim_map"], sxt.fx(d, "ssim_map"), m, "ssim_map")
    sxt.assert_all_close(np.array([out["ssim"]]), sxt.fx(d, "ssim"), m, "ssim")
    for k, v in m["hand_check"].items():
        _, y, x, ch = k.split("_")
        assert abs(out["ssim_map"][0, int(y[1:]), int(x[1:]), int(ch[2:])] - v) <= 1e-5 + 1e-3 * abs(v), k
    v = ops.ssim_bwd(img1, img2, out["coeff_mu"], out["coeff_sigma"], out["coeff_cross"], 1.0)
    sxt.assert_all_close(v, sxt.fx(d, "v_img1"), m, "v_img1")


def check_relocation(ops):
    d = "relocation_basic"
    m = sxt.meta(d)
    binoms = sxt.fx(d, "binoms").ravel()
    no, ns = ops.mcmc_relocation(sxt.fx(d, "opacities"), sxt.fx(d, "scales"), sxt.fx(d, "ratios"), binoms,
                                 int(m["n_max"]), m["min_opacity"])
    sxt.assert_all_close(no, sxt.fx(d, "new_opacities"), m, "new_opacities")
    sxt.assert_all_close(ns, sxt.fx(d, "new_scales"), m, "new_scales")


def check_perturb(ops):
    d = "perturb_basic"
    m = sxt.meta(d)
    pos = sxt.fx(d, "positions").copy()
    ops.mcmc_perturb_positions(pos, sxt.fx(d, "quats"), sxt.fx(d, "scales_log"), sxt.fx(d, "opacities_logit"),
                               sxt.fx(d, "noise"), m["noise_scale"], m["t"], m["k"])
    sxt.assert_all_close(pos, sxt.fx(d, "positions_out"), m, "positions_out")


# McmcTests.cpp:44-63 — Random123 philox4x32-10 known-answer vector with counter (0,0,0,0), key 0,
# reachable through the (t, offset, seed) stream mapping at t=0, offset=0, seed=0.
PHILOX_KAT0 = np.array([0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8], np.uint32)


def check_rng(ops):
    u = ops.rng_philox_u32(0, 0, 4)
    assert np.array_equal(u, PHILOX_KAT0)
    z = ops.rng_normal_f32(0xDEADBEEFCAFEF00D, 7, 1021)
    assert np.isfinite(z).all() and z.size == 1021
