"""gfx950 backend (through the C ABI) against the golden fixtures and the CPU oracle.

Bar: bit-exact for integer, key and index outputs and for every deterministic forward
(projection, SH, isect, scan, sort, offsets, raster fwd, SSIM, Adam, RNG, relocation, perturb —
the device code follows the oracle's operation order with the same transcendental layer);
gradients whose device accumulation order differs (raster bwd atomics, float SH/projection VJPs vs
the oracle's double accumulation) are held to rel_l2 <= 1e-4 (north star: rel 1e-4 for gradients).
"""
import hashlib

import numpy as np
import pytest

import golden_checks as gc
import inputs
import splatx_hip as sh

pytestmark = pytest.mark.gpu

GOLDEN = [gc.check_adam, gc.check_projection_fwd, gc.check_projection_bwd, gc.check_sh, gc.check_isect_sort_offsets,
          gc.check_raster_fwd, gc.check_raster_bwd, gc.check_ssim, gc.check_relocation, gc.check_perturb,
          gc.check_rng]


@pytest.mark.parametrize("check", GOLDEN, ids=lambda c: c.__name__)
def test_gpu_goldens(gpu, check):
    check(gpu)


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.dtype.kind == "f":
        return np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else np.uint64),
                              b.view(np.uint32 if b.dtype == np.float32 else np.uint64))
    return np.array_equal(a, b)


def rel_l2(a, e):
    a = np.asarray(a, np.float64).ravel()
    e = np.asarray(e, np.float64).ravel()
    den = np.sqrt((e * e).sum())
    return float(np.sqrt(((a - e) ** 2).sum()) / den) if den > 0 else float(np.sqrt(((a - e) ** 2).sum()))


# ---- projection ----------------------------------------------------------------------------
PROJ_CASES = [dict(), dict(aa=True), dict(covars=True, n=1500), dict(C=3), dict(opacities=False),
              dict(C=2, aa=True, n=2500)]


@pytest.mark.parametrize("case", PROJ_CASES, ids=str)
def test_projection_fwd_bitexact(gpu, oracle, case):
    kw = inputs.proj_kwargs(seed=11, **case)
    g = gpu.projection_fused_fwd(**kw)
    o = oracle.projection_fused_fwd(**kw)
    v = gc.valid_mask(o["radii"])
    assert 0 < v.sum() < v.size
    for k in ("radii", "means2d", "depths", "conics"):
        assert same_bits(g[k], o[k]), k
    if kw["calc_compensations"]:
        assert same_bits(g["compensations"], o["compensations"])


@pytest.mark.parametrize("case", [dict(), dict(aa=True), dict(covars=True, n=1500), dict(C=3)], ids=str)
def test_projection_bwd_close(gpu, oracle, case):
    kw = inputs.proj_kwargs(seed=12, **case)
    f = oracle.projection_fused_fwd(**kw)
    r = inputs.rng(5)
    CN = f["depths"].size
    v = gc.valid_mask(f["radii"]).reshape(f["depths"].shape)
    gin = dict(radii=f["radii"], conics=f["conics"],
               v_means2d=(r.standard_normal(f["means2d"].shape) * v[..., None]).astype(np.float32),
               v_depths=(r.standard_normal(f["depths"].shape) * v).astype(np.float32),
               v_conics=(r.standard_normal(f["conics"].shape) * v[..., None]).astype(np.float32),
               viewmats_grad=True)
    if kw["calc_compensations"]:
        gin["compensations"] = f["compensations"]
        gin["v_compensations"] = (r.standard_normal(CN) * v.ravel()).astype(np.float32).reshape(f["depths"].shape)
    a = gpu.projection_fused_bwd(**gin, **kw)
    b = oracle.projection_fused_bwd(**gin, **kw)
    for k in ("v_means", "v_covars", "v_quats", "v_scales", "v_viewmats"):
        if b[k] is not None:
            assert rel_l2(a[k], b[k]) <= 1e-4, (k, rel_l2(a[k], b[k]))


# ---- SH --------------------------------------------------------------------------------------------
@pytest.mark.parametrize("deg,K,B", [(0, 1, 1), (1, 4, 1), (2, 9, 1), (3, 16, 1), (3, 16, 2), (4, 25, 1), (2, 16, 1)])
def test_sh_fwd_bitexact_bwd_close(gpu, oracle, deg, K, B):
    r = inputs.rng(deg * 10 + K + B)
    N = 3000
    dirs = r.standard_normal((B * N, 3)).astype(np.float32)
    coeffs = r.standard_normal((N, K, 3)).astype(np.float32)
    masks = (r.uniform(0, 1, B * N) > 0.3).astype(np.uint8)
    a = gpu.sh_fwd(dirs, coeffs, deg, masks=masks, B=B)
    b = oracle.sh_fwd(dirs, coeffs, deg, masks=masks, B=B)
    assert same_bits(a, b)
    vc = r.standard_normal((B * N, 3)).astype(np.float32)
    ga = gpu.sh_bwd(dirs, coeffs, deg, vc, masks=masks, B=B)
    gb = oracle.sh_bwd(dirs, coeffs, deg, vc, masks=masks, B=B)
    assert rel_l2(ga["v_coeffs"], gb["v_coeffs"]) <= 1e-5
    if deg > 0:
        assert rel_l2(ga["v_dirs"], gb["v_dirs"]) <= 1e-5


# ---- intersection / scan / sort / offsets ----------------------------------------------------------
@pytest.mark.parametrize("accu,I", [(True, 1), (False, 1), (True, 2), (False, 2)])
def test_isect_bitexact(gpu, oracle, accu, I):
    kw = inputs.isect_kwargs(oracle, n=5000, seed=21 + I, accutile=accu, I=I)
    a = gpu.isect_tiles(**kw)
    b = oracle.isect_tiles(**kw)
    assert a["n_isects"] == b["n_isects"] > 0
    for k in ("tiles_per_gauss", "isect_ids", "flatten_ids"):
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.parametrize("n", [1, 7, 255, 256, 4095, 4096, 4097, 100_000, 1_000_003])
def test_scan_exact(gpu, n):
    r = inputs.rng(n)
    x = r.integers(0, 3000, n).astype(np.int32)
    if n > 10:
        x[r.integers(0, n, 3)] = 2_000_000_000  # int64 promotion
    assert np.array_equal(gpu.prefix_scan_i64(x), np.cumsum(x.astype(np.int64)))


@pytest.mark.parametrize("n", [0, 1, 255, 256, 1023, 1024, 4095, 4096, 4097, 65_537, 300_001])
@pytest.mark.parametrize("bits", [4, 13, 36, 45, 64])
def test_sort_matches_stable_sort(gpu, n, bits):
    keys, vals = inputs.sort_inputs(n, bits, seed=n + bits)
    ks, vs = gpu.sort_isect(keys, vals, bits)
    rk, rv = inputs.stable_sort_ref(keys, vals)
    assert np.array_equal(ks, rk) and np.array_equal(vs, rv)


def test_sort_3m_with_ties_and_determinism(gpu):
    keys, vals = inputs.sort_inputs(3_000_000, 45, seed=3)
    rk, rv = inputs.stable_sort_ref(keys, vals)
    digests = set()
    for _ in range(5):
        ks, vs = gpu.sort_isect(keys, vals, 45)
        assert np.array_equal(ks, rk) and np.array_equal(vs, rv)
        digests.add(hashlib.sha1(ks.tobytes() + vs.tobytes()).hexdigest())
    assert len(digests) == 1


# From 256 tiles of 4096 keys on (1 M keys) every pass takes its prefixes from a scan of the tiles'
# digit counts instead of the look-back chain (below, the 300,001-key cases above take the chain): the
# same stable order, checked at the threshold, with a ragged last tile, at config-5 scale in tiles,
# and for 2, 6 and 8 passes; and all keys equal (every tile's run of one digit).
@pytest.mark.parametrize("n,bits", [(1_048_576, 13), (1_048_577, 45), (9_000_001, 45), (9_000_001, 64)])
def test_sort_reduce_then_scan_matches_stable_sort(gpu, n, bits):
    keys, vals = inputs.sort_inputs(n, bits, seed=n + bits)
    ks, vs = gpu.sort_isect(keys, vals, bits)
    rk, rv = inputs.stable_sort_ref(keys, vals)
    assert np.array_equal(ks, rk) and np.array_equal(vs, rv)


def _run_keys(n, key_bits, seed):
    """Keys in runs, the way an emit lays out tile ids: runs of 1-40 keys that repeat a key or step by
    2^s (s at a digit boundary or not), so some pass sees runs of equal digits and runs of consecutive
    digits that wrap past the last digit into the next one."""
    r = inputs.rng(seed)
    top = np.uint64(2**min(key_bits, 63) - 1) if key_bits < 64 else np.uint64(2**64 - 1)
    keys = np.empty(n, np.uint64)
    i = 0
    while i < n:
        length = int(r.integers(1, 41))
        start = np.uint64(r.integers(0, 2**min(key_bits, 62)))
        s = int(r.choice([0, 0, 1, 5, 6, 7, 8, 13, 16, 24, 32, 40])) % max(1, key_bits)
        step = np.uint64(0) if r.random() < 0.3 else np.uint64(1) << np.uint64(s)
        k = min(length, n - i)
        keys[i:i + k] = (start + step * np.arange(k, dtype=np.uint64)) & top
        i += k
    return keys, np.arange(n, dtype=np.int32)


# Keys laid out in runs (an emit's tile ids along a row, repeated keys): the digit counts add a thread's
# runs of equal digits at once, and the passes see runs of consecutive digits wrapping past the last
# digit, for digit ranges from 16 (the first pass of 9 bits: 4 + 5) to 256.
@pytest.mark.parametrize("n,bits", [(1_048_577, 9), (1_048_577, 13), (1_048_576, 36), (2_000_003, 45),
                                    (1_100_000, 64)])
def test_sort_reduce_then_scan_runs(gpu, n, bits):
    keys, vals = _run_keys(n, bits, seed=n + bits)
    ks, vs = gpu.sort_isect(keys, vals, bits)
    rk, rv = inputs.stable_sort_ref(keys, vals)
    assert np.array_equal(ks, rk) and np.array_equal(vs, rv)


def test_sort_reduce_then_scan_equal_keys(gpu):
    n = 8_500_000
    keys = np.full(n, (np.uint64(5) << np.uint64(32)) | np.uint64(77), np.uint64)
    vals = np.arange(n, dtype=np.int32)[::-1].copy()
    ks, vs = gpu.sort_isect(keys, vals, 45)
    assert np.array_equal(ks, keys) and np.array_equal(vs, vals)


def test_offsets_doc_example_and_edges(gpu, oracle):
    # IsectTests/ScanTests doc example: tile ids [1,1,1,3,3] over 6 tiles -> [0,0,3,3,5,5]
    ids = (np.array([1, 1, 1, 3, 3], np.uint64) << np.uint64(32))
    assert list(gpu.isect_offset_encode(ids, 1, 6, 1)) == [0, 0, 3, 3, 5, 5]
    assert list(gpu.isect_offset_encode(np.zeros(0, np.uint64), 1, 6, 1)) == [0] * 6
    kw = inputs.isect_kwargs(oracle, n=4000, seed=31, I=2)
    it = oracle.isect_tiles(**kw)
    ks, _ = oracle.sort_isect(it["isect_ids"], it["flatten_ids"], 32 + it["tile_n_bits"] + it["image_n_bits"])
    a = gpu.isect_offset_encode(ks, 2, kw["tile_width"], kw["tile_height"])
    b = oracle.isect_offset_encode(ks, 2, kw["tile_width"], kw["tile_height"])
    assert np.array_equal(a, b)


# ---- raster ----------------------------------------------------------------------------------------------
RASTER_CASES = [dict(), dict(backgrounds=True), dict(masks=True, backgrounds=True), dict(I=2), dict(accutile=False),
                dict(n=12000, width=333, height=171)]


@pytest.mark.parametrize("case", RASTER_CASES, ids=str)
def test_raster_fwd_bitexact_bwd_close(gpu, oracle, case):
    kw = inputs.raster_kwargs(oracle, seed=41, **case)
    a = gpu.rasterize_fwd(**kw)
    b = oracle.rasterize_fwd(**kw)
    for k in ("render_colors", "render_alphas", "last_ids"):
        assert same_bits(a[k], b[k]), k
    a2 = gpu.rasterize_fwd(**kw)
    assert same_bits(a2["render_colors"], a["render_colors"])  # run-to-run determinism
    r = inputs.rng(9)
    gin = dict(render_alphas=b["render_alphas"], last_ids=b["last_ids"],
               v_render_colors=r.standard_normal(b["render_colors"].shape).astype(np.float32),
               v_render_alphas=r.standard_normal(b["render_alphas"].shape).astype(np.float32))
    ga = gpu.rasterize_bwd(absgrad=True, **gin, **kw)
    gb = oracle.rasterize_bwd(absgrad=True, **gin, **kw)
    for k in ("v_means2d", "v_conics", "v_colors", "v_opacities", "v_means2d_abs"):
        assert rel_l2(ga[k], gb[k]) <= 1e-4, (k, rel_l2(ga[k], gb[k]))
    gc2 = gpu.rasterize_bwd(absgrad=True, **gin, **kw)  # self-consistency of the atomic path
    for k in ("v_means2d", "v_conics", "v_colors", "v_opacities"):
        assert rel_l2(gc2[k], ga[k]) <= 1e-5


def extreme_splats(seed, n=400, width=80, height=56):
    """Splats of every shape the rasterisers' block lists must keep or drop correctly: needle-thin ellipses
    (aspect up to 1000:1) at every angle, sub-pixel and image-sized footprints, opacities from just above
    1/255 (tiny cutoffs) to 0.99, centres inside, on tile and block edges and outside the image. Every
    tile's list holds every splat (index order), so the lists, not the intersection test, decide which
    pairs are evaluated."""
    r = inputs.rng(seed)
    s1 = np.exp(r.uniform(np.log(0.15), np.log(60.0), n))
    s2 = s1 * np.exp(r.uniform(np.log(1e-3), 0.0, n))
    th = r.uniform(0.0, np.pi, n)
    c, s = np.cos(th), np.sin(th)
    cxx = c * c * s1 ** 2 + s * s * s2 ** 2
    cyy = s * s * s1 ** 2 + c * c * s2 ** 2
    cxy = c * s * (s1 ** 2 - s2 ** 2)
    det = cxx * cyy - cxy ** 2
    conics = np.stack([cyy / det, -cxy / det, cxx / det], 1).astype(np.float32)[None]
    means = np.stack([r.uniform(-10, width + 10, n), r.uniform(-10, height + 10, n)], 1)
    snap = r.uniform(size=n) < 0.3  # a share of centres exactly on a 4-pixel block or tile boundary
    means[snap] = np.round(means[snap] / 4.0) * 4.0
    opac = np.exp(r.uniform(np.log(1.05 / 255.0), np.log(0.99), n)).astype(np.float32)[None]
    tw, th_ = (width + 15) // 16, (height + 15) // 16
    n_tiles = tw * th_
    flat = np.tile(np.arange(n, dtype=np.int32), n_tiles)
    off = (np.arange(n_tiles, dtype=np.int32) * n).reshape(1, th_, tw)
    colors = r.uniform(0.0, 1.0, (1, n, 3)).astype(np.float32)
    return dict(means2d=means.astype(np.float32)[None], conics=conics, colors=colors, opacities=opac,
                isect_offsets=off, flatten_ids=flat, I=1, N=n, n_isects=int(flat.size), width=width, height=height,
                tile_width=tw, tile_height=th_)


@pytest.mark.parametrize("seed", [3, 4, 5])
def test_raster_extreme_shapes(gpu, oracle, seed):
    """The block lists (bounding box and exact per-row ellipse ranges) must keep every block a splat's
    cutoff set reaches: any block dropped wrongly changes a pixel of the bit-exact forward."""
    kw = extreme_splats(seed)
    a = gpu.rasterize_fwd(**kw)
    b = oracle.rasterize_fwd(**kw)
    assert b["render_alphas"].max() > 0.5
    for k in ("render_colors", "render_alphas", "last_ids"):
        assert same_bits(a[k], b[k]), k
    r = inputs.rng(seed + 100)
    gin = dict(render_alphas=b["render_alphas"], last_ids=b["last_ids"],
               v_render_colors=r.standard_normal(b["render_colors"].shape).astype(np.float32),
               v_render_alphas=r.standard_normal(b["render_alphas"].shape).astype(np.float32))
    ga = gpu.rasterize_bwd(absgrad=False, **gin, **kw)
    gb = oracle.rasterize_bwd(absgrad=False, **gin, **kw)
    for k in ("v_means2d", "v_conics", "v_colors", "v_opacities"):
        assert rel_l2(ga[k], gb[k]) <= 1e-4, (k, rel_l2(ga[k], gb[k]))


def test_raster_general_exponential(gpu, oracle):
    """Opacities above ~1e35 put a splat's cutoff past the range of the rasterisers' branch-free
    exponential (and at 5e37 make it infinite): the batches holding one take the general exponential,
    so the forward stays bit-exact and the backward within tolerance."""
    kw = extreme_splats(6)
    r = inputs.rng(106)
    # small footprints late in the order (their cutoff radius is ~13 standard deviations), so that most
    # pixels still composite the other splats first
    con = kw["conics"][0]
    small = np.flatnonzero((np.minimum(con[:, 0], con[:, 2]) > 4.0) & (np.arange(kw["N"]) > kw["N"] // 3))
    huge = r.choice(small, 8, replace=False)
    op = kw["opacities"].copy()
    op[0, huge[:6]] = np.exp(r.uniform(np.log(1e35), np.log(1e36), 6)).astype(np.float32)
    op[0, huge[6:]] = 5e37
    kw["opacities"] = op
    a = gpu.rasterize_fwd(**kw)
    b = oracle.rasterize_fwd(**kw)
    for k in ("render_colors", "render_alphas", "last_ids"):
        assert same_bits(a[k], b[k]), k
    gin = dict(render_alphas=b["render_alphas"], last_ids=b["last_ids"],
               v_render_colors=r.standard_normal(b["render_colors"].shape).astype(np.float32),
               v_render_alphas=r.standard_normal(b["render_alphas"].shape).astype(np.float32))
    ga = gpu.rasterize_bwd(absgrad=False, **gin, **kw)
    gb = oracle.rasterize_bwd(absgrad=False, **gin, **kw)
    for k in ("v_means2d", "v_conics", "v_colors", "v_opacities"):
        assert rel_l2(ga[k], gb[k]) <= 1e-4, (k, rel_l2(ga[k], gb[k]))


def test_raster_empty_and_background(gpu, oracle):
    kw = inputs.raster_kwargs(oracle, seed=43, backgrounds=True)
    kw["n_isects"] = 0
    kw["flatten_ids"] = np.zeros(0, np.int32)
    kw["isect_offsets"] = np.zeros_like(kw["isect_offsets"])
    a = gpu.rasterize_fwd(**kw)
    b = oracle.rasterize_fwd(**kw)
    assert same_bits(a["render_colors"], b["render_colors"])
    assert np.allclose(a["render_colors"][0], kw["backgrounds"][0])


# ---- SSIM -------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(1, 24, 24, 3), (1, 37, 53, 3), (2, 16, 40, 1), (1, 200, 301, 3), (2, 30, 41, 3),
                                   (1, 19, 27, 4)])
def test_ssim_bitexact(gpu, oracle, shape):
    r = inputs.rng(sum(shape))
    x = r.uniform(0, 1, shape).astype(np.float32)
    y = np.clip(x * 0.9 + r.normal(0, 0.05, shape), 0, 1).astype(np.float32)
    a = gpu.ssim_fwd(x, y, need_coeffs=True)
    b = oracle.ssim_fwd(x, y, need_coeffs=True)
    for k in ("ssim_map", "coeff_mu", "coeff_sigma", "coeff_cross"):
        assert same_bits(a[k], b[k]), k
    assert a["ssim"] == b["ssim"]
    va = gpu.ssim_bwd(x, y, a["coeff_mu"], a["coeff_sigma"], a["coeff_cross"], 0.2)
    vb = oracle.ssim_bwd(x, y, b["coeff_mu"], b["coeff_sigma"], b["coeff_cross"], 0.2)
    assert same_bits(va, vb)


# ---- Adam / RNG / MCMC -------------------------------------------------------------------------------------
def test_adam_bitexact(gpu, oracle):
    r = inputs.rng(3)
    N, D = 50_000, 7
    p, g = r.standard_normal((N, D)).astype(np.float32), r.standard_normal((N, D)).astype(np.float32)
    m, v = r.standard_normal((N, D)).astype(np.float32), np.abs(r.standard_normal((N, D))).astype(np.float32)
    valid = (r.uniform(0, 1, N) > 0.4).astype(np.uint8)
    outs = []
    for ops in (gpu, oracle):
        pp, mm, vv = p.copy(), m.copy(), v.copy()
        ops.fused_adam(pp, g, mm, vv, valid, N, 1e-3, 0.9, 0.999, 1e-15)
        outs.append((pp, mm, vv))
    for x, y in zip(*outs):
        assert same_bits(x, y)


def test_rng_bitexact(gpu, oracle):
    for seed, off, count in ((0, 0, 4), (0xDEADBEEFCAFEF00D, 7, 1021), (0x853C49E6748FEA9B, 2**33 + 5, 100_003)):
        assert np.array_equal(gpu.rng_philox_u32(seed, off, count), oracle.rng_philox_u32(seed, off, count))
        assert same_bits(gpu.rng_normal_f32(seed, off, count), oracle.rng_normal_f32(seed, off, count))
    z = gpu.rng_normal_f32(1, 0, 1_000_000)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3


def test_relocation_and_perturb_bitexact(gpu, oracle):
    r = inputs.rng(4)
    N = 5000
    op = r.uniform(0.001, 0.999, N).astype(np.float32)
    sc = np.exp(r.normal(-3, 1, (N, 3))).astype(np.float32)
    ratios = r.integers(1, 52, N).astype(np.int32)
    binoms = oracle.make_binoms_lut(51)
    assert same_bits(gpu.make_binoms_lut(51), binoms)
    a = gpu.mcmc_relocation(op, sc, ratios, binoms)
    b = oracle.mcmc_relocation(op, sc, ratios, binoms)
    assert same_bits(a[0], b[0]) and same_bits(a[1], b[1])
    pos = r.standard_normal((N, 3)).astype(np.float32)
    args = (r.standard_normal((N, 4)).astype(np.float32), r.normal(-3, 1, (N, 3)).astype(np.float32),
            r.standard_normal(N).astype(np.float32), r.standard_normal((N, 3)).astype(np.float32))
    pa, pb = pos.copy(), pos.copy()
    gpu.mcmc_perturb_positions(pa, *args, 0.05)
    oracle.mcmc_perturb_positions(pb, *args, 0.05)
    assert same_bits(pa, pb)


# ---- error contract (Validate.h) -----------------------------------------------------------------------
def test_validation_errors(gpu):
    kw = inputs.proj_kwargs(n=10)
    with pytest.raises(sh.SxRuntimeError):
        gpu.projection_fused_fwd(**dict(kw, camera_model=1))
    with pytest.raises(sh.SxInvalidArgument):
        gpu.sort_isect(np.zeros(4, np.uint64), np.zeros(4, np.int32), 65)
    with pytest.raises(sh.SxInvalidArgument):
        gpu.sh_fwd(np.zeros((4, 3), np.float32), np.zeros((4, 4, 3), np.float32), 2)
    with pytest.raises(sh.SxInvalidArgument):
        gpu.mcmc_relocation(np.full(3, 0.5, np.float32), np.ones((3, 3), np.float32), np.array([1, 0, 2], np.int32),
                            gpu.make_binoms_lut(51))
    x = np.zeros((1, 10, 20, 3), np.float32)
    with pytest.raises(sh.SxInvalidArgument):
        gpu.ssim_fwd(x, x)
