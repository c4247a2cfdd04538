"""Formats either side of the step on the device, against the reference's own PlyIO.cpp and
Checkpoint.cpp (oracle/_ref, prebuilt; skipped where it was not built) and the CPU oracle:

- export: filter_cloud_for_export + write_inria_ply of the executor's live rows give a file byte for
  byte identical to the reference's (degrees 0-3, f_rest padding on and off, non-finite and
  low-opacity rows, count below the arena, count 0), with the same filter statistics;
- checkpoints: the device-packed file is byte for byte the reference's save_checkpoint_file output
  (fp32, and fp16 with its clamp and sqrt compression); reference files load into the arena as the
  reference's load_checkpoint_file reads them (fp16 paired zeroing included), the tail rows are
  zero, and a fingerprint mismatch, a file that does not fit the arena or a corrupt file changes
  nothing on the device;
- render sessions: every frame equals the oracle's forward render of the PLY's cloud quantized as
  sx_render_session_frame quantizes (NaN and v <= 0 -> 0, v > 1 -> 1, round-half-even of 255 v).
"""
import numpy as np
import pytest

import oracle_py
import scene
import splatx_hip as sh
from inputs import make_cloud

pytestmark = pytest.mark.gpu

F = np.float32
THRESH_LOGIT = np.log(0.005 / 0.995)


def same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def cloud(n, cap, deg, seed, specials=True):
    p, m, v = make_cloud(n, cap, deg, seed)
    # keep logits off the filter's threshold by more than float noise (libm vs correctly rounded exp)
    lg = p[3][:n, 0]
    near = np.abs(lg - THRESH_LOGIT) < 1e-3
    lg[near] += 0.01
    if specials and n > 40:
        p[0][3, 2] = np.nan
        p[2][11, 0] = np.inf
        if deg:
            p[5][17, -1] = -np.inf
        p[3][23, 0] = np.nan
    return p, m, v


@pytest.fixture(scope="module")
def ref():
    if not oracle_py.Reference.available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return oracle_py.Reference()


@pytest.mark.parametrize("deg,pad,n,cap", [(0, True, 3000, 3000), (1, True, 2500, 4000), (1, False, 2500, 2500),
                                           (2, True, 1000, 1200), (3, True, 5000, 6000), (3, True, 0, 10)])
def test_export_ply_matches_reference(gpu, ref, tmp_path, deg, pad, n, cap):
    p, m, v = cloud(n, cap, deg, 50 + deg)
    ex = gpu.make_train_step_executor(arena_rows=cap, sh_degree=deg)
    ex.upload_params(p, m, v, cap)
    mine, theirs = str(tmp_path / "mine.ply"), str(tmp_path / "ref.ply")
    st = ex.export_ply(n, mine, pad_sh_full=pad)
    st_ref = ref.export_ply([x[:n] for x in p], n, deg, theirs, pad_sh_full=pad)
    assert st == st_ref
    assert open(mine, "rb").read() == open(theirs, "rb").read()
    if n:
        assert st["removed_nonfinite"] == (4 if deg else 3) and st["removed_low_opacity"] > 0
    ex.close()


@pytest.mark.parametrize("fp16", [False, True])
def test_save_checkpoint_matches_reference(gpu, ref, tmp_path, fp16):
    n, cap, deg = 4000, 5000, 3
    p, m, v = cloud(n, cap, deg, 60, specials=False)
    # values the fp16 path clamps, underflows and rounds at ties
    p[0][:n][7] = [70000.0, -1e9, 65519.0]
    v[2][:n][9] = [1e-18, 0.0, 4e-16]
    ex = gpu.make_train_step_executor(arena_rows=cap, sh_degree=deg)
    ex.upload_params(p, m, v, cap)
    cfg = sh.CkptConfig.make(sh_degree=deg, total_iters=30000, mcmc_enabled=1, cap_max=cap, mcmc_seed=42,
                             scene_scale=1.25, ssim_weight=0.2)
    rng = " ".join(str(x) for x in range(313))
    mine, theirs = str(tmp_path / "mine.sxck"), str(tmp_path / "ref.sxck")
    ex.save_checkpoint(cfg, 777, n, mine, rng_state=rng, fp16=fp16)
    ref.save_checkpoint(cfg, 777, [x[:n] for x in p], [x[:n] for x in m], [x[:n] for x in v], n, deg, theirs,
                        rng_state=rng, fp16=fp16)
    assert open(mine, "rb").read() == open(theirs, "rb").read()
    ex.close()


def download(ex, cap, deg):
    dims = scene.group_dims(deg)
    out = [[np.zeros((cap, d), F) for d in dims] for _ in range(3)]
    ex.download_params(*out, cap)
    return out


@pytest.mark.parametrize("fp16", [False, True])
def test_load_checkpoint_matches_reference(gpu, ref, tmp_path, fp16):
    n, cap, deg = 3000, 3500, 2
    p, m, v = cloud(n, n, deg, 70, specials=False)
    v[1][5] = 1e-20  # underflows in fp16: its exp_avg is zeroed on load
    cfg = sh.CkptConfig.make(sh_degree=deg, total_iters=500, mcmc_enabled=1, cap_max=cap, mcmc_seed=3)
    path = str(tmp_path / "ref.sxck")
    rng = "9 8 7"
    ref.save_checkpoint(cfg, 42, p, m, v, n, deg, path, rng_state=rng, fp16=fp16)
    want = ref.load_checkpoint(path, n)
    ex = gpu.make_train_step_executor(arena_rows=cap, sh_degree=deg)
    junk = [[np.full((cap, d), 3.0, F) for d in scene.group_dims(deg)] for _ in range(3)]
    ex.upload_params(*junk, cap)
    got = ex.load_checkpoint(path, current=cfg)
    assert got["iter"] == 42 and got["alive_count"] == n and got["fp16"] == int(fp16) and got["rng_state"] == rng
    dp, dm, dv = download(ex, cap, deg)
    for g in range(6):
        if not dp[g].size:
            continue
        assert same(dp[g][:n], want["params"][g]), g
        assert same(dm[g][:n], want["exp_avg"][g]), g
        assert same(dv[g][:n], want["exp_avg_sq"][g]), g
        assert not dp[g][n:].any() and not dm[g][n:].any() and not dv[g][n:].any()
    if fp16:
        assert not want["exp_avg"][1][5].any()
    # a device save of what was loaded is the same file again (fp32: exact round trip)
    if not fp16:
        again = str(tmp_path / "again.sxck")
        ex.save_checkpoint(cfg, 42, n, again, rng_state=rng)
        assert open(again, "rb").read() == open(path, "rb").read()
    ex.close()


def test_load_checkpoint_rejections_leave_arena(gpu, ref, tmp_path):
    n, deg = 800, 1
    p, m, v = cloud(n, n, deg, 80, specials=False)
    cfg = sh.CkptConfig.make(sh_degree=deg, total_iters=500)
    path = str(tmp_path / "c.sxck")
    ref.save_checkpoint(cfg, 1, p, m, v, n, deg, path)
    small = gpu.make_train_step_executor(arena_rows=n - 1, sh_degree=deg)
    with pytest.raises(sh.SxInvalidArgument):
        small.load_checkpoint(path)
    small.close()
    ex = gpu.make_train_step_executor(arena_rows=n, sh_degree=deg)
    fill = [[np.full((n, d), 5.0, F) for d in scene.group_dims(deg)] for _ in range(3)]
    ex.upload_params(*fill, n)
    with pytest.raises(sh.SxRuntimeError):  # fingerprint mismatch
        ex.load_checkpoint(path, current=sh.CkptConfig.make(sh_degree=deg, total_iters=501))
    data = open(path, "rb").read()
    for name, bad in (("trailing", data + b"\0"), ("truncated", data[:-3])):
        bp = str(tmp_path / f"{name}.sxck")
        open(bp, "wb").write(bad)
        with pytest.raises(sh.SxRuntimeError):
            ex.load_checkpoint(bp)
    other = gpu.make_train_step_executor(arena_rows=n, sh_degree=3)
    with pytest.raises(sh.SxInvalidArgument):
        other.load_checkpoint(path)
    other.close()
    dp, dm, dv = download(ex, n, deg)
    for arrs in (dp, dm, dv):
        for a in arrs:
            assert np.all(a == 5.0)
    ex.close()


def quantize(rgb):
    v = np.where(rgb > 0, rgb, F(0)).astype(F)
    v = np.minimum(v, F(1))
    q = np.rint(v * F(255)).astype(np.uint8)
    return np.concatenate([q, np.full(q.shape[:2] + (1,), 255, np.uint8)], axis=2)


@pytest.mark.parametrize("deg,session_deg,aa", [(0, 0, False), (3, 0, False), (3, 1, True), (2, 2, False)])
def test_render_session_frames(gpu, oracle, tmp_path, deg, session_deg, aa):
    sc = scene.make_scene(n=5000, sh_degree=deg, width=150, height=110, fx=120.0, seed=90 + deg)
    path = str(tmp_path / "c.ply")
    ex = gpu.make_train_step_executor(arena_rows=sc.n, sh_degree=deg)
    p, m, v = scene.copy_state(sc)
    ex.upload_params(p, m, v, sc.n)
    ex.export_ply(sc.n, path, min_opacity=0.0, pad_sh_full=False)  # keeps every finite row
    ex.close()
    cl = sh.ply_read(path)
    eff = session_deg or cl["sh_degree"]
    sess = gpu.render_session(path, antialiased=aa, sh_degree=session_deg)
    rng = np.random.Generator(np.random.PCG64(5))
    kt = (eff + 1) ** 2
    params = [x.copy() for x in cl["params"]]
    params[5] = params[5][:, : (kt - 1) * 3].copy()
    for k in range(3):
        vm = scene.jittered_view(rng)
        W, H = (150, 110) if k < 2 else (97, 64)  # the frame size may change between frames
        fx, fy, cx, cy = 120.0, 118.0, W / 2.0, H / 2.0 + 1.5
        got = sess.frame(vm, fx, fy, cx, cy, W, H)
        K = np.array([[fx, 0, cx], [0, fy, cy], [0, 0, 1]], F)
        pp, mm, vv = [x.copy() for x in params], [np.zeros_like(x) for x in params], [np.zeros_like(x) for x in params]
        r = oracle.train_step(pp, mm, vv, cl["count"], eff, vm, K, W, H, None, eff, [0.0] * 6, forward_only=True,
                              antialiased=aa)
        assert np.array_equal(got, quantize(r["render_colors"])), k
    for bad in (dict(fx=0.0), dict(cx=np.nan), dict(width=0)):
        kw = dict(viewmat=np.eye(4, dtype=F), fx=100.0, fy=100.0, cx=10.0, cy=10.0, width=20, height=20)
        kw.update(bad)
        with pytest.raises(sh.SxInvalidArgument):
            sess.frame(**kw)
    sess.close()
    if deg < 3:
        with pytest.raises(sh.SxInvalidArgument):
            gpu.render_session(path, sh_degree=deg + 1)
