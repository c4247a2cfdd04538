"""Benchmark of the resident 3DGS training step on one MI355X (BASELINE.json metric).

Workload (the headline): N = 1,000,000 Gaussians, SH degree 3, 1297x840
pinhole (fx = fy = 1150, principal point centred), means x,y ~ U[-4,4], z ~ U[1.5,20],
log-scales ~ N(ln 0.01, 0.7), AccuTile intersection, loss 0.8 L1 + 0.2 (1 - SSIM), fused Adam.
Every step uses its own seeded camera pose (rotation <= 5 deg, translation <= 0.2); its target is
the render of a second seeded scene from that pose, held in the device-resident GT cache.
A step = graph of kernels from preprocess to Adam with its two host syncs (n_isects, loss).

Prints one JSON line. `roofline` is for the kernel with the largest share of GPU time in the timed
region (HIP events on the executor's stream); `cpu_baseline` times the CPU oracle (this repo's
single-threaded restatement of the reference CPU path plus its own backward) on two full steps.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "splatx-metal_amd", "python"))

import scene  # noqa: E402
import splatx_hip as sh  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def algorithmic_bytes(name: str, n: int, v: int, i: int, px: int, sh_k: int, shape: dict) -> float:
    """Minimum HBM bytes one launch of `name` must move (the per-unit figures of each case below). shape:
    index_first (the step's intersection order: emit in index order, then per-tile depth sorts; else
    depth first), depth_passes / tile_passes (radix passes of the depth sort over the Gaussians with tiles
    and of the tile sort over the i intersections) and key_b (bytes of a tile id: 2 up to 2^16 tiles,
    else 4). The Gaussians with tiles, which the emit steps run over, are counted as the v visible ones
    (a visible Gaussian without a tile is rare)."""
    pd = 3 + 4 + 3 + 1 + 3 + (sh_k - 1) * 3  # parameter floats per Gaussian (59 at SH3)
    kb = shape["key_b"]
    if shape.get("index_first"):
        if name == "emit":
            # the compaction in the same launch: every Gaussian's tile count (4 B) in, the list of those with
            # tiles (4 B) and their inclusive offsets (8 B) out; their 32-B conic/mean record; per entry the
            # tile id, the Gaussian (4 B) and its depth bits (4 B) out
            return 4.0 * n + v * (12.0 + 32.0) + i * (kb + 8.0)
        if name == "tile_depth_sort":
            # per entry: the emit position in and out (8 B), its depth bits (4 B, carried by the tile sort)
            return 12.0 * i
        if name == "sort":
            # as below, plus each entry's depth bits (4 B) read and written with it by every pass
            return i * (kb + 2.0 * (kb + 4.0 + 4.0) * shape["tile_passes"] - 4.0)
    if name == "preprocess":
        # params of every Gaussian (44 B) + SH coefficients of visible ones; writes radii+count (12 B),
        # and for visible ones the 48-B splat record
        return 44.0 * n + 4.0 * 3 * sh_k * v + 12.0 * n + 48.0 * v
    if name == "postprocess":
        # every row's meta word and touched flag; visible: read params, both moments, grads (36 B) and
        # conic/comp/meta (20 B); write params+moments
        return 5.0 * n + v * (4.0 * pd * 3 + 36 + 20 + 4.0 * pd * 3)
    if name == "update_preprocess":
        # the previous step's postprocess and this step's preprocess in one pass: the postprocess's bytes
        # and the preprocess's writes (radii + count 12 B per row, the 48-B record per visible one); the
        # preprocess reads nothing again
        return algorithmic_bytes("postprocess", n, v, i, px, sh_k, shape) + 12.0 * n + 48.0 * v
    if name == "raster_fwd":
        # the measurement plan's per-unit figures: 40 B read per intersection (its sorted id and the splat's record),
        # 20 B written per pixel (colour, alpha, last id)
        return i * 40.0 + px * 20.0
    if name == "raster_bwd":
        # the measurement plan's per-unit figures: 40 B read and 36 B of gradient sums scattered per intersection,
        # 20 B read per pixel (alpha, last id, v_render)
        return i * (40.0 + 36.0) + px * 20.0
    if name == "gather":
        # order, offset and touched flag per Gaussian with tiles (13 B), the 36-B sums and stamp of the
        # entries, the 48-B gradient record of the visible Gaussians
        return v * 13.0 + i * 40.0 + v * 48.0
    if name == "depth_sort":
        # compaction: every tile count (4 B) in, the list of Gaussians with tiles (4 B) out; keys: their
        # depths (4 B) in, (key, index) out (8 B); the onesweep sort of those (u32, i32) pairs: one histogram
        # read (4 B), per pass a read and a write (16 B)
        return 4.0 * n + v * (4.0 + 4.0 + 8.0) + v * (4.0 + 16.0 * shape["depth_passes"])
    if name == "scan":
        # tile counts gathered through the depth order: order (4 B) + count (4 B) in, offset (8 B) out
        return v * 16.0
    if name == "emit":
        # order (4 B) and offset (8 B) per position, the 32-B conic/mean record, and the (tile id, emit
        # position's Gaussian) entries out
        return v * (12.0 + 32.0) + i * (kb + 4.0)
    if name == "sort":
        # tile sort: one histogram read of the ids, per pass a read and a write of (id, emit position); the
        # first pass takes the positions from the key index instead of reading them
        return i * (kb + 2.0 * (kb + 4.0) * shape["tile_passes"] - 4.0)
    if name == "offsets":
        return 4.0 * (px / 256.0)
    if name == "ssim_fwd":
        return px * 3 * (4 + 4) + (px * 3) * 16.0
    if name == "ssim_bwd_l1":
        return px * 3 * (4 + 4) + (px * 3) * 12.0 + px * 3 * 4.0
    return 0.0


# The oracle's backward stages are this build's own code: the reference's CPU path has no backward
# (its raster, SH, projection and SSIM VJPs exist only as GPU kernels), so these are reported apart from
# the stages the reference's CPU kernels also run.
OWN_BACKWARD_STAGES = ("raster_bwd", "sh_bwd", "projection_bwd", "ssim_bwd")


def cpu_model() -> str:
    """The host CPU's model name (first `model name` of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(sc, pose, gt, lr) -> dict:
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle_py

    orc = oracle_py.Oracle(libm=False)
    p, m, v = scene.copy_state(sc)
    n_steps = 2
    stages = {}
    t0 = time.perf_counter()
    for _ in range(n_steps):
        r = orc.train_step(p, m, v, sc.n, sc.sh_degree, pose, sc.K, sc.width, sc.height, gt, sc.sh_degree, lr,
                           ssim_weight=0.2, want_render=False)
        for k, x in r["stage_ms"].items():
            stages[k] = stages.get(k, 0.0) + x / n_steps
    dt = (time.perf_counter() - t0) * 1000.0 / n_steps
    return {"value": round(dt, 1), "unit": "ms/iter", "cores": 1, "kind": "port",
            "sample": f"{n_steps} consecutive full fwd+bwd+Adam steps of the same config-3 workload (N=1M, SH3, "
                      "1297x840, AccuTile, SSIM; first timed pose and its target) by the single-threaded CPU oracle",
            "n_isects": r["n_isects"], "cpu_model": cpu_model(),
            "stages_ms": {k: round(x, 1) for k, x in stages.items() if x > 0 and k not in OWN_BACKWARD_STAGES},
            "own_backward_stages_ms": {k: round(stages[k], 1) for k in OWN_BACKWARD_STAGES if stages.get(k, 0) > 0},
            "own_backward_note": "the reference has no CPU backward; these stages are this build's own CPU code"}


def calibrate_copy(mib: int, reps: int = 4) -> None:
    """Device-to-device copies of a known size (the runtime's copy kernel), as the yardstick that scales
    the FETCH_SIZE / WRITE_SIZE counters of a `rocprofv3 --pmc` run into HBM bytes."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    n = mib << 20
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    for p in (a, b):
        if hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(n)) != 0:
            raise RuntimeError("hipMalloc failed")
    if hip.hipMemset(a, 1, ctypes.c_size_t(n)) != 0:
        raise RuntimeError("hipMemset failed")
    for _ in range(reps):
        if hip.hipMemcpy(b, a, ctypes.c_size_t(n), 3) != 0:  # hipMemcpyDeviceToDevice
            raise RuntimeError("hipMemcpy failed")
    hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)
    print(json.dumps({"calibrate_copy_bytes": n, "reps": reps}), flush=True)


def bench_formats(cfg_id: int) -> None:
    """Wall-clock ms of the data formats on the config's scene (files under $TMPDIR): the device export filter +
    INRIA PLY write, SXCK checkpoint save and load (fp32 and fp16, with fsync), and render-session frames."""
    import tempfile

    sc, cfg = scene.config_scene(cfg_id, seed=0)
    b = sh.Backend(0)
    ex = b.make_train_step_executor(arena_rows=sc.n, sh_degree=sc.sh_degree)
    p, m, v = scene.copy_state(sc)
    ex.upload_params(p, m, v, sc.n)
    d = tempfile.mkdtemp(prefix="splatx_formats_")
    out = {"workload": f"config {cfg_id}: N={sc.n}, SH{sc.sh_degree}", "ms": {}, "bytes": {}}

    def timed(name, fn, reps=3):
        best = None
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            dt = (time.perf_counter() - t0) * 1000.0
            best = dt if best is None else min(best, dt)
        out["ms"][name] = round(best, 2)

    ply = os.path.join(d, "c.ply")
    timed("export_ply", lambda: ex.export_ply(sc.n, ply))
    out["bytes"]["ply"] = os.path.getsize(ply)
    ck = sh.CkptConfig.make(sh_degree=sc.sh_degree, total_iters=30000)
    for fp16 in (False, True):
        path = os.path.join(d, f"c{16 if fp16 else 32}.sxck")
        timed(f"save_checkpoint_fp{16 if fp16 else 32}", lambda: ex.save_checkpoint(ck, 100, sc.n, path, fp16=fp16))
        timed(f"load_checkpoint_fp{16 if fp16 else 32}", lambda: ex.load_checkpoint(path, current=ck))
        out["bytes"][f"checkpoint_fp{16 if fp16 else 32}"] = os.path.getsize(path)
    ex.close()
    sess = b.render_session(ply)
    rng = np.random.Generator(np.random.PCG64(7))
    views = [scene.jittered_view(rng) for _ in range(20)]
    K = sc.K
    sess.frame(views[0], K[0, 0], K[1, 1], K[0, 2], K[1, 2], sc.width, sc.height)
    t0 = time.perf_counter()
    for vm in views:
        sess.frame(vm, K[0, 0], K[1, 1], K[0, 2], K[1, 2], sc.width, sc.height)
    out["ms"]["render_session_frame"] = round((time.perf_counter() - t0) * 1000.0 / len(views), 3)
    sess.close()
    b.close()
    for f in os.listdir(d):
        os.remove(os.path.join(d, f))
    os.rmdir(d)
    print(json.dumps(out), flush=True)


def load_traffic(kernel: str, cfg: int):
    """HBM bytes per launch of `kernel`, as measured by the counter runs recorded in profiles/traffic.json
    (FETCH_SIZE and WRITE_SIZE per training step, each scaled by the copy-kernel yardstick, divided by the
    kernel's dispatches per step); None if not recorded for this configuration."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    # the counter tables label kernels by what they run; bench.py's event intervals by step stage
    label = {"update_preprocess": "update + preprocess"}.get(kernel, kernel)
    k = rec.get("configs", {}).get(str(cfg), {}).get("kernels", {}).get(label)
    if k is None:
        return None
    return round(k["hbm_bytes"] / max(1, k["dispatches"]))


# Cycles a SIMD spends per wave-level VALU instruction (measured by --calibrate-valu on MI355X): 4 for
# f32 arithmetic, bitwise and DPP moves, 8 for transcendentals (v_exp_f32, v_rcp_f32, ...). v_add_u32
# and plain v_mov_b32 issue at about twice the f32 rate, so the bound below is an upper estimate when
# a kernel has many of them.
VALU_CYCLES, TRANS_CYCLES, SIMDS, CLOCK_HZ = 4, 8, 1024, 2.4e9


def load_valu(kernel: str, cfg: int):
    """VALU issue bound of one training step's launches of `kernel` from the counter runs recorded in
    profiles/counters.json (SQ_INSTS_VALU and SQ_INSTS_VALU_TRANS_F32 over training-step dispatches);
    None if not recorded for this configuration."""
    path = os.path.join(REPO, "profiles", "counters.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    k = rec.get("configs", {}).get(str(cfg), {}).get("kernels", {}).get(kernel)
    if k is None or "SQ_INSTS_VALU" not in k:
        return None
    v, t = k["SQ_INSTS_VALU"], k.get("SQ_INSTS_VALU_TRANS_F32", 0)
    cycles = VALU_CYCLES * (v - t) + TRANS_CYCLES * t
    return {"valu_insts": v, "trans_insts": t, "bound_ms": round(cycles / (SIMDS * CLOCK_HZ) * 1e3, 4),
            "simds": SIMDS, "clock_hz": CLOCK_HZ, "cycles_per_wave_instr": VALU_CYCLES,
            "cycles_per_trans_instr": TRANS_CYCLES}


def calibrate_valu(blocks: int = 8192, reps: int = 5) -> None:
    """VALU issue rates per instruction class on device 0 (the yardstick kernels of
    splatx-metal_amd/yardstick/k_yardstick.hip, a library of their own): wave-level instructions per SIMD
    per 4 cycles at CLOCK_HZ, and the cycles per instruction."""
    import ctypes
    path = os.path.join(REPO, "splatx-metal_amd", "build", "libsplatx_yardstick.so")
    if not os.path.exists(path):
        raise RuntimeError(f"yardstick library not built: {path} (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    lib.sxy_valu_name.restype = ctypes.c_char_p
    lib.sxy_valu.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                             ctypes.POINTER(ctypes.c_double)]
    out = {"blocks": blocks, "waves": blocks * 4, "clock_hz": CLOCK_HZ, "simds": SIMDS, "ops": {}}
    for op in range(lib.sxy_valu_count()):
        name = lib.sxy_valu_name(op).decode()
        slow = "exp" in name or "rcp" in name
        iters = 1024 if slow else 4096
        ms = ctypes.c_double()
        if lib.sxy_valu(0, op, blocks, iters, reps, ctypes.byref(ms)) != 0:
            raise RuntimeError(f"yardstick {name} failed")
        insts = blocks * 4 * iters * 8
        rate = insts / SIMDS / (ms.value * 1e-3 * CLOCK_HZ / 4.0)
        out["ops"][name] = {"iters": iters, "wave_instrs": insts, "ms": round(ms.value, 4),
                            "per_simd_per_4_cycles": round(rate, 3), "cycles_per_instr": round(4.0 / rate, 2)}
        print(f"{name:40s} {ms.value:8.4f} ms  {rate:6.3f} per SIMD per 4 cycles", file=sys.stderr, flush=True)
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--formats", action="store_true",
                    help="time the formats either side of the step (PLY export, checkpoint save/load, render-session "
                         "frames) on the config's arena instead of the training step, and exit")
    ap.add_argument("--calibrate-valu", action="store_true",
                    help="only time the VALU yardstick kernels (issue rate per instruction class) and exit")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run device copies of MIB MiB (yardstick for the HBM byte counters) and exit")
    ap.add_argument("--row-order", choices=("auto", "original", "spatial"), default="auto",
                    help="how the executor keeps the rows in HBM (sxh_exec_set_row_order; the same results)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the step has no multi-GPU "
              f"path — run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy > 0:
        calibrate_copy(args.calibrate_copy)
        return
    if args.calibrate_valu:
        calibrate_valu()
        return

    if args.formats:
        bench_formats(args.config)
        return

    sc, cfg = scene.config_scene(args.config, seed=0)
    tgt, _ = scene.config_scene(args.config, seed=1)
    mcmc = "cap_max" in cfg  # config 4: MCMC arena, a device refine after every step
    arena = cfg.get("cap_max", sc.n)
    n_poses = args.steps + args.warmup
    rng = np.random.Generator(np.random.PCG64(1234))
    poses = [scene.jittered_view(rng) for _ in range(n_poses)]
    lr = list(sc.lr)
    isect = sh.SXH_ISECT_ACCUTILE if cfg["isect"] == "accutile" else sh.SXH_ISECT_AABB
    aa = bool(cfg.get("antialiased", False))

    b = sh.Backend(0)
    ex = b.make_train_step_executor(arena_rows=arena, sh_degree=sc.sh_degree, ssim_weight=cfg["ssim"],
                                    antialiased=aa, isect_mode=isect)
    ex.set_row_order({"auto": sh.SXH_ROW_ORDER_SPATIAL_AUTO, "original": sh.SXH_ROW_ORDER_ORIGINAL,
                      "spatial": sh.SXH_ROW_ORDER_SPATIAL}[args.row_order])
    # targets: the second scene rendered from every pose into the device GT cache
    ex.set_gt_cache(np.zeros((n_poses, sc.height, sc.width, 3), np.float32))
    tp, tm, tv = scene.copy_state(tgt)
    ex.upload_params(tp, tm, tv, sc.n)
    base = scene.step_kwargs(sc)
    gt_first = None
    for k in range(n_poses):
        ex.render_to_gt_cache(k, **dict(base, viewmat=poses[k]))
        if k == args.warmup:  # host copy of the first timed target, for the CPU baseline
            gt_first = ex.step(want_render=True, forward_only=True, **dict(base, viewmat=poses[k]))["render_colors"]
    p, m, v = scene.copy_state(sc)
    if mcmc:  # the arena beyond the live rows starts at zero (Trainer.cpp:686-709)
        p, m, v = ([np.concatenate([x.reshape(sc.n, -1), np.zeros((arena - sc.n, x.reshape(sc.n, -1).shape[1]),
                                                                  np.float32)]) for x in grp] for grp in (p, m, v))
    ex.upload_params(p, m, v, arena)

    # pre-built step arguments (no host work inside the timed loop beyond the step itself)
    count = sc.n

    def step_inputs(k, count):
        extra = {}
        if mcmc:  # Trainer.cpp:920-935: regularization weights over the live count; no noise on refine steps
            extra = dict(count=count, opacity_reg_w=cfg["opacity_reg"] / count,
                         scale_reg_w=cfg["scale_reg"] / (3 * count))
        return ex.make_step_inputs(**dict(base, viewmat=poses[k], **extra), gt_index=k)

    steps = [step_inputs(k, count) for k in range(n_poses)]
    steps0 = list(steps)  # the timed region's inputs as first built (MCMC rebuilds them as the count grows)
    n_tiles = ((sc.width + 15) // 16) * ((sc.height + 15) // 16)
    tile_bits = int(n_tiles - 1).bit_length()  # the tile id's bits (bits_for_count)
    out = sh.StepOutputs()
    for k in range(args.warmup):
        rc = ex.step_raw(steps[k][0], out)
        assert rc == 0, b.lib.sxh_last_error()

    refine_ms, counts = [], []
    if mcmc:
        binoms = b.make_binoms_lut(51)
        rng_state = b.mt64_seed(42)
        noise_lr = 5e5  # McmcOptions::noise_lr (Trainer.h:195); noise_scale = lr_means * noise_lr

    # timed loop: the product path (segment B of each step replayed as a captured hipGraph)
    totals = {}
    n_isects, n_vis, losses, passes, step_ms = [], [], [], [], []
    ex.sync()  # the warm-up's last parameter update is done before the clock starts
    t0 = time.perf_counter()
    for k in range(args.warmup, n_poses):
        if mcmc and count != sc.n:
            steps[k] = step_inputs(k, count)
        ts = time.perf_counter()
        rc = ex.step_raw(steps[k][0], out)
        step_ms.append((time.perf_counter() - ts) * 1000.0)  # the step returns after its loss readback
        if rc != 0:
            raise RuntimeError(b.lib.sxh_last_error())
        n_isects.append(out.n_isects)
        n_vis.append(out.n_visible)
        passes.append(((out.sort_key_bits - tile_bits) + 7) // 8)  # depth sort passes
        losses.append(out.loss)
        if mcmc:  # the refine step of Trainer::step_resident (Trainer.cpp:957-967): refine, then noise
            tr = time.perf_counter()
            r = ex.mcmc_refine(count, arena, rng_state, binoms, min_opacity=cfg["min_opacity"], inject_noise=True,
                               noise_seed=42, noise_offset=k, noise_scale=lr[0] * noise_lr)
            refine_ms.append((time.perf_counter() - tr) * 1000.0)
            count = r["count"]
            counts.append(count)
    ex.sync()  # a step returns at its loss: the last parameter update is inside the timed region
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1000.0 / args.steps
    # per-kernel times: the timed region's work again — the same start state, warm-up and poses — with
    # HIP events between the kernels (profiling launches the kernels directly; their durations are
    # those of the graph replays, which rocprof confirms). With MCMC the steps follow the timed loop's
    # final state instead (its refines are not replayed).
    if not mcmc:
        ex.upload_params(p, m, v, arena)
        for k in range(args.warmup):
            if ex.step_raw(steps0[k][0], out) != 0:
                raise RuntimeError(b.lib.sxh_last_error())
    ex.set_profiling(True)
    for k in range(args.warmup, n_poses):
        rc = ex.step_raw((steps if mcmc else steps0)[k][0], out)
        if rc != 0:
            raise RuntimeError(b.lib.sxh_last_error())
        for name, ms in ex.get_timing().items():
            totals[name] = totals.get(name, 0.0) + ms
    ex.set_profiling(False)
    avg = {k: x / args.steps for k, x in totals.items()}
    # raster pair counts: the timed region's work once more with the counting raster kernels
    pair_tot = {}
    if not mcmc:
        ex.upload_params(p, m, v, arena)
        for k in range(args.warmup):
            if ex.step_raw(steps0[k][0], out) != 0:
                raise RuntimeError(b.lib.sxh_last_error())
        ex.set_profiling(False, pair_stats=True)
        for k in range(args.warmup, n_poses):
            if ex.step_raw(steps0[k][0], out) != 0:
                raise RuntimeError(b.lib.sxh_last_error())
            for name, x in ex.get_raster_stats().items():
                pair_tot[name] = pair_tot.get(name, 0) + x
        ex.set_profiling(False)

    I, V = float(np.mean(n_isects)), float(np.mean(n_vis))
    px = sc.width * sc.height
    sh_k = (sc.sh_degree + 1) ** 2
    # the step's intersection order, as the profiled steps ran it (index first: a per-tile depth sort, no
    # depth sort of the Gaussians)
    index_first = "tile_depth_sort" in avg
    shape = {"index_first": index_first, "depth_passes": 0.0 if index_first else float(np.mean(passes)),
             "tile_passes": (tile_bits + 7) // 8, "key_b": 2 if tile_bits <= 16 else 4}
    kernel_names = [k for k in avg if not k.startswith("host_")]
    per_kernel = {}
    for k in kernel_names:
        by = algorithmic_bytes(k, sc.n, V, I, px, sh_k, shape)
        per_kernel[k] = {"ms": round(avg[k], 4), "alg_GB": round(by / 1e9, 4),
                         "GBps": round(by / 1e9 / (avg[k] / 1e3), 1) if by > 0 and avg[k] > 0 else None}
    dom = max(kernel_names, key=lambda k: avg[k])
    dom_bytes = algorithmic_bytes(dom, sc.n, V, I, px, sh_k, shape)
    achieved = dom_bytes / 1e9 / (avg[dom] / 1e3)
    step_bytes = sum(algorithmic_bytes(k, sc.n, V, I, px, sh_k, shape) for k in kernel_names)
    ref_step_bytes = 84.0 * sc.n + 1708.0 * V + 288.0 * I + 160.0 * px

    res = {
        "metric": "train-step ms/iter (fwd+bwd+Adam) at N=1M, 1297x840; % HBM roofline",
        "value": round(ms_per_step, 4),
        "unit": "ms/iter",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generator of BASELINE.json configs; target = second seeded scene rendered per pose)",
        "config": {"workload": f"config {args.config}: N={sc.n}, SH{sc.sh_degree}, {sc.width}x{sc.height}, "
                               f"fx=fy={cfg['fx']}, {cfg['isect']} isect, ssim_weight={cfg['ssim']}, "
                               f"pose jittered per step", "gaussians": sc.n, "width": sc.width,
                   "height": sc.height, "sh_degree": sc.sh_degree, "parallelism": "single GPU",
                   "row_order": args.row_order},
        "ms_p50": round(float(np.percentile(step_ms, 50)), 4),
        "ms_p90": round(float(np.percentile(step_ms, 90)), 4),
        "gaussians_per_s": round(sc.n / (ms_per_step / 1e3), 1),
        "mean_n_isects": round(I, 1),
        "mean_visible": round(V, 1),
        "isect_order": "index_first" if index_first else "depth_first",
        "sort_passes": {"depth": round(shape["depth_passes"], 2), "tile": shape["tile_passes"]},
        "final_loss": round(float(losses[-1]), 6),
        "step_alg_GB": round(step_bytes / 1e9, 4),
        "step_hbm_roofline_frac": round(step_bytes / 1e9 / (ms_per_step / 1e3) / HBM_PEAK_GBS, 5),
        # the reference design's step bytes, 84 N + 1708 V + 288 I + 160 P (an unfused 8-bit sort over 45-bit
        # keys, a perturb pass), over the measured step time
        "step_alg_GB_reference_design": round(ref_step_bytes / 1e9, 4),
        "step_hbm_roofline_frac_reference_design": round(ref_step_bytes / 1e9 / (ms_per_step / 1e3)
                                                         / HBM_PEAK_GBS, 5),
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(dom, args.config), "alg_bytes": round(dom_bytes)},
        "kernels": per_kernel,
        "valu_issue": None,
        "host_waits_ms": {k: round(avg[k], 4) for k in avg if k.startswith("host_")},
    }
    if pair_tot:  # per-step means; a list entry is one splat against the 64 pixels of a wave
        pm = {k: x / args.steps for k, x in pair_tot.items()}
        rp = {"fwd_lane_pairs": round(pm["fwd_iters"] * 64), "fwd_block_entries": round(pm["fwd_entries"]),
              "fwd_composited": round(pm["fwd_taken"]), "bwd_lane_pairs": round(pm["bwd_chunks"] * 256),
              "bwd_block_entries": round(pm["bwd_entries"]), "bwd_in_cutoff": round(pm["bwd_in_cutoff"]),
              "bwd_contributing": round(pm["bwd_contrib"]), "bwd_chunks": round(pm["bwd_chunks"]),
              "bwd_empty_chunks": round(pm["bwd_empty_chunks"]), "upper_bound_256I": round(256 * I)}
        vb = load_valu("raster_bwd", args.config)
        if vb is not None and pm["bwd_chunks"] > 0:  # wave-level VALU instructions per 4-iteration chunk
            rp["bwd_valu_per_chunk"] = round(vb["valu_insts"] / pm["bwd_chunks"], 1)
        res["raster_pairs"] = rp
    vi = load_valu(dom, args.config)
    if vi is not None:  # the dominant kernel's own bound when it is compute-, not memory-bound
        vi["kernel"] = dom
        vi["frac"] = round(vi["bound_ms"] / avg[dom], 4)
        res["valu_issue"] = vi
    if mcmc:
        res["config"]["workload"] = (f"config 4: {sc.n} live of a {arena}-row arena, SH{sc.sh_degree}, "
                                     f"{sc.width}x{sc.height}, AccuTile, SSIM, opacity/scale reg 1e-2; every step "
                                     f"is a refine step (step, device MCMC refine, noise)")
        res["mcmc"] = {"refine_ms_mean": round(float(np.mean(refine_ms)), 3),
                       "refine_ms_median": round(float(np.median(refine_ms)), 3),
                       "count_first": int(counts[0]), "count_last": int(counts[-1])}
    ex.close()
    b.close()
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(sc, poses[args.warmup], gt_first, lr)
        res["cpu_baseline"]["cores_available"] = os.cpu_count()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
