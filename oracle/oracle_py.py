"""ctypes access to the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker
or the timed CPU baseline. `Oracle(libm=False)` uses the deterministic transcendental layer shared
with the device code; `Oracle(libm=True)` uses glibc exactly like the reference CPU code;
`Reference()` calls the reference's own CPU code (CpuKernels.cpp, and the Trainer on the CPU
backend for the MCMC refine) built under oracle/_ref (when present).
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(REPO, "splatx-metal_amd", "python"))

import splatx_hip as sh  # noqa: E402  (struct layouts of include/splatx_hip.h)


class StepArgs(C.Structure):
    _fields_ = [("params", sh.fp * 6), ("exp_avg", sh.fp * 6), ("exp_avg_sq", sh.fp * 6),
                ("count", C.c_int64), ("sh_degree", C.c_int32), ("viewmat", sh.fp), ("K", sh.fp),
                ("width", C.c_int32), ("height", C.c_int32), ("gt_rgb", sh.fp),
                ("degrees_to_use", C.c_uint32), ("lr", C.c_float * 6), ("opacity_reg_w", C.c_float),
                ("scale_reg_w", C.c_float), ("eps2d", C.c_float), ("near_plane", C.c_float),
                ("far_plane", C.c_float), ("radius_clip", C.c_float), ("b1", C.c_float),
                ("b2", C.c_float), ("eps", C.c_float), ("ssim_weight", C.c_float),
                ("antialiased", C.c_uint8), ("isect_mode", C.c_uint8), ("forward_only", C.c_uint8),
                ("inject_noise", C.c_uint8), ("noise_seed", C.c_uint64), ("noise_offset", C.c_uint64),
                ("noise_scale", C.c_float), ("loss", C.c_float), ("n_isects", C.c_int64),
                ("n_visible", C.c_int64), ("render_colors", sh.fp), ("stage_ms", C.c_double * 16)]


class RefineArgs(C.Structure):
    _fields_ = [("params", sh.fp * 6), ("exp_avg", sh.fp * 6), ("exp_avg_sq", sh.fp * 6), ("count", C.c_int64),
                ("cap_max", C.c_int64), ("sh_degree", C.c_int32), ("min_opacity", C.c_float), ("n_max", C.c_int32),
                ("binoms", sh.fp), ("rng", C.POINTER(sh.MtState)), ("new_count", C.c_int64),
                ("n_relocated", C.c_int64), ("n_added", C.c_int64), ("relocated_dead", sh.i64p),
                ("relocation_src", sh.i64p), ("added_src", sh.i64p), ("capacity", C.c_int64)]


class RefCase(C.Structure):
    _fields_ = [("params", sh.fp * 6), ("exp_avg", sh.fp * 6), ("exp_avg_sq", sh.fp * 6), ("count", C.c_int64),
                ("cap_max", C.c_int64), ("sh_degree", C.c_int32), ("min_opacity", C.c_float), ("seed", C.c_uint64),
                ("n_refine", C.c_int32), ("out_params", sh.fp * 6), ("out_exp_avg", sh.fp * 6),
                ("out_exp_avg_sq", sh.fp * 6), ("counts", sh.i64p), ("n_relocated", sh.i64p), ("n_added", sh.i64p),
                ("relocated_dead", sh.i64p), ("relocation_src", sh.i64p), ("added_src", sh.i64p),
                ("capacity", C.c_int64), ("rng_out", C.POINTER(sh.MtState))]


class HipTrainCase(C.Structure):
    _fields_ = [("params", sh.fp * 6), ("count", C.c_int64), ("sh_degree", C.c_int32), ("viewmat", sh.fp),
                ("K", sh.fp), ("width", C.c_int32), ("height", C.c_int32), ("gt_rgb", sh.fp), ("steps", C.c_int32),
                ("total_iters", C.c_int32), ("lr", C.c_float * 6), ("ssim_weight", C.c_float),
                ("opacity_reg", C.c_float), ("scale_reg", C.c_float), ("antialiased", C.c_uint8),
                ("resident", C.c_uint8), ("mcmc", C.c_uint8), ("cap_max", C.c_int64), ("seed", C.c_uint64),
                ("refine_start_ratio", C.c_float), ("refine_stop_ratio", C.c_float),
                ("refine_every_ratio", C.c_float), ("out_params", sh.fp * 6), ("losses", sh.fp),
                ("n_isects", sh.i64p), ("render0", sh.fp), ("out_count", C.c_int64), ("n_refined", C.c_int32),
                ("n_cams", C.c_int32), ("viewmats", sh.fp), ("Ks", sh.fp), ("gts", sh.fp), ("start_iter", C.c_int32),
                ("scene_scale", C.c_float), ("sh_degree_interval_ratio", C.c_float)]


class RefSchedule(C.Structure):
    _fields_ = [("total_iters", C.c_int32), ("scene_scale", C.c_float), ("lr_means", C.c_float),
                ("sh_degree_interval_ratio", C.c_float), ("mcmc_enabled", C.c_uint8), ("refine_start_ratio", C.c_float),
                ("refine_stop_ratio", C.c_float), ("refine_every_ratio", C.c_float)]


class RefCloudIn(C.Structure):
    _fields_ = [("params", sh.fp * 6), ("count", C.c_int64), ("sh_degree", C.c_int32)]


class RefCloudOut(C.Structure):
    _fields_ = [("params", sh.fp * 6), ("count", C.c_int64), ("sh_degree", C.c_int32)]


class HipRefineCase(C.Structure):
    _fields_ = [("params", sh.fp * 6), ("exp_avg", sh.fp * 6), ("exp_avg_sq", sh.fp * 6), ("count", C.c_int64),
                ("cap_max", C.c_int64), ("sh_degree", C.c_int32), ("n_refine", C.c_int32), ("seed", C.c_uint64),
                ("binoms", sh.fp), ("counts", sh.i64p), ("last_lists", sh.i64p), ("last_sizes", C.c_int64 * 3),
                ("rng_out", C.POINTER(sh.MtState))]


def _ptr_or_null(a):
    return sh.ptr(a) if a is not None and a.size else None


def lib_path(libm: bool) -> str:
    return os.path.join(HERE, "liboracle_libm.so" if libm else "liboracle.so")


class Oracle(sh.Ops):
    def __init__(self, libm: bool = False):
        p = lib_path(libm)
        if not os.path.exists(p):
            raise RuntimeError(f"oracle not built: {p}")
        lib = C.CDLL(p)
        super().__init__(lib, "sxo_")
        self.libm = libm

    def make_binoms_lut(self, n_max=51):
        out = np.zeros(n_max * n_max, np.float32)
        self._call("make_binoms_lut", n_max, sh.ptr(out))
        return out

    TRAIN_DEFAULT_FIELDS = ("total_iters", "scene_scale", "lr_means", "lr_quats", "lr_scales", "lr_opacities", "lr_sh0",
                            "lr_shN", "sh_degree_interval_ratio", "opacity_reg", "scale_reg", "cap_max",
                            "min_opacity", "refine_start_ratio", "refine_stop_ratio", "refine_every_ratio",
                            "noise_lr", "mcmc_seed")

    def train_defaults(self) -> dict:
        """TrainConfig / McmcOptions defaults of the reference's Trainer.h."""
        out = np.zeros(18, np.float64)
        self._call("train_defaults", out.ctypes.data_as(C.POINTER(C.c_double)))
        return dict(zip(self.TRAIN_DEFAULT_FIELDS, out.tolist()))

    def train_plans(self, total_iters, scene_scale, lr_means, sh_degree_interval_ratio, mcmc_enabled,
                    refine_start_ratio, refine_stop_ratio, refine_every_ratio, sh_degree, iters):
        """means_lr_at, sh_degree_at and Trainer::mcmc_refine_due of the reference for `iters`."""
        s = RefSchedule(total_iters, scene_scale, lr_means, sh_degree_interval_ratio, int(bool(mcmc_enabled)),
                        refine_start_ratio, refine_stop_ratio, refine_every_ratio)
        it = np.ascontiguousarray(iters, np.int32)
        lr0 = np.zeros(it.size, np.float32)
        deg = np.zeros(it.size, np.uint32)
        due = np.zeros(it.size, np.uint8)
        self._call("train_plans", C.byref(s), sh_degree, it.size, sh.ptr(it), sh.ptr(lr0), sh.ptr(deg), sh.ptr(due))
        return lr0, deg, due

    def quat_scale_to_covar(self, quats, scales):
        q, s = sh.f32(quats), sh.f32(scales)
        out = np.zeros((q.shape[0], 3, 3), np.float32)
        self._call("quat_scale_to_covar", sh.ptr(q), sh.ptr(s), q.shape[0], sh.ptr(out))
        return out

    def _arr(self, name, x, *extra):
        x = sh.f32(x)
        outs = [np.zeros_like(x) for _ in range(2 if name == "sincosf_array" else 1)]
        f = getattr(self.lib, "sxo_" + name)
        f.restype = None
        f(sh.ptr(x), *[sh.ptr(sh.f32(e)) for e in extra], *[sh.ptr(o) for o in outs], C.c_int64(x.size))
        return outs if len(outs) > 1 else outs[0]

    def logf(self, x):
        return self._arr("logf_array", x)

    def expf(self, x):
        return self._arr("expf_array", x)

    def expf_fast(self, x):
        return self._arr("expf_fast_array", x)

    def powf(self, x, p):
        return self._arr("powf_array", x, p)

    def sincosf(self, x):
        return self._arr("sincosf_array", x)

    def train_step(self, params, exp_avg, exp_avg_sq, count, sh_degree, viewmat, K, width, height,
                   gt_rgb, degrees_to_use, lr, opacity_reg_w=0.0, scale_reg_w=0.0, eps2d=0.3,
                   near_plane=0.01, far_plane=1e10, radius_clip=0.0, b1=0.9, b2=0.999, eps=1e-15,
                   ssim_weight=0.2, antialiased=False, isect_mode=sh.SXH_ISECT_ACCUTILE,
                   forward_only=False, inject_noise=False, noise_seed=0, noise_offset=0,
                   noise_scale=0.0, want_render=True):
        a = StepArgs()
        for g in range(6):
            a.params[g] = sh.ptr(params[g]) if params[g] is not None and params[g].size else None
            a.exp_avg[g] = sh.ptr(exp_avg[g]) if exp_avg[g] is not None and exp_avg[g].size else None
            a.exp_avg_sq[g] = sh.ptr(exp_avg_sq[g]) if exp_avg_sq[g] is not None and exp_avg_sq[g].size else None
        keep = [sh.f32(viewmat), sh.f32(K), sh.f32(gt_rgb)]
        render = np.zeros((height, width, 3), np.float32) if want_render else None
        a.count, a.sh_degree = count, sh_degree
        a.viewmat, a.K, a.gt_rgb = sh.ptr(keep[0]), sh.ptr(keep[1]), sh.ptr(keep[2])
        a.width, a.height, a.degrees_to_use = width, height, degrees_to_use
        for g in range(6):
            a.lr[g] = lr[g]
        a.opacity_reg_w, a.scale_reg_w = opacity_reg_w, scale_reg_w
        a.eps2d, a.near_plane, a.far_plane, a.radius_clip = eps2d, near_plane, far_plane, radius_clip
        a.b1, a.b2, a.eps, a.ssim_weight = b1, b2, eps, ssim_weight
        a.antialiased, a.isect_mode = int(bool(antialiased)), isect_mode
        a.forward_only, a.inject_noise = int(bool(forward_only)), int(bool(inject_noise))
        a.noise_seed, a.noise_offset, a.noise_scale = noise_seed, noise_offset, noise_scale
        a.render_colors = sh.ptr(render)
        self._call("train_step", C.byref(a))
        stage_fn = self.lib.sxo_stage_name
        stage_fn.restype = C.c_char_p
        stages = {stage_fn(i).decode(): a.stage_ms[i] for i in range(16)}
        return dict(loss=float(a.loss), n_isects=int(a.n_isects), n_visible=int(a.n_visible),
                    render_colors=render, stage_ms=stages)

    def mt64_seed(self, seed):
        st = sh.MtState()
        self._call("mt64_seed", C.c_uint64(seed), C.byref(st))
        return st

    def mt64_draw(self, st, n):
        out = np.zeros(n, np.uint64)
        self._call("mt64_draw", C.byref(st), C.c_int64(n), sh.ptr(out))
        return out

    def running_sum_f64(self, w):
        w = sh.f32(w)
        out = np.zeros(w.size, np.float64)
        f = self.lib.sxo_running_sum_f64
        f.restype = C.c_int32
        f(sh.ptr(w), C.c_int64(w.size), out.ctypes.data_as(C.POINTER(C.c_double)))
        return out

    def mcmc_refine(self, params, exp_avg, exp_avg_sq, count, cap_max, sh_degree, rng, binoms, min_opacity=0.005,
                    n_max=51, want_lists=True):
        """Trainer::mcmc_refine on AoS arena arrays [rows, dim] in place; `rng` (MtState) advanced in place."""
        a = RefineArgs()
        for g in range(6):
            a.params[g] = _ptr_or_null(params[g])
            a.exp_avg[g] = _ptr_or_null(exp_avg[g])
            a.exp_avg_sq[g] = _ptr_or_null(exp_avg_sq[g])
        keep = sh.f32(binoms)
        a.count, a.cap_max, a.sh_degree, a.min_opacity, a.n_max = count, cap_max, sh_degree, min_opacity, n_max
        a.binoms, a.rng = sh.ptr(keep), C.pointer(rng)
        lists = None
        if want_lists:
            cap = params[3].shape[0]
            lists = [np.zeros(cap, np.int64) for _ in range(3)]
            a.relocated_dead, a.relocation_src, a.added_src = (sh.ptr(x) for x in lists)
            a.capacity = cap
        self._call("mcmc_refine", C.byref(a))
        o = sh.RefineOutputs(a.new_count, a.n_relocated, a.n_added)
        return sh.refine_lists(o, lists)


class Reference(sh.Ops):
    """The reference's own CPU kernels (oracle/_ref/libsx_ref.so, built from /root/reference)."""

    PATH = os.path.join(HERE, "_ref", "libsx_ref.so")

    def __init__(self):
        if not os.path.exists(self.PATH):
            raise RuntimeError("oracle/_ref not built (reference tree absent)")
        super().__init__(C.CDLL(self.PATH), "sxr_")

    def quat_scale_to_covar(self, quats, scales):
        q, s = sh.f32(quats), sh.f32(scales)
        out = np.zeros((q.shape[0], 3, 3), np.float32)
        self._call("quat_scale_to_covar", sh.ptr(q), sh.ptr(s), q.shape[0], sh.ptr(out))
        return out

    def make_binoms_lut(self, n_max=51):
        out = np.zeros(n_max * n_max, np.float32)
        self._call("make_binoms_lut", n_max, sh.ptr(out))
        return out

    TRAIN_DEFAULT_FIELDS = ("total_iters", "scene_scale", "lr_means", "lr_quats", "lr_scales", "lr_opacities", "lr_sh0",
                            "lr_shN", "sh_degree_interval_ratio", "opacity_reg", "scale_reg", "cap_max",
                            "min_opacity", "refine_start_ratio", "refine_stop_ratio", "refine_every_ratio",
                            "noise_lr", "mcmc_seed")

    def train_defaults(self) -> dict:
        """TrainConfig / McmcOptions defaults of the reference's Trainer.h."""
        out = np.zeros(18, np.float64)
        self._call("train_defaults", out.ctypes.data_as(C.POINTER(C.c_double)))
        return dict(zip(self.TRAIN_DEFAULT_FIELDS, out.tolist()))

    def train_plans(self, total_iters, scene_scale, lr_means, sh_degree_interval_ratio, mcmc_enabled,
                    refine_start_ratio, refine_stop_ratio, refine_every_ratio, sh_degree, iters):
        """means_lr_at, sh_degree_at and Trainer::mcmc_refine_due of the reference for `iters`."""
        s = RefSchedule(total_iters, scene_scale, lr_means, sh_degree_interval_ratio, int(bool(mcmc_enabled)),
                        refine_start_ratio, refine_stop_ratio, refine_every_ratio)
        it = np.ascontiguousarray(iters, np.int32)
        lr0 = np.zeros(it.size, np.float32)
        deg = np.zeros(it.size, np.uint32)
        due = np.zeros(it.size, np.uint8)
        self._call("train_plans", C.byref(s), sh_degree, it.size, sh.ptr(it), sh.ptr(lr0), sh.ptr(deg), sh.ptr(due))
        return lr0, deg, due

    def trainer_mcmc_refine(self, params, exp_avg, exp_avg_sq, count, cap_max, sh_degree, seed, n_refine,
                            min_opacity=0.005):
        """The reference's Trainer (CPU backend, MCMC on) after n_refine calls of mcmc_refine.

        params: count-row AoS arrays; exp_avg / exp_avg_sq: cap_max-row arrays. Returns cap_max-row
        arrays, the count and list sizes after every refine, the last refine's lists and the
        engine state."""
        c = RefCase()
        dims = sh.GROUP_DIMS(sh_degree)
        outs = [[np.zeros((cap_max, d), np.float32) for d in dims] for _ in range(3)]
        keep = [[sh.f32(x) for x in grp] for grp in (params, exp_avg, exp_avg_sq)]
        for g in range(6):
            c.params[g] = _ptr_or_null(keep[0][g])
            c.exp_avg[g] = _ptr_or_null(keep[1][g])
            c.exp_avg_sq[g] = _ptr_or_null(keep[2][g])
            c.out_params[g] = _ptr_or_null(outs[0][g])
            c.out_exp_avg[g] = _ptr_or_null(outs[1][g])
            c.out_exp_avg_sq[g] = _ptr_or_null(outs[2][g])
        c.count, c.cap_max, c.sh_degree, c.min_opacity, c.seed, c.n_refine = (count, cap_max, sh_degree, min_opacity,
                                                                              seed, n_refine)
        per = [np.zeros(n_refine, np.int64) for _ in range(3)]
        c.counts, c.n_relocated, c.n_added = (sh.ptr(x) for x in per)
        lists = [np.zeros(cap_max, np.int64) for _ in range(3)]
        c.relocated_dead, c.relocation_src, c.added_src = (sh.ptr(x) for x in lists)
        c.capacity = cap_max
        st = sh.MtState()
        c.rng_out = C.pointer(st)
        self._call("trainer_mcmc_refine", C.byref(c))
        nr, na = int(per[1][-1]), int(per[2][-1])
        return dict(params=outs[0], exp_avg=outs[1], exp_avg_sq=outs[2], counts=per[0], n_relocated=per[1],
                    n_added=per[2], relocated_dead=lists[0][:nr], relocation_src=lists[1][:nr],
                    added_src=lists[2][:na], rng=st)

    # -- formats (PlyIO.cpp, Checkpoint.cpp) ----------------------------------------------------
    @staticmethod
    def _cloud_in(params, count, sh_degree):
        keep = [sh.f32(x).reshape(count, -1) if x is not None and count > 0 else None for x in params]
        c = RefCloudIn()
        for g in range(6):
            c.params[g] = _ptr_or_null(keep[g]) if keep[g] is not None else None
        c.count, c.sh_degree = count, sh_degree
        return c, keep

    def export_ply(self, params, count, sh_degree, path, min_opacity=0.005, pad_sh_full=True):
        c, keep = self._cloud_in(params, count, sh_degree)
        st = sh.ExportStats()
        self._call("export_ply", C.byref(c), C.c_float(min_opacity), int(bool(pad_sh_full)), path.encode(),
                   C.byref(st))
        return st.as_dict()

    def read_ply(self, path, capacity):
        o = RefCloudOut()
        outs = [np.zeros((capacity, d), np.float32) for d in sh.GROUP_DIMS(3)]
        for g in range(6):
            o.params[g] = sh.ptr(outs[g])
        o.count = capacity
        self._call("read_ply", path.encode(), C.byref(o))
        n, deg = int(o.count), int(o.sh_degree)
        dims = sh.GROUP_DIMS(deg)
        return dict(count=n, sh_degree=deg,
                    params=[outs[g].ravel()[: n * dims[g]].reshape(n, dims[g]) for g in range(6)])

    def save_checkpoint(self, config, iter, params, exp_avg, exp_avg_sq, count, sh_degree, path, rng_state=None,
                        fp16=False):
        c, keep = self._cloud_in(params, count, sh_degree)
        mk = [sh.f32(x).reshape(count, -1) for x in exp_avg]
        vk = [sh.f32(x).reshape(count, -1) for x in exp_avg_sq]
        m = (sh.fp * 6)(*[_ptr_or_null(x) for x in mk])
        v = (sh.fp * 6)(*[_ptr_or_null(x) for x in vk])
        self._call("save_checkpoint", C.byref(config), iter, C.byref(c), m, v,
                   rng_state.encode() if rng_state else None, int(bool(fp16)), path.encode())

    def load_checkpoint(self, path, capacity):
        h = sh.CkptHeader()
        o = RefCloudOut()
        dims = sh.GROUP_DIMS(3)
        outs = [np.zeros((capacity, d), np.float32) for d in dims]
        ms = [np.zeros((capacity, d), np.float32) for d in dims]
        vs = [np.zeros((capacity, d), np.float32) for d in dims]
        for g in range(6):
            o.params[g] = sh.ptr(outs[g])
        o.count = capacity
        buf = C.create_string_buffer(1 << 16)
        self._call("load_checkpoint", path.encode(), C.byref(h), C.byref(o), (sh.fp * 6)(*[sh.ptr(x) for x in ms]),
                   (sh.fp * 6)(*[sh.ptr(x) for x in vs]), buf, C.c_int64(1 << 16))
        n, deg = int(o.count), int(o.sh_degree)
        dd = sh.GROUP_DIMS(deg)
        cut = lambda arrs: [arrs[g].ravel()[: n * dd[g]].reshape(n, dd[g]) for g in range(6)]
        return dict(header=h.as_dict(), params=cut(outs), exp_avg=cut(ms), exp_avg_sq=cut(vs),
                    rng_state=buf.value.decode())

    def checkpoint_verify_config(self, saved, current):
        self._call("checkpoint_verify_config", C.byref(saved), C.byref(current))

    @staticmethod
    def available() -> bool:
        return os.path.exists(Reference.PATH)


class ReferenceTrainerOnHip:
    """The reference's Trainer (Trainer.cpp, unchanged) on this repository's backend through the C++
    KernelBackend adapter: oracle/_ref/libsx_ref_hip.so. Needs a GPU at run time."""

    PATH = os.path.join(HERE, "_ref", "libsx_ref_hip.so")

    def __init__(self):
        if not os.path.exists(self.PATH):
            raise RuntimeError("oracle/_ref/libsx_ref_hip.so not built (reference tree absent)")
        self.lib = C.CDLL(self.PATH)
        self.lib.sxr_hip_trainer_run.restype = C.c_int32
        self.lib.sxr_hip_last_error.restype = C.c_char_p

    @staticmethod
    def available() -> bool:
        return os.path.exists(ReferenceTrainerOnHip.PATH)

    def adapter_refine(self, params, exp_avg, exp_avg_sq, count, cap_max, sh_degree, seed, n_refine, binoms):
        """hip_mcmc_refine through the C++ adapter; arrays ([cap_max, dim]) are updated in place."""
        c = HipRefineCase()
        for g in range(6):
            c.params[g] = _ptr_or_null(params[g])
            c.exp_avg[g] = _ptr_or_null(exp_avg[g])
            c.exp_avg_sq[g] = _ptr_or_null(exp_avg_sq[g])
        keep = sh.f32(binoms)
        c.count, c.cap_max, c.sh_degree, c.n_refine, c.seed, c.binoms = (count, cap_max, sh_degree, n_refine, seed,
                                                                        sh.ptr(keep))
        counts = np.zeros(n_refine, np.int64)
        lists = np.zeros((3, cap_max), np.int64)
        st = sh.MtState()
        c.counts, c.last_lists, c.rng_out = sh.ptr(counts), sh.ptr(lists), C.pointer(st)
        self.lib.sxr_hip_adapter_refine.restype = C.c_int32
        rc = self.lib.sxr_hip_adapter_refine(C.byref(c))
        if rc != sh.SXH_OK:
            raise sh.SxRuntimeError(self.lib.sxr_hip_last_error().decode(errors="replace"))
        sizes = list(c.last_sizes)
        return dict(counts=counts, relocated_dead=lists[0][:sizes[0]], relocation_src=lists[1][:sizes[1]],
                    added_src=lists[2][:sizes[2]], rng=st)

    def run(self, params, count, sh_degree, viewmat, K, width, height, gt, steps, lr, total_iters=100,
            ssim_weight=0.2, opacity_reg=0.0, scale_reg=0.0, antialiased=False, resident=True, mcmc=False,
            cap_max=0, seed=42, refine_start_ratio=0.0, refine_stop_ratio=1.0, refine_every_ratio=0.02,
            cameras=None, start_iter=0, scene_scale=0.0, sh_degree_interval_ratio=0.0):
        """Steps start_iter .. start_iter + steps of Trainer::step; with cameras = (viewmats [n,16],
        Ks [n,9], gts [n,H,W,3]) step it uses camera it % n (viewmat/K/gt are then ignored)."""
        c = HipTrainCase()
        if cameras is not None:
            cv, ck, cg = (sh.f32(x) for x in cameras)
            self._cams = (cv, ck, cg)
            c.n_cams, c.viewmats, c.Ks, c.gts = cv.shape[0], sh.ptr(cv), sh.ptr(ck), sh.ptr(cg)
            viewmat, K, gt = cv[0], ck[0], cg[0]
        c.start_iter, c.scene_scale, c.sh_degree_interval_ratio = start_iter, scene_scale, sh_degree_interval_ratio
        keep = [sh.f32(x).reshape(count, -1) for x in params]
        for g in range(6):
            c.params[g] = _ptr_or_null(keep[g])
        rows = cap_max if mcmc else count
        dims = sh.GROUP_DIMS(sh_degree)
        outs = [np.zeros((rows, d), np.float32) for d in dims]
        for g in range(6):
            c.out_params[g] = _ptr_or_null(outs[g])
        vm, KK, gg = sh.f32(viewmat), sh.f32(K), sh.f32(gt)
        c.count, c.sh_degree, c.viewmat, c.K, c.width, c.height = count, sh_degree, sh.ptr(vm), sh.ptr(KK), width, height
        c.gt_rgb, c.steps, c.total_iters = sh.ptr(gg), steps, total_iters
        for g in range(6):
            c.lr[g] = lr[g]
        c.ssim_weight, c.opacity_reg, c.scale_reg = ssim_weight, opacity_reg, scale_reg
        c.antialiased, c.resident, c.mcmc = int(bool(antialiased)), int(bool(resident)), int(bool(mcmc))
        c.cap_max, c.seed = cap_max, seed
        c.refine_start_ratio, c.refine_stop_ratio, c.refine_every_ratio = (refine_start_ratio, refine_stop_ratio,
                                                                           refine_every_ratio)
        losses = np.zeros(steps, np.float32)
        n_isects = np.zeros(steps, np.int64)
        render0 = np.zeros((height, width, 3), np.float32)
        c.losses, c.n_isects, c.render0 = sh.ptr(losses), sh.ptr(n_isects), sh.ptr(render0)
        rc = self.lib.sxr_hip_trainer_run(C.byref(c))
        if rc != sh.SXH_OK:
            msg = self.lib.sxr_hip_last_error().decode(errors="replace")
            raise (sh.SxInvalidArgument if rc == sh.SXH_ERR_INVALID_ARGUMENT else sh.SxRuntimeError)(msg)
        return dict(params=outs, losses=losses, n_isects=n_isects, render0=render0, count=int(c.out_count),
                    n_refined=int(c.n_refined))
