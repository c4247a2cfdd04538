"""ctypes binding of the splatx MI355X backend C ABI (include/splatx_hip.h).

`Backend` mirrors the reference operator boundary `splatx::KernelBackend`
(Sources/SplatXCore/include/splatx/KernelBackend.h:396-509): one method per op, numpy arrays in,
numpy arrays out, the reference's exception classes mapped to `SxInvalidArgument` (ValueError,
for std::invalid_argument) and `SxRuntimeError` (RuntimeError, for std::runtime_error).
`Executor` mirrors `splatx::TrainStepExecutor` (KernelBackend.h:386-392).

The generic `Ops` class drives any library exporting the same structs with a name prefix; the
product library uses prefix "sxh_" and a backend handle. Loading fails loudly when the compiled
library is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_ROOT, "build", "libsplatx_hip.so")

SXH_OK = 0
SXH_ERR_INVALID_ARGUMENT = 1
SXH_ERR_RUNTIME = 2
SXH_ERR_CAPACITY = 3
SXH_ISECT_ACCUTILE = 0
SXH_ISECT_AABB = 1
SXH_ISECT_ORDER_AUTO = 0
SXH_ISECT_ORDER_DEPTH_FIRST = 1
SXH_ISECT_ORDER_INDEX_FIRST = 2
SXH_ROW_ORDER_SPATIAL_AUTO = 0
SXH_ROW_ORDER_ORIGINAL = 1
SXH_ROW_ORDER_SPATIAL = 2


class SxInvalidArgument(ValueError):
    """std::invalid_argument in the reference (Validate.h:23)."""


class SxRuntimeError(RuntimeError):
    """std::runtime_error in the reference (device, allocation or unsupported-camera failures)."""


class SxCapacityError(RuntimeError):
    pass


fp = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)
u32p = C.POINTER(C.c_uint32)
i64p = C.POINTER(C.c_int64)
u64p = C.POINTER(C.c_uint64)
u8p = C.POINTER(C.c_uint8)


class AdamInputs(C.Structure):
    _fields_ = [("param", fp), ("grad", fp), ("exp_avg", fp), ("exp_avg_sq", fp), ("valid", u8p),
                ("n_elems", C.c_int64), ("n_gauss", C.c_int64), ("lr", C.c_float), ("b1", C.c_float),
                ("b2", C.c_float), ("eps", C.c_float)]


class ProjectionInputs(C.Structure):
    _fields_ = [("means", fp), ("covars", fp), ("quats", fp), ("scales", fp), ("opacities", fp),
                ("viewmats", fp), ("Ks", fp), ("N", C.c_int64), ("C", C.c_int64), ("width", C.c_int32),
                ("height", C.c_int32), ("eps2d", C.c_float), ("near_plane", C.c_float),
                ("far_plane", C.c_float), ("radius_clip", C.c_float), ("camera_model", C.c_uint32),
                ("calc_compensations", C.c_uint8)]


class ProjectionOutputs(C.Structure):
    _fields_ = [("radii", i32p), ("means2d", fp), ("depths", fp), ("conics", fp), ("compensations", fp)]


class ProjectionGradsIn(C.Structure):
    _fields_ = [("radii", i32p), ("conics", fp), ("compensations", fp), ("v_means2d", fp),
                ("v_depths", fp), ("v_conics", fp), ("v_compensations", fp), ("viewmats_grad", C.c_uint8)]


class ProjectionGrads(C.Structure):
    _fields_ = [("v_means", fp), ("v_covars", fp), ("v_quats", fp), ("v_scales", fp), ("v_viewmats", fp)]


class ShInputs(C.Structure):
    _fields_ = [("dirs", fp), ("coeffs", fp), ("masks", u8p), ("degrees_to_use", C.c_uint32),
                ("B", C.c_int64), ("N", C.c_int64), ("K", C.c_int64), ("D", C.c_uint32),
                ("compute_v_dirs", C.c_uint8)]


class IsectInputs(C.Structure):
    _fields_ = [("means2d", fp), ("radii", i32p), ("depths", fp), ("conics", fp), ("opacities", fp),
                ("I", C.c_int64), ("N", C.c_int64), ("tile_size", C.c_uint32), ("tile_width", C.c_uint32),
                ("tile_height", C.c_uint32)]


class IsectOutputs(C.Structure):
    _fields_ = [("tiles_per_gauss", i32p), ("isect_ids", u64p), ("flatten_ids", i32p),
                ("capacity", C.c_int64), ("n_isects", C.c_int64), ("tile_n_bits", C.c_uint32),
                ("image_n_bits", C.c_uint32)]


class SortInputs(C.Structure):
    _fields_ = [("keys", u64p), ("values", i32p), ("n", C.c_int64), ("key_n_bits", C.c_uint32)]


class OffsetInputs(C.Structure):
    _fields_ = [("isect_ids", u64p), ("n_isects", C.c_int64), ("I", C.c_int64),
                ("tile_width", C.c_uint32), ("tile_height", C.c_uint32)]


class RasterInputs(C.Structure):
    _fields_ = [("means2d", fp), ("conics", fp), ("colors", fp), ("opacities", fp), ("backgrounds", fp),
                ("masks", u8p), ("isect_offsets", i32p), ("flatten_ids", i32p), ("I", C.c_int64),
                ("N", C.c_int64), ("n_isects", C.c_int64), ("image_width", C.c_uint32),
                ("image_height", C.c_uint32), ("tile_size", C.c_uint32), ("tile_width", C.c_uint32),
                ("tile_height", C.c_uint32)]


class RasterOutputs(C.Structure):
    _fields_ = [("render_colors", fp), ("render_alphas", fp), ("last_ids", i32p)]


class RasterGradsIn(C.Structure):
    _fields_ = [("render_alphas", fp), ("last_ids", i32p), ("v_render_colors", fp),
                ("v_render_alphas", fp), ("absgrad", C.c_uint8)]


class RasterGrads(C.Structure):
    _fields_ = [("v_means2d", fp), ("v_conics", fp), ("v_colors", fp), ("v_opacities", fp),
                ("v_means2d_abs", fp)]


class RngInputs(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("offset", C.c_uint64), ("count", C.c_int64)]


class RelocationInputs(C.Structure):
    _fields_ = [("opacities", fp), ("scales", fp), ("ratios", i32p), ("binoms", fp), ("N", C.c_int64),
                ("n_max", C.c_int32), ("min_opacity", C.c_float)]


class PerturbInputs(C.Structure):
    _fields_ = [("positions", fp), ("quats", fp), ("scales_log", fp), ("opacities_logit", fp),
                ("noise", fp), ("N", C.c_int64), ("noise_scale", C.c_float), ("t", C.c_float),
                ("k", C.c_float)]


class SsimInputs(C.Structure):
    _fields_ = [("img1", fp), ("img2", fp), ("I", C.c_int64), ("H", C.c_int64), ("W", C.c_int64),
                ("C", C.c_int64), ("need_coeffs", C.c_uint8)]


class SsimOutputs(C.Structure):
    _fields_ = [("ssim", C.c_double), ("ssim_map", fp), ("coeff_mu", fp), ("coeff_sigma", fp),
                ("coeff_cross", fp)]


class SsimGradsIn(C.Structure):
    _fields_ = [("coeff_mu", fp), ("coeff_sigma", fp), ("coeff_cross", fp), ("v_loss", C.c_float)]


class ExecDesc(C.Structure):
    _fields_ = [("arena_rows", C.c_int64), ("sh_degree", C.c_int32), ("eps2d", C.c_float),
                ("near_plane", C.c_float), ("far_plane", C.c_float), ("radius_clip", C.c_float),
                ("b1", C.c_float), ("b2", C.c_float), ("eps", C.c_float), ("ssim_weight", C.c_float),
                ("antialiased", C.c_uint8), ("isect_mode", C.c_uint8)]


class ParamSync(C.Structure):
    _fields_ = [("params", fp * 6), ("exp_avg", fp * 6), ("exp_avg_sq", fp * 6), ("rows", C.c_int64)]


class StepInputs(C.Structure):
    _fields_ = [("viewmat", fp), ("K", fp), ("width", C.c_int32), ("height", C.c_int32), ("gt_rgb", fp),
                ("gt_index", C.c_int32), ("count", C.c_int64), ("degrees_to_use", C.c_uint32),
                ("lr", C.c_float * 6), ("opacity_reg_w", C.c_float), ("scale_reg_w", C.c_float),
                ("forward_only", C.c_uint8), ("inject_noise", C.c_uint8), ("noise_seed", C.c_uint64),
                ("noise_offset", C.c_uint64), ("noise_scale", C.c_float)]


class StepOutputs(C.Structure):
    _fields_ = [("loss", C.c_float), ("n_isects", C.c_int64), ("n_visible", C.c_int64),
                ("render_colors", fp), ("sort_key_bits", C.c_uint32)]


class MtState(C.Structure):
    """std::mt19937_64 in libstdc++'s layout: 312 words and the next-word position."""
    _fields_ = [("x", C.c_uint64 * 312), ("p", C.c_uint32)]

    def copy(self) -> "MtState":
        c = MtState()
        C.memmove(C.byref(c), C.byref(self), C.sizeof(MtState))
        return c

    def equals(self, other: "MtState") -> bool:
        return self.p == other.p and list(self.x) == list(other.x)


class RefineInputs(C.Structure):
    _fields_ = [("count", C.c_int64), ("cap_max", C.c_int64), ("min_opacity", C.c_float), ("n_max", C.c_int32),
                ("binoms", fp), ("rng", C.POINTER(MtState)), ("inject_noise", C.c_uint8),
                ("noise_seed", C.c_uint64), ("noise_offset", C.c_uint64), ("noise_scale", C.c_float)]


class RefineOutputs(C.Structure):
    _fields_ = [("count", C.c_int64), ("n_relocated", C.c_int64), ("n_added", C.c_int64),
                ("relocated_dead", i64p), ("relocation_src", i64p), ("added_src", i64p), ("capacity", C.c_int64)]


def refine_lists(out: RefineOutputs, lists) -> dict:
    r = dict(count=int(out.count), n_relocated=int(out.n_relocated), n_added=int(out.n_added))
    if lists is not None:
        r["relocated_dead"] = lists[0][:out.n_relocated].copy()
        r["relocation_src"] = lists[1][:out.n_relocated].copy()
        r["added_src"] = lists[2][:out.n_added].copy()
    return r


class ExportStats(C.Structure):
    _fields_ = [("input", C.c_int64), ("removed_nonfinite", C.c_int64), ("removed_low_opacity", C.c_int64),
                ("kept", C.c_int64)]

    def as_dict(self):
        return {k: int(getattr(self, k)) for k, _ in self._fields_}


class CkptConfig(C.Structure):
    _fields_ = [("sh_degree", C.c_int32), ("factor", C.c_int32), ("test_split", C.c_int32), ("total_iters", C.c_int32),
                ("mcmc_enabled", C.c_uint8), ("antialiased", C.c_uint8), ("cap_max", C.c_int64),
                ("mcmc_seed", C.c_uint64), ("scene_scale", C.c_float), ("ssim_weight", C.c_float)]

    @staticmethod
    def make(**kw):
        c = CkptConfig()
        c.scene_scale = 1.0
        for k, v in kw.items():
            setattr(c, k, v)
        return c

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class CkptHeader(C.Structure):
    _fields_ = [("config", CkptConfig), ("iter", C.c_int32), ("alive_count", C.c_int64), ("fp16", C.c_uint8),
                ("version", C.c_uint32)]

    def as_dict(self):
        return dict(config=self.config.as_dict(), iter=int(self.iter), alive_count=int(self.alive_count),
                    fp16=int(self.fp16), version=int(self.version))


class RenderSessionArgs(C.Structure):
    _fields_ = [("ply_path", C.c_char_p), ("antialiased", C.c_int32), ("sh_degree", C.c_int32)]


class TrainCamera(C.Structure):
    """TrainingCamera with its image's slot in the GT cache (sxh_train_camera)."""
    _fields_ = [("viewmat", C.c_float * 16), ("K", C.c_float * 9), ("width", C.c_int32), ("height", C.c_int32),
                ("gt_index", C.c_int32)]

    @staticmethod
    def make(viewmat, K, width, height, gt_index):
        c = TrainCamera()
        c.viewmat[:] = [float(x) for x in np.asarray(viewmat, np.float32).ravel()]
        c.K[:] = [float(x) for x in np.asarray(K, np.float32).ravel()]
        c.width, c.height, c.gt_index = width, height, gt_index
        return c


class TrainSchedule(C.Structure):
    """TrainConfig / McmcOptions fields the caller loop reads (sxh_train_schedule)."""
    _fields_ = [("total_iters", C.c_int32), ("scene_scale", C.c_float), ("lr_means", C.c_float),
                ("lr_quats", C.c_float), ("lr_scales", C.c_float), ("lr_opacities", C.c_float), ("lr_sh0", C.c_float),
                ("lr_shN", C.c_float), ("sh_degree_interval_ratio", C.c_float), ("opacity_reg", C.c_float),
                ("scale_reg", C.c_float), ("mcmc_enabled", C.c_uint8), ("cap_max", C.c_int64),
                ("min_opacity", C.c_float), ("refine_start_ratio", C.c_float), ("refine_stop_ratio", C.c_float),
                ("refine_every_ratio", C.c_float), ("noise_lr", C.c_float), ("mcmc_seed", C.c_uint64)]


class TrainProgress(C.Structure):
    """SxTrainProgress (sxh_train_progress)."""
    _fields_ = [("iter", C.c_int32), ("run_until", C.c_int32), ("total_iters", C.c_int32), ("loss", C.c_float),
                ("psnr", C.c_float), ("step_ms", C.c_double), ("n_isects", C.c_int64), ("splat_count", C.c_int64),
                ("thermal_state", C.c_int32), ("mcmc_refined", C.c_int32), ("n_relocated", C.c_int64),
                ("n_added", C.c_int64)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class SplatSnapshot(C.Structure):
    """SxSplatSnapshot (sxh_splat_snapshot)."""
    _fields_ = [("iter", C.c_int32), ("sh_degree", C.c_int32), ("count", C.c_int64), ("means", fp), ("quats", fp),
                ("scales", fp), ("opacities", fp), ("sh0", fp), ("shN", fp)]


class TrainPlan(C.Structure):
    """One iteration's step arguments under a schedule (sxh_train_plan)."""
    _fields_ = [("degrees_to_use", C.c_uint32), ("lr", C.c_float * 6), ("opacity_reg_w", C.c_float),
                ("scale_reg_w", C.c_float), ("refine_due", C.c_uint8), ("inject_noise", C.c_uint8),
                ("noise_scale", C.c_float)]


def train_schedule_defaults(lib=None) -> TrainSchedule:
    lib = lib or load_library()
    s = TrainSchedule()
    lib.sxh_train_schedule_defaults.restype = C.c_int32
    _raise(lib, lib.sxh_train_schedule_defaults(C.byref(s)))
    return s


def train_plan_at(schedule: TrainSchedule, iter: int, sh_degree: int, count: int, lib=None) -> TrainPlan:
    """Trainer::step_resident's arguments for iteration `iter` (sxh_train_plan_at, host only)."""
    lib = lib or load_library()
    p = TrainPlan()
    lib.sxh_train_plan_at.restype = C.c_int32
    _raise(lib, lib.sxh_train_plan_at(C.byref(schedule), iter, sh_degree, C.c_int64(count), C.byref(p)))
    return p


PROGRESS_FN = C.CFUNCTYPE(None, C.POINTER(TrainProgress), C.c_void_p)
SNAPSHOT_FN = C.CFUNCTYPE(None, C.POINTER(SplatSnapshot), C.c_void_p)


class TrainLoopArgs(C.Structure):
    _fields_ = [("cameras", C.POINTER(TrainCamera)), ("n_cameras", C.c_int32),
                ("eval_cameras", C.POINTER(TrainCamera)), ("n_eval_cameras", C.c_int32), ("eval_every", C.c_int32),
                ("start_iter", C.c_int32), ("run_until", C.c_int32), ("count", C.c_int64), ("sched", TrainSchedule),
                ("binoms", fp), ("n_max", C.c_int32), ("rng", C.POINTER(MtState)), ("jitter_max_deg", C.c_float),
                ("jitter_max_t", C.c_float), ("jitter_seed", C.c_uint64), ("progress", PROGRESS_FN),
                ("progress_user", C.c_void_p), ("snapshot", SNAPSHOT_FN), ("snapshot_user", C.c_void_p),
                ("snapshot_every", C.c_int32), ("live_ply_every", C.c_int32), ("live_ply_path", C.c_char_p),
                ("checkpoint_every", C.c_int32), ("checkpoint_path", C.c_char_p),
                ("checkpoint_config", C.POINTER(CkptConfig)), ("checkpoint_fp16", C.c_uint8)]


class TrainLoopResult(C.Structure):
    _fields_ = [("completed_iters", C.c_int32), ("count", C.c_int64), ("first_loss", C.c_float),
                ("last_loss", C.c_float), ("last_eval_psnr", C.c_float), ("train_seconds", C.c_double),
                ("stopped", C.c_int32)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


def _raise(lib, rc):
    if rc != SXH_OK:
        msg = lib.sxh_last_error().decode(errors="replace")
        if rc == SXH_ERR_INVALID_ARGUMENT:
            raise SxInvalidArgument(msg)
        if rc == SXH_ERR_CAPACITY:
            raise SxCapacityError(msg)
        raise SxRuntimeError(msg)


def ply_read(path, lib=None):
    """read_inria_ply (sxh_ply_read): dict(count, sh_degree, params = 6 AoS arrays)."""
    lib = lib or load_library()
    lib.sxh_last_error.restype = C.c_char_p
    f = lib.sxh_ply_read
    f.restype = C.c_int32
    n, deg = C.c_int64(), C.c_int32()
    _raise(lib, f(path.encode(), C.byref(n), C.byref(deg), None))
    dims = GROUP_DIMS(deg.value)
    params = [np.zeros((n.value, d), np.float32) for d in dims]
    arr = (fp * 6)(*[ptr(x) if x.size else None for x in params])
    _raise(lib, f(path.encode(), C.byref(n), C.byref(deg), arr))
    return dict(count=n.value, sh_degree=deg.value, params=params)


def checkpoint_read_header(path, lib=None):
    lib = lib or load_library()
    lib.sxh_last_error.restype = C.c_char_p
    h = CkptHeader()
    lib.sxh_checkpoint_read_header.restype = C.c_int32
    _raise(lib, lib.sxh_checkpoint_read_header(path.encode(), C.byref(h)))
    return h.as_dict()


def checkpoint_verify_config(saved: CkptConfig, current: CkptConfig, lib=None):
    lib = lib or load_library()
    lib.sxh_last_error.restype = C.c_char_p
    lib.sxh_checkpoint_verify_config.restype = C.c_int32
    _raise(lib, lib.sxh_checkpoint_verify_config(C.byref(saved), C.byref(current)))


class RenderSession:
    """sx_render_session_* (splatx_train_c.h:604-682) over sxh_render_session_*."""

    def __init__(self, backend, ply_path, antialiased=False, sh_degree=0):
        self.lib = backend.lib
        self.h = C.c_void_p()
        self._path = ply_path.encode()
        a = RenderSessionArgs(self._path, int(bool(antialiased)), sh_degree)
        self.lib.sxh_render_session_open.restype = C.c_int32
        _raise(self.lib, self.lib.sxh_render_session_open(backend.handle, C.byref(a), C.byref(self.h)))
        self.lib.sxh_render_session_frame.restype = C.c_int32
        self.lib.sxh_render_session_close.argtypes = [C.c_void_p]

    def frame(self, viewmat, fx, fy, cx, cy, width, height):
        vm = f32(viewmat)
        out = np.zeros((height, width, 4), np.uint8)
        _raise(self.lib, self.lib.sxh_render_session_frame(self.h, ptr(vm), C.c_float(fx), C.c_float(fy), C.c_float(cx),
                                                          C.c_float(cy), width, height, ptr(out)))
        return out

    def close(self):
        if self.h is not None and self.h.value is not None:
            self.lib.sxh_render_session_close(self.h)
        self.h = None


class RasterStats(C.Structure):
    _fields_ = [(k, C.c_uint64) for k in ("fwd_iters", "fwd_entries", "fwd_taken", "bwd_chunks", "bwd_entries",
                                          "bwd_empty_chunks", "bwd_in_cutoff", "bwd_contrib")]


class ExecTiming(C.Structure):
    _fields_ = [("n", C.c_int32), ("names", C.c_char_p * 32), ("ms", C.c_float * 32)]


# ---------------------------------------------------------------------------------------------
def ptr(a: Optional[np.ndarray], ctype=None):
    """Pointer to a C-contiguous numpy array (None -> NULL)."""
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    t = {np.float32: fp, np.int32: i32p, np.uint32: u32p, np.int64: i64p, np.uint64: u64p,
         np.uint8: u8p}[a.dtype.type]
    return a.ctypes.data_as(t)


def f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def i32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


def u8(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.uint8)


def u64(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.uint64)


def bits_for_count(count: int) -> int:
    """CpuKernels.h:69-74."""
    if count <= 1:
        return 0
    return int(count - 1).bit_length()


class Ops:
    """One method per KernelBackend op over a library exporting `<prefix><op>` functions.

    `handle` is prepended to every call when not None (the product's backend pointer)."""

    def __init__(self, lib, prefix: str, handle=None, err_fn: str = "last_error"):
        self.lib = lib
        self.prefix = prefix
        self.handle = handle
        self._err = getattr(lib, prefix + err_fn)
        self._err.restype = C.c_char_p
        self._err.argtypes = []

    def _fn(self, name):
        f = getattr(self.lib, self.prefix + name)
        f.restype = C.c_int32
        return f

    def _call(self, name, *args):
        f = self._fn(name)
        rc = f(self.handle, *args) if self.handle is not None else f(*args)
        if rc != SXH_OK:
            msg = (self._err() or b"").decode(errors="replace")
            if rc == SXH_ERR_INVALID_ARGUMENT:
                raise SxInvalidArgument(msg)
            if rc == SXH_ERR_CAPACITY:
                raise SxCapacityError(msg)
            raise SxRuntimeError(msg)
        return rc

    # -- fused_adam (in place) -------------------------------------------------------------
    def fused_adam(self, param, grad, exp_avg, exp_avg_sq, valid, n_gauss, lr, b1=0.9, b2=0.999, eps=1e-8):
        a = AdamInputs(ptr(param), ptr(f32(grad)), ptr(exp_avg), ptr(exp_avg_sq), ptr(u8(valid)),
                       param.size, n_gauss, lr, b1, b2, eps)
        self._call("fused_adam", C.byref(a))

    # -- projection --------------------------------------------------------------------------
    def _proj_in(self, means, viewmats, Ks, width, height, covars=None, quats=None, scales=None,
                 opacities=None, eps2d=0.3, near_plane=0.01, far_plane=1e10, radius_clip=0.0,
                 camera_model=0, calc_compensations=False):
        keep = [f32(means), f32(covars), f32(quats), f32(scales), f32(opacities), f32(viewmats), f32(Ks)]
        N = keep[0].shape[0] if keep[0] is not None else 0
        Cn = keep[5].reshape(-1, 16).shape[0]
        p = ProjectionInputs(*(ptr(k) for k in keep), N, Cn, width, height, eps2d, near_plane, far_plane,
                             radius_clip, camera_model, int(bool(calc_compensations)))
        return p, keep, N, Cn

    def projection_fused_fwd(self, **kw):
        p, keep, N, Cn = self._proj_in(**kw)
        radii = np.zeros((Cn, N, 2), np.int32)
        means2d = np.zeros((Cn, N, 2), np.float32)
        depths = np.zeros((Cn, N), np.float32)
        conics = np.zeros((Cn, N, 3), np.float32)
        comps = np.zeros((Cn, N), np.float32) if kw.get("calc_compensations") else None
        o = ProjectionOutputs(ptr(radii), ptr(means2d), ptr(depths), ptr(conics), ptr(comps))
        self._call("projection_fused_fwd", C.byref(p), C.byref(o))
        return dict(radii=radii, means2d=means2d, depths=depths, conics=conics, compensations=comps)

    def projection_fused_bwd(self, radii, conics, v_means2d, v_depths, v_conics, compensations=None,
                             v_compensations=None, viewmats_grad=False, **kw):
        p, keep, N, Cn = self._proj_in(**kw)
        g_keep = [i32(radii), f32(conics), f32(compensations), f32(v_means2d), f32(v_depths), f32(v_conics),
                  f32(v_compensations)]
        g = ProjectionGradsIn(*(ptr(k) for k in g_keep), int(bool(viewmats_grad)))
        use_cov = kw.get("covars") is not None
        v_means = np.zeros((N, 3), np.float32)
        v_covars = np.zeros((N, 6), np.float32) if use_cov else None
        v_quats = None if use_cov else np.zeros((N, 4), np.float32)
        v_scales = None if use_cov else np.zeros((N, 3), np.float32)
        v_view = np.zeros((Cn, 16), np.float32) if viewmats_grad else None
        o = ProjectionGrads(ptr(v_means), ptr(v_covars), ptr(v_quats), ptr(v_scales), ptr(v_view))
        self._call("projection_fused_bwd", C.byref(p), C.byref(g), C.byref(o))
        return dict(v_means=v_means, v_covars=v_covars, v_quats=v_quats, v_scales=v_scales, v_viewmats=v_view)

    # -- SH ----------------------------------------------------------------------------------
    def _sh_in(self, dirs, coeffs, degrees_to_use, masks=None, B=1, compute_v_dirs=False):
        keep = [f32(dirs), f32(coeffs), u8(masks)]
        N, K, D = keep[1].shape
        s = ShInputs(ptr(keep[0]), ptr(keep[1]), ptr(keep[2]), degrees_to_use, B, N, K, D,
                     int(bool(compute_v_dirs)))
        return s, keep, N, K, D

    def sh_fwd(self, dirs, coeffs, degrees_to_use, masks=None, B=1):
        s, keep, N, K, D = self._sh_in(dirs, coeffs, degrees_to_use, masks, B)
        colors = np.zeros((B * N, D), np.float32)
        self._call("sh_fwd", C.byref(s), ptr(colors))
        return colors

    def sh_bwd(self, dirs, coeffs, degrees_to_use, v_colors, masks=None, B=1, compute_v_dirs=True):
        s, keep, N, K, D = self._sh_in(dirs, coeffs, degrees_to_use, masks, B, compute_v_dirs)
        vc = f32(v_colors)
        v_coeffs = np.zeros((N, K, D), np.float32)
        v_dirs = np.zeros((B * N, 3), np.float32) if compute_v_dirs else None
        self._call("sh_bwd", C.byref(s), ptr(vc), ptr(v_coeffs), ptr(v_dirs))
        return dict(v_coeffs=v_coeffs, v_dirs=v_dirs)

    # -- isect / scan / sort / offsets -----------------------------------------------------------
    def isect_tiles(self, means2d, radii, depths, I, N, tile_width, tile_height, conics=None,
                    opacities=None, tile_size=16):
        keep = [f32(means2d), i32(radii), f32(depths), f32(conics), f32(opacities)]
        i = IsectInputs(ptr(keep[0]), ptr(keep[1]), ptr(keep[2]), ptr(keep[3]), ptr(keep[4]), I, N,
                        tile_size, tile_width, tile_height)
        tiles = np.zeros(I * N, np.int32)
        o = IsectOutputs(ptr(tiles), None, None, 0, 0, 0, 0)
        try:
            self._call("isect_tiles", C.byref(i), C.byref(o))
        except SxCapacityError:
            pass
        n = int(o.n_isects)
        ids = np.zeros(n, np.uint64)
        flat = np.zeros(n, np.int32)
        if n > 0:
            o = IsectOutputs(ptr(tiles), ptr(ids), ptr(flat), n, 0, 0, 0)
            self._call("isect_tiles", C.byref(i), C.byref(o))
        return dict(tiles_per_gauss=tiles, isect_ids=ids, flatten_ids=flat, n_isects=n,
                    tile_n_bits=int(o.tile_n_bits), image_n_bits=int(o.image_n_bits))

    def prefix_scan_i64(self, x):
        x = i32(x)
        out = np.zeros(x.size, np.int64)
        self._call("prefix_scan_i64", ptr(x), x.size, ptr(out))
        return out

    def sort_isect(self, keys, values, key_n_bits=64):
        keys, values = u64(keys), i32(values)
        n = keys.size
        ks = np.zeros(n, np.uint64)
        vs = np.zeros(n, np.int32)
        s = SortInputs(ptr(keys), ptr(values), n, key_n_bits)
        self._call("sort_isect", C.byref(s), ptr(ks), ptr(vs))
        return ks, vs

    def isect_offset_encode(self, isect_ids, I, tile_width, tile_height, n_isects=None):
        ids = u64(isect_ids)
        n = ids.size if n_isects is None else n_isects
        off = np.zeros(I * tile_width * tile_height, np.int32)
        s = OffsetInputs(ptr(ids), n, I, tile_width, tile_height)
        self._call("isect_offset_encode", C.byref(s), ptr(off))
        return off

    # -- raster --------------------------------------------------------------------------------
    def _raster_in(self, means2d, conics, colors, opacities, isect_offsets, flatten_ids, I, N, n_isects,
                   width, height, tile_width, tile_height, backgrounds=None, masks=None, tile_size=16):
        keep = [f32(means2d), f32(conics), f32(colors), f32(opacities), f32(backgrounds), u8(masks),
                i32(isect_offsets), i32(flatten_ids)]
        r = RasterInputs(*(ptr(k) for k in keep), I, N, n_isects, width, height, tile_size, tile_width,
                         tile_height)
        return r, keep

    def rasterize_fwd(self, **kw):
        r, keep = self._raster_in(**kw)
        I, H, W = kw["I"], kw["height"], kw["width"]
        rc = np.zeros((I, H, W, 3), np.float32)
        ra = np.zeros((I, H, W, 1), np.float32)
        li = np.zeros((I, H, W), np.int32)
        o = RasterOutputs(ptr(rc), ptr(ra), ptr(li))
        self._call("rasterize_fwd", C.byref(r), C.byref(o))
        return dict(render_colors=rc, render_alphas=ra, last_ids=li)

    def rasterize_bwd(self, render_alphas, last_ids, v_render_colors, v_render_alphas, absgrad=False, **kw):
        r, keep = self._raster_in(**kw)
        I, N = kw["I"], kw["N"]
        gk = [f32(render_alphas), i32(last_ids), f32(v_render_colors), f32(v_render_alphas)]
        g = RasterGradsIn(*(ptr(k) for k in gk), int(bool(absgrad)))
        out = dict(v_means2d=np.zeros((I * N, 2), np.float32), v_conics=np.zeros((I * N, 3), np.float32),
                   v_colors=np.zeros((I * N, 3), np.float32), v_opacities=np.zeros(I * N, np.float32),
                   v_means2d_abs=np.zeros((I * N, 2), np.float32) if absgrad else None)
        o = RasterGrads(ptr(out["v_means2d"]), ptr(out["v_conics"]), ptr(out["v_colors"]),
                        ptr(out["v_opacities"]), ptr(out["v_means2d_abs"]))
        self._call("rasterize_bwd", C.byref(r), C.byref(g), C.byref(o))
        return out

    # -- RNG / MCMC ---------------------------------------------------------------------------
    def rng_normal_f32(self, seed, offset, count):
        out = np.zeros(count, np.float32)
        self._call("rng_normal_f32", C.byref(RngInputs(seed, offset, count)), ptr(out))
        return out

    def rng_philox_u32(self, seed, offset, count):
        out = np.zeros(count, np.uint32)
        self._call("rng_philox_u32", C.byref(RngInputs(seed, offset, count)), ptr(out))
        return out

    def mcmc_relocation(self, opacities, scales, ratios, binoms, n_max=51, min_opacity=0.005):
        keep = [f32(opacities), f32(scales), i32(ratios), f32(binoms)]
        N = keep[0].size
        r = RelocationInputs(ptr(keep[0]), ptr(keep[1]), ptr(keep[2]), ptr(keep[3]), N, n_max, min_opacity)
        no = np.zeros(N, np.float32)
        ns = np.zeros((N, 3), np.float32)
        self._call("mcmc_relocation", C.byref(r), ptr(no), ptr(ns))
        return no, ns

    def mcmc_perturb_positions(self, positions, quats, scales_log, opacities_logit, noise, noise_scale,
                               t=0.005, k=100.0):
        keep = [f32(quats), f32(scales_log), f32(opacities_logit), f32(noise)]
        p = PerturbInputs(ptr(positions), *(ptr(x) for x in keep), positions.shape[0], noise_scale, t, k)
        self._call("mcmc_perturb_positions", C.byref(p))

    # -- SSIM ----------------------------------------------------------------------------------
    def ssim_fwd(self, img1, img2, need_coeffs=False):
        a, b = f32(img1), f32(img2)
        I, H, W, Cc = a.shape
        s = SsimInputs(ptr(a), ptr(b), I, H, W, Cc, int(bool(need_coeffs)))
        shp = (I, max(H - 10, 0), max(W - 10, 0), Cc)
        smap = np.zeros(shp, np.float32)
        co = [np.zeros(shp, np.float32) for _ in range(3)] if need_coeffs else [None] * 3
        o = SsimOutputs(0.0, ptr(smap), *(ptr(c) for c in co))
        self._call("ssim_fwd", C.byref(s), C.byref(o))
        return dict(ssim=float(o.ssim), ssim_map=smap, coeff_mu=co[0], coeff_sigma=co[1], coeff_cross=co[2])

    def ssim_bwd(self, img1, img2, coeff_mu, coeff_sigma, coeff_cross, v_loss=1.0):
        a, b = f32(img1), f32(img2)
        I, H, W, Cc = a.shape
        s = SsimInputs(ptr(a), ptr(b), I, H, W, Cc, 1)
        keep = [f32(coeff_mu), f32(coeff_sigma), f32(coeff_cross)]
        g = SsimGradsIn(*(ptr(k) for k in keep), v_loss)
        out = np.zeros_like(a)
        self._call("ssim_bwd", C.byref(s), C.byref(g), ptr(out))
        return out


def load_library(path: str = LIB_PATH):
    if not os.path.exists(path):
        raise SxRuntimeError(f"splatx HIP library not built: {path} (run __graft_entry__.build())")
    lib = C.CDLL(path)
    lib.sxh_last_error.restype = C.c_char_p
    return lib


class Backend(Ops):
    """The gfx950 backend (replaces make_metal_backend, MetalBackend.h:38-57)."""

    def __init__(self, device_ordinal: int = 0, lib=None):
        lib = lib or load_library()
        h = C.c_void_p()
        lib.sxh_backend_create.restype = C.c_int32
        lib.sxh_backend_create.argtypes = [C.c_int32, C.POINTER(C.c_void_p)]
        lib.sxh_last_error.restype = C.c_char_p
        rc = lib.sxh_backend_create(device_ordinal, C.byref(h))
        if rc != SXH_OK:
            raise SxRuntimeError(lib.sxh_last_error().decode())
        super().__init__(lib, "sxh_", handle=h)
        lib.sxh_backend_destroy.argtypes = [C.c_void_p]
        lib.sxh_backend_name.restype = C.c_char_p
        lib.sxh_backend_name.argtypes = [C.c_void_p]

    def name(self) -> str:
        return self.lib.sxh_backend_name(self.handle).decode()

    def close(self):
        if self.handle is not None:
            self.lib.sxh_backend_destroy(self.handle)
            self.handle = None

    def make_binoms_lut(self, n_max=51):
        out = np.zeros(n_max * n_max, np.float32)
        f = self.lib.sxh_make_binoms_lut
        f.restype = C.c_int32
        if f(n_max, ptr(out)) != SXH_OK:
            raise SxInvalidArgument(self.lib.sxh_last_error().decode())
        return out

    def make_train_step_executor(self, **desc) -> "Executor":
        return Executor(self, **desc)

    def running_sum_f64(self, w):
        """The multinomial's left-to-right f64 running sum on the device (sxh_running_sum_f64)."""
        w = f32(w).ravel()
        out = np.zeros(w.size, np.float64)
        self._call("running_sum_f64", ptr(w), C.c_int64(w.size), out.ctypes.data_as(C.POINTER(C.c_double)))
        return out

    def mt64_draw(self, st: MtState, n: int):
        """n draws of std::mt19937_64 on the device (sxh_mt64_draw); `st` advanced in place."""
        out = np.zeros(n, np.uint64)
        self._call("mt64_draw", C.byref(st), C.c_int64(n), ptr(out))
        return out

    def render_session(self, ply_path, antialiased=False, sh_degree=0) -> "RenderSession":
        return RenderSession(self, ply_path, antialiased, sh_degree)

    def mt64_seed(self, seed: int) -> MtState:
        """std::mt19937_64(seed) state (sxh_mt64_seed)."""
        st = MtState()
        f = self.lib.sxh_mt64_seed
        f.restype = C.c_int32
        f.argtypes = [C.c_uint64, C.POINTER(MtState)]
        if f(seed, C.byref(st)) != SXH_OK:
            raise SxInvalidArgument(self.lib.sxh_last_error().decode())
        return st


GROUP_DIMS = lambda sh_degree: [3, 4, 3, 1, 3, ((sh_degree + 1) ** 2 - 1) * 3]


class Executor:
    """Resident train-step executor (TrainStepExecutor, KernelBackend.h:386-392)."""

    def __init__(self, backend: Backend, arena_rows: int, sh_degree: int = 3, eps2d=0.3, near_plane=0.01,
                 far_plane=1e10, radius_clip=0.0, b1=0.9, b2=0.999, eps=1e-15, ssim_weight=0.2,
                 antialiased=False, isect_mode=SXH_ISECT_ACCUTILE):
        self.b = backend
        self.lib = backend.lib
        self.sh_degree = sh_degree
        self.arena_rows = arena_rows
        d = ExecDesc(arena_rows, sh_degree, eps2d, near_plane, far_plane, radius_clip, b1, b2, eps,
                     ssim_weight, int(bool(antialiased)), isect_mode)
        h = C.c_void_p()
        self.lib.sxh_exec_create.restype = C.c_int32
        self.lib.sxh_exec_create.argtypes = [C.c_void_p, C.POINTER(ExecDesc), C.POINTER(C.c_void_p)]
        self._check(self.lib.sxh_exec_create(backend.handle, C.byref(d), C.byref(h)))
        self.h = h
        for n in ("sxh_exec_upload", "sxh_exec_download", "sxh_exec_step", "sxh_exec_set_gt_cache",
                  "sxh_exec_render_to_gt_cache", "sxh_exec_set_profiling", "sxh_exec_get_timing", "sxh_exec_set_graph",
                  "sxh_exec_set_isect_order", "sxh_exec_set_row_order", "sxh_exec_mcmc_refine", "sxh_exec_sync"):
            getattr(self.lib, n).restype = C.c_int32
        self.lib.sxh_exec_destroy.argtypes = [C.c_void_p]

    def _check(self, rc):
        if rc != SXH_OK:
            msg = self.lib.sxh_last_error().decode(errors="replace")
            if rc == SXH_ERR_INVALID_ARGUMENT:
                raise SxInvalidArgument(msg)
            if rc == SXH_ERR_CAPACITY:
                raise SxCapacityError(msg)
            raise SxRuntimeError(msg)

    def close(self):
        if self.h is not None:
            self.lib.sxh_exec_destroy(self.h)
            self.h = None

    def _sync(self, params, exp_avg, exp_avg_sq, rows):
        """ParamSync over the caller's arrays. The library copies rows * dim floats per group from or
        into each array, so every array given must hold at least that many elements."""
        s = ParamSync()
        dims = GROUP_DIMS(self.sh_degree)
        for g in range(6):
            for name, arrs, field in (("params", params, s.params), ("exp_avg", exp_avg, s.exp_avg),
                                      ("exp_avg_sq", exp_avg_sq, s.exp_avg_sq)):
                a = arrs[g]
                if a is not None and a.size:
                    if a.size < rows * dims[g]:
                        raise ValueError(f"{name}[{g}] holds {a.size} floats; rows * dim = {rows * dims[g]}")
                    field[g] = ptr(a)
                else:
                    field[g] = None
        s.rows = rows
        return s

    def upload_params(self, params, exp_avg, exp_avg_sq, rows):
        s = self._sync(params, exp_avg, exp_avg_sq, rows)
        self._check(self.lib.sxh_exec_upload(self.h, C.byref(s)))

    def download_params(self, params, exp_avg, exp_avg_sq, rows):
        s = self._sync(params, exp_avg, exp_avg_sq, rows)
        self._check(self.lib.sxh_exec_download(self.h, C.byref(s)))

    def make_step_inputs(self, viewmat, K, width, height, count, degrees_to_use, lr, gt_rgb=None,
                         gt_index=-1, opacity_reg_w=0.0, scale_reg_w=0.0, forward_only=False,
                         inject_noise=False, noise_seed=0, noise_offset=0, noise_scale=0.0):
        keep = [f32(viewmat), f32(K), f32(gt_rgb)]
        if keep[0].size != 16 or keep[1].size != 9:
            raise ValueError("viewmat must hold 16 floats and K 9")
        if gt_rgb is not None and keep[2].size != width * height * 3:
            raise ValueError(f"gt_rgb holds {keep[2].size} floats; width * height * 3 = {width * height * 3}")
        s = StepInputs(ptr(keep[0]), ptr(keep[1]), width, height, ptr(keep[2]), gt_index, count,
                       degrees_to_use, (C.c_float * 6)(*lr), opacity_reg_w, scale_reg_w,
                       int(bool(forward_only)), int(bool(inject_noise)), noise_seed, noise_offset,
                       noise_scale)
        return s, keep

    def step(self, want_render=False, **kw):
        s, keep = self.make_step_inputs(**kw)
        render = np.zeros((kw["height"], kw["width"], 3), np.float32) if want_render else None
        o = StepOutputs(0.0, 0, 0, ptr(render))
        self._check(self.lib.sxh_exec_step(self.h, C.byref(s), C.byref(o)))
        return dict(loss=float(o.loss), n_isects=int(o.n_isects), n_visible=int(o.n_visible),
                    render_colors=render)

    def step_raw(self, s: StepInputs, o: StepOutputs):
        return self.lib.sxh_exec_step(self.h, C.byref(s), C.byref(o))

    def set_gt_cache(self, images: np.ndarray):
        images = f32(images)
        n, h, w, _ = images.shape
        self._check(self.lib.sxh_exec_set_gt_cache(self.h, ptr(images), n, w, h))

    def render_to_gt_cache(self, index, **kw):
        s, keep = self.make_step_inputs(**kw)
        self._check(self.lib.sxh_exec_render_to_gt_cache(self.h, C.byref(s), index))

    def mcmc_refine(self, count, cap_max, rng: MtState, binoms, min_opacity=0.005, n_max=51, inject_noise=False,
                    noise_seed=0, noise_offset=0, noise_scale=0.0, want_lists=False, capacity=None):
        """Trainer::mcmc_refine on the arena (sxh_exec_mcmc_refine); `rng` is advanced in place."""
        binoms = f32(binoms)
        i = RefineInputs(count, cap_max, min_opacity, n_max, ptr(binoms), C.pointer(rng), int(bool(inject_noise)),
                         noise_seed, noise_offset, noise_scale)
        lists = None
        o = RefineOutputs()
        if want_lists:
            cap = self.arena_rows if capacity is None else capacity
            lists = [np.zeros(max(cap, 1), np.int64) for _ in range(3)]
            o.relocated_dead, o.relocation_src, o.added_src = (ptr(a) for a in lists)
            o.capacity = cap
        self._check(self.lib.sxh_exec_mcmc_refine(self.h, C.byref(i), C.byref(o)))
        return refine_lists(o, lists)

    def export_ply(self, count, path, min_opacity=0.005, pad_sh_full=True):
        """filter_cloud_for_export + write_inria_ply of the live rows (sxh_exec_export_ply)."""
        st = ExportStats()
        f = self.lib.sxh_exec_export_ply
        f.restype = C.c_int32
        self._check(f(self.h, C.c_int64(count), C.c_float(min_opacity), int(bool(pad_sh_full)), path.encode(),
                      C.byref(st)))
        return st.as_dict()

    def save_checkpoint(self, config: CkptConfig, iter, count, path, rng_state=None, fp16=False):
        f = self.lib.sxh_exec_save_checkpoint
        f.restype = C.c_int32
        rng = rng_state.encode() if rng_state else None
        self._check(f(self.h, C.byref(config), iter, C.c_int64(count), rng, int(bool(fp16)), path.encode()))

    def load_checkpoint(self, path, current: CkptConfig = None, rng_capacity=1 << 16):
        f = self.lib.sxh_exec_load_checkpoint
        f.restype = C.c_int32
        h = CkptHeader()
        buf = C.create_string_buffer(rng_capacity)
        self._check(f(self.h, path.encode(), C.byref(current) if current is not None else None, C.byref(h), buf,
                      C.c_int64(rng_capacity)))
        d = h.as_dict()
        d["rng_state"] = buf.value.decode()
        return d

    def train_schedule_defaults(self) -> TrainSchedule:
        s = TrainSchedule()
        f = self.lib.sxh_train_schedule_defaults
        f.restype = C.c_int32
        self._check(f(C.byref(s)))
        return s

    def train_loop(self, cameras, start_iter, run_until, count, schedule: TrainSchedule, rng: MtState = None,
                   binoms=None, n_max=51, eval_cameras=(), eval_every=0, jitter=None, progress=None,
                   snapshot=None, snapshot_every=0, live_ply_every=0, live_ply_path=None, checkpoint_every=0,
                   checkpoint_path=None, checkpoint_config: CkptConfig = None, checkpoint_fp16=False):
        """The caller loop (sxh_exec_train_loop) over `cameras` (TrainCamera, GT in the cache).
        progress(dict) is called at every step boundary; snapshot(dict of arrays) every
        snapshot_every steps; jitter = (max_deg, max_t, seed) or None. `rng` is advanced in place."""
        cams = (TrainCamera * len(cameras))(*cameras)
        ecams = (TrainCamera * max(1, len(eval_cameras)))(*eval_cameras) if eval_cameras else None
        a = TrainLoopArgs()
        a.cameras, a.n_cameras = cams, len(cameras)
        if ecams is not None:
            a.eval_cameras, a.n_eval_cameras = ecams, len(eval_cameras)
        a.eval_every = eval_every
        a.start_iter, a.run_until, a.count, a.sched = start_iter, run_until, count, schedule
        keep = []
        if binoms is not None:
            b = f32(binoms)
            keep.append(b)
            a.binoms, a.n_max = ptr(b), n_max
        if rng is not None:
            a.rng = C.pointer(rng)
        if jitter is not None:
            a.jitter_max_deg, a.jitter_max_t, a.jitter_seed = jitter
        if progress is not None:
            cb = PROGRESS_FN(lambda p, _u: progress(p.contents.as_dict()))
            keep.append(cb)
            a.progress = cb
        if snapshot is not None:
            def snap(sp, _u):
                s = sp.contents
                n = int(s.count)
                k = (s.sh_degree + 1) ** 2 - 1
                def arr(pp, dim):
                    return np.ctypeslib.as_array(pp, shape=(n, dim)).copy() if n and pp else np.zeros((n, dim), np.float32)
                snapshot(dict(iter=int(s.iter), sh_degree=int(s.sh_degree), count=n, means=arr(s.means, 3),
                              quats=arr(s.quats, 4), scales=arr(s.scales, 3), opacities=arr(s.opacities, 1)[:, 0],
                              sh0=arr(s.sh0, 3), shN=arr(s.shN, 3 * k) if k else None))
            cb = SNAPSHOT_FN(snap)
            keep.append(cb)
            a.snapshot, a.snapshot_every = cb, snapshot_every
        a.live_ply_every = live_ply_every
        a.live_ply_path = live_ply_path.encode() if live_ply_path else None
        a.checkpoint_every = checkpoint_every
        a.checkpoint_path = checkpoint_path.encode() if checkpoint_path else None
        if checkpoint_config is not None:
            a.checkpoint_config = C.pointer(checkpoint_config)
        a.checkpoint_fp16 = int(bool(checkpoint_fp16))
        out = TrainLoopResult()
        f = self.lib.sxh_exec_train_loop
        f.restype = C.c_int32
        self._check(f(self.h, C.byref(a), C.byref(out)))
        return out.as_dict()

    def request_stop(self):
        f = self.lib.sxh_exec_request_stop
        f.restype = C.c_int32
        self._check(f(self.h))

    def set_profiling(self, enable: bool, pair_stats: bool = False):
        """Per-kernel HIP-event times of each step (enable); with pair_stats also the rasterisers' pair
        counts (counting kernels: use the counts, not the times, of such steps)."""
        flags = (1 if enable else 0) | (2 if pair_stats else 0)
        self._check(self.lib.sxh_exec_set_profiling(self.h, flags))

    def get_raster_stats(self) -> dict:
        st = RasterStats()
        f = self.lib.sxh_exec_get_raster_stats
        f.restype = C.c_int32
        self._check(f(self.h, C.byref(st)))
        return {k: int(getattr(st, k)) for k, _ in RasterStats._fields_}

    def sync(self):
        """Wait until the executor's device work has finished (a step returns once its loss is read
        back, possibly before its parameter update completes on the device)."""
        self._check(self.lib.sxh_exec_sync(self.h))

    def set_graph(self, enable: bool):
        """Run the step's second segment as a captured hipGraph (default) or as direct launches."""
        self._check(self.lib.sxh_exec_set_graph(self.h, int(bool(enable))))

    def set_isect_order(self, mode: int):
        """SXH_ISECT_ORDER_AUTO (default), _DEPTH_FIRST or _INDEX_FIRST: how the step
        builds each tile's (depth, index)-ordered intersection list (the same lists either way)."""
        self._check(self.lib.sxh_exec_set_isect_order(self.h, int(mode)))

    def set_row_order(self, mode: int):
        """SXH_ROW_ORDER_SPATIAL_AUTO (default), _ORIGINAL or _SPATIAL: the order in which the executor keeps
        the live rows in HBM (the same results in every mode)."""
        self._check(self.lib.sxh_exec_set_row_order(self.h, int(mode)))

    def get_timing(self):
        t = ExecTiming()
        self._check(self.lib.sxh_exec_get_timing(self.h, C.byref(t)))
        return {t.names[i].decode(): float(t.ms[i]) for i in range(t.n)}
