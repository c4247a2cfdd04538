"""The boundary's error contract: the reference's negative-case table for its shared validators
(Sources/SplatXTests/ValidateTests.cpp:173-420 over Validate.h:40-267), run through the C ABI.

Each case mutates one field of a valid baseline input (the reference's baselines, ValidateTests.cpp:34-
168) and calls the per-op entry point; it must fail with the reference's status (SXH_ERR_INVALID_ARGUMENT
for std::invalid_argument, SXH_ERR_RUNTIME for the projection's camera model, which the reference
throws as std::runtime_error) and a message that starts with the op name and holds the reference's
substring. The entry points validate their inputs before they look at the backend, so:
- on the CPU, with a null backend, every unmutated baseline gets past validation and fails only on
  the missing backend ("null backend"), and every mutation fails on its own check;
- on the GPU, with a real backend, every mutation fails before any device work.
The pointers are small host arrays; the validators only test them for null.
The readback guard of the resident step (validate_n_isects_readback, ValidateTests.cpp:421-470) is
compiled from the library's header into a small host program and checked on the same boundaries.
"""
import ctypes as C
import os
import shutil
import subprocess

import numpy as np
import pytest

import splatx_hip as sh

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INT32_MAX = 2 ** 31 - 1
UINT32_MAX = 2 ** 32 - 1

_keep = []


def buf(dtype, n=64):
    a = np.zeros(n, dtype)
    _keep.append(a)
    return a


F = sh.ptr(buf(np.float32))
I32 = sh.ptr(buf(np.int32))
U64 = sh.ptr(buf(np.uint64))
U32 = sh.ptr(buf(np.uint32))
NULL_F = sh.fp()
NULL_I32 = sh.i32p()
NULL_U64 = sh.u64p()


# ---- the reference's valid baselines (ValidateTests.cpp:34-168) ---------------------------------
def adam_ok():
    return sh.AdamInputs(param=F, grad=F, exp_avg=F, exp_avg_sq=F, n_elems=6, n_gauss=2, lr=1e-3, b1=0.9,
                         b2=0.999, eps=1e-8)


def proj_ok():
    return sh.ProjectionInputs(means=F, quats=F, scales=F, viewmats=F, Ks=F, N=4, C=1, width=160, height=120,
                               eps2d=0.3, near_plane=0.01, far_plane=1e10)


def grads_ok():
    return sh.ProjectionGradsIn(radii=I32, conics=F, v_means2d=F, v_depths=F, v_conics=F)


def sh_ok():
    return sh.ShInputs(dirs=F, coeffs=F, degrees_to_use=3, B=1, N=4, K=16, D=3)


def isect_ok():
    return sh.IsectInputs(means2d=F, radii=I32, depths=F, I=1, N=4, tile_size=16, tile_width=10, tile_height=8)


def sort_ok():
    return sh.SortInputs(keys=U64, values=I32, n=1, key_n_bits=36)


def offset_ok():
    return sh.OffsetInputs(isect_ids=U64, n_isects=1, I=1, tile_width=10, tile_height=8)


def rast_ok():
    return sh.RasterInputs(means2d=F, conics=F, colors=F, opacities=F, isect_offsets=I32, flatten_ids=I32, I=1, N=4,
                           n_isects=1, image_width=160, image_height=120, tile_size=16, tile_width=10, tile_height=8)


def rast_bwd_ok():
    return sh.RasterGradsIn(render_alphas=F, last_ids=I32, v_render_colors=F, v_render_alphas=F)


def rng_ok():
    return sh.RngInputs(seed=1, offset=2, count=8)


def reloc_ok():
    return sh.RelocationInputs(opacities=F, scales=F, ratios=I32, binoms=F, N=4, n_max=51, min_opacity=0.005)


def perturb_ok():
    return sh.PerturbInputs(positions=F, quats=F, scales_log=F, opacities_logit=F, noise=F, N=4, noise_scale=1.0,
                            t=0.005, k=100.0)


def ssim_ok():
    return sh.SsimInputs(img1=F, img2=F, I=1, H=24, W=24, C=3, need_coeffs=1)


def ssim_grads_ok():
    return sh.SsimGradsIn(coeff_mu=F, coeff_sigma=F, coeff_cross=F, v_loss=1.0)


# ---- calls through the C ABI ---------------------------------------------------------------------
def call(lib, b, op, *structs, extra=()):
    f = getattr(lib, "sxh_" + op)
    f.restype = C.c_int32
    args = [b] + [C.byref(s) if s is not None else None for s in structs] + list(extra)
    rc = f(*args)
    return rc, lib.sxh_last_error().decode(errors="replace")


def proj_out():
    return sh.ProjectionOutputs(radii=I32, means2d=F, depths=F, conics=F, compensations=F)


def run(lib, b, op, a=None, g=None):
    """One entry point with the given inputs (the others at their baselines)."""
    if op == "fused_adam":
        return call(lib, b, op, a or adam_ok())
    if op == "projection_fused_fwd":
        return call(lib, b, op, a or proj_ok(), proj_out())
    if op == "projection_fused_bwd":
        out = sh.ProjectionGrads(v_means=F, v_quats=F, v_scales=F)
        return call(lib, b, op, a or proj_ok(), g or grads_ok(), out)
    if op == "sh_fwd":
        return call(lib, b, op, a or sh_ok(), extra=(F,))
    if op == "isect_tiles":
        out = sh.IsectOutputs(tiles_per_gauss=I32, isect_ids=U64, flatten_ids=I32, capacity=64)
        return call(lib, b, op, a or isect_ok(), out)
    if op == "sort_isect":
        return call(lib, b, op, a or sort_ok(), extra=(U64, I32))
    if op == "isect_offset_encode":
        return call(lib, b, op, a or offset_ok(), extra=(I32,))
    if op == "rasterize_fwd":
        return call(lib, b, op, a or rast_ok(), sh.RasterOutputs(render_colors=F, render_alphas=F, last_ids=I32))
    if op == "rasterize_bwd":
        out = sh.RasterGrads(v_means2d=F, v_conics=F, v_colors=F, v_opacities=F)
        return call(lib, b, op, a or rast_ok(), g or rast_bwd_ok(), out)
    if op == "rng_normal_f32":
        return call(lib, b, op, a or rng_ok(), extra=(F,))
    if op == "rng_philox_u32":
        return call(lib, b, op, a or rng_ok(), extra=(U32,))
    if op == "mcmc_relocation":
        return call(lib, b, op, a or reloc_ok(), extra=(F, F))
    if op == "mcmc_perturb_positions":
        return call(lib, b, op, a or perturb_ok())
    if op == "ssim_fwd":
        out = sh.SsimOutputs(ssim_map=F, coeff_mu=F, coeff_sigma=F, coeff_cross=F)
        return call(lib, b, op, a or ssim_ok(), out)
    if op == "ssim_bwd":
        return call(lib, b, op, a or ssim_ok(), g or ssim_grads_ok(), extra=(F,))
    raise KeyError(op)


def mut(factory, **fields):
    s = factory()
    for k, v in fields.items():
        setattr(s, k, v)
    return s


INV, RT = sh.SXH_ERR_INVALID_ARGUMENT, sh.SXH_ERR_RUNTIME

# (name, op, inputs, grads-in, expected message substring, expected status)
CASES = [
    # general-purpose primitives (validate_nonnull, validate_range_u32)
    ("nonnull", "sort_isect", "null-inputs", None, "null inputs", INV),
    ("range_u32", "sort_isect", mut(sort_ok, key_n_bits=65), None, "key_n_bits must be 1..64", INV),
    # validate_adam_inputs
    ("adam null tensor", "fused_adam", mut(adam_ok, grad=NULL_F), None, "null tensor", INV),
    ("adam n_elems % n_gauss", "fused_adam", mut(adam_ok, n_elems=5), None,
     "n_elems must be a positive multiple of n_gauss", INV),
    ("adam n_gauss <= 0", "fused_adam", mut(adam_ok, n_gauss=0), None, "positive multiple of n_gauss", INV),
    # validate_projection_fused_inputs
    ("proj camera_model", "projection_fused_fwd", mut(proj_ok, camera_model=2), None,
     "only PINHOLE (camera_model=0) supported", RT),
    ("proj null means", "projection_fused_fwd", mut(proj_ok, means=NULL_F), None, "null means/viewmats/Ks", INV),
    ("proj no covar path", "projection_fused_fwd", mut(proj_ok, quats=NULL_F), None,
     "need covars (6-triu) or quats+scales", INV),
    ("proj negative N", "projection_fused_fwd", mut(proj_ok, N=-1), None, "negative N or C", INV),
    # validate_projection_fused_grads_in
    ("grads null radii", "projection_fused_bwd", None, mut(grads_ok, radii=NULL_I32),
     "null radii/conics/v_means2d/v_depths/v_conics", INV),
    ("grads v_comp without comp", "projection_fused_bwd", None, mut(grads_ok, v_compensations=F),
     "v_compensations requires compensations", INV),
    # validate_sh_inputs
    ("sh null dirs", "sh_fwd", mut(sh_ok, dirs=NULL_F), None, "null dirs/coeffs", INV),
    ("sh negative B", "sh_fwd", mut(sh_ok, B=-1), None, "negative B or N", INV),
    ("sh K < 1", "sh_fwd", mut(sh_ok, K=0), None, "K and D must be positive", INV),
    ("sh degrees > 4", "sh_fwd", mut(sh_ok, degrees_to_use=5), None, "degrees_to_use must be 0..4", INV),
    ("sh bands^2 > K", "sh_fwd", mut(sh_ok, degrees_to_use=4), None, "(degrees_to_use+1)^2 must be <= K", INV),
    # validate_isect_tiles_inputs
    ("isect null means2d", "isect_tiles", mut(isect_ok, means2d=NULL_F), None, "null means2d/radii/depths", INV),
    ("isect conics without opacities", "isect_tiles", mut(isect_ok, conics=F), None,
     "conics and opacities must be given together", INV),
    ("isect negative I", "isect_tiles", mut(isect_ok, I=-1), None, "negative I or N", INV),
    ("isect tile_size 0", "isect_tiles", mut(isect_ok, tile_size=0), None,
     "tile_size/tile_width/tile_height must be positive", INV),
    ("isect bit budget", "isect_tiles", mut(isect_ok, I=1 << 20, tile_width=4096, tile_height=4096), None,
     "image_n_bits + tile_n_bits must be <= 32", INV),
    ("isect I*N overflow", "isect_tiles", mut(isect_ok, I=1 << 30, N=4, tile_width=1, tile_height=1), None,
     "I*N must fit in int32", INV),
    # validate_sort_isect_inputs
    ("sort negative n", "sort_isect", mut(sort_ok, n=-1), None, "negative n", INV),
    ("sort null keys", "sort_isect", mut(sort_ok, keys=NULL_U64), None, "null keys/values", INV),
    ("sort n > int32", "sort_isect", mut(sort_ok, n=INT32_MAX + 1), None, "n must fit in int32", INV),
    ("sort key_n_bits 0", "sort_isect", mut(sort_ok, key_n_bits=0), None, "key_n_bits must be 1..64", INV),
    # validate_isect_offset_inputs
    ("offset negative n_isects", "isect_offset_encode", mut(offset_ok, n_isects=-1), None, "negative n_isects", INV),
    ("offset null isect_ids", "isect_offset_encode", mut(offset_ok, isect_ids=NULL_U64), None, "null isect_ids",
     INV),
    ("offset negative I", "isect_offset_encode", mut(offset_ok, I=-1), None, "negative I", INV),
    ("offset I == 0", "isect_offset_encode", mut(offset_ok, I=0), None, "n_isects > 0 requires I > 0", INV),
    ("offset tile_width 0", "isect_offset_encode", mut(offset_ok, tile_width=0), None,
     "tile_width/tile_height must be positive", INV),
    ("offset bit budget", "isect_offset_encode", mut(offset_ok, I=1 << 20, tile_width=4096, tile_height=4096),
     None, "image_n_bits + tile_n_bits must be <= 32", INV),
    ("offset n_isects > int32", "isect_offset_encode",
     mut(offset_ok, n_isects=INT32_MAX + 1, tile_width=1, tile_height=1), None, "n_isects must fit in int32", INV),
    ("offset I*n_tiles overflow", "isect_offset_encode", mut(offset_ok, I=1 << 20, tile_width=64, tile_height=64),
     None, "I*n_tiles must fit in int32", INV),
    # validate_rasterize_fwd_inputs
    ("rast null conics", "rasterize_fwd", mut(rast_ok, conics=NULL_F), None,
     "null means2d/conics/colors/opacities/isect_offsets", INV),
    ("rast null flatten_ids", "rasterize_fwd", mut(rast_ok, flatten_ids=NULL_I32), None, "null flatten_ids", INV),
    ("rast negative n_isects", "rasterize_fwd", mut(rast_ok, n_isects=-1), None, "negative I/N/n_isects", INV),
    ("rast n_isects without N", "rasterize_fwd", mut(rast_ok, N=0), None, "n_isects > 0 requires N > 0", INV),
    ("rast tile_size 4", "rasterize_fwd", mut(rast_ok, tile_size=4), None, "tile_size must be 16", INV),
    ("rast image 0", "rasterize_fwd", mut(rast_ok, image_width=0), None,
     "image_width/image_height must be positive", INV),
    ("rast grid uncovered", "rasterize_fwd", mut(rast_ok, tile_width=9), None, "tile grid must cover the image",
     INV),
    ("rast n_isects > int32", "rasterize_fwd", mut(rast_ok, n_isects=INT32_MAX + 1), None,
     "n_isects must fit in int32", INV),
    # validate_rasterize_bwd_inputs
    ("rast bwd fwd rule pass-through", "rasterize_bwd", mut(rast_ok, tile_size=4), None, "tile_size must be 16",
     INV),
    ("rast bwd null last_ids", "rasterize_bwd", None, mut(rast_bwd_ok, last_ids=NULL_I32),
     "null render_alphas/last_ids (fwd outputs)", INV),
    ("rast bwd null v_render", "rasterize_bwd", None, mut(rast_bwd_ok, v_render_alphas=NULL_F),
     "null v_render_colors/v_render_alphas", INV),
    # validate_rng_inputs
    ("rng negative count", "rng_normal_f32", mut(rng_ok, count=-1), None, "negative count", INV),
    ("rng count > uint32", "rng_normal_f32", mut(rng_ok, count=UINT32_MAX + 1), None, "count must fit in uint32",
     INV),
    # validate_relocation_inputs
    ("reloc null binoms", "mcmc_relocation", mut(reloc_ok, binoms=NULL_F), None,
     "null opacities/scales/ratios/binoms", INV),
    ("reloc negative N", "mcmc_relocation", mut(reloc_ok, N=-1), None, "negative N", INV),
    ("reloc n_max < 1", "mcmc_relocation", mut(reloc_ok, n_max=0), None, "n_max must be >= 1", INV),
    # validate_perturb_inputs
    ("perturb null noise", "mcmc_perturb_positions", mut(perturb_ok, noise=NULL_F), None,
     "null positions/quats/scales_log/opacities_logit/noise", INV),
    ("perturb negative N", "mcmc_perturb_positions", mut(perturb_ok, N=-1), None, "negative N", INV),
    ("perturb N > uint32", "mcmc_perturb_positions", mut(perturb_ok, N=UINT32_MAX + 1), None, "N exceeds uint32",
     INV),
    # SSIM validators (Validate.h, validate_ssim_inputs / validate_ssim_grads_in; not in the reference's table)
    ("ssim null img2", "ssim_fwd", mut(ssim_ok, img2=NULL_F), None, "null img1/img2", INV),
    ("ssim C 0", "ssim_fwd", mut(ssim_ok, C=0), None, "I and C must be positive", INV),
    ("ssim H < 11", "ssim_fwd", mut(ssim_ok, H=10), None, "H and W must be >= 11", INV),
    ("ssim bwd null coeffs", "ssim_bwd", None, mut(ssim_grads_ok, coeff_cross=NULL_F), "null coeff maps", INV),
]

OPS = sorted({c[1] for c in CASES})
REFERENCE_TABLE_SIZE = 53  # ValidateTests.cpp:196-362


def invoke(lib, b, case):
    name, op, a, g, _, _ = case
    if a == "null-inputs":
        f = getattr(lib, "sxh_" + op)
        f.restype = C.c_int32
        rc = f(b, None, U64, I32)
        return rc, lib.sxh_last_error().decode(errors="replace")
    return run(lib, b, op, a, g)


def check(case, rc, msg):
    name, op, _, _, expect, status = case
    assert rc == status, (name, rc, msg)
    assert msg.startswith(op + ": "), (name, msg)
    assert expect in msg, (name, msg, expect)


@pytest.fixture(scope="module")
def lib():
    return sh.load_library()


def test_table_covers_the_reference_cases():
    assert len([c for c in CASES if not c[0].startswith("ssim")]) == REFERENCE_TABLE_SIZE


@pytest.mark.parametrize("op", OPS)
def test_baselines_pass_validation(lib, op):
    """An unmutated baseline gets through validation and stops only at the null backend."""
    rc, msg = run(lib, None, op)
    assert rc == sh.SXH_ERR_INVALID_ARGUMENT and msg == f"{op}: null backend", (op, rc, msg)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_negative_case_null_backend(lib, case):
    rc, msg = invoke(lib, None, case)
    check(case, rc, msg)


@pytest.mark.gpu
def test_negative_table_with_backend(gpu):
    """The whole table against a live backend: every mutation fails before any device work, and the
    backend keeps working afterwards."""
    b = gpu.handle
    for case in CASES:
        print(f"case: {case[0]}", flush=True)
        rc, msg = invoke(gpu.lib, b, case)
        check(case, rc, msg)
    # the backend is unaffected: a valid call still runs
    out = gpu.rng_philox_u32(1, 2, 8)
    assert out.dtype == np.uint32 and out.size == 8


READBACK_PROGRAM = r"""
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include "sx_host.h"
namespace sxh { void set_last_error(const std::string&) {} }
int main() {
    int bad = 0;
    const int64_t ok[] = {0, 12345, INT32_MAX};
    for (int64_t v : ok)
        if (sxh::validate_n_isects_readback(v, "vt") != static_cast<uint32_t>(v)) bad++;
    struct Case { int64_t v; const char* expect; };
    const Case cases[] = {{-1, "negative n_isects"}, {int64_t{INT32_MAX} + 1, "n_isects must fit in int32"},
                          {int64_t{UINT32_MAX}, "n_isects must fit in int32"},
                          {int64_t{UINT32_MAX} + 1, "n_isects must fit in int32"}};
    for (const Case& c : cases) {
        try {
            (void)sxh::validate_n_isects_readback(c.v, "vt");
            std::printf("no throw for %lld\n", static_cast<long long>(c.v));
            bad++;
        } catch (const std::invalid_argument& e) {
            const std::string m = e.what();
            if (m.rfind("vt: ", 0) != 0 || m.find(c.expect) == std::string::npos) {
                std::printf("bad message for %lld: %s\n", static_cast<long long>(c.v), m.c_str());
                bad++;
            }
        }
    }
    std::printf("failures %d\n", bad);
    return bad == 0 ? 0 : 1;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None or not os.path.isdir("/opt/rocm/include"),
                    reason="needs g++ and the ROCm headers")
def test_n_isects_readback_guard(tmp_path):
    """validate_n_isects_readback (the step's sync-1 guard): 0, 12345 and INT32_MAX pass unchanged;
    negative values and everything past int32 (including the uint32 range) are rejected with the
    reference's message (ValidateTests.cpp:421-470)."""
    src = tmp_path / "readback.cpp"
    src.write_text(READBACK_PROGRAM)
    exe = tmp_path / "readback"
    cmd = ["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I", os.path.join(REPO, "include"), "-I", os.path.join(REPO, "splatx-metal_amd", "csrc"),
           str(src), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
