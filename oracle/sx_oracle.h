/*
 * sx_oracle.h — CPU oracle of the splatx 3DGS training step. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker (or the timed CPU baseline); the product path never calls it.
 *
 * The forward ops restate the reference CPU code (Sources/SplatXCore/CpuKernels.cpp, Math.cpp,
 * RngPhilox.h) op for op; the small step glue restates Trainer.cpp; the backward ops (raster, SH,
 * projection, SSIM), which the reference has no CPU version of, restate the reference kernels'
 * mathematics (Rasterize3DGSBwd.metal, SphericalHarmonics.metal, ProjectionEWA.metal, Ssim.metal)
 * in scalar C++. Every function takes the same structs as the product C ABI (include/splatx_hip.h).
 *
 * Transcendentals: built twice. liboracle.so uses the deterministic functions of
 * splatx-metal_amd/csrc/sx_fmath.h (so GPU and oracle can be compared bit for bit);
 * liboracle_libm.so uses glibc (std::exp/log/pow/sin/cos) exactly as the reference does. Both
 * variants are checked against the golden fixtures.
 *
 * Parity status per function (what pins it) is listed in sxo_pins below and in the tests.
 */
#ifndef SX_ORACLE_H
#define SX_ORACLE_H

#include <stdint.h>
#include "splatx_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

const char* sxo_last_error(void);
int32_t sxo_uses_libm(void);

int32_t sxo_fused_adam(const sxh_adam_inputs* in);
int32_t sxo_projection_fused_fwd(const sxh_projection_inputs* in, sxh_projection_outputs* out);
int32_t sxo_projection_fused_bwd(const sxh_projection_inputs* in, const sxh_projection_grads_in* gin,
                                 sxh_projection_grads* out);
int32_t sxo_sh_fwd(const sxh_sh_inputs* in, float* colors);
int32_t sxo_sh_bwd(const sxh_sh_inputs* in, const float* v_colors, float* v_coeffs, float* v_dirs);
int32_t sxo_isect_tiles(const sxh_isect_inputs* in, sxh_isect_outputs* out);
int32_t sxo_prefix_scan_i64(const int32_t* in, int64_t n, int64_t* out);
int32_t sxo_sort_isect(const sxh_sort_inputs* in, uint64_t* keys_sorted, int32_t* values_sorted);
int32_t sxo_isect_offset_encode(const sxh_offset_inputs* in, int32_t* offsets);
int32_t sxo_rasterize_fwd(const sxh_raster_inputs* in, sxh_raster_outputs* out);
int32_t sxo_rasterize_bwd(const sxh_raster_inputs* in, const sxh_raster_grads_in* gin,
                          sxh_raster_grads* out);
int32_t sxo_rng_normal_f32(const sxh_rng_inputs* in, float* out);
int32_t sxo_rng_philox_u32(const sxh_rng_inputs* in, uint32_t* out);
int32_t sxo_make_binoms_lut(int32_t n_max, float* out);
int32_t sxo_mcmc_relocation(const sxh_relocation_inputs* in, float* new_opacities, float* new_scales);
int32_t sxo_mcmc_perturb_positions(const sxh_perturb_inputs* in);
int32_t sxo_ssim_fwd(const sxh_ssim_inputs* in, sxh_ssim_outputs* out);
int32_t sxo_ssim_bwd(const sxh_ssim_inputs* in, const sxh_ssim_grads_in* gin, float* v_img1);

/* Math.cpp quat_scale_to_covar: out is a row-major 3x3 per Gaussian. */
int32_t sxo_quat_scale_to_covar(const float* quats, const float* scales, int64_t n, float* out);

/* Scalar primitives, for pinning the transcendental layer. */
void sxo_logf_array(const float* x, float* y, int64_t n);
void sxo_expf_array(const float* x, float* y, int64_t n);
void sxo_expf_fast_array(const float* x, float* y, int64_t n);
void sxo_powf_array(const float* x, const float* p, float* y, int64_t n);
void sxo_sincosf_array(const float* x, float* s, float* c, int64_t n);

/* One full host-path training step (Trainer.cpp:971-1131 + the noise tail of the resident path,
 * MetalBackend.cpp:2198-2229), on host arrays, in place on params and moments. */
typedef struct {
    float* params[6];
    float* exp_avg[6];
    float* exp_avg_sq[6];
    int64_t count;
    int32_t sh_degree;
    const float* viewmat;
    const float* K;
    int32_t width, height;
    const float* gt_rgb;
    uint32_t degrees_to_use;
    float lr[6];
    float opacity_reg_w, scale_reg_w;
    float eps2d, near_plane, far_plane, radius_clip;
    float b1, b2, eps;
    float ssim_weight;
    uint8_t antialiased, isect_mode, forward_only, inject_noise;
    uint64_t noise_seed, noise_offset;
    float noise_scale;
    /* outputs */
    float loss;
    int64_t n_isects;
    int64_t n_visible;
    float* render_colors; /* optional [H,W,3] */
    double stage_ms[16];  /* see sxo_stage_name */
} sxo_step_args;

int32_t sxo_train_step(sxo_step_args* a);

/* Trainer::mcmc_refine (Trainer.cpp:1273-1435) on host AoS arrays of arena rows, in place. */
typedef struct {
    float* params[6];
    float* exp_avg[6];
    float* exp_avg_sq[6];
    int64_t count, cap_max;
    int32_t sh_degree;
    float min_opacity;
    int32_t n_max;
    const float* binoms;
    sxh_mt64_state* rng; /* in/out */
    /* outputs */
    int64_t new_count, n_relocated, n_added;
    int64_t* relocated_dead; /* optional, `capacity` entries each */
    int64_t* relocation_src;
    int64_t* added_src;
    int64_t capacity;
} sxo_refine_args;
int32_t sxo_mcmc_refine(sxo_refine_args* r);
/* std::mt19937_64 helpers: the seeded state, n raw draws (advancing the state). */
int32_t sxo_mt64_seed(uint64_t seed, sxh_mt64_state* out);
int32_t sxo_mt64_draw(sxh_mt64_state* st, int64_t n, uint64_t* out);
/* The left-to-right f64 running sum of float weights. */
int32_t sxo_running_sum_f64(const float* w, int64_t n, double* out);
const char* sxo_stage_name(int32_t i);

#ifdef __cplusplus
}
#endif

#endif
