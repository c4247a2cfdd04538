/*
 * splatx_hip.h — the C ABI of the MI355X (gfx950) backend for the splatx 3DGS training step.
 *
 * Pure C (C99, POD structs, int32 status codes) so that a Swift module map, a C++ adapter, or
 * Python ctypes can bind it directly. Every entry point replaces one virtual op of the reference
 * operator boundary `splatx::KernelBackend`
 * (Sources/SplatXCore/include/splatx/KernelBackend.h:396-509) or one method of the resident
 * `splatx::TrainStepExecutor` (KernelBackend.h:386-392). Struct fields keep the reference field
 * names (which are the gsplat kernel argument names) and their meaning.
 *
 * Ownership (mirrors KernelBackend.h): inputs are borrowed host pointers valid for the duration of
 * the call; outputs are caller-allocated host buffers of the documented sizes. Ops that are
 * in-place in the reference (fused_adam, mcmc_perturb_positions) are in-place here.
 * Calls are blocking and not thread-safe per backend (KernelBackend.h threading contract:
 * one backend per process, calls commit and wait).
 *
 * Errors: every function returns SXH_OK or an error code; the message of the last failing call on
 * the calling thread is available from sxh_last_error(). The codes map onto the reference's
 * exception types (Validate.h:23 std::invalid_argument; MetalBackend.cpp:52-54 std::runtime_error).
 */
#ifndef SPLATX_HIP_H
#define SPLATX_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SXH_ABI_VERSION 1

/* Status codes. */
enum {
    SXH_OK = 0,
    SXH_ERR_INVALID_ARGUMENT = 1, /* reference: std::invalid_argument (Validate.h:23) */
    SXH_ERR_RUNTIME = 2,          /* reference: std::runtime_error (device, allocation, unsupported camera) */
    SXH_ERR_CAPACITY = 3          /* output capacity too small: required size is reported, nothing written */
};

/* ------------------------------------------------------------------------------------------ */
/* Backend lifetime                                                                           */
/* ------------------------------------------------------------------------------------------ */

typedef struct sxh_backend sxh_backend;

/* Replaces make_metal_backend(void* device, const MetalBackendDesc&) (MetalBackend.h:38-57).
 * device_ordinal selects the HIP device. */
int32_t sxh_backend_create(int32_t device_ordinal, sxh_backend** out);
void sxh_backend_destroy(sxh_backend* b);
/* Replaces KernelBackend::name() (KernelBackend.h:399). */
const char* sxh_backend_name(const sxh_backend* b);
/* Message of the last failing call on this thread ("" if none). */
const char* sxh_last_error(void);
int32_t sxh_abi_version(void);

/* ------------------------------------------------------------------------------------------ */
/* fused_adam — KernelBackend::fused_adam (KernelBackend.h:404), AdamInputs (:18-27)          */
/* In place, no bias correction, eps outside sqrt(v), valid[g]==0 skips param and moments.    */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    float* param;           /* [n_elems] in/out */
    const float* grad;      /* [n_elems] */
    float* exp_avg;         /* [n_elems] in/out */
    float* exp_avg_sq;      /* [n_elems] in/out */
    const uint8_t* valid;   /* [n_gauss] 0/1, may be NULL */
    int64_t n_elems;        /* N*D */
    int64_t n_gauss;        /* N */
    float lr, b1, b2, eps;
} sxh_adam_inputs;
int32_t sxh_fused_adam(sxh_backend* b, const sxh_adam_inputs* in);

/* ------------------------------------------------------------------------------------------ */
/* projection_fused_fwd / _bwd — KernelBackend.h:407-413, ProjectionFusedInputs (:31-45),      */
/* ProjectionFusedOutputs (:47-54), ProjectionFusedGradsIn (:57-66), ProjectionFusedGrads      */
/* (:68-74). PINHOLE only (camera_model must be 0; anything else is SXH_ERR_RUNTIME, as the    */
/* reference's runtime_error at Validate.h:51-55).                                            */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float* means;      /* [N,3] world */
    const float* covars;     /* [N,6] triu (c00,c01,c02,c11,c12,c22); NULL selects quats+scales */
    const float* quats;      /* [N,4] (w,x,y,z), unnormalized */
    const float* scales;     /* [N,3] linear */
    const float* opacities;  /* [N] post-sigmoid, may be NULL (fwd only: opacity-aware radius) */
    const float* viewmats;   /* [C,16] world->cam row-major */
    const float* Ks;         /* [C,9] row-major */
    int64_t N, C;
    int32_t width, height;
    float eps2d, near_plane, far_plane, radius_clip;
    uint32_t camera_model;   /* 0 = PINHOLE */
    uint8_t calc_compensations;
} sxh_projection_inputs;

/* Caller-allocated. Culled slots: radii = 0, compensations = 0, other outputs unspecified
 * (this implementation writes 0 there). */
typedef struct {
    int32_t* radii;          /* [C,N,2] */
    float* means2d;          /* [C,N,2] */
    float* depths;           /* [C,N] */
    float* conics;           /* [C,N,3] */
    float* compensations;    /* [C,N], required iff calc_compensations */
} sxh_projection_outputs;

typedef struct {
    const int32_t* radii;          /* [C,N,2] fwd output */
    const float* conics;           /* [C,N,3] fwd output */
    const float* compensations;    /* [C,N] fwd output, required iff v_compensations != NULL */
    const float* v_means2d;        /* [C,N,2] */
    const float* v_depths;         /* [C,N] */
    const float* v_conics;         /* [C,N,3] */
    const float* v_compensations;  /* [C,N] or NULL */
    uint8_t viewmats_grad;
} sxh_projection_grads_in;

typedef struct {
    float* v_means;     /* [N,3] */
    float* v_covars;    /* [N,6]  covars path only (else may be NULL) */
    float* v_quats;     /* [N,4]  quats/scales path only */
    float* v_scales;    /* [N,3]  quats/scales path only */
    float* v_viewmats;  /* [C,16] only when viewmats_grad */
} sxh_projection_grads;

int32_t sxh_projection_fused_fwd(sxh_backend* b, const sxh_projection_inputs* in,
                                 sxh_projection_outputs* out);
int32_t sxh_projection_fused_bwd(sxh_backend* b, const sxh_projection_inputs* in,
                                 const sxh_projection_grads_in* gin, sxh_projection_grads* out);

/* ------------------------------------------------------------------------------------------ */
/* sh_fwd / sh_bwd — KernelBackend.h:414-419, ShInputs (:77-86), ShOutputs/ShGrads (:88-95)   */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float* dirs;       /* [B*N,3] unnormalized */
    const float* coeffs;     /* [N,K,D] */
    const uint8_t* masks;    /* [B*N] 0/1 or NULL; masked elements are left unwritten */
    uint32_t degrees_to_use; /* 0..4 */
    int64_t B, N, K;
    uint32_t D;
    uint8_t compute_v_dirs;  /* bwd only */
} sxh_sh_inputs;
int32_t sxh_sh_fwd(sxh_backend* b, const sxh_sh_inputs* in, float* colors /* [B*N,D] */);
int32_t sxh_sh_bwd(sxh_backend* b, const sxh_sh_inputs* in, const float* v_colors /* [B*N,D] */,
                   float* v_coeffs /* [N,K,D] */, float* v_dirs /* [B*N,3] or NULL */);

/* ------------------------------------------------------------------------------------------ */
/* isect_tiles — KernelBackend.h:420-422, IsectTilesInputs (:106-115), IsectTilesOutputs       */
/* (:121-128). conics+opacities given -> AccuTile; both NULL -> AABB.                         */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float* means2d;    /* [I,N,2] */
    const int32_t* radii;    /* [I,N,2] */
    const float* depths;     /* [I,N] */
    const float* conics;     /* [I,N,3] (AccuTile) or NULL */
    const float* opacities;  /* [I,N] (AccuTile) or NULL */
    int64_t I, N;
    uint32_t tile_size, tile_width, tile_height;
} sxh_isect_inputs;

typedef struct {
    int32_t* tiles_per_gauss; /* [I,N] caller-allocated */
    uint64_t* isect_ids;      /* [capacity] raw emit order */
    int32_t* flatten_ids;     /* [capacity] */
    int64_t capacity;         /* in: size of isect_ids/flatten_ids */
    int64_t n_isects;         /* out (also on SXH_ERR_CAPACITY) */
    uint32_t tile_n_bits;     /* out */
    uint32_t image_n_bits;    /* out */
} sxh_isect_outputs;
int32_t sxh_isect_tiles(sxh_backend* b, const sxh_isect_inputs* in, sxh_isect_outputs* out);

/* prefix_scan_i64 — KernelBackend.h:428-430: int32 -> inclusive int64 cumsum. */
int32_t sxh_prefix_scan_i64(sxh_backend* b, const int32_t* in, int64_t n, int64_t* out);

/* sort_isect — KernelBackend.h:435-437, SortIsectInputs (:143-148): stable ascending sort of
 * (u64 key, i32 value) on key bits [0, key_n_bits). */
typedef struct {
    const uint64_t* keys;
    const int32_t* values;
    int64_t n;
    uint32_t key_n_bits;
} sxh_sort_inputs;
int32_t sxh_sort_isect(sxh_backend* b, const sxh_sort_inputs* in, uint64_t* keys_sorted,
                       int32_t* values_sorted);

/* sort_isect_noalloc — no counterpart in the reference. For callers that cannot allocate device
 * memory (code under stream capture, tight serving loops): the same sort as sxh_sort_isect, on
 * DEVICE buffers of the backend's device (keys, values in; keys_sorted, values_sorted out; no
 * aliasing), that allocates nothing. Its working memory is a fixed per-device array of the
 * library (26 MiB, held until the process ends), so n is limited to 2,097,152 keys (larger n:
 * SXH_ERR_INVALID_ARGUMENT; so are buffers whose allocation holds fewer than n elements and outputs
 * that overlap an input or each other). It runs on the backend's stream and returns when the sort
 * is done. Calls on one device share that array; a per-device lock inside the call serialises calls
 * from several host threads. */
int32_t sxh_sort_isect_noalloc(sxh_backend* b, const uint64_t* keys, const int32_t* values, int64_t n,
                               uint32_t key_n_bits, uint64_t* keys_sorted, int32_t* values_sorted);

/* isect_offset_encode — KernelBackend.h:441-443, IsectOffsetInputs (:161-166). */
typedef struct {
    const uint64_t* isect_ids; /* [n_isects] sorted */
    int64_t n_isects;
    int64_t I;
    uint32_t tile_width, tile_height;
} sxh_offset_inputs;
int32_t sxh_isect_offset_encode(sxh_backend* b, const sxh_offset_inputs* in,
                                int32_t* offsets /* [I*tile_height*tile_width] */);

/* ------------------------------------------------------------------------------------------ */
/* rasterize_fwd / _bwd — KernelBackend.h:450-461, RasterizeFwdInputs (:175-188),              */
/* RasterizeFwdOutputs (:195-199), RasterizeBwdGradsIn (:207-213), RasterizeBwdGrads (:220-226) */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float* means2d;         /* [I,N,2] */
    const float* conics;          /* [I,N,3] */
    const float* colors;          /* [I,N,3] */
    const float* opacities;       /* [I,N] */
    const float* backgrounds;     /* [I,3] or NULL */
    const uint8_t* masks;         /* [I,TH,TW] or NULL */
    const int32_t* isect_offsets; /* [I,TH,TW] */
    const int32_t* flatten_ids;   /* [n_isects] sorted */
    int64_t I, N, n_isects;
    uint32_t image_width, image_height;
    uint32_t tile_size, tile_width, tile_height;
} sxh_raster_inputs;

typedef struct {
    float* render_colors;  /* [I,H,W,3] */
    float* render_alphas;  /* [I,H,W,1] */
    int32_t* last_ids;     /* [I,H,W] */
} sxh_raster_outputs;

typedef struct {
    const float* render_alphas;
    const int32_t* last_ids;
    const float* v_render_colors;  /* [I,H,W,3] */
    const float* v_render_alphas;  /* [I,H,W,1] */
    uint8_t absgrad;
} sxh_raster_grads_in;

typedef struct {
    float* v_means2d;      /* [I,N,2] */
    float* v_conics;       /* [I,N,3] */
    float* v_colors;       /* [I,N,3] */
    float* v_opacities;    /* [I,N] */
    float* v_means2d_abs;  /* [I,N,2] only when absgrad (else may be NULL) */
} sxh_raster_grads;

int32_t sxh_rasterize_fwd(sxh_backend* b, const sxh_raster_inputs* in, sxh_raster_outputs* out);
int32_t sxh_rasterize_bwd(sxh_backend* b, const sxh_raster_inputs* in,
                          const sxh_raster_grads_in* gin, sxh_raster_grads* out);

/* ------------------------------------------------------------------------------------------ */
/* RNG — rng_normal_f32 / rng_philox_u32 (KernelBackend.h:466-474), RngNormalInputs (:234-238) */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    uint64_t seed;
    uint64_t offset;
    int64_t count;
} sxh_rng_inputs;
int32_t sxh_rng_normal_f32(sxh_backend* b, const sxh_rng_inputs* in, float* out /* [count] */);
int32_t sxh_rng_philox_u32(sxh_backend* b, const sxh_rng_inputs* in, uint32_t* out /* [count] */);

/* ------------------------------------------------------------------------------------------ */
/* MCMC — mcmc_relocation (KernelBackend.h:478-480, RelocationInputs :246-254) and             */
/* mcmc_perturb_positions (:483-485, PerturbInputs :265-275).                                 */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float* opacities;  /* [N] post-sigmoid */
    const float* scales;     /* [N,3] linear */
    const int32_t* ratios;   /* [N] in 1..n_max */
    const float* binoms;     /* [n_max*n_max] */
    int64_t N;
    int32_t n_max;
    float min_opacity;
} sxh_relocation_inputs;
int32_t sxh_mcmc_relocation(sxh_backend* b, const sxh_relocation_inputs* in,
                            float* new_opacities /* [N] */, float* new_scales /* [N,3] */);

typedef struct {
    float* positions;              /* [N,3] in/out */
    const float* quats;            /* [N,4] */
    const float* scales_log;       /* [N,3] */
    const float* opacities_logit;  /* [N] */
    const float* noise;            /* [N,3] */
    int64_t N;
    float noise_scale, t, k;
} sxh_perturb_inputs;
int32_t sxh_mcmc_perturb_positions(sxh_backend* b, const sxh_perturb_inputs* in);

/* Host helper: make_binoms_lut (CpuKernels.h:166) — out has n_max*n_max floats. */
int32_t sxh_make_binoms_lut(int32_t n_max, float* out);

/* ------------------------------------------------------------------------------------------ */
/* SSIM — ssim_fwd / ssim_bwd (KernelBackend.h:491-501), SsimInputs (:283-291),               */
/* SsimFwdOutputs (:299-305), SsimGradsIn (:313-318). Layout [I,H,W,C], valid padding.        */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float* img1;  /* [I,H,W,C] render */
    const float* img2;  /* [I,H,W,C] GT */
    int64_t I, H, W, C;
    uint8_t need_coeffs;
} sxh_ssim_inputs;

typedef struct {
    double ssim;         /* out: mean of the map, f64 sum in ascending index order */
    float* ssim_map;     /* [I,H-10,W-10,C] */
    float* coeff_mu;     /* same shape, only when need_coeffs */
    float* coeff_sigma;
    float* coeff_cross;
} sxh_ssim_outputs;

typedef struct {
    const float* coeff_mu;
    const float* coeff_sigma;
    const float* coeff_cross;
    float v_loss;
} sxh_ssim_grads_in;

int32_t sxh_ssim_fwd(sxh_backend* b, const sxh_ssim_inputs* in, sxh_ssim_outputs* out);
int32_t sxh_ssim_bwd(sxh_backend* b, const sxh_ssim_inputs* in, const sxh_ssim_grads_in* gin,
                     float* v_img1 /* [I,H,W,C] */);

/* ------------------------------------------------------------------------------------------ */
/* Resident train-step executor — TrainStepExecutor (KernelBackend.h:386-392) created by       */
/* KernelBackend::make_train_step_executor (:505-508); TrainStepExecutorDesc (:338-346),       */
/* ResidentParamSync (:354-359), ResidentStepInputs (:361-378), ResidentStepOutputs (:380-384) */
/* ------------------------------------------------------------------------------------------ */
typedef struct sxh_executor sxh_executor;

enum { SXH_ISECT_ACCUTILE = 0, SXH_ISECT_AABB = 1 };

typedef struct {
    int64_t arena_rows;    /* parameter rows (MCMC cap_max) — never reallocated */
    int32_t sh_degree;     /* 0..3 */
    float eps2d, near_plane, far_plane, radius_clip;
    float b1, b2, eps;
    float ssim_weight;     /* lambda; 0 bypasses SSIM */
    uint8_t antialiased;
    uint8_t isect_mode;    /* SXH_ISECT_ACCUTILE (the reference step) or SXH_ISECT_AABB */
} sxh_exec_desc;

/* Group order: 0 means[3], 1 quats[4], 2 scales[3] (log), 3 opacities[1] (logit), 4 sh0[3],
 * 5 shN[(K-1)*3] (NULL when sh_degree == 0). */
typedef struct {
    float* params[6];
    float* exp_avg[6];
    float* exp_avg_sq[6];
    int64_t rows;
} sxh_param_sync;

typedef struct {
    const float* viewmat;     /* [16] world->cam row-major */
    const float* K;           /* [9] */
    int32_t width, height;
    const float* gt_rgb;      /* [H,W,3] host, or NULL when gt_index >= 0 or forward_only */
    int32_t gt_index;         /* >= 0: use the device-resident GT cache entry (sxh_exec_set_gt_cache) */
    int64_t count;            /* alive rows <= arena_rows */
    uint32_t degrees_to_use;
    float lr[6];
    float opacity_reg_w, scale_reg_w;
    uint8_t forward_only;
    uint8_t inject_noise;
    uint64_t noise_seed, noise_offset;
    float noise_scale;
} sxh_step_inputs;

typedef struct {
    float loss;              /* 0 when forward_only */
    int64_t n_isects;        /* the sync-point readback */
    int64_t n_visible;       /* Gaussians with radii > 0 (device counter) */
    float* render_colors;    /* in: [H,W,3] host buffer to fill, or NULL for no readback */
    uint32_t sort_key_bits;  /* out: significant bits of the step's sort keys (tile bits + 32 depth bits) */
} sxh_step_outputs;

int32_t sxh_exec_create(sxh_backend* b, const sxh_exec_desc* desc, sxh_executor** out);
void sxh_exec_destroy(sxh_executor* e);
/* TrainStepExecutor::upload_params / download_params. */
int32_t sxh_exec_upload(sxh_executor* e, const sxh_param_sync* s);
int32_t sxh_exec_download(sxh_executor* e, const sxh_param_sync* s);
/* TrainStepExecutor::step: two host sync points (n_isects, loss). It returns once the loss is read
 * back; without a render read-back the device may still be finishing the step's parameter update,
 * which every later call on the executor (the next step, a download, a refine) is ordered after. */
int32_t sxh_exec_step(sxh_executor* e, const sxh_step_inputs* in, sxh_step_outputs* out);
/* Waits until the executor's device work has finished (for a caller that times steps). No
 * counterpart in the reference (its step returns after its command buffers complete). */
int32_t sxh_exec_sync(sxh_executor* e);
/* Device-resident GT cache: n_images images of [height,width,3] floats, uploaded once. */
int32_t sxh_exec_set_gt_cache(sxh_executor* e, const float* images, int32_t n_images,
                              int32_t width, int32_t height);
/* Renders the current parameters into GT cache entry `index` (synthetic-target helper). */
int32_t sxh_exec_render_to_gt_cache(sxh_executor* e, const sxh_step_inputs* in, int32_t index);

/* ------------------------------------------------------------------------------------------ */
/* MCMC refine on the device — replaces the host orchestration Trainer::mcmc_refine           */
/* (Trainer.cpp:1273-1280) = mcmc_relocate (:1284-1338) + mcmc_add (:1342-1395) with          */
/* mcmc_zero_adam_rows (:1422-1435) and the helpers multinomial_with_replacement (:1199-1218) */
/* and run_relocation_for (:1231-1258), plus the noise tail mcmc_inject_noise (:1400-1418)    */
/* that step_resident runs after a refine (:960-967). The reference downloads and re-uploads  */
/* the whole arena for this (sync_host_for_mutation, :911-914); here it runs in place in HBM. */
/* ------------------------------------------------------------------------------------------ */

/* The multinomial engine, std::mt19937_64 (Trainer.h:495 mcmc_rng_), in libstdc++'s layout:  */
/* x[312] state words and p, the index of the next word to temper (p == 312: the next draw    */
/* twists first). A standard textual state (the 312 most recent words, as libc++ writes it)   */
/* is x = those words with p = 312.                                                            */
typedef struct {
    uint64_t x[312];
    uint32_t p;
} sxh_mt64_state;

/* std::mt19937_64::seed(seed) (Trainer.cpp:713). Host only. */
int32_t sxh_mt64_seed(uint64_t seed, sxh_mt64_state* out);

typedef struct {
    int64_t count;           /* live rows before the refine (cloud_.count) */
    int64_t cap_max;         /* growth cap, <= arena_rows (McmcOptions::cap_max, Trainer.h:190) */
    float min_opacity;       /* dead = sigmoid(logit) <= min_opacity, in (0,1) (Trainer.h:191) */
    int32_t n_max;           /* ratio clamp of the relocation (kMcmcNMax = 51) */
    const float* binoms;     /* [n_max*n_max] host LUT (sxh_make_binoms_lut) */
    sxh_mt64_state* rng;     /* in/out: advanced by exactly the draws the reference makes */
    uint8_t inject_noise;    /* after the refine: mcmc_inject_noise over the new count */
    uint64_t noise_seed, noise_offset;
    float noise_scale;
} sxh_refine_inputs;

typedef struct {
    int64_t count;           /* out: live rows after the refine */
    int64_t n_relocated;     /* out: McmcRefineResult.relocated_dead.size() */
    int64_t n_added;         /* out: McmcRefineResult.added_src.size() */
    /* Optional (NULL = not wanted) copies of McmcRefineResult (Trainer.h:414-420), each with
     * `capacity` entries; SXH_ERR_CAPACITY before any mutation when a wanted list would not fit. */
    int64_t* relocated_dead;
    int64_t* relocation_src;
    int64_t* added_src;
    int64_t capacity;
} sxh_refine_outputs;

/* Errors follow the reference: NaN weights or a zero weight sum (multinomial, :1205-1209) and a
 * non-positive new scale (:1318-1319) fail before that phase mutates anything. */
int32_t sxh_exec_mcmc_refine(sxh_executor* e, const sxh_refine_inputs* in, sxh_refine_outputs* out);

/* The refine's two sequential primitives on the device, exposed for verification like the other
 * ops: the multinomial's running f64 sum of float weights (Trainer.cpp:1202-1208: acc +=
 * double(w[i]), left to right; out[i] = the sum after w[i]), and `n` raw 64-bit draws of the
 * engine (advancing `st`). */
int32_t sxh_running_sum_f64(sxh_backend* b, const float* w, int64_t n, double* out /* [n] */);
int32_t sxh_mt64_draw(sxh_backend* b, sxh_mt64_state* st, int64_t n, uint64_t* out /* [n] */);

/* ------------------------------------------------------------------------------------------ */
/* Data formats either side of the step: the INRIA PLY export with its filter (PlyIO.h:20-51),  */
/* SXCK checkpoints (Checkpoint.h:11-147; Trainer::make_checkpoint / restore_checkpoint,        */
/* Trainer.cpp:1450-1570) and forward-only render sessions (splatx_train_c.h:604-682). The      */
/* filter, the compaction and the packing of PLY rows and checkpoint tensors run on the device  */
/* arena; only the packed bytes cross PCIe.                                                     */
/* ------------------------------------------------------------------------------------------ */

/* ExportFilterStats (PlyIO.h:43-48). */
typedef struct {
    int64_t input, removed_nonfinite, removed_low_opacity, kept;
} sxh_export_stats;

/* filter_cloud_for_export (PlyIO.h:49-51) + write_inria_ply (:20) of the executor's live rows
 * [0, count): rows with a non-finite parameter and rows with sigmoid(opacity) <= min_opacity are
 * dropped; f_rest is zero-padded to 45 coefficients when 0 < K < 15 and pad_sh_full is set. */
int32_t sxh_exec_export_ply(sxh_executor* e, int64_t count, float min_opacity, uint8_t pad_sh_full,
                            const char* path, sxh_export_stats* stats /* may be NULL */);

/* read_inria_ply (PlyIO.h:21), host only: with params == NULL it reports count and sh_degree;
 * then params[6] = AoS arrays of [count, dim] in group order (shN NULL when the degree is 0). */
int32_t sxh_ply_read(const char* path, int64_t* count, int32_t* sh_degree, float* const* params);

/* CheckpointConfig (Checkpoint.h:86-97). */
typedef struct {
    int32_t sh_degree, factor, test_split, total_iters;
    uint8_t mcmc_enabled, antialiased;
    int64_t cap_max;
    uint64_t mcmc_seed;
    float scene_scale, ssim_weight;
} sxh_checkpoint_config;

/* CheckpointHeader (Checkpoint.h:133-139). */
typedef struct {
    sxh_checkpoint_config config;
    int32_t iter;
    int64_t alive_count;
    uint8_t fp16;
    uint32_t version;
} sxh_checkpoint_header;

/* verify_checkpoint_config (Checkpoint.h:117): SXH_ERR_RUNTIME naming the first mismatching field. */
int32_t sxh_checkpoint_verify_config(const sxh_checkpoint_config* saved, const sxh_checkpoint_config* current);
/* load_checkpoint_header (Checkpoint.h:140), host only. */
int32_t sxh_checkpoint_read_header(const char* path, sxh_checkpoint_header* out);
/* make_checkpoint + save_checkpoint_file (Trainer.cpp:1465-1511, Checkpoint.h:121): rows [0, count)
 * of the parameters and both moments, fp32 verbatim or fp16 (half, clamped to +-65504; exp_avg_sq
 * stored as sqrt), written atomically (temp file, fsync, rename, directory fsync). rng_state is the
 * multinomial engine's text form (NULL or "" without MCMC). */
int32_t sxh_exec_save_checkpoint(sxh_executor* e, const sxh_checkpoint_config* config, int32_t iter,
                                 int64_t count, const char* rng_state, uint8_t fp16, const char* path);
/* load_checkpoint_file + restore_checkpoint (Checkpoint.h:122, Trainer.cpp:1513-1570): the file's
 * fingerprint is verified against `current` (skipped when NULL), rows [0, alive_count) of the arena
 * are restored (fp16: exp_avg_sq squared back, exp_avg zeroed where exp_avg_sq decoded to 0), rows
 * beyond are zeroed; `out` gets the header, rng_state (capacity bytes, NUL-terminated) the engine
 * text. A file that does not fit the arena is rejected before any device write. */
int32_t sxh_exec_load_checkpoint(sxh_executor* e, const char* path, const sxh_checkpoint_config* current,
                                 sxh_checkpoint_header* out, char* rng_state, int64_t rng_capacity);

/* Render sessions (sx_render_session_open / _frame / _close, splatx_train_c.h:604-682): a PLY is
 * read and uploaded once; each frame is the resident forward at the cloud's SH degree (as
 * Trainer::render, Trainer.cpp:1133-1151), quantized to RGBA8 on the device (NaN and v <= 0 -> 0,
 * v > 1 -> 1, round-to-nearest-even of 255 v, alpha 255). */
typedef struct sxh_render_session sxh_render_session;
typedef struct {
    const char* ply_path;
    int32_t antialiased;
    int32_t sh_degree;  /* 0: the PLY's degree; 1..3: an upper bound (above the PLY's degree is an error) */
} sxh_render_session_args;
int32_t sxh_render_session_open(sxh_backend* b, const sxh_render_session_args* args, sxh_render_session** out);
int32_t sxh_render_session_frame(sxh_render_session* s, const float* viewmat, float fx, float fy, float cx, float cy,
                                 int32_t width, int32_t height, uint8_t* out_rgba /* [height*width*4] */);
void sxh_render_session_close(sxh_render_session* s);

/* ------------------------------------------------------------------------------------------ */
/* The caller loop: the training loop of sx_train_run_ex (TrainC.cpp:743-906) over           */
/* Trainer::step_resident (Trainer.cpp:916-969), every GT image resident in the executor's   */
/* GT cache. Per iteration it: uses camera it % n_cameras (TrainC.cpp:785); takes the         */
/* schedules means_lr_at / sh_degree_at (Trainer.cpp:496-508) and the regularization weights */
/* (:933-940); injects noise with Philox offset = it unless a refine is due (:942-950); runs */
/* the MCMC refine when Trainer::mcmc_refine_due (:1261-1271) holds, on the device           */
/* (sxh_exec_mcmc_refine, noise after it over the new count, :957-967); evaluates, saves a   */
/* checkpoint, writes the live PLY and calls the snapshot and progress callbacks at the step */
/* boundary in the reference's order (TrainC.cpp:820-905).                                    */
/* ------------------------------------------------------------------------------------------ */

/* TrainingCamera (Trainer.h) with its image's slot in the GT cache. */
typedef struct {
    float viewmat[16];       /* world->camera, row-major */
    float K[9];
    int32_t width, height;   /* must be the GT cache's image size */
    int32_t gt_index;        /* its image in the GT cache (sxh_exec_set_gt_cache) */
} sxh_train_camera;

/* The TrainConfig (Trainer.h:206-243) and McmcOptions (Trainer.h:186-198) fields the loop reads;
 * sxh_train_schedule_defaults fills the reference's defaults. */
typedef struct {
    int32_t total_iters;
    float scene_scale;
    float lr_means, lr_quats, lr_scales, lr_opacities, lr_sh0, lr_shN;
    float sh_degree_interval_ratio;
    float opacity_reg, scale_reg;
    uint8_t mcmc_enabled;
    int64_t cap_max;         /* <= arena_rows */
    float min_opacity;
    float refine_start_ratio, refine_stop_ratio, refine_every_ratio;
    float noise_lr;
    uint64_t mcmc_seed;      /* the Philox noise key (the generator state comes in `rng`) */
} sxh_train_schedule;
int32_t sxh_train_schedule_defaults(sxh_train_schedule* out);

/* One iteration's step arguments under the schedule, as Trainer::step_resident forms them
 * (Trainer.cpp:920-952): means_lr_at and sh_degree_at (:496-508), the regularization weights
 * over the live count, Trainer::mcmc_refine_due (:1261-1271). Host only; the loop uses it. */
typedef struct {
    uint32_t degrees_to_use;
    float lr[6];
    float opacity_reg_w, scale_reg_w;
    uint8_t refine_due;      /* the MCMC refine runs after this iteration's step */
    uint8_t inject_noise;    /* MCMC on and no refine due: the step injects the noise */
    float noise_scale;       /* means_lr_at(iter) * noise_lr (also the refine's noise) */
} sxh_train_plan;
int32_t sxh_train_plan_at(const sxh_train_schedule* s, int32_t iter, int32_t sh_degree, int64_t count,
                          sxh_train_plan* out);

/* SxTrainProgress (splatx_train_c.h:185-195), plus the tick's refine (TrainC.cpp:804-810). */
typedef struct {
    int32_t iter;            /* completed iterations, this step included */
    int32_t run_until, total_iters;
    float loss;
    float psnr;              /* mean PSNR of the eval views if an eval ran on this tick, else NaN */
    double step_ms;          /* the step, and the refine when one ran */
    int64_t n_isects;
    int64_t splat_count;     /* live rows after this tick */
    int32_t thermal_state;   /* 0: no thermal governor here */
    int32_t mcmc_refined;
    int64_t n_relocated, n_added;
} sxh_train_progress;
typedef void (*sxh_train_progress_fn)(const sxh_train_progress* p, void* user);

/* SxSplatSnapshot (splatx_train_c.h:236-246): the filtered rows (filter_cloud_for_export,
 * min opacity 0.005) in the raw domain, valid only during the callback. */
typedef struct {
    int32_t iter, sh_degree;
    int64_t count;
    const float* means;      /* [count,3] */
    const float* quats;      /* [count,4] */
    const float* scales;     /* [count,3] log */
    const float* opacities;  /* [count] logit */
    const float* sh0;        /* [count,3] */
    const float* shN;        /* [count,K,3]; NULL at degree 0 */
} sxh_splat_snapshot;
typedef void (*sxh_snapshot_fn)(const sxh_splat_snapshot* s, void* user);

typedef struct {
    const sxh_train_camera* cameras;  /* the train split in order */
    int32_t n_cameras;
    const sxh_train_camera* eval_cameras;  /* the test split (NULL when n_eval_cameras is 0) */
    int32_t n_eval_cameras;
    int32_t eval_every;      /* eval after iteration it when (it + 1) % eval_every == 0; 0: never */
    int32_t start_iter, run_until;
    int64_t count;           /* live rows at start_iter */
    sxh_train_schedule sched;
    const float* binoms;     /* MCMC: the relocation LUT [n_max * n_max] (sxh_make_binoms_lut) */
    int32_t n_max;
    sxh_mt64_state* rng;     /* MCMC: the multinomial generator, advanced in place */
    /* seeded pose jitter (0: none): iteration it composes a rotation by at most jitter_max_deg
     * about a random axis and a translation of length at most jitter_max_t, drawn from
     * (jitter_seed, it), with the camera's view (the config-3 workload's per-step jitter) */
    float jitter_max_deg, jitter_max_t;
    uint64_t jitter_seed;
    sxh_train_progress_fn progress;  /* may be NULL */
    void* progress_user;
    sxh_snapshot_fn snapshot;        /* with snapshot_every > 0 */
    void* snapshot_user;
    int32_t snapshot_every;
    int32_t live_ply_every;          /* (it + 1) % every == 0: write live_ply_path via "<path>.tmp" */
    const char* live_ply_path;
    int32_t checkpoint_every;        /* (it + 1) % every == 0 and it + 1 < run_until */
    const char* checkpoint_path;
    const sxh_checkpoint_config* checkpoint_config;
    uint8_t checkpoint_fp16;
} sxh_train_loop_args;

typedef struct {
    int32_t completed_iters; /* the next iteration to run (SxTrainStats.completed_iters) */
    int64_t count;           /* live rows at the end */
    float first_loss, last_loss;
    float last_eval_psnr;    /* NaN when no eval ran */
    double train_seconds;
    int32_t stopped;         /* 1 when sxh_exec_request_stop ended the loop early */
} sxh_train_loop_result;

/* Live PLY, snapshot and eval failures warn on stderr and training continues (TrainC.cpp:840-889);
 * a step, refine or checkpoint failure ends the loop with its error (out->completed_iters says
 * where). Callbacks run synchronously on the calling thread and must not re-enter the loop. */
int32_t sxh_exec_train_loop(sxh_executor* e, const sxh_train_loop_args* a, sxh_train_loop_result* out);
/* sx_train_request_stop: from any thread (a callback included); the loop ends at the next step
 * boundary with stopped = 1. A new sxh_exec_train_loop call clears the request. */
int32_t sxh_exec_request_stop(sxh_executor* e);

/* Per-kernel timing of the last step (HIP events on the executor's stream), enabled by
 * sxh_exec_set_profiling(e, enable) with bit 0 of enable. Names are stable strings; times are
 * milliseconds. Bit 1 of enable also counts the rasterisers' pair work of each step (counting
 * instantiations of the raster kernels, slower than the production ones: use the counts, not the
 * times, of such steps). No counterpart in the reference (its per-segment timing probe is
 * MetalBackend.cpp:56-69). */
typedef struct {
    int32_t n;
    const char* names[32];
    float ms[32];
} sxh_exec_timing;
typedef struct {
    uint64_t fwd_iters;         /* forward wave iterations (x 64 = lane pairs evaluated) */
    uint64_t fwd_entries;       /* block-list entries walked: one splat against a 4x4 pixel block */
    uint64_t fwd_taken;         /* pairs composited (alpha >= 1/255, T not yet spent) */
    uint64_t bwd_chunks;        /* backward 4-iteration chunks (x 256 = lane pairs evaluated) */
    uint64_t bwd_entries;       /* block-list entries in those chunks */
    uint64_t bwd_empty_chunks;  /* chunks in which no lane's pair is inside the cutoff (skipped) */
    uint64_t bwd_in_cutoff;     /* lane pairs inside the cutoff and at or before the pixel's last contributor */
    uint64_t bwd_contrib;       /* pairs that contribute a gradient (alpha >= 1/255) */
} sxh_raster_stats;
int32_t sxh_exec_set_profiling(sxh_executor* e, int32_t enable);
int32_t sxh_exec_get_timing(sxh_executor* e, sxh_exec_timing* out);
/* The pair counts of the last step run with bit 1 of profiling set (zeros otherwise). */
int32_t sxh_exec_get_raster_stats(sxh_executor* e, sxh_raster_stats* out);
/* Whether the step's second segment (everything after the intersection-count readback) runs as a
 * captured hipGraph (default 1) or as direct launches (0). Profiling always launches directly. No
 * counterpart in the reference (its Metal command buffers are encoded per step). */
int32_t sxh_exec_set_graph(sxh_executor* e, int32_t enable);
/* How the step orders its intersections (both give the reference's per-tile (depth, index) order,
 * bit for bit): SXH_ISECT_ORDER_DEPTH_FIRST sorts the Gaussians by depth, emits in that order and
 * sorts the tile ids; SXH_ISECT_ORDER_INDEX_FIRST emits in index order, sorts the tile ids and then
 * each tile's list by depth in LDS (cheaper while tiles hold at most a few thousand entries);
 * SXH_ISECT_ORDER_AUTO (default) takes index-first once the previous step's largest tile held at
 * most 4096 entries. No counterpart in the reference (a tuning choice of this backend). */
#define SXH_ISECT_ORDER_AUTO 0
#define SXH_ISECT_ORDER_DEPTH_FIRST 1
#define SXH_ISECT_ORDER_INDEX_FIRST 2
int32_t sxh_exec_set_isect_order(sxh_executor* e, int32_t mode);
/* The order in which the executor keeps the live rows in HBM. SXH_ROW_ORDER_SPATIAL_AUTO (default):
 * from the second training step after the last call that exchanged rows with the caller (upload,
 * download, refine, checkpoint, export), for clouds of at least 65536 rows, along a Morton curve over
 * the means, so that the rows a camera culls fill whole waves that the parameter update skips;
 * SXH_ROW_ORDER_ORIGINAL: always the caller's order; SXH_ROW_ORDER_SPATIAL: along the curve from the
 * next training step on, at any size. Every result is the same bit for bit in every mode (the
 * intersection lists order equal depths, and the MCMC noise is drawn, by original row; every call that
 * exchanges rows restores the caller's order first). No counterpart in the reference (a layout choice of this
 * backend). */
#define SXH_ROW_ORDER_SPATIAL_AUTO 0
#define SXH_ROW_ORDER_ORIGINAL 1
#define SXH_ROW_ORDER_SPATIAL 2
int32_t sxh_exec_set_row_order(sxh_executor* e, int32_t mode);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* SPLATX_HIP_H */
