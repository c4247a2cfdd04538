// ref_shim.cpp — C entry points over the reference's own CPU code (TEST INFRASTRUCTURE ONLY).
//
// Compiled by oracle/Makefile together with Sources/SplatXCore/{CpuKernels,Math,CpuBackend,Trainer,
// Checkpoint}.cpp taken in place from the reference tree, into oracle/_ref/libsx_ref.so. It
// converts the C structs of include/splatx_hip.h to the reference's KernelBackend.h structs and
// calls the reference's functions unchanged (for the MCMC refine: a reference Trainer on the
// reference CPU backend), so tests can cross-check the oracle restatement against the real thing.
#include <cstring>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>

#include "splatx/Checkpoint.h"
#include "splatx/CpuKernels.h"
#include "splatx/KernelBackend.h"
#include "splatx/Math.h"
#include "splatx/PlyIO.h"
#include "splatx/Trainer.h"
#include "splatx_hip.h"

extern "C" {
/* One reference Trainer with MCMC on (CPU backend): n_refine calls of Trainer::mcmc_refine on a
 * cloud of `count` rows and cap_max-row Adam moments. Outputs are cap_max-row arrays. */
typedef struct {
    const float* params[6];   /* [count, dim] */
    const float* exp_avg[6];  /* [cap_max, dim] */
    const float* exp_avg_sq[6];
    int64_t count, cap_max;
    int32_t sh_degree;
    float min_opacity;
    uint64_t seed;
    int32_t n_refine;
    /* outputs */
    float* out_params[6];     /* [cap_max, dim] */
    float* out_exp_avg[6];
    float* out_exp_avg_sq[6];
    int64_t* counts;          /* [n_refine] count after each refine */
    int64_t* n_relocated;     /* [n_refine] */
    int64_t* n_added;         /* [n_refine] */
    int64_t* relocated_dead;  /* last refine's lists, `capacity` entries each */
    int64_t* relocation_src;
    int64_t* added_src;
    int64_t capacity;
    sxh_mt64_state* rng_out;  /* the engine after the last refine (its checkpoint text) */
} sxr_refine_case;

/* A cloud as AoS group arrays of `count` rows (shN NULL at degree 0). */
typedef struct {
    const float* params[6];
    int64_t count;
    int32_t sh_degree;
} sxr_cloud_in;
typedef struct {
    float* params[6];
    int64_t count;      /* in: capacity rows, out: rows */
    int32_t sh_degree;  /* out */
} sxr_cloud_out;
}

namespace {
thread_local std::string g_err;
struct CapacityError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
template <class F>
int32_t guarded(F&& f) {
    try {
        f();
        return SXH_OK;
    } catch (const std::invalid_argument& e) {
        g_err = e.what();
        return SXH_ERR_INVALID_ARGUMENT;
    } catch (const CapacityError& e) {
        g_err = e.what();
        return SXH_ERR_CAPACITY;
    } catch (const std::exception& e) {
        g_err = e.what();
        return SXH_ERR_RUNTIME;
    }
}
template <class T>
void put(T* dst, const std::vector<T>& v) {
    if (dst && !v.empty()) std::memcpy(dst, v.data(), v.size() * sizeof(T));
}
} // namespace

extern "C" {

const char* sxr_last_error(void) { return g_err.c_str(); }

int32_t sxr_fused_adam(const sxh_adam_inputs* in) {
    return guarded([&] {
        splatx::AdamInputs a;
        a.param = in->param; a.grad = in->grad; a.exp_avg = in->exp_avg;
        a.exp_avg_sq = in->exp_avg_sq; a.valid = in->valid; a.n_elems = in->n_elems;
        a.n_gauss = in->n_gauss; a.lr = in->lr; a.b1 = in->b1; a.b2 = in->b2; a.eps = in->eps;
        splatx::fused_adam_cpu(a);
    });
}

int32_t sxr_projection_fused_fwd(const sxh_projection_inputs* in, sxh_projection_outputs* out) {
    return guarded([&] {
        splatx::ProjectionFusedInputs p;
        p.means = in->means; p.covars = in->covars; p.quats = in->quats; p.scales = in->scales;
        p.opacities = in->opacities; p.viewmats = in->viewmats; p.Ks = in->Ks; p.N = in->N;
        p.C = in->C; p.width = in->width; p.height = in->height; p.eps2d = in->eps2d;
        p.near_plane = in->near_plane; p.far_plane = in->far_plane; p.radius_clip = in->radius_clip;
        p.camera_model = in->camera_model; p.calc_compensations = in->calc_compensations != 0;
        const splatx::ProjectionFusedOutputs o = splatx::projection_fused_fwd_cpu(p);
        put(out->radii, o.radii);
        put(out->means2d, o.means2d);
        put(out->depths, o.depths);
        put(out->conics, o.conics);
        if (in->calc_compensations) put(out->compensations, o.compensations);
    });
}

int32_t sxr_sh_fwd(const sxh_sh_inputs* in, float* colors) {
    return guarded([&] {
        splatx::ShInputs s;
        s.dirs = in->dirs; s.coeffs = in->coeffs; s.masks = in->masks;
        s.degrees_to_use = in->degrees_to_use; s.B = in->B; s.N = in->N; s.K = in->K; s.D = in->D;
        put(colors, splatx::sh_fwd_cpu(s).colors);
    });
}

int32_t sxr_isect_tiles(const sxh_isect_inputs* in, sxh_isect_outputs* out) {
    return guarded([&] {
        splatx::IsectTilesInputs i;
        i.means2d = in->means2d; i.radii = in->radii; i.depths = in->depths; i.conics = in->conics;
        i.opacities = in->opacities; i.I = in->I; i.N = in->N; i.tile_size = in->tile_size;
        i.tile_width = in->tile_width; i.tile_height = in->tile_height;
        const splatx::IsectTilesOutputs o = splatx::isect_tiles_cpu(i);
        put(out->tiles_per_gauss, o.tiles_per_gauss);
        out->n_isects = o.n_isects;
        out->tile_n_bits = o.tile_n_bits;
        out->image_n_bits = o.image_n_bits;
        if (out->capacity < o.n_isects) throw CapacityError("capacity too small");
        put(out->isect_ids, o.isect_ids);
        put(out->flatten_ids, o.flatten_ids);
    });
}

int32_t sxr_sort_isect(const sxh_sort_inputs* in, uint64_t* keys_sorted, int32_t* values_sorted) {
    return guarded([&] {
        splatx::SortIsectInputs s;
        s.keys = in->keys; s.values = in->values; s.n = in->n; s.key_n_bits = in->key_n_bits;
        const splatx::SortIsectOutputs o = splatx::sort_isect_cpu(s);
        put(keys_sorted, o.keys_sorted);
        put(values_sorted, o.values_sorted);
    });
}

int32_t sxr_isect_offset_encode(const sxh_offset_inputs* in, int32_t* offsets) {
    return guarded([&] {
        splatx::IsectOffsetInputs i;
        i.isect_ids = in->isect_ids; i.n_isects = in->n_isects; i.I = in->I;
        i.tile_width = in->tile_width; i.tile_height = in->tile_height;
        put(offsets, splatx::isect_offset_encode_cpu(i));
    });
}

int32_t sxr_rasterize_fwd(const sxh_raster_inputs* in, sxh_raster_outputs* out) {
    return guarded([&] {
        splatx::RasterizeFwdInputs r;
        r.means2d = in->means2d; r.conics = in->conics; r.colors = in->colors;
        r.opacities = in->opacities; r.backgrounds = in->backgrounds; r.masks = in->masks;
        r.isect_offsets = in->isect_offsets; r.flatten_ids = in->flatten_ids; r.I = in->I;
        r.N = in->N; r.n_isects = in->n_isects; r.image_width = in->image_width;
        r.image_height = in->image_height; r.tile_size = in->tile_size;
        r.tile_width = in->tile_width; r.tile_height = in->tile_height;
        const splatx::RasterizeFwdOutputs o = splatx::rasterize_fwd_cpu(r);
        put(out->render_colors, o.render_colors);
        put(out->render_alphas, o.render_alphas);
        put(out->last_ids, o.last_ids);
    });
}

int32_t sxr_rng_normal_f32(const sxh_rng_inputs* in, float* out) {
    return guarded([&] {
        splatx::RngNormalInputs r;
        r.seed = in->seed; r.offset = in->offset; r.count = in->count;
        put(out, splatx::rng_normal_f32_cpu(r));
    });
}

int32_t sxr_rng_philox_u32(const sxh_rng_inputs* in, uint32_t* out) {
    return guarded([&] {
        splatx::RngNormalInputs r;
        r.seed = in->seed; r.offset = in->offset; r.count = in->count;
        put(out, splatx::rng_philox_u32_cpu(r));
    });
}

int32_t sxr_make_binoms_lut(int32_t n_max, float* out) {
    return guarded([&] { put(out, splatx::make_binoms_lut(n_max)); });
}

int32_t sxr_mcmc_relocation(const sxh_relocation_inputs* in, float* new_op, float* new_sc) {
    return guarded([&] {
        splatx::RelocationInputs r;
        r.opacities = in->opacities; r.scales = in->scales; r.ratios = in->ratios;
        r.binoms = in->binoms; r.N = in->N; r.n_max = in->n_max; r.min_opacity = in->min_opacity;
        const splatx::RelocationOutputs o = splatx::mcmc_relocation_cpu(r);
        put(new_op, o.new_opacities);
        put(new_sc, o.new_scales);
    });
}

int32_t sxr_mcmc_perturb_positions(const sxh_perturb_inputs* in) {
    return guarded([&] {
        splatx::PerturbInputs p;
        p.positions = in->positions; p.quats = in->quats; p.scales_log = in->scales_log;
        p.opacities_logit = in->opacities_logit; p.noise = in->noise; p.N = in->N;
        p.noise_scale = in->noise_scale; p.t = in->t; p.k = in->k;
        splatx::mcmc_perturb_positions_cpu(p);
    });
}

int32_t sxr_ssim_fwd(const sxh_ssim_inputs* in, sxh_ssim_outputs* out) {
    return guarded([&] {
        splatx::SsimInputs s;
        s.img1 = in->img1; s.img2 = in->img2; s.I = in->I; s.H = in->H; s.W = in->W; s.C = in->C;
        s.need_coeffs = in->need_coeffs != 0;
        const splatx::SsimFwdOutputs o = splatx::ssim_fwd_cpu(s);
        out->ssim = o.ssim;
        put(out->ssim_map, o.ssim_map);
        if (in->need_coeffs) {
            put(out->coeff_mu, o.coeff_mu);
            put(out->coeff_sigma, o.coeff_sigma);
            put(out->coeff_cross, o.coeff_cross);
        }
    });
}

int32_t sxr_quat_scale_to_covar(const float* quats, const float* scales, int64_t n, float* out) {
    return guarded([&] {
        for (int64_t i = 0; i < n; i++) {
            const splatx::Mat3 c = splatx::quat_scale_to_covar(quats + i * 4, scales + i * 3);
            std::memcpy(out + i * 9, c.m, sizeof(c.m));
        }
    });
}

namespace {
splatx::SplatCloud cloud_from(const sxr_cloud_in* c) {
    splatx::SplatCloud cl;
    cl.count = c->count;
    cl.sh_degree = c->sh_degree;
    std::vector<float>* vs[6] = {&cl.means, &cl.quats, &cl.scales, &cl.opacities, &cl.sh0, &cl.shN};
    const int64_t dims[6] = {3, 4, 3, 1, 3, static_cast<int64_t>(cl.sh_rest_coeffs()) * 3};
    for (int g = 0; g < 6; g++)
        if (dims[g]) vs[g]->assign(c->params[g], c->params[g] + c->count * dims[g]);
    return cl;
}
void cloud_to(const splatx::SplatCloud& cl, sxr_cloud_out* o) {
    if (cl.count > o->count) throw CapacityError("cloud capacity");
    o->count = cl.count;
    o->sh_degree = cl.sh_degree;
    const std::vector<float>* vs[6] = {&cl.means, &cl.quats, &cl.scales, &cl.opacities, &cl.sh0, &cl.shN};
    for (int g = 0; g < 6; g++)
        if (o->params[g]) put(o->params[g], *vs[g]);
}
splatx::CheckpointConfig config_from(const sxh_checkpoint_config* c) {
    splatx::CheckpointConfig k;
    k.sh_degree = c->sh_degree;
    k.factor = c->factor;
    k.test_split = c->test_split;
    k.total_iters = c->total_iters;
    k.mcmc_enabled = c->mcmc_enabled;
    k.antialiased = c->antialiased;
    k.cap_max = c->cap_max;
    k.mcmc_seed = c->mcmc_seed;
    k.scene_scale = c->scene_scale;
    k.ssim_weight = c->ssim_weight;
    return k;
}
}  // namespace

/* filter_cloud_for_export + write_inria_ply (PlyIO.h:20-51) */
int32_t sxr_export_ply(const sxr_cloud_in* c, float min_opacity, uint8_t pad_sh_full, const char* path,
                       sxh_export_stats* stats) {
    return guarded([&] {
        splatx::ExportFilterStats st;
        const splatx::SplatCloud f = splatx::filter_cloud_for_export(cloud_from(c), min_opacity, &st);
        splatx::write_inria_ply(f, path, pad_sh_full != 0);
        if (stats) {
            stats->input = st.input;
            stats->removed_nonfinite = st.removed_nonfinite;
            stats->removed_low_opacity = st.removed_low_opacity;
            stats->kept = st.kept;
        }
    });
}

/* read_inria_ply */
int32_t sxr_read_ply(const char* path, sxr_cloud_out* o) {
    return guarded([&] { cloud_to(splatx::read_inria_ply(path), o); });
}

/* TrainerCheckpoint of count rows -> save_checkpoint_file */
int32_t sxr_save_checkpoint(const sxh_checkpoint_config* cfg, int32_t iter, const sxr_cloud_in* c,
                            const float* const* exp_avg, const float* const* exp_avg_sq, const char* rng_state,
                            uint8_t fp16, const char* path) {
    return guarded([&] {
        splatx::TrainerCheckpoint ck;
        ck.config = config_from(cfg);
        ck.iter = iter;
        ck.cloud = cloud_from(c);
        const int64_t dims[6] = {3, 4, 3, 1, 3, static_cast<int64_t>(ck.cloud.sh_rest_coeffs()) * 3};
        for (int g = 0; g < 6; g++) {
            const int64_t n = c->count * dims[g];
            if (n) {
                ck.moments[g].exp_avg.assign(exp_avg[g], exp_avg[g] + n);
                ck.moments[g].exp_avg_sq.assign(exp_avg_sq[g], exp_avg_sq[g] + n);
            }
        }
        ck.mcmc_rng_state = rng_state ? rng_state : "";
        splatx::save_checkpoint_file(ck, path, fp16 != 0);
    });
}

/* load_checkpoint_file: the header, the cloud and the moments of count rows, the engine text */
int32_t sxr_load_checkpoint(const char* path, sxh_checkpoint_header* h, sxr_cloud_out* o, float* const* exp_avg,
                            float* const* exp_avg_sq, char* rng_state, int64_t rng_capacity) {
    return guarded([&] {
        const splatx::TrainerCheckpoint ck = splatx::load_checkpoint_file(path);
        const splatx::CheckpointHeader hh = splatx::load_checkpoint_header(path);
        h->config.sh_degree = hh.config.sh_degree;
        h->config.factor = hh.config.factor;
        h->config.test_split = hh.config.test_split;
        h->config.total_iters = hh.config.total_iters;
        h->config.mcmc_enabled = hh.config.mcmc_enabled;
        h->config.antialiased = hh.config.antialiased;
        h->config.cap_max = hh.config.cap_max;
        h->config.mcmc_seed = hh.config.mcmc_seed;
        h->config.scene_scale = hh.config.scene_scale;
        h->config.ssim_weight = hh.config.ssim_weight;
        h->iter = hh.iter;
        h->alive_count = hh.alive_count;
        h->fp16 = hh.fp16 ? 1 : 0;
        h->version = hh.version;
        cloud_to(ck.cloud, o);
        for (int g = 0; g < 6; g++) {
            if (exp_avg && exp_avg[g]) put(exp_avg[g], ck.moments[g].exp_avg);
            if (exp_avg_sq && exp_avg_sq[g]) put(exp_avg_sq[g], ck.moments[g].exp_avg_sq);
        }
        if (rng_state) {
            if (static_cast<int64_t>(ck.mcmc_rng_state.size()) + 1 > rng_capacity) throw CapacityError("rng capacity");
            std::memcpy(rng_state, ck.mcmc_rng_state.c_str(), ck.mcmc_rng_state.size() + 1);
        }
    });
}

int32_t sxr_checkpoint_verify_config(const sxh_checkpoint_config* saved, const sxh_checkpoint_config* current) {
    return guarded([&] { splatx::verify_checkpoint_config(config_from(saved), config_from(current)); });
}

int32_t sxr_trainer_mcmc_refine(sxr_refine_case* c) {
    return guarded([&] {
        auto cpu = splatx::make_cpu_backend();
        splatx::SplatCloud cloud;
        cloud.count = c->count;
        cloud.sh_degree = c->sh_degree;
        std::vector<float>* vs[6] = {&cloud.means, &cloud.quats, &cloud.scales,
                                     &cloud.opacities, &cloud.sh0, &cloud.shN};
        const int64_t dims[6] = {3, 4, 3, 1, 3, static_cast<int64_t>(cloud.sh_rest_coeffs()) * 3};
        for (int g = 0; g < 6; g++) vs[g]->assign(c->params[g], c->params[g] + c->count * dims[g]);
        splatx::TrainConfig cfg;
        cfg.total_iters = 1000;
        cfg.mcmc.enabled = true;
        cfg.mcmc.cap_max = c->cap_max;
        cfg.mcmc.min_opacity = c->min_opacity;
        cfg.mcmc.seed = c->seed;
        splatx::Trainer tr(*cpu, std::move(cloud), cfg);
        const splatx::Trainer::ParamGroup groups[6] = {
            splatx::Trainer::ParamGroup::Means, splatx::Trainer::ParamGroup::Quats,
            splatx::Trainer::ParamGroup::Scales, splatx::Trainer::ParamGroup::Opacities,
            splatx::Trainer::ParamGroup::Sh0, splatx::Trainer::ParamGroup::ShN};
        for (int g = 0; g < 6; g++) {
            splatx::AdamState& st = tr.adam_state(groups[g]);
            st.exp_avg.assign(c->exp_avg[g], c->exp_avg[g] + c->cap_max * dims[g]);
            st.exp_avg_sq.assign(c->exp_avg_sq[g], c->exp_avg_sq[g] + c->cap_max * dims[g]);
        }
        splatx::Trainer::McmcRefineResult last;
        for (int r = 0; r < c->n_refine; r++) {
            last = tr.mcmc_refine();
            c->counts[r] = tr.splat_count();
            c->n_relocated[r] = static_cast<int64_t>(last.relocated_dead.size());
            c->n_added[r] = static_cast<int64_t>(last.added_src.size());
        }
        const splatx::SplatCloud& out = tr.cloud();
        const std::vector<float>* os[6] = {&out.means, &out.quats, &out.scales,
                                           &out.opacities, &out.sh0, &out.shN};
        for (int g = 0; g < 6; g++) {
            put(c->out_params[g], *os[g]);
            const splatx::AdamState& st = tr.adam_state(groups[g]);
            put(c->out_exp_avg[g], st.exp_avg);
            put(c->out_exp_avg_sq[g], st.exp_avg_sq);
        }
        const auto put_list = [&](int64_t* dst, const std::vector<int64_t>& v) {
            if (!dst) return;
            if (static_cast<int64_t>(v.size()) > c->capacity) throw CapacityError("refine list capacity");
            put(dst, v);
        };
        put_list(c->relocated_dead, last.relocated_dead);
        put_list(c->relocation_src, last.relocation_src);
        put_list(c->added_src, last.added_src);
        // the engine state as the reference serializes it into a checkpoint (Trainer.cpp:1500-1510)
        const splatx::TrainerCheckpoint ck = tr.make_checkpoint(0);
        std::istringstream is(ck.mcmc_rng_state);
        for (int i = 0; i < 312; i++) is >> c->rng_out->x[i];
        is >> c->rng_out->p;
        if (!is) throw std::runtime_error("unexpected mt19937_64 text layout");
    });
}

} // extern "C"

// ---- the caller loop's schedule: the reference's own functions ----------------------------------
extern "C" {

typedef struct {
    int32_t total_iters;
    float scene_scale, lr_means, sh_degree_interval_ratio;
    uint8_t mcmc_enabled;
    float refine_start_ratio, refine_stop_ratio, refine_every_ratio;
} sxr_schedule;

/* TrainConfig / McmcOptions defaults (Trainer.h), as floats in sxh_train_schedule's order:
 * total_iters, scene_scale, lr_means, lr_quats, lr_scales, lr_opacities, lr_sh0, lr_shN,
 * sh_degree_interval_ratio, opacity_reg, scale_reg, cap_max, min_opacity, refine_start_ratio,
 * refine_stop_ratio, refine_every_ratio, noise_lr, seed (18 values) */
int32_t sxr_train_defaults(double* out) {
    const splatx::TrainConfig c;
    const splatx::McmcOptions m;
    const double v[18] = {static_cast<double>(c.total_iters), c.scene_scale, c.lr_means, c.lr_quats, c.lr_scales,
                          c.lr_opacities, c.lr_sh0, c.lr_shN, c.sh_degree_interval_ratio, c.opacity_reg, c.scale_reg,
                          static_cast<double>(m.cap_max), m.min_opacity, m.refine_start_ratio, m.refine_stop_ratio,
                          m.refine_every_ratio, m.noise_lr, static_cast<double>(m.seed)};
    std::memcpy(out, v, sizeof(v));
    return SXH_OK;
}

/* means_lr_at, sh_degree_at and Trainer::mcmc_refine_due for iterations iters[0 .. n) */
int32_t sxr_train_plans(const sxr_schedule* s, int32_t sh_degree, int32_t n, const int32_t* iters, float* lr0,
                        uint32_t* degrees, uint8_t* due) {
    return guarded([&] {
        splatx::TrainConfig cfg;
        cfg.total_iters = s->total_iters;
        cfg.scene_scale = s->scene_scale;
        cfg.lr_means = s->lr_means;
        cfg.sh_degree_interval_ratio = s->sh_degree_interval_ratio;
        cfg.mcmc.enabled = s->mcmc_enabled != 0;
        cfg.mcmc.refine_start_ratio = s->refine_start_ratio;
        cfg.mcmc.refine_stop_ratio = s->refine_stop_ratio;
        cfg.mcmc.refine_every_ratio = s->refine_every_ratio;
        cfg.mcmc.cap_max = 4;
        auto cpu = splatx::make_cpu_backend();
        splatx::SplatCloud cloud;  // one Gaussian: the Trainer only has to exist
        cloud.count = 1;
        cloud.sh_degree = sh_degree;
        cloud.means = {0.f, 0.f, 3.f};
        cloud.quats = {1.f, 0.f, 0.f, 0.f};
        cloud.scales = {-3.f, -3.f, -3.f};
        cloud.opacities = {0.f};
        cloud.sh0 = {0.f, 0.f, 0.f};
        cloud.shN.assign(static_cast<size_t>(cloud.sh_rest_coeffs()) * 3, 0.f);
        splatx::Trainer tr(*cpu, std::move(cloud), cfg);
        for (int32_t k = 0; k < n; k++) {
            lr0[k] = splatx::means_lr_at(cfg, iters[k]);
            degrees[k] = splatx::sh_degree_at(cfg, iters[k], sh_degree);
            due[k] = tr.mcmc_refine_due(iters[k]) ? 1 : 0;
        }
    });
}

}  // extern "C"
