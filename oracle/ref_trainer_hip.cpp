// ref_trainer_hip.cpp — the reference's own Trainer driving this repository's backend (TEST
// INFRASTRUCTURE ONLY).
//
// Compiled by oracle/Makefile (target `ref`) with Sources/SplatXCore/{Trainer,CpuKernels,Math}.cpp
// taken in place from the reference tree and splatx-metal_amd/host/hip_kernel_backend.cpp (the
// C++ KernelBackend adapter over the C ABI), linked against splatx-metal_amd/build/libsplatx_hip.so,
// into oracle/_ref/libsx_ref_hip.so. The Trainer code is the reference's, unchanged: it is the
// caller a maintainer would point at make_hip_backend, so a run here exercises the drop-in
// boundary end to end — the host path through the per-op virtuals, the resident path through
// make_train_step_executor, the MCMC refine through the executor's download/upload.
#include <cstring>
#include <memory>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "hip_kernel_backend.h"
#include "splatx/KernelBackend.h"
#include "splatx/Trainer.h"
#include "splatx_hip.h"

namespace {
thread_local std::string g_err;
}

extern "C" {

typedef struct {
    const float* params[6];  /* [count, dim] */
    int64_t count;
    int32_t sh_degree;
    const float* viewmat;    /* [16] */
    const float* K;          /* [9] */
    int32_t width, height;
    const float* gt_rgb;     /* [H,W,3] */
    int32_t steps, total_iters;
    float lr[6];             /* means, quats, scales, opacities, sh0, shN */
    float ssim_weight, opacity_reg, scale_reg;
    uint8_t antialiased, resident, mcmc;
    int64_t cap_max;
    uint64_t seed;
    float refine_start_ratio, refine_stop_ratio, refine_every_ratio;
    /* outputs */
    float* out_params[6];    /* [rows, dim] with rows = cap_max when mcmc else count */
    float* losses;           /* [steps] */
    int64_t* n_isects;       /* [steps] */
    float* render0;          /* [H,W,3]: the first step's render */
    int64_t out_count;
    int32_t n_refined;
    /* optional: a camera list (step it uses camera it % n_cams and its own GT) and a first iteration */
    int32_t n_cams;
    const float* viewmats;   /* [n_cams,16] */
    const float* Ks;         /* [n_cams,9] */
    const float* gts;        /* [n_cams,H,W,3] */
    int32_t start_iter;
    float scene_scale, sh_degree_interval_ratio;
} sxr_hip_train_case;

const char* sxr_hip_last_error(void) { return g_err.c_str(); }

int32_t sxr_hip_trainer_run(sxr_hip_train_case* c) {
    try {
        auto backend = splatx::make_hip_backend({});
        splatx::SplatCloud cloud;
        cloud.count = c->count;
        cloud.sh_degree = c->sh_degree;
        std::vector<float>* vs[6] = {&cloud.means, &cloud.quats, &cloud.scales,
                                     &cloud.opacities, &cloud.sh0, &cloud.shN};
        const int64_t dims[6] = {3, 4, 3, 1, 3, static_cast<int64_t>(cloud.sh_rest_coeffs()) * 3};
        for (int g = 0; g < 6; g++) vs[g]->assign(c->params[g], c->params[g] + c->count * dims[g]);
        splatx::TrainConfig cfg;
        cfg.total_iters = c->total_iters;
        if (c->scene_scale > 0.0f) cfg.scene_scale = c->scene_scale;
        if (c->sh_degree_interval_ratio > 0.0f) cfg.sh_degree_interval_ratio = c->sh_degree_interval_ratio;
        cfg.lr_means = c->lr[0];
        cfg.lr_quats = c->lr[1];
        cfg.lr_scales = c->lr[2];
        cfg.lr_opacities = c->lr[3];
        cfg.lr_sh0 = c->lr[4];
        cfg.lr_shN = c->lr[5];
        cfg.ssim_weight = c->ssim_weight;
        cfg.opacity_reg = c->opacity_reg;
        cfg.scale_reg = c->scale_reg;
        cfg.antialiased = c->antialiased != 0;
        cfg.resident = c->resident != 0;
        if (c->mcmc) {
            cfg.mcmc.enabled = true;
            cfg.mcmc.cap_max = c->cap_max;
            cfg.mcmc.seed = c->seed;
            cfg.mcmc.refine_start_ratio = c->refine_start_ratio;
            cfg.mcmc.refine_stop_ratio = c->refine_stop_ratio;
            cfg.mcmc.refine_every_ratio = c->refine_every_ratio;
        }
        splatx::Trainer tr(*backend, std::move(cloud), cfg);
        const int n_cams = c->n_cams > 0 ? c->n_cams : 1;
        std::vector<splatx::TrainingCamera> cams(static_cast<size_t>(n_cams));
        for (int k = 0; k < n_cams; k++) {
            std::memcpy(cams[k].viewmat, c->n_cams > 0 ? c->viewmats + 16 * k : c->viewmat, sizeof(cams[k].viewmat));
            std::memcpy(cams[k].K, c->n_cams > 0 ? c->Ks + 9 * k : c->K, sizeof(cams[k].K));
            cams[k].width = c->width;
            cams[k].height = c->height;
        }
        const size_t img = static_cast<size_t>(c->width) * c->height * 3;
        c->n_refined = 0;
        for (int s = 0; s < c->steps; s++) {
            const int it = c->start_iter + s;
            const int k = it % n_cams;
            const float* gt = c->n_cams > 0 ? c->gts + img * static_cast<size_t>(k) : c->gt_rgb;
            const splatx::TrainStepResult r = tr.step(cams[static_cast<size_t>(k)], gt, it);
            c->losses[s] = r.loss;
            c->n_isects[s] = r.n_isects;
            if (r.mcmc_refined) c->n_refined++;
            if (s == 0 && c->render0 && !r.render_colors.empty())
                std::memcpy(c->render0, r.render_colors.data(), r.render_colors.size() * sizeof(float));
        }
        const splatx::SplatCloud& out = tr.cloud();
        c->out_count = out.count;
        const std::vector<float>* os[6] = {&out.means, &out.quats, &out.scales, &out.opacities, &out.sh0, &out.shN};
        for (int g = 0; g < 6; g++)
            if (c->out_params[g] && !os[g]->empty())
                std::memcpy(c->out_params[g], os[g]->data(), os[g]->size() * sizeof(float));
        return SXH_OK;
    } catch (const std::invalid_argument& e) {
        g_err = e.what();
        return SXH_ERR_INVALID_ARGUMENT;
    } catch (const std::exception& e) {
        g_err = e.what();
        return SXH_ERR_RUNTIME;
    }
}

/* hip_mcmc_refine (the adapter's device refine) on an executor made through the adapter: params
 * and moments ([rows, dim], rows = cap_max) are uploaded, n_refine refines run from
 * std::mt19937_64(seed), everything is downloaded back in place; rng_out = the engine after. */
typedef struct {
    float* params[6];
    float* exp_avg[6];
    float* exp_avg_sq[6];
    int64_t count, cap_max;
    int32_t sh_degree, n_refine;
    uint64_t seed;
    const float* binoms;     /* [51*51] */
    int64_t* counts;         /* [n_refine] */
    int64_t* last_lists;     /* [3, cap_max]: relocated_dead, relocation_src, added_src of the last refine */
    int64_t last_sizes[3];
    sxh_mt64_state* rng_out;
} sxr_hip_refine_case;

int32_t sxr_hip_adapter_refine(sxr_hip_refine_case* c) {
    try {
        auto backend = splatx::make_hip_backend({});
        splatx::TrainStepExecutorDesc d;
        d.arena_rows = c->cap_max;
        d.sh_degree = c->sh_degree;
        auto exec = backend->make_train_step_executor(d);
        if (!exec) throw std::runtime_error("no executor");
        splatx::ResidentParamSync sync;
        sync.rows = c->cap_max;
        for (int g = 0; g < 6; g++) {
            sync.params[g] = c->params[g];
            sync.exp_avg[g] = c->exp_avg[g];
            sync.exp_avg_sq[g] = c->exp_avg_sq[g];
        }
        exec->upload_params(sync);
        std::mt19937_64 rng(c->seed);
        const std::vector<float> binoms(c->binoms, c->binoms + 51 * 51);
        splatx::HipMcmcRefineInputs in;
        in.count = c->count;
        in.cap_max = c->cap_max;
        in.binoms = &binoms;
        for (int r = 0; r < c->n_refine; r++) {
            const splatx::HipMcmcRefineResult res = splatx::hip_mcmc_refine(*exec, rng, in);
            in.count = res.count;
            c->counts[r] = res.count;
            const std::vector<int64_t>* ls[3] = {&res.relocated_dead, &res.relocation_src, &res.added_src};
            for (int k = 0; k < 3; k++) {
                c->last_sizes[k] = static_cast<int64_t>(ls[k]->size());
                std::memcpy(c->last_lists + k * c->cap_max, ls[k]->data(), ls[k]->size() * sizeof(int64_t));
            }
        }
        exec->download_params(sync);
        std::ostringstream os;
        os << rng;
        std::istringstream is(os.str());
        for (int i = 0; i < 312; i++) is >> c->rng_out->x[i];
        is >> c->rng_out->p;
        return SXH_OK;
    } catch (const std::invalid_argument& e) {
        g_err = e.what();
        return SXH_ERR_INVALID_ARGUMENT;
    } catch (const std::exception& e) {
        g_err = e.what();
        return SXH_ERR_RUNTIME;
    }
}

} // extern "C"
