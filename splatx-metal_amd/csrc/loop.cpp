// loop.cpp — the caller loop: the training loop of sx_train_run_ex (TrainC.cpp:743-906) over
// Trainer::step_resident (Trainer.cpp:916-969), on the executor. The GT images live in the
// executor's GT cache, the step and the MCMC refine run on the device, and per iteration the host
// only evaluates the schedules (a few scalars), reads back the two sync-point values and calls
// the hooks. The schedules are the reference's expressions, evaluated in the same float/double
// types, so a run here takes the same learning rates, SH degrees, refine iterations and noise
// offsets as the reference's loop.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <limits>
#include <string>
#include <vector>

#include "splatx_hip.h"
#include "sx_exec.h"
#include "sx_host.h"
#include "sx_io.h"
#include "sx_kernels.h"

using namespace sxh;

namespace {

using Clock = std::chrono::steady_clock;

double ms_since(Clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

// means_lr_at (Trainer.cpp:496-501): lr_means * scene_scale * 0.01^(iter / total_iters)
float means_lr_at(const sxh_train_schedule& s, int iter) {
    const float p = s.total_iters > 0 ? static_cast<float>(iter) / static_cast<float>(s.total_iters) : 0.0f;
    return s.lr_means * s.scene_scale * std::pow(0.01f, p);
}

// sh_degree_at (Trainer.cpp:503-508)
uint32_t sh_degree_at(const sxh_train_schedule& s, int iter, int sh_degree) {
    if (sh_degree <= 0 || iter < 0) return 0;
    const int interval =
        std::max(1, static_cast<int>(static_cast<float>(s.total_iters) * s.sh_degree_interval_ratio));
    return static_cast<uint32_t>(std::min(iter / interval, sh_degree));
}

// Trainer::mcmc_refine_due (Trainer.cpp:1261-1271): strictly between start and stop, every `every`
bool refine_due(const sxh_train_schedule& s, int iter) {
    if (!s.mcmc_enabled) return false;
    const double total = static_cast<double>(s.total_iters);
    const int start = static_cast<int>(std::lround(total * s.refine_start_ratio));
    const int stop = static_cast<int>(std::lround(total * s.refine_stop_ratio));
    const int every = std::max(1, static_cast<int>(std::lround(total * s.refine_every_ratio)));
    return iter > start && iter < stop && iter % every == 0;
}

// Trainer::step_resident's per-iteration arguments (Trainer.cpp:920-952)
sxh_train_plan plan_at(const sxh_train_schedule& s, int iter, int sh_degree, int64_t count) {
    sxh_train_plan p{};
    p.degrees_to_use = sh_degree_at(s, iter, sh_degree);
    p.lr[0] = means_lr_at(s, iter);
    p.lr[1] = s.lr_quats;
    p.lr[2] = s.lr_scales;
    p.lr[3] = s.lr_opacities;
    p.lr[4] = s.lr_sh0;
    p.lr[5] = s.lr_shN;
    p.opacity_reg_w = s.opacity_reg > 0.0f ? s.opacity_reg / static_cast<float>(count) : 0.0f;
    p.scale_reg_w = s.scale_reg > 0.0f ? s.scale_reg / static_cast<float>(count * 3) : 0.0f;
    p.refine_due = refine_due(s, iter) ? 1 : 0;
    p.inject_noise = (s.mcmc_enabled && !p.refine_due) ? 1 : 0;
    p.noise_scale = means_lr_at(s, iter) * s.noise_lr;
    return p;
}

// a failed C entry point, rethrown with its error class
[[noreturn]] void rethrow(int32_t rc) {
    const std::string msg = sxh_last_error();
    if (rc == SXH_ERR_INVALID_ARGUMENT) throw InvalidArgument(msg);
    if (rc == SXH_ERR_CAPACITY) throw CapacityError(msg);
    throw std::runtime_error(msg);
}

// std::mt19937_64 operator<< in libstdc++'s form (the 312 words, then the position): the text a
// reference checkpoint holds (Trainer::make_checkpoint, Trainer.cpp:1500-1510)
std::string mt_text(const sxh_mt64_state& st) {
    std::string s;
    s.reserve(312 * 21);
    for (int i = 0; i < 312; i++) {
        s += std::to_string(st.x[i]);
        s += ' ';
    }
    s += std::to_string(st.p);
    return s;
}

// splitmix64 (Steele, Lea, Flood 2014): the pose-jitter stream of (seed, iteration)
struct SplitMix {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return static_cast<double>(next() >> 11) * 0x1.0p-53; }  // [0, 1)
    double normal() {  // Box-Muller
        const double u1 = 1.0 - uniform(), u2 = uniform();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

// out = J * vm with J = [R t; 0 1]: R a rotation by an angle in [-max_deg, max_deg] degrees about a
// uniformly random axis (Rodrigues), t a uniformly random direction times a length in [0, max_t]
void jitter_view(const float* vm, float max_deg, float max_t, uint64_t seed, int iter, float* out) {
    SplitMix g{seed ^ (0xD1B54A32D192ED03ull * (static_cast<uint64_t>(iter) + 1))};
    double ax[3] = {g.normal(), g.normal(), g.normal()};
    double n = std::sqrt(ax[0] * ax[0] + ax[1] * ax[1] + ax[2] * ax[2]);
    if (!(n > 0)) ax[0] = 1, ax[1] = ax[2] = 0, n = 1;
    for (double& v : ax) v /= n;
    const double ang = (2.0 * g.uniform() - 1.0) * static_cast<double>(max_deg) * 3.141592653589793 / 180.0;
    const double c = std::cos(ang), s = std::sin(ang), C = 1.0 - c;
    const double R[3][3] = {{c + ax[0] * ax[0] * C, ax[0] * ax[1] * C - ax[2] * s, ax[0] * ax[2] * C + ax[1] * s},
                            {ax[1] * ax[0] * C + ax[2] * s, c + ax[1] * ax[1] * C, ax[1] * ax[2] * C - ax[0] * s},
                            {ax[2] * ax[0] * C - ax[1] * s, ax[2] * ax[1] * C + ax[0] * s, c + ax[2] * ax[2] * C}};
    double td[3] = {g.normal(), g.normal(), g.normal()};
    const double tn = std::sqrt(td[0] * td[0] + td[1] * td[1] + td[2] * td[2]);
    const double tl = g.uniform() * static_cast<double>(max_t);
    double J[4][4] = {};
    for (int r = 0; r < 3; r++) {
        for (int k = 0; k < 3; k++) J[r][k] = R[r][k];
        J[r][3] = tn > 0 ? td[r] / tn * tl : 0.0;
    }
    J[3][3] = 1.0;
    for (int r = 0; r < 4; r++)
        for (int k = 0; k < 4; k++) {
            double acc = 0.0;
            for (int q = 0; q < 4; q++) acc += J[r][q] * static_cast<double>(vm[q * 4 + k]);
            out[r * 4 + k] = static_cast<float>(acc);
        }
}

void check_camera(const sxh_executor* e, const sxh_train_camera& c, const char* what) {
    if (!(c.width == e->gt_w && c.height == e->gt_h)) invalid(what, "camera size differs from the GT cache's");
    if (c.gt_index < 0 || c.gt_index >= e->gt_n) invalid(what, "camera gt_index out of the GT cache");
}

// The loop's device scratch and pinned readback of one call.
struct LoopState {
    DevBuf<double> sq;
    PinnedHost sq_host{sizeof(double) * 1024};
    LoopState() : sq(static_cast<size_t>(sxk::sq_err_blocks())) {}
};

// eval (TrainC.cpp:653-680, the raw PSNR): every eval view rendered at the full SH degree, clamped
// to [0,1], PSNR = 10 log10(1 / mse) per view (psnr, Trainer.cpp:349-360), then the mean
double eval_psnr(sxh_executor* e, const sxh_train_loop_args& a, int64_t count, LoopState& ls) {
    hipStream_t s = e->b->stream;
    const int64_t n = static_cast<int64_t>(e->gt_w) * e->gt_h * 3;
    double sum = 0.0;
    for (int v = 0; v < a.n_eval_cameras; v++) {
        const sxh_train_camera& cam = a.eval_cameras[v];
        sxh_step_inputs in{};
        in.viewmat = cam.viewmat;
        in.K = cam.K;
        in.width = cam.width;
        in.height = cam.height;
        in.gt_index = -1;
        in.count = count;
        in.degrees_to_use = static_cast<uint32_t>(e->d.sh_degree);
        in.forward_only = 1;
        sxh_step_outputs out{};
        sxh_detail::run_step(e, &in, &out, nullptr);
        sxk::sq_err(e->render.p, e->gt_cache.p + static_cast<size_t>(cam.gt_index) * static_cast<size_t>(n), n,
                    ls.sq.p, s);
        SXH_HIP(hipMemcpyAsync(ls.sq_host.p, ls.sq.p, sizeof(double) * ls.sq.n, hipMemcpyDeviceToHost, s));
        SXH_HIP(hipStreamSynchronize(s));
        const double* part = static_cast<const double*>(ls.sq_host.p);
        double acc = 0.0;
        for (size_t b = 0; b < ls.sq.n; b++) acc += part[b];
        const double mse = acc / static_cast<double>(n);
        const float p = mse <= 0.0 ? std::numeric_limits<float>::infinity()
                                   : static_cast<float>(10.0 * std::log10(1.0 / mse));
        sum += static_cast<double>(p);
    }
    return sum / static_cast<double>(a.n_eval_cameras);
}

// filter_cloud_for_export (min opacity 0.005) of the live rows into host arrays, raw domain
int64_t filtered_rows(sxh_executor* e, int64_t count, std::vector<float> (&host)[6]) {
    sxh_detail::canonicalize(e);
    hipStream_t s = e->b->stream;
    const int N = static_cast<int>(count);
    DevBuf<unsigned long long> removed(2);
    DevBuf<int32_t> list(std::max<size_t>(1, static_cast<size_t>(N)));
    sxk::Dims6 dims{};
    for (int g = 0; g < 6; g++) dims.d[g] = e->dims[g];
    const sxk::Arena A = e->arena();
    sxk::export_flags(A, dims, N, 0.005f, e->tiles.p, removed.p, s);
    sxk::scan_i32_i64(e->tiles.p, e->cum.p, N, e->scan_scratch.p, s);
    sxk::export_list(e->tiles.p, e->cum.p, N, list.p, s);
    int64_t kept = 0;
    SXH_HIP(hipMemcpyAsync(&kept, e->cum.p + (N - 1), 8, hipMemcpyDeviceToHost, s));
    SXH_HIP(hipStreamSynchronize(s));
    for (int g = 0; g < 6; g++) {
        host[g].assign(static_cast<size_t>(kept) * e->dims[g], 0.0f);
        if (!kept || !e->dims[g]) continue;
        sxk::gather_rows(A.p[g], e->rows, e->dims[g], list.p, kept, e->staging.p, s);
        SXH_HIP(hipMemcpyAsync(host[g].data(), e->staging.p, host[g].size() * 4, hipMemcpyDeviceToHost, s));
    }
    SXH_HIP(hipStreamSynchronize(s));
    return kept;
}

}  // namespace

extern "C" {

int32_t sxh_train_schedule_defaults(sxh_train_schedule* out) {
    return guarded([&] {
        if (!out) invalid("train_schedule_defaults", "null argument");
        *out = sxh_train_schedule{};
        // TrainConfig (Trainer.h:206-220, 231-232) and McmcOptions (Trainer.h:186-198) defaults
        out->total_iters = 300;
        out->scene_scale = 1.0f;
        out->lr_means = 1.6e-4f;
        out->lr_scales = 5e-3f;
        out->lr_quats = 1e-3f;
        out->lr_opacities = 5e-2f;
        out->lr_sh0 = 2.5e-3f;
        out->lr_shN = 2.5e-3f / 20.0f;
        out->sh_degree_interval_ratio = 1.0f / 30.0f;
        out->opacity_reg = 0.0f;
        out->scale_reg = 0.0f;
        out->mcmc_enabled = 0;
        out->cap_max = 1000000;
        out->min_opacity = 0.005f;
        out->refine_start_ratio = 500.0f / 30000.0f;
        out->refine_stop_ratio = 25000.0f / 30000.0f;
        out->refine_every_ratio = 100.0f / 30000.0f;
        out->noise_lr = 5e5f;
        out->mcmc_seed = 42;
    });
}

int32_t sxh_train_plan_at(const sxh_train_schedule* s, int32_t iter, int32_t sh_degree, int64_t count,
                          sxh_train_plan* out) {
    return guarded([&] {
        if (!s || !out) invalid("train_plan_at", "null argument");
        if (count < 1) invalid("train_plan_at", "count must be >= 1");
        *out = plan_at(*s, iter, sh_degree, count);
    });
}

int32_t sxh_exec_request_stop(sxh_executor* e) {
    return guarded([&] {
        if (!e) invalid("train_loop", "null executor");
        e->stop_requested.store(1, std::memory_order_release);
    });
}

int32_t sxh_exec_train_loop(sxh_executor* e, const sxh_train_loop_args* a, sxh_train_loop_result* out) {
    return guarded([&] {
        const char* what = "train_loop";
        if (!e || !a || !out) invalid(what, "null argument");
        *out = sxh_train_loop_result{};
        out->completed_iters = a->start_iter;
        out->count = a->count;
        out->first_loss = out->last_loss = 0.0f;
        out->last_eval_psnr = std::numeric_limits<float>::quiet_NaN();
        if (!a->cameras || a->n_cameras < 1) invalid(what, "no train cameras");
        if (a->start_iter < 0 || a->run_until < a->start_iter) invalid(what, "need 0 <= start_iter <= run_until");
        if (a->count < 1 || a->count > e->rows) invalid(what, "count out of [1, arena_rows]");
        if (a->sched.total_iters < 1) invalid(what, "total_iters must be >= 1");
        for (int c = 0; c < a->n_cameras; c++) check_camera(e, a->cameras[c], what);
        if (a->eval_every > 0 && a->n_eval_cameras > 0) {
            if (!a->eval_cameras) invalid(what, "null eval cameras");
            for (int c = 0; c < a->n_eval_cameras; c++) check_camera(e, a->eval_cameras[c], what);
        }
        const sxh_train_schedule& sc = a->sched;
        if (sc.mcmc_enabled) {
            if (!a->rng || !a->binoms || a->n_max < 1) invalid(what, "MCMC needs rng, binoms and n_max");
            if (sc.cap_max < a->count || sc.cap_max > e->rows) invalid(what, "cap_max out of [count, arena_rows]");
        }
        if (a->checkpoint_every > 0 && (!a->checkpoint_path || !a->checkpoint_config))
            invalid(what, "checkpoint_every needs checkpoint_path and checkpoint_config");
        if (a->live_ply_every > 0 && !a->live_ply_path) invalid(what, "live_ply_every needs live_ply_path");
        if (a->snapshot_every > 0 && !a->snapshot) invalid(what, "snapshot_every needs a snapshot callback");
        SXH_HIP(hipSetDevice(e->b->device));
        e->stop_requested.store(0, std::memory_order_release);
        LoopState ls;
        int64_t count = a->count;
        const auto t_train = Clock::now();
        float vm_j[16];
        for (int it = a->start_iter; it < a->run_until; it++) {
            if (e->stop_requested.load(std::memory_order_acquire)) {
                out->stopped = 1;
                break;
            }
            const sxh_train_camera& cam = a->cameras[static_cast<size_t>(it) % static_cast<size_t>(a->n_cameras)];
            const float* vm = cam.viewmat;
            if (a->jitter_max_deg > 0.0f || a->jitter_max_t > 0.0f) {
                jitter_view(cam.viewmat, a->jitter_max_deg, a->jitter_max_t, a->jitter_seed, it, vm_j);
                vm = vm_j;
            }
            // Trainer::step_resident (Trainer.cpp:920-952)
            const sxh_train_plan pl = plan_at(sc, it, e->d.sh_degree, count);
            sxh_step_inputs in{};
            in.viewmat = vm;
            in.K = cam.K;
            in.width = cam.width;
            in.height = cam.height;
            in.gt_index = cam.gt_index;
            in.count = count;
            in.degrees_to_use = pl.degrees_to_use;
            for (int g = 0; g < 6; g++) in.lr[g] = pl.lr[g];
            in.opacity_reg_w = pl.opacity_reg_w;
            in.scale_reg_w = pl.scale_reg_w;
            const bool refine = pl.refine_due != 0;
            if (pl.inject_noise) {
                in.inject_noise = 1;
                in.noise_seed = sc.mcmc_seed;
                in.noise_offset = static_cast<uint64_t>(it);
                in.noise_scale = pl.noise_scale;
            }
            const auto t_it = Clock::now();
            sxh_step_outputs so{};
            sxh_detail::run_step(e, &in, &so, nullptr);
            sxh_train_progress p{};
            if (refine) {  // refine, then the noise over the new count (Trainer.cpp:957-967)
                sxh_refine_inputs ri{};
                ri.count = count;
                ri.cap_max = sc.cap_max;
                ri.min_opacity = sc.min_opacity;
                ri.n_max = a->n_max;
                ri.binoms = a->binoms;
                ri.rng = a->rng;
                ri.inject_noise = 1;
                ri.noise_seed = sc.mcmc_seed;
                ri.noise_offset = static_cast<uint64_t>(it);
                ri.noise_scale = pl.noise_scale;
                sxh_refine_outputs ro{};
                const int32_t rc = sxh_exec_mcmc_refine(e, &ri, &ro);
                if (rc != SXH_OK) rethrow(rc);
                count = ro.count;
                p.mcmc_refined = 1;
                p.n_relocated = ro.n_relocated;
                p.n_added = ro.n_added;
            }
            const double step_ms = ms_since(t_it);
            if (it == a->start_iter) out->first_loss = so.loss;
            out->last_loss = so.loss;
            out->completed_iters = it + 1;
            out->count = count;
            // step-boundary hooks in the reference's order: eval, checkpoint, live PLY + snapshot,
            // progress (TrainC.cpp:820-905)
            bool eval_tick = false;
            double psnr = 0.0;
            if (a->eval_every > 0 && a->n_eval_cameras > 0 && (it + 1) % a->eval_every == 0) {
                try {
                    psnr = eval_psnr(e, *a, count, ls);
                    eval_tick = true;
                    out->last_eval_psnr = static_cast<float>(psnr);
                } catch (const std::exception& ex) {
                    std::fprintf(stderr, "warning: eval failed (iter %d): %s — training continues\n", it + 1,
                                 ex.what());
                }
            }
            if (a->checkpoint_every > 0 && (it + 1) % a->checkpoint_every == 0 && it + 1 < a->run_until) {
                const std::string rng = sc.mcmc_enabled ? mt_text(*a->rng) : std::string();
                const int32_t rc = sxh_exec_save_checkpoint(e, a->checkpoint_config, it + 1, count,
                                                            sc.mcmc_enabled ? rng.c_str() : nullptr,
                                                            a->checkpoint_fp16, a->checkpoint_path);
                if (rc != SXH_OK) rethrow(rc);
            }
            const bool live_tick = a->live_ply_every > 0 && (it + 1) % a->live_ply_every == 0;
            const bool snap_tick = a->snapshot_every > 0 && a->snapshot && (it + 1) % a->snapshot_every == 0;
            if (live_tick) {  // "<path>.tmp", then an atomic rename (TrainC.cpp:846-862)
                const std::string path = a->live_ply_path, tmp = path + ".tmp";
                const int32_t rc = sxh_exec_export_ply(e, count, 0.005f, 1, tmp.c_str(), nullptr);
                if (rc != SXH_OK || std::rename(tmp.c_str(), path.c_str()) != 0) {
                    std::remove(tmp.c_str());
                    std::fprintf(stderr, "warning: live PLY export failed (iter %d): %s — training continues\n",
                                 it + 1, rc != SXH_OK ? sxh_last_error() : ("rename to " + path + " failed").c_str());
                }
            }
            if (snap_tick) {
                try {
                    std::vector<float> rows[6];
                    const int64_t kept = filtered_rows(e, count, rows);
                    sxh_splat_snapshot snap{};
                    snap.iter = it + 1;
                    snap.sh_degree = e->d.sh_degree;
                    snap.count = kept;
                    snap.means = rows[0].data();
                    snap.quats = rows[1].data();
                    snap.scales = rows[2].data();
                    snap.opacities = rows[3].data();
                    snap.sh0 = rows[4].data();
                    snap.shN = e->d.sh_degree > 0 ? rows[5].data() : nullptr;
                    a->snapshot(&snap, a->snapshot_user);
                } catch (const std::exception& ex) {
                    std::fprintf(stderr, "warning: live snapshot failed (iter %d): %s — training continues\n",
                                 it + 1, ex.what());
                }
            }
            if (a->progress) {
                p.iter = it + 1;
                p.run_until = a->run_until;
                p.total_iters = sc.total_iters;
                p.loss = so.loss;
                p.psnr = eval_tick ? static_cast<float>(psnr) : std::numeric_limits<float>::quiet_NaN();
                p.step_ms = step_ms;
                p.n_isects = so.n_isects;
                p.splat_count = count;
                p.thermal_state = 0;
                a->progress(&p, a->progress_user);
            }
        }
        out->train_seconds = ms_since(t_train) / 1000.0;
    });
}

}  // extern "C"
