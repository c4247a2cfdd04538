// hip_kernel_backend.cpp — splatx::KernelBackend (KernelBackend.h:396-509) implemented by forwarding
// every op to the splatx-hip C ABI (include/splatx_hip.h). Output std::vectors are sized here and
// handed to the C calls as caller-allocated buffers; C status codes become the reference's
// exception types (std::invalid_argument for validation, Validate.h:23; std::runtime_error for
// everything else, MetalBackend.cpp:52-54).
#include "hip_kernel_backend.h"

#include <cmath>
#include <locale>
#include <sstream>
#include <stdexcept>
#include <string>

#include "splatx_hip.h"

namespace splatx {
namespace {

void check(int32_t rc) {
    if (rc == SXH_OK) return;
    const std::string msg = sxh_last_error();
    if (rc == SXH_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

template <class T> T* data_or_null(std::vector<T>& v) { return v.empty() ? nullptr : v.data(); }

sxh_projection_inputs to_c(const ProjectionFusedInputs& in) {
    sxh_projection_inputs c{};
    c.means = in.means;
    c.covars = in.covars;
    c.quats = in.quats;
    c.scales = in.scales;
    c.opacities = in.opacities;
    c.viewmats = in.viewmats;
    c.Ks = in.Ks;
    c.N = in.N;
    c.C = in.C;
    c.width = in.width;
    c.height = in.height;
    c.eps2d = in.eps2d;
    c.near_plane = in.near_plane;
    c.far_plane = in.far_plane;
    c.radius_clip = in.radius_clip;
    c.camera_model = in.camera_model;
    c.calc_compensations = in.calc_compensations ? 1 : 0;
    return c;
}

sxh_sh_inputs to_c(const ShInputs& in) {
    sxh_sh_inputs c{};
    c.dirs = in.dirs;
    c.coeffs = in.coeffs;
    c.masks = in.masks;
    c.degrees_to_use = in.degrees_to_use;
    c.B = in.B;
    c.N = in.N;
    c.K = in.K;
    c.D = in.D;
    c.compute_v_dirs = in.compute_v_dirs ? 1 : 0;
    return c;
}

sxh_raster_inputs to_c(const RasterizeFwdInputs& in) {
    sxh_raster_inputs c{};
    c.means2d = in.means2d;
    c.conics = in.conics;
    c.colors = in.colors;
    c.opacities = in.opacities;
    c.backgrounds = in.backgrounds;
    c.masks = in.masks;
    c.isect_offsets = in.isect_offsets;
    c.flatten_ids = in.flatten_ids;
    c.I = in.I;
    c.N = in.N;
    c.n_isects = in.n_isects;
    c.image_width = in.image_width;
    c.image_height = in.image_height;
    c.tile_size = in.tile_size;
    c.tile_width = in.tile_width;
    c.tile_height = in.tile_height;
    return c;
}

sxh_ssim_inputs to_c(const SsimInputs& in) {
    sxh_ssim_inputs c{};
    c.img1 = in.img1;
    c.img2 = in.img2;
    c.I = in.I;
    c.H = in.H;
    c.W = in.W;
    c.C = in.C;
    c.need_coeffs = in.need_coeffs ? 1 : 0;
    return c;
}

size_t sz(int64_t n) { return n > 0 ? static_cast<size_t>(n) : 0; }

class HipTrainStepExecutor final : public TrainStepExecutor {
public:
    explicit HipTrainStepExecutor(sxh_executor* e) : e_(e) {}
    ~HipTrainStepExecutor() override { sxh_exec_destroy(e_); }

    void upload_params(const ResidentParamSync& s) override {
        const sxh_param_sync c = to_c(s);
        check(sxh_exec_upload(e_, &c));
    }
    void download_params(const ResidentParamSync& s) override {
        const sxh_param_sync c = to_c(s);
        check(sxh_exec_download(e_, &c));
    }
    ResidentStepOutputs step(const ResidentStepInputs& in) override {
        sxh_step_inputs c{};
        c.viewmat = in.viewmat;
        c.K = in.K;
        c.width = in.width;
        c.height = in.height;
        c.gt_rgb = in.gt_rgb;
        c.gt_index = -1;
        c.count = in.count;
        c.degrees_to_use = in.degrees_to_use;
        for (int g = 0; g < 6; g++) c.lr[g] = in.lr[g];
        c.opacity_reg_w = in.opacity_reg_w;
        c.scale_reg_w = in.scale_reg_w;
        c.forward_only = in.forward_only ? 1 : 0;
        c.inject_noise = in.inject_noise ? 1 : 0;
        c.noise_seed = in.noise_seed;
        c.noise_offset = in.noise_offset;
        c.noise_scale = in.noise_scale;
        ResidentStepOutputs out;
        if (in.want_render) out.render_colors.resize(sz(int64_t{in.width} * in.height * 3));
        sxh_step_outputs o{};
        o.render_colors = data_or_null(out.render_colors);
        check(sxh_exec_step(e_, &c, &o));
        out.loss = o.loss;
        out.n_isects = o.n_isects;
        return out;
    }

    sxh_executor* handle() const { return e_; }

private:
    static sxh_param_sync to_c(const ResidentParamSync& s) {
        sxh_param_sync c{};
        for (int g = 0; g < 6; g++) {
            c.params[g] = s.params[g];
            c.exp_avg[g] = s.exp_avg[g];
            c.exp_avg_sq[g] = s.exp_avg_sq[g];
        }
        c.rows = s.rows;
        return c;
    }
    sxh_executor* e_;
};

class HipKernelBackend final : public KernelBackend {
public:
    explicit HipKernelBackend(int device) {
        if (sxh_abi_version() != SXH_ABI_VERSION) throw std::runtime_error("splatx-hip: ABI version mismatch");
        check(sxh_backend_create(device, &b_));
        name_ = sxh_backend_name(b_);
    }
    ~HipKernelBackend() override { sxh_backend_destroy(b_); }

    const char* name() const override { return name_.c_str(); }

    ProjectionOutputs projection_ewa_fwd(const ProjectionInputs&) override {
        throw std::runtime_error("projection_ewa_fwd: unimplemented on hip backend");
    }

    void fused_adam(const AdamInputs& in) override {
        sxh_adam_inputs c{in.param, in.grad, in.exp_avg, in.exp_avg_sq, in.valid, in.n_elems, in.n_gauss,
                          in.lr, in.b1, in.b2, in.eps};
        check(sxh_fused_adam(b_, &c));
    }

    ProjectionFusedOutputs projection_fused_fwd(const ProjectionFusedInputs& in) override {
        const sxh_projection_inputs c = to_c(in);
        const size_t cn = sz(in.C) * sz(in.N);
        ProjectionFusedOutputs out;
        out.radii.resize(cn * 2);
        out.means2d.resize(cn * 2);
        out.depths.resize(cn);
        out.conics.resize(cn * 3);
        if (in.calc_compensations) out.compensations.resize(cn);
        sxh_projection_outputs o{data_or_null(out.radii), data_or_null(out.means2d), data_or_null(out.depths),
                                 data_or_null(out.conics), data_or_null(out.compensations)};
        check(sxh_projection_fused_fwd(b_, &c, &o));
        return out;
    }

    ProjectionFusedGrads projection_fused_bwd(const ProjectionFusedInputs& in,
                                              const ProjectionFusedGradsIn& g) override {
        const sxh_projection_inputs c = to_c(in);
        sxh_projection_grads_in gc{g.radii,    g.conics,   g.compensations,  g.v_means2d,
                                   g.v_depths, g.v_conics, g.v_compensations, g.viewmats_grad ? uint8_t{1} : uint8_t{0}};
        ProjectionFusedGrads out;
        out.v_means.resize(sz(in.N) * 3);
        if (in.covars) out.v_covars.resize(sz(in.N) * 6);
        else {
            out.v_quats.resize(sz(in.N) * 4);
            out.v_scales.resize(sz(in.N) * 3);
        }
        if (g.viewmats_grad) out.v_viewmats.resize(sz(in.C) * 16);
        sxh_projection_grads o{data_or_null(out.v_means), data_or_null(out.v_covars), data_or_null(out.v_quats),
                               data_or_null(out.v_scales), data_or_null(out.v_viewmats)};
        check(sxh_projection_fused_bwd(b_, &c, &gc, &o));
        return out;
    }

    ShOutputs sh_fwd(const ShInputs& in) override {
        const sxh_sh_inputs c = to_c(in);
        ShOutputs out;
        out.colors.resize(sz(in.B) * sz(in.N) * in.D);
        check(sxh_sh_fwd(b_, &c, data_or_null(out.colors)));
        return out;
    }

    ShGrads sh_bwd(const ShInputs& in, const float* v_colors) override {
        const sxh_sh_inputs c = to_c(in);
        ShGrads out;
        out.v_coeffs.resize(sz(in.N) * sz(in.K) * in.D);
        if (in.compute_v_dirs) out.v_dirs.resize(sz(in.B) * sz(in.N) * 3);
        check(sxh_sh_bwd(b_, &c, v_colors, data_or_null(out.v_coeffs), data_or_null(out.v_dirs)));
        return out;
    }

    IsectTilesOutputs isect_tiles(const IsectTilesInputs& in) override {
        sxh_isect_inputs c{in.means2d, in.radii,     in.depths,    in.conics,     in.opacities,
                           in.I,       in.N,         in.tile_size, in.tile_width, in.tile_height};
        IsectTilesOutputs out;
        out.tiles_per_gauss.resize(sz(in.I) * sz(in.N));
        // first attempt sized for a typical density; the C call reports the exact count when short
        int64_t cap = 4 * in.I * in.N + 1024;
        for (int attempt = 0; attempt < 2; attempt++) {
            out.isect_ids.resize(sz(cap));
            out.flatten_ids.resize(sz(cap));
            sxh_isect_outputs o{};
            o.tiles_per_gauss = data_or_null(out.tiles_per_gauss);
            o.isect_ids = data_or_null(out.isect_ids);
            o.flatten_ids = data_or_null(out.flatten_ids);
            o.capacity = cap;
            const int32_t rc = sxh_isect_tiles(b_, &c, &o);
            if (rc == SXH_ERR_CAPACITY && attempt == 0) {
                cap = o.n_isects;
                continue;
            }
            check(rc);
            out.n_isects = o.n_isects;
            out.tile_n_bits = o.tile_n_bits;
            out.image_n_bits = o.image_n_bits;
            out.isect_ids.resize(sz(o.n_isects));
            out.flatten_ids.resize(sz(o.n_isects));
            return out;
        }
        throw std::runtime_error("isect_tiles: intersection count changed between attempts");
    }

    std::vector<int64_t> prefix_scan_i64(const int32_t* in, int64_t n) override {
        std::vector<int64_t> out(sz(n));
        check(sxh_prefix_scan_i64(b_, in, n, data_or_null(out)));
        return out;
    }

    SortIsectOutputs sort_isect(const SortIsectInputs& in) override {
        sxh_sort_inputs c{in.keys, in.values, in.n, in.key_n_bits};
        SortIsectOutputs out;
        out.keys_sorted.resize(sz(in.n));
        out.values_sorted.resize(sz(in.n));
        check(sxh_sort_isect(b_, &c, data_or_null(out.keys_sorted), data_or_null(out.values_sorted)));
        return out;
    }

    std::vector<int32_t> isect_offset_encode(const IsectOffsetInputs& in) override {
        sxh_offset_inputs c{in.isect_ids, in.n_isects, in.I, in.tile_width, in.tile_height};
        std::vector<int32_t> out(sz(in.I) * in.tile_width * in.tile_height);
        check(sxh_isect_offset_encode(b_, &c, data_or_null(out)));
        return out;
    }

    RasterizeFwdOutputs rasterize_fwd(const RasterizeFwdInputs& in) override {
        const sxh_raster_inputs c = to_c(in);
        const size_t px = sz(in.I) * in.image_width * in.image_height;
        RasterizeFwdOutputs out;
        out.render_colors.resize(px * 3);
        out.render_alphas.resize(px);
        out.last_ids.resize(px);
        sxh_raster_outputs o{data_or_null(out.render_colors), data_or_null(out.render_alphas),
                             data_or_null(out.last_ids)};
        check(sxh_rasterize_fwd(b_, &c, &o));
        return out;
    }

    RasterizeBwdGrads rasterize_bwd(const RasterizeFwdInputs& in, const RasterizeBwdGradsIn& g) override {
        const sxh_raster_inputs c = to_c(in);
        sxh_raster_grads_in gc{g.render_alphas, g.last_ids, g.v_render_colors, g.v_render_alphas,
                               g.absgrad ? uint8_t{1} : uint8_t{0}};
        const size_t n = sz(in.I) * sz(in.N);
        RasterizeBwdGrads out;
        out.v_means2d.resize(n * 2);
        out.v_conics.resize(n * 3);
        out.v_colors.resize(n * 3);
        out.v_opacities.resize(n);
        if (g.absgrad) out.v_means2d_abs.resize(n * 2);
        sxh_raster_grads o{data_or_null(out.v_means2d), data_or_null(out.v_conics), data_or_null(out.v_colors),
                           data_or_null(out.v_opacities), data_or_null(out.v_means2d_abs)};
        check(sxh_rasterize_bwd(b_, &c, &gc, &o));
        return out;
    }

    std::vector<float> rng_normal_f32(const RngNormalInputs& in) override {
        sxh_rng_inputs c{in.seed, in.offset, in.count};
        std::vector<float> out(sz(in.count));
        check(sxh_rng_normal_f32(b_, &c, data_or_null(out)));
        return out;
    }

    std::vector<uint32_t> rng_philox_u32(const RngNormalInputs& in) override {
        sxh_rng_inputs c{in.seed, in.offset, in.count};
        std::vector<uint32_t> out(sz(in.count));
        check(sxh_rng_philox_u32(b_, &c, data_or_null(out)));
        return out;
    }

    RelocationOutputs mcmc_relocation(const RelocationInputs& in) override {
        sxh_relocation_inputs c{in.opacities, in.scales, in.ratios, in.binoms, in.N, in.n_max, in.min_opacity};
        RelocationOutputs out;
        out.new_opacities.resize(sz(in.N));
        out.new_scales.resize(sz(in.N) * 3);
        check(sxh_mcmc_relocation(b_, &c, data_or_null(out.new_opacities), data_or_null(out.new_scales)));
        return out;
    }

    void mcmc_perturb_positions(const PerturbInputs& in) override {
        sxh_perturb_inputs c{in.positions, in.quats, in.scales_log, in.opacities_logit, in.noise,
                             in.N,         in.noise_scale, in.t,    in.k};
        check(sxh_mcmc_perturb_positions(b_, &c));
    }

    SsimFwdOutputs ssim_fwd(const SsimInputs& in) override {
        const sxh_ssim_inputs c = to_c(in);
        const int64_t hm = in.H - 10, wm = in.W - 10;
        const size_t m = (hm > 0 && wm > 0) ? sz(in.I) * sz(hm) * sz(wm) * sz(in.C) : 0;
        SsimFwdOutputs out;
        out.ssim_map.resize(m);
        if (in.need_coeffs) {
            out.coeff_mu.resize(m);
            out.coeff_sigma.resize(m);
            out.coeff_cross.resize(m);
        }
        sxh_ssim_outputs o{};
        o.ssim_map = data_or_null(out.ssim_map);
        o.coeff_mu = data_or_null(out.coeff_mu);
        o.coeff_sigma = data_or_null(out.coeff_sigma);
        o.coeff_cross = data_or_null(out.coeff_cross);
        check(sxh_ssim_fwd(b_, &c, &o));
        out.ssim = o.ssim;
        return out;
    }

    std::vector<float> ssim_bwd(const SsimInputs& in, const SsimGradsIn& g) override {
        const sxh_ssim_inputs c = to_c(in);
        sxh_ssim_grads_in gc{g.coeff_mu, g.coeff_sigma, g.coeff_cross, g.v_loss};
        std::vector<float> out(sz(in.I) * sz(in.H) * sz(in.W) * sz(in.C));
        check(sxh_ssim_bwd(b_, &c, &gc, data_or_null(out)));
        return out;
    }

    std::unique_ptr<TrainStepExecutor> make_train_step_executor(const TrainStepExecutorDesc& d) override {
        sxh_exec_desc c{};
        c.arena_rows = d.arena_rows;
        c.sh_degree = d.sh_degree;
        c.eps2d = d.eps2d;
        c.near_plane = d.near_plane;
        c.far_plane = d.far_plane;
        c.radius_clip = d.radius_clip;
        c.b1 = d.b1;
        c.b2 = d.b2;
        c.eps = d.eps;
        c.ssim_weight = d.ssim_weight;
        c.antialiased = d.antialiased ? 1 : 0;
        c.isect_mode = SXH_ISECT_ACCUTILE; // the reference's resident step (MetalBackend.cpp:1835)
        sxh_executor* e = nullptr;
        check(sxh_exec_create(b_, &c, &e));
        return std::make_unique<HipTrainStepExecutor>(e);
    }

private:
    sxh_backend* b_ = nullptr;
    std::string name_;
};

} // namespace

namespace {

// The engine's state through its text form (the C++ standard's stream operators): libstdc++ writes
// its 312 words and the position (313 numbers), libc++ the 312 most recent words (then p = 312).
sxh_mt64_state mt_state_of(const std::mt19937_64& g) {
    std::ostringstream os;
    os.imbue(std::locale::classic());
    os << g;
    std::istringstream is(os.str());
    is.imbue(std::locale::classic());
    std::vector<uint64_t> v;
    uint64_t x;
    while (is >> x) v.push_back(x);
    if (v.size() != 312 && v.size() != 313) throw std::runtime_error("hip_mcmc_refine: unknown mt19937_64 text layout");
    sxh_mt64_state st{};
    for (int i = 0; i < 312; i++) st.x[i] = v[static_cast<size_t>(i)];
    st.p = v.size() == 313 ? static_cast<uint32_t>(v[312]) : 312u;
    return st;
}

void mt_state_to(const sxh_mt64_state& st, std::mt19937_64& g) {
    std::ostringstream probe;
    probe.imbue(std::locale::classic());
    probe << g;
    std::istringstream count_is(probe.str());
    size_t n = 0;
    for (uint64_t x; count_is >> x;) n++;
    std::ostringstream os;
    os.imbue(std::locale::classic());
    for (int i = 0; i < 312; i++) os << st.x[i] << (i + 1 < 312 ? " " : "");
    if (n == 313) os << ' ' << st.p;
    else if (st.p != 312)  // this library's text form holds no position
        throw std::runtime_error("hip_mcmc_refine: engine position not expressible in this C++ library's text form");
    std::istringstream is(os.str());
    is.imbue(std::locale::classic());
    is >> g;
    if (!is) throw std::runtime_error("hip_mcmc_refine: engine state rejected");
}

} // namespace

sxh_executor* hip_executor_handle(TrainStepExecutor& exec) {
    auto* hx = dynamic_cast<HipTrainStepExecutor*>(&exec);
    if (!hx) throw std::invalid_argument("hip_executor_handle: executor was not made by make_hip_backend");
    return hx->handle();
}

HipMcmcRefineResult hip_mcmc_refine(TrainStepExecutor& exec, std::mt19937_64& rng, const HipMcmcRefineInputs& in) {
    auto* hx = dynamic_cast<HipTrainStepExecutor*>(&exec);
    if (!hx) throw std::invalid_argument("hip_mcmc_refine: executor was not made by make_hip_backend");
    if (!in.binoms) throw std::invalid_argument("hip_mcmc_refine: null binoms");
    sxh_mt64_state st = mt_state_of(rng);
    sxh_refine_inputs c{};
    c.count = in.count;
    c.cap_max = in.cap_max;
    c.min_opacity = in.min_opacity;
    c.n_max = static_cast<int32_t>(std::lround(std::sqrt(static_cast<double>(in.binoms->size()))));
    c.binoms = in.binoms->data();
    c.rng = &st;
    c.inject_noise = in.inject_noise ? 1 : 0;
    c.noise_seed = in.noise_seed;
    c.noise_offset = in.noise_offset;
    c.noise_scale = in.noise_scale;
    HipMcmcRefineResult r;
    const size_t cap = sz(in.cap_max);
    r.relocated_dead.resize(cap);
    r.relocation_src.resize(cap);
    r.added_src.resize(cap);
    sxh_refine_outputs o{};
    o.relocated_dead = data_or_null(r.relocated_dead);
    o.relocation_src = data_or_null(r.relocation_src);
    o.added_src = data_or_null(r.added_src);
    o.capacity = in.cap_max;
    const int32_t rc = sxh_exec_mcmc_refine(hx->handle(), &c, &o);
    mt_state_to(st, rng);  // the engine advanced by the draws made, also when a phase failed
    check(rc);
    r.count = o.count;
    r.relocated_dead.resize(sz(o.n_relocated));
    r.relocation_src.resize(sz(o.n_relocated));
    r.added_src.resize(sz(o.n_added));
    return r;
}

std::unique_ptr<KernelBackend> make_hip_backend(const HipBackendDesc& desc) {
    return std::make_unique<HipKernelBackend>(desc.device_ordinal);
}

} // namespace splatx
