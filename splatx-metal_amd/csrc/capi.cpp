// capi.cpp — the C ABI per-op entry points (include/splatx_hip.h): the verification surface that
// replaces the reference's per-op KernelBackend methods (MetalBackend.cpp:247-1412).
//
// Each call validates like Validate.h, stages the host inputs into device memory on the backend's
// stream, runs the gfx950 kernels, copies the outputs back and synchronizes — the blocking,
// commit-and-wait semantics of the reference boundary.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <numeric>
#include <string>

#include "splatx_hip.h"
#include "sx_host.h"
#include "sx_kernels.h"

namespace sxh {
namespace {
thread_local std::string g_last_error;

void sync(sxh_backend* b) { SXH_HIP(hipStreamSynchronize(b->stream)); }
void need(const void* p, const char* what, const char* name) {
    if (!p) invalid(what, std::string("null ") + name);
}
sxk::ProjArgs proj_args(const sxh_projection_inputs& in, const float* means, const float* covars,
                        const float* quats, const float* scales, const float* opac, const float* vm,
                        const float* Ks) {
    sxk::ProjArgs a{};
    a.means = means; a.covars = covars; a.quats = quats; a.scales = scales; a.opacities = opac;
    a.viewmats = vm; a.Ks = Ks;
    a.N = static_cast<int>(in.N); a.C = static_cast<int>(in.C);
    a.width = in.width; a.height = in.height;
    a.eps2d = in.eps2d; a.near_plane = in.near_plane; a.far_plane = in.far_plane;
    a.radius_clip = in.radius_clip; a.calc_comp = in.calc_compensations ? 1 : 0;
    return a;
}
} // namespace
void set_last_error(const std::string& msg) { g_last_error = msg; }
const char* last_error() { return g_last_error.c_str(); }
} // namespace sxh

using namespace sxh;

extern "C" {

int32_t sxh_abi_version(void) { return SXH_ABI_VERSION; }
const char* sxh_last_error(void) { return sxh::last_error(); }

int32_t sxh_backend_create(int32_t device_ordinal, sxh_backend** out) {
    return guarded([&] {
        if (!out) invalid("sxh_backend_create", "null out");
        int count = 0;
        SXH_HIP(hipGetDeviceCount(&count));
        if (device_ordinal < 0 || device_ordinal >= count)
            throw std::runtime_error("sxh_backend_create: no HIP device " + std::to_string(device_ordinal));
        SXH_HIP(hipSetDevice(device_ordinal));
        hipDeviceProp_t prop;
        SXH_HIP(hipGetDeviceProperties(&prop, device_ordinal));
        auto* b = new sxh_backend();
        b->device = device_ordinal;
        b->name = std::string("hip-gfx950:") + prop.gcnArchName;
        try {
            SXH_HIP(hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking));
            SXH_HIP(hipHostMalloc(reinterpret_cast<void**>(&b->pinned_word), sizeof(uint32_t), hipHostMallocDefault));
            noalloc_init(device_ordinal);  // the allocation-free entry points' scratch on this device
        } catch (...) {
            sxh_backend_destroy(b);
            throw;
        }
        *out = b;
    });
}

void sxh_backend_destroy(sxh_backend* b) {
    if (!b) return;
    if (b->stream) (void)hipStreamDestroy(b->stream);
    if (b->pinned_word) (void)hipHostFree(b->pinned_word);
    delete b;
}

const char* sxh_backend_name(const sxh_backend* b) { return b ? b->name.c_str() : ""; }

int32_t sxh_make_binoms_lut(int32_t n_max, float* out) {
    return guarded([&] {
        if (n_max < 1) invalid("make_binoms_lut", "n_max must be >= 1");
        need(out, "make_binoms_lut", "out");
        // Pascal's triangle in u64 (exact up to n_max = 51), cast to float (CpuKernels.cpp:906-917)
        std::vector<uint64_t> row(static_cast<size_t>(n_max), 0);
        std::fill(out, out + static_cast<size_t>(n_max) * n_max, 0.0f);
        for (int n = 0; n < n_max; n++) {
            for (int k = n; k >= 1; k--) row[k] += row[k - 1];
            row[0] = 1;
            for (int k = 0; k <= n; k++) out[static_cast<size_t>(n) * n_max + k] = static_cast<float>(row[k]);
        }
    });
}

// ---- fused_adam --------------------------------------------------------------------------------
int32_t sxh_fused_adam(sxh_backend* b, const sxh_adam_inputs* in) {
    return guarded([&] {
        need(in, "fused_adam", "inputs");
        if (in->n_elems != 0) validate_adam(*in, "fused_adam");  // empty: dispatch skip before validation (D8-6)
        need(b, "fused_adam", "backend");
        if (in->n_elems == 0) return;
        SXH_HIP(hipSetDevice(b->device));
        const size_t n = static_cast<size_t>(in->n_elems);
        auto p = upload(in->param, n, b->stream);
        auto g = upload(in->grad, n, b->stream);
        auto m = upload(in->exp_avg, n, b->stream);
        auto v = upload(in->exp_avg_sq, n, b->stream);
        DevBuf<uint8_t> valid;
        if (in->valid) valid = upload(in->valid, static_cast<size_t>(in->n_gauss), b->stream);
        sxk::adam(p.p, g.p, m.p, v.p, valid.p, in->n_elems, in->n_elems / in->n_gauss, in->lr, in->b1, in->b2,
                  in->eps, b->stream);
        SXH_HIP(hipGetLastError());
        download(in->param, p, n, b->stream);
        download(in->exp_avg, m, n, b->stream);
        download(in->exp_avg_sq, v, n, b->stream);
        sync(b);
    });
}

// ---- projection ------------------------------------------------------------------------------
int32_t sxh_projection_fused_fwd(sxh_backend* b, const sxh_projection_inputs* in, sxh_projection_outputs* out) {
    return guarded([&] {
        need(in, "projection_fused_fwd", "inputs");
        need(out, "projection_fused_fwd", "outputs");
        validate_projection(*in, "projection_fused_fwd");
        const size_t N = static_cast<size_t>(in->N), C = static_cast<size_t>(in->C), CN = N * C;
        if (!out->radii || !out->means2d || !out->depths || !out->conics ||
            (in->calc_compensations && !out->compensations))
            invalid("projection_fused_fwd", "null output buffer");
        need(b, "projection_fused_fwd", "backend");
        if (CN == 0) return;
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto means = upload(in->means, N * 3, s);
        DevBuf<float> covars, quats, scales, opac;
        if (in->covars) covars = upload(in->covars, N * 6, s);
        else {
            quats = upload(in->quats, N * 4, s);
            scales = upload(in->scales, N * 3, s);
        }
        if (in->opacities) opac = upload(in->opacities, N, s);
        auto vm = upload(in->viewmats, C * 16, s);
        auto K = upload(in->Ks, C * 9, s);
        auto radii = zeros<int32_t>(CN * 2, s);
        auto m2 = zeros<float>(CN * 2, s);
        auto dep = zeros<float>(CN, s);
        auto con = zeros<float>(CN * 3, s);
        auto comp = zeros<float>(in->calc_compensations ? CN : 0, s);
        sxk::projection_fwd(proj_args(*in, means.p, covars.p, quats.p, scales.p, opac.p, vm.p, K.p), radii.p, m2.p,
                            dep.p, con.p, comp.p, s);
        SXH_HIP(hipGetLastError());
        download(out->radii, radii, CN * 2, s);
        download(out->means2d, m2, CN * 2, s);
        download(out->depths, dep, CN, s);
        download(out->conics, con, CN * 3, s);
        if (in->calc_compensations) download(out->compensations, comp, CN, s);
        sync(b);
    });
}

int32_t sxh_projection_fused_bwd(sxh_backend* b, const sxh_projection_inputs* in, const sxh_projection_grads_in* g,
                                 sxh_projection_grads* out) {
    return guarded([&] {
        need(in, "projection_fused_bwd", "inputs");
        need(g, "projection_fused_bwd", "grads_in");
        need(out, "projection_fused_bwd", "outputs");
        validate_projection(*in, "projection_fused_bwd");
        validate_projection_grads(*g, "projection_fused_bwd");
        const size_t N = static_cast<size_t>(in->N), C = static_cast<size_t>(in->C), CN = N * C;
        const bool cov = in->covars != nullptr;
        need(out->v_means, "projection_fused_bwd", "v_means");
        if (cov) need(out->v_covars, "projection_fused_bwd", "v_covars");
        else {
            need(out->v_quats, "projection_fused_bwd", "v_quats");
            need(out->v_scales, "projection_fused_bwd", "v_scales");
        }
        if (g->viewmats_grad) need(out->v_viewmats, "projection_fused_bwd", "v_viewmats");
        need(b, "projection_fused_bwd", "backend");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto means = upload(in->means, N * 3, s);
        DevBuf<float> covars, quats, scales, comps, vcomps;
        if (cov) covars = upload(in->covars, N * 6, s);
        else {
            quats = upload(in->quats, N * 4, s);
            scales = upload(in->scales, N * 3, s);
        }
        auto vm = upload(in->viewmats, C * 16, s);
        auto K = upload(in->Ks, C * 9, s);
        auto radii = upload(g->radii, CN * 2, s);
        auto con = upload(g->conics, CN * 3, s);
        if (g->v_compensations) {
            comps = upload(g->compensations, CN, s);
            vcomps = upload(g->v_compensations, CN, s);
        }
        auto vm2 = upload(g->v_means2d, CN * 2, s);
        auto vdep = upload(g->v_depths, CN, s);
        auto vcon = upload(g->v_conics, CN * 3, s);
        auto v_means = zeros<float>(N * 3, s);
        auto v_covars = zeros<float>(cov ? N * 6 : 0, s);
        auto v_quats = zeros<float>(cov ? 0 : N * 4, s);
        auto v_scales = zeros<float>(cov ? 0 : N * 3, s);
        auto v_view = zeros<float>(g->viewmats_grad ? C * 16 : 0, s);
        sxk::ProjBwdArgs ga{radii.p, con.p, comps.p, vm2.p, vdep.p, vcon.p, vcomps.p, g->viewmats_grad ? 1 : 0};
        sxk::projection_bwd(proj_args(*in, means.p, covars.p, quats.p, scales.p, nullptr, vm.p, K.p), ga,
                            v_means.p, v_covars.p, v_quats.p, v_scales.p, v_view.p, s);
        SXH_HIP(hipGetLastError());
        download(out->v_means, v_means, N * 3, s);
        if (cov) download(out->v_covars, v_covars, N * 6, s);
        else {
            download(out->v_quats, v_quats, N * 4, s);
            download(out->v_scales, v_scales, N * 3, s);
        }
        if (g->viewmats_grad) download(out->v_viewmats, v_view, C * 16, s);
        sync(b);
    });
}

// ---- SH --------------------------------------------------------------------------------------------
int32_t sxh_sh_fwd(sxh_backend* b, const sxh_sh_inputs* in, float* colors) {
    return guarded([&] {
        need(in, "sh_fwd", "inputs");
        validate_sh(*in, "sh_fwd");
        const size_t BN = static_cast<size_t>(in->B * in->N);
        need(b, "sh_fwd", "backend");
        if (BN == 0) return;
        need(colors, "sh_fwd", "colors");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto dirs = upload(in->dirs, BN * 3, s);
        auto co = upload(in->coeffs, static_cast<size_t>(in->N * in->K) * in->D, s);
        DevBuf<uint8_t> masks;
        if (in->masks) masks = upload(in->masks, BN, s);
        // masked elements are left unwritten: stage the caller's buffer so untouched slots survive
        auto out = upload(colors, BN * in->D, s);
        sxk::sh_fwd(dirs.p, co.p, masks.p, in->degrees_to_use, static_cast<int>(in->B), static_cast<int>(in->N),
                    static_cast<int>(in->K), static_cast<int>(in->D), out.p, s);
        SXH_HIP(hipGetLastError());
        download(colors, out, BN * in->D, s);
        sync(b);
    });
}

int32_t sxh_sh_bwd(sxh_backend* b, const sxh_sh_inputs* in, const float* v_colors, float* v_coeffs, float* v_dirs) {
    return guarded([&] {
        need(in, "sh_bwd", "inputs");
        validate_sh(*in, "sh_bwd");
        const size_t BN = static_cast<size_t>(in->B * in->N);
        const size_t NKD = static_cast<size_t>(in->N * in->K) * in->D;
        need(v_coeffs, "sh_bwd", "v_coeffs");
        if (in->compute_v_dirs) need(v_dirs, "sh_bwd", "v_dirs");
        need(b, "sh_bwd", "backend");
        if (BN == 0) {
            std::fill(v_coeffs, v_coeffs + NKD, 0.0f);
            return;
        }
        need(v_colors, "sh_bwd", "v_colors");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto dirs = upload(in->dirs, BN * 3, s);
        auto co = upload(in->coeffs, NKD, s);
        DevBuf<uint8_t> masks;
        if (in->masks) masks = upload(in->masks, BN, s);
        auto vc = upload(v_colors, BN * in->D, s);
        auto vco = zeros<float>(NKD, s);
        auto vd = zeros<float>(in->compute_v_dirs ? BN * 3 : 0, s);
        sxk::sh_bwd(dirs.p, co.p, masks.p, in->degrees_to_use, static_cast<int>(in->B), static_cast<int>(in->N),
                    static_cast<int>(in->K), static_cast<int>(in->D), vc.p, vco.p,
                    in->compute_v_dirs ? vd.p : nullptr, s);
        SXH_HIP(hipGetLastError());
        download(v_coeffs, vco, NKD, s);
        if (in->compute_v_dirs) download(v_dirs, vd, BN * 3, s);
        sync(b);
    });
}

// ---- isect / scan / sort / offsets ---------------------------------------------------------------
int32_t sxh_isect_tiles(sxh_backend* b, const sxh_isect_inputs* in, sxh_isect_outputs* out) {
    return guarded([&] {
        need(in, "isect_tiles", "inputs");
        need(out, "isect_tiles", "outputs");
        validate_isect(*in, "isect_tiles");
        const int64_t n_el = in->I * in->N;
        out->tile_n_bits = sx::bits_for_count(static_cast<int64_t>(in->tile_width) * in->tile_height);
        out->image_n_bits = sx::bits_for_count(in->I);
        out->n_isects = 0;
        need(b, "isect_tiles", "backend");
        if (n_el == 0) return;
        need(out->tiles_per_gauss, "isect_tiles", "tiles_per_gauss");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        const size_t n = static_cast<size_t>(n_el);
        auto m2 = upload(in->means2d, n * 2, s);
        auto radii = upload(in->radii, n * 2, s);
        auto dep = upload(in->depths, n, s);
        DevBuf<float> con, op;
        if (in->conics) {
            con = upload(in->conics, n * 3, s);
            op = upload(in->opacities, n, s);
        }
        DevBuf<int32_t> tiles(n);
        DevBuf<int64_t> cum(n);
        DevBuf<uint8_t> scratch(sxk::scan_scratch_bytes(n_el));
        sxk::IsectArgs a{m2.p, radii.p, dep.p, con.p, op.p, static_cast<int>(in->I), static_cast<int>(in->N),
                         static_cast<int>(in->tile_size), static_cast<int>(in->tile_width),
                         static_cast<int>(in->tile_height), out->tile_n_bits};
        // The reference validates depth >= 0 before emit (CpuKernels.cpp:635-637): check on the host.
        sxk::isect_count(a, tiles.p, s);
        sxk::scan_i32_i64(tiles.p, cum.p, n_el, scratch.p, s);
        SXH_HIP(hipGetLastError());
        download(out->tiles_per_gauss, tiles, n, s);
        int64_t total = 0;
        SXH_HIP(hipMemcpyAsync(&total, cum.p + (n - 1), sizeof(int64_t), hipMemcpyDeviceToHost, s));
        sync(b);
        out->n_isects = total;
        if (total == 0) return;
        for (size_t i = 0; i < n; i++)
            if (in->radii[i * 2] > 0 && in->radii[i * 2 + 1] > 0 && !(in->depths[i] >= 0.f))
                invalid("isect_tiles", "depth must be >= 0 at idx " + std::to_string(i));
        if (out->capacity < total)
            throw CapacityError("isect_tiles: capacity " + std::to_string(out->capacity) + " < n_isects " +
                                std::to_string(total));
        need(out->isect_ids, "isect_tiles", "isect_ids");
        need(out->flatten_ids, "isect_tiles", "flatten_ids");
        DevBuf<uint64_t> keys(static_cast<size_t>(total));
        DevBuf<int32_t> vals(static_cast<size_t>(total));
        sxk::isect_emit(a, cum.p, keys.p, vals.p, s);
        SXH_HIP(hipGetLastError());
        download(out->isect_ids, keys, static_cast<size_t>(total), s);
        download(out->flatten_ids, vals, static_cast<size_t>(total), s);
        sync(b);
    });
}

int32_t sxh_prefix_scan_i64(sxh_backend* b, const int32_t* in, int64_t n, int64_t* out) {
    return guarded([&] {
        if (n < 0) invalid("prefix_scan_i64", "negative n");
        need(b, "prefix_scan_i64", "backend");
        if (n == 0) return;
        need(in, "prefix_scan_i64", "in");
        need(out, "prefix_scan_i64", "out");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto d_in = upload(in, static_cast<size_t>(n), s);
        DevBuf<int64_t> d_out(static_cast<size_t>(n));
        DevBuf<uint8_t> scratch(sxk::scan_scratch_bytes(n));
        sxk::scan_i32_i64(d_in.p, d_out.p, n, scratch.p, s);
        SXH_HIP(hipGetLastError());
        download(out, d_out, static_cast<size_t>(n), s);
        sync(b);
    });
}

int32_t sxh_sort_isect(sxh_backend* b, const sxh_sort_inputs* in, uint64_t* keys_sorted, int32_t* values_sorted) {
    return guarded([&] {
        need(in, "sort_isect", "inputs");
        validate_sort(*in, "sort_isect");
        const size_t n = static_cast<size_t>(in->n);
        need(b, "sort_isect", "backend");
        if (n == 0) return;
        need(keys_sorted, "sort_isect", "keys_sorted");
        need(values_sorted, "sort_isect", "values_sorted");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto ka = upload(in->keys, n, s);
        auto va = upload(in->values, n, s);
        DevBuf<uint64_t> kb(n);
        DevBuf<int32_t> vb(n);
        DevBuf<uint8_t> scratch(sxk::sort_scratch_bytes(in->n));
        const int which = sxk::radix_sort(ka.p, va.p, kb.p, vb.p, in->n, in->key_n_bits, scratch.p, s);
        uint32_t sort_err = 0;
        SXH_HIP(hipMemcpyAsync(&sort_err, sxk::sort_error_flag(scratch.p), 4, hipMemcpyDeviceToHost, s));
        SXH_HIP(hipStreamSynchronize(s));
        if (sort_err) throw std::runtime_error("sort_isect: radix sort look-back did not complete");
        SXH_HIP(hipGetLastError());
        download(keys_sorted, which ? kb : ka, n, s);
        download(values_sorted, which ? vb : va, n, s);
        sync(b);
    });
}

int32_t sxh_isect_offset_encode(sxh_backend* b, const sxh_offset_inputs* in, int32_t* offsets) {
    return guarded([&] {
        need(in, "isect_offset_encode", "inputs");
        validate_offsets(*in, "isect_offset_encode");
        const int64_t n_tiles = static_cast<int64_t>(in->tile_width) * in->tile_height;
        const size_t total = static_cast<size_t>(in->I * n_tiles);
        need(b, "isect_offset_encode", "backend");
        if (total == 0) return;
        need(offsets, "isect_offset_encode", "offsets");
        if (in->n_isects == 0) {  // offsets.fill_(0) (CpuKernels.cpp:713)
            std::fill(offsets, offsets + total, 0);
            return;
        }
        // keys are caller data: their (image, tile) field must address the offsets table
        const uint32_t tnb = sx::bits_for_count(n_tiles);
        for (int64_t k = 0; k < in->n_isects; k++) {
            const uint64_t id = in->isect_ids[k] >> 32;
            const uint64_t flat = (id >> tnb) * static_cast<uint64_t>(n_tiles) + (id & ((1ull << tnb) - 1));
            if ((id & ((1ull << tnb) - 1)) >= static_cast<uint64_t>(n_tiles) || flat >= total)
                invalid("isect_offset_encode", "isect_ids[" + std::to_string(k) + "] addresses no tile");
        }
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto keys = upload(in->isect_ids, static_cast<size_t>(in->n_isects), s);
        auto off = zeros<int32_t>(total, s);
        sxk::offset_encode(keys.p, in->n_isects, static_cast<int>(in->I), static_cast<int>(n_tiles),
                           sx::bits_for_count(n_tiles), off.p, s);
        SXH_HIP(hipGetLastError());
        download(offsets, off, total, s);
        sync(b);
    });
}

// ---- raster -----------------------------------------------------------------------------------------
namespace {
struct RasterStage {
    DevBuf<float4> splats;
    DevBuf<int32_t> offsets, flat;
    DevBuf<float> bg;
    DevBuf<uint8_t> masks;
    sxk::RasterArgs args{};
};
void stage_raster(const sxh_raster_inputs& in, hipStream_t s, RasterStage& st) {
    const size_t n = static_cast<size_t>(in.I * in.N);
    const size_t n_tiles = static_cast<size_t>(in.tile_width) * in.tile_height;
    // Index inputs are caller data: keep every device gather in bounds.
    for (size_t t = 0; t < static_cast<size_t>(in.I) * n_tiles; t++)
        if (in.isect_offsets[t] < 0 || in.isect_offsets[t] > in.n_isects)
            invalid("rasterize", "isect_offsets[" + std::to_string(t) + "] outside [0, n_isects]");
    for (int64_t k = 0; k < in.n_isects; k++)
        if (in.flatten_ids[k] < 0 || static_cast<size_t>(in.flatten_ids[k]) >= n)
            invalid("rasterize", "flatten_ids[" + std::to_string(k) + "] outside [0, I*N)");
    auto m2 = upload(in.means2d, n * 2, s);
    auto cn = upload(in.conics, n * 3, s);
    auto col = upload(in.colors, n * 3, s);
    auto op = upload(in.opacities, n, s);
    st.splats.alloc(std::max<size_t>(n, 1) * 3);
    sxk::pack_splats(m2.p, cn.p, col.p, op.p, static_cast<int>(n), st.splats.p, s);
    st.offsets = upload(in.isect_offsets, static_cast<size_t>(in.I) * n_tiles, s);
    if (in.n_isects > 0) st.flat = upload(in.flatten_ids, static_cast<size_t>(in.n_isects), s);
    if (in.backgrounds) st.bg = upload(in.backgrounds, static_cast<size_t>(in.I) * 3, s);
    if (in.masks) st.masks = upload(in.masks, static_cast<size_t>(in.I) * n_tiles, s);
    st.args.splats = st.splats.p;
    st.args.offsets = st.offsets.p;
    st.args.flatten_ids = st.flat.p;
    st.args.backgrounds = st.bg.p;
    st.args.masks = st.masks.p;
    st.args.I = static_cast<int>(in.I);
    st.args.width = static_cast<int>(in.image_width);
    st.args.height = static_cast<int>(in.image_height);
    st.args.tile_width = static_cast<int>(in.tile_width);
    st.args.tile_height = static_cast<int>(in.tile_height);
    st.args.n_isects = static_cast<int32_t>(in.n_isects);
    SXH_HIP(hipStreamSynchronize(s));  // the temporary SoA inputs go out of scope here
}
} // namespace

int32_t sxh_rasterize_fwd(sxh_backend* b, const sxh_raster_inputs* in, sxh_raster_outputs* out) {
    return guarded([&] {
        need(in, "rasterize_fwd", "inputs");
        need(out, "rasterize_fwd", "outputs");
        validate_raster(*in, "rasterize_fwd");
        const size_t P = static_cast<size_t>(in->I) * in->image_width * in->image_height;
        need(b, "rasterize_fwd", "backend");
        if (P == 0) return;
        if (!out->render_colors || !out->render_alphas || !out->last_ids) invalid("rasterize_fwd", "null output buffer");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        RasterStage st;
        stage_raster(*in, s, st);
        DevBuf<float> rgb(P * 3), alpha(P);
        DevBuf<int32_t> last(P);
        sxk::raster_fwd(st.args, rgb.p, alpha.p, last.p, s);  // always runs: background of empty tiles
        SXH_HIP(hipGetLastError());
        download(out->render_colors, rgb, P * 3, s);
        download(out->render_alphas, alpha, P, s);
        download(out->last_ids, last, P, s);
        sync(b);
    });
}

int32_t sxh_rasterize_bwd(sxh_backend* b, const sxh_raster_inputs* in, const sxh_raster_grads_in* g,
                          sxh_raster_grads* out) {
    return guarded([&] {
        need(in, "rasterize_bwd", "inputs");
        need(g, "rasterize_bwd", "grads_in");
        need(out, "rasterize_bwd", "outputs");
        validate_raster(*in, "rasterize_bwd");
        validate_raster_grads(*g, "rasterize_bwd");
        const size_t n = static_cast<size_t>(in->I * in->N);
        const size_t P = static_cast<size_t>(in->I) * in->image_width * in->image_height;
        if (!out->v_means2d || !out->v_conics || !out->v_colors || !out->v_opacities ||
            (g->absgrad && !out->v_means2d_abs))
            invalid("rasterize_bwd", "null output buffer");
        need(b, "rasterize_bwd", "backend");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto vm2 = zeros<float>(n * 2, s);
        auto vcn = zeros<float>(n * 3, s);
        auto vcol = zeros<float>(n * 3, s);
        auto vop = zeros<float>(n, s);
        auto vabs = zeros<float>(g->absgrad ? n * 2 : 0, s);
        if (in->n_isects > 0 && P > 0) {
            RasterStage st;
            stage_raster(*in, s, st);
            auto ra = upload(g->render_alphas, P, s);
            auto li = upload(g->last_ids, P, s);
            auto vrc = upload(g->v_render_colors, P * 3, s);
            auto vra = upload(g->v_render_alphas, P, s);
            sxk::RasterBwdGrads gg{vm2.p, vcn.p, vcol.p, vop.p, g->absgrad ? vabs.p : nullptr, nullptr};
            sxk::raster_bwd(st.args, ra.p, li.p, vrc.p, vra.p, gg, s);
            SXH_HIP(hipGetLastError());
            sync(b);
        }
        download(out->v_means2d, vm2, n * 2, s);
        download(out->v_conics, vcn, n * 3, s);
        download(out->v_colors, vcol, n * 3, s);
        download(out->v_opacities, vop, n, s);
        if (g->absgrad) download(out->v_means2d_abs, vabs, n * 2, s);
        sync(b);
    });
}

// ---- RNG / MCMC ---------------------------------------------------------------------------------------
int32_t sxh_rng_normal_f32(sxh_backend* b, const sxh_rng_inputs* in, float* out) {
    return guarded([&] {
        need(in, "rng_normal_f32", "inputs");
        validate_rng(*in, "rng_normal_f32");
        need(b, "rng_normal_f32", "backend");
        if (in->count == 0) return;
        need(out, "rng_normal_f32", "out");
        SXH_HIP(hipSetDevice(b->device));
        DevBuf<float> d(static_cast<size_t>(in->count));
        sxk::rng_normal_f32(in->seed, in->offset, in->count, d.p, b->stream);
        SXH_HIP(hipGetLastError());
        download(out, d, static_cast<size_t>(in->count), b->stream);
        sync(b);
    });
}

int32_t sxh_rng_philox_u32(sxh_backend* b, const sxh_rng_inputs* in, uint32_t* out) {
    return guarded([&] {
        need(in, "rng_philox_u32", "inputs");
        validate_rng(*in, "rng_philox_u32");
        need(b, "rng_philox_u32", "backend");
        if (in->count == 0) return;
        need(out, "rng_philox_u32", "out");
        SXH_HIP(hipSetDevice(b->device));
        DevBuf<uint32_t> d(static_cast<size_t>(in->count));
        sxk::rng_philox_u32(in->seed, in->offset, in->count, d.p, b->stream);
        SXH_HIP(hipGetLastError());
        download(out, d, static_cast<size_t>(in->count), b->stream);
        sync(b);
    });
}

int32_t sxh_mcmc_relocation(sxh_backend* b, const sxh_relocation_inputs* in, float* new_op, float* new_sc) {
    return guarded([&] {
        need(in, "mcmc_relocation", "inputs");
        validate_relocation(*in, "mcmc_relocation");
        const size_t N = static_cast<size_t>(in->N);
        need(b, "mcmc_relocation", "backend");
        if (N == 0) return;
        need(new_op, "mcmc_relocation", "new_opacities");
        need(new_sc, "mcmc_relocation", "new_scales");
        // the host clamp contract (relocation.py:61-62), checked on the host before launch
        for (size_t i = 0; i < N; i++)
            if (in->ratios[i] < 1 || in->ratios[i] > in->n_max)
                invalid("mcmc_relocation", "ratios[" + std::to_string(i) + "] out of [1, n_max] (host clamp contract)");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto op = upload(in->opacities, N, s);
        auto sc = upload(in->scales, N * 3, s);
        auto ra = upload(in->ratios, N, s);
        auto bi = upload(in->binoms, static_cast<size_t>(in->n_max) * in->n_max, s);
        DevBuf<float> no(N), ns(N * 3);
        sxk::mcmc_relocation(op.p, sc.p, ra.p, bi.p, static_cast<int>(N), in->n_max, in->min_opacity, no.p, ns.p, s);
        SXH_HIP(hipGetLastError());
        download(new_op, no, N, s);
        download(new_sc, ns, N * 3, s);
        sync(b);
    });
}

int32_t sxh_mcmc_perturb_positions(sxh_backend* b, const sxh_perturb_inputs* in) {
    return guarded([&] {
        need(in, "mcmc_perturb_positions", "inputs");
        if (in->N != 0) validate_perturb(*in, "mcmc_perturb_positions");  // empty: skip before validation
        need(b, "mcmc_perturb_positions", "backend");
        if (in->N == 0) return;
        const size_t N = static_cast<size_t>(in->N);
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto pos = upload(in->positions, N * 3, s);
        auto q = upload(in->quats, N * 4, s);
        auto sl = upload(in->scales_log, N * 3, s);
        auto lg = upload(in->opacities_logit, N, s);
        auto nz = upload(in->noise, N * 3, s);
        sxk::mcmc_perturb(pos.p, q.p, sl.p, lg.p, nz.p, static_cast<int>(N), in->noise_scale, in->t, in->k, s);
        SXH_HIP(hipGetLastError());
        download(in->positions, pos, N * 3, s);
        sync(b);
    });
}

// ---- SSIM ---------------------------------------------------------------------------------------------
int32_t sxh_ssim_fwd(sxh_backend* b, const sxh_ssim_inputs* in, sxh_ssim_outputs* out) {
    return guarded([&] {
        need(in, "ssim_fwd", "inputs");
        need(out, "ssim_fwd", "outputs");
        validate_ssim(*in, "ssim_fwd");
        const int I = static_cast<int>(in->I), H = static_cast<int>(in->H), W = static_cast<int>(in->W),
                  C = static_cast<int>(in->C);
        const size_t n = static_cast<size_t>(I) * H * W * C;
        const size_t M = static_cast<size_t>(I) * (H - 10) * (W - 10) * C;
        if (!out->ssim_map || (in->need_coeffs && (!out->coeff_mu || !out->coeff_sigma || !out->coeff_cross)))
            invalid("ssim_fwd", "null output buffer");
        need(b, "ssim_fwd", "backend");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto a = upload(in->img1, n, s);
        auto g = upload(in->img2, n, s);
        DevBuf<float> map(M), mu(in->need_coeffs ? M : 0), sg(in->need_coeffs ? M : 0), cr(in->need_coeffs ? M : 0);
        sxk::ssim_fwd(a.p, g.p, I, H, W, C, in->need_coeffs ? 1 : 0, map.p, mu.p, sg.p, cr.p, nullptr, s);
        SXH_HIP(hipGetLastError());
        download(out->ssim_map, map, M, s);
        if (in->need_coeffs) {
            download(out->coeff_mu, mu, M, s);
            download(out->coeff_sigma, sg, M, s);
            download(out->coeff_cross, cr, M, s);
        }
        sync(b);
        double sum = 0.0;  // ssim_reduce_mean_f64 (CpuKernels.h:198-202): ascending-index f64 sum
        for (size_t i = 0; i < M; i++) sum += static_cast<double>(out->ssim_map[i]);
        out->ssim = sum / static_cast<double>(M);
    });
}

int32_t sxh_ssim_bwd(sxh_backend* b, const sxh_ssim_inputs* in, const sxh_ssim_grads_in* gin, float* v_img1) {
    return guarded([&] {
        need(in, "ssim_bwd", "inputs");
        need(gin, "ssim_bwd", "grads_in");
        validate_ssim(*in, "ssim_bwd");
        validate_ssim_grads(*gin, "ssim_bwd");
        need(v_img1, "ssim_bwd", "v_img1");
        const int I = static_cast<int>(in->I), H = static_cast<int>(in->H), W = static_cast<int>(in->W),
                  C = static_cast<int>(in->C);
        const size_t n = static_cast<size_t>(I) * H * W * C;
        const size_t M = static_cast<size_t>(I) * (H - 10) * (W - 10) * C;
        need(b, "ssim_bwd", "backend");
        SXH_HIP(hipSetDevice(b->device));
        hipStream_t s = b->stream;
        auto a = upload(in->img1, n, s);
        auto g = upload(in->img2, n, s);
        auto mu = upload(gin->coeff_mu, M, s);
        auto sg = upload(gin->coeff_sigma, M, s);
        auto cr = upload(gin->coeff_cross, M, s);
        DevBuf<float> v(n);
        const float G = static_cast<float>(-static_cast<double>(gin->v_loss) / static_cast<double>(M));
        sxk::ssim_bwd(a.p, g.p, mu.p, sg.p, cr.p, I, H, W, C, G, v.p, s);
        SXH_HIP(hipGetLastError());
        download(v_img1, v, n, s);
        sync(b);
    });
}

} // extern "C"
