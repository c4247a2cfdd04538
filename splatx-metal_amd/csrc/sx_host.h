// sx_host.h — host runtime helpers of the C ABI: error mapping, device buffers, entry validation.
//
// Validation restates the reference's shared validators (Sources/SplatXCore/include/splatx/
// Validate.h:40-263) on the C structs: the same conditions raise InvalidArgument (SXH_ERR_INVALID_
// ARGUMENT, the reference's std::invalid_argument) with the same messages; device and allocation
// failures raise RuntimeError (SXH_ERR_RUNTIME).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "splatx_hip.h"
#include "sx_common.h"

namespace sxh {

struct InvalidArgument : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct CapacityError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] inline void invalid(const char* what, const std::string& msg) {
    throw InvalidArgument(std::string(what) + ": " + msg);
}

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
}
#define SXH_HIP(call) ::sxh::hip_check((call), #call)

void set_last_error(const std::string& msg);

template <class F>
int32_t guarded(F&& f) {
    try {
        f();
        return SXH_OK;
    } catch (const std::invalid_argument& e) {
        set_last_error(e.what());
        return SXH_ERR_INVALID_ARGUMENT;
    } catch (const CapacityError& e) {
        set_last_error(e.what());
        return SXH_ERR_CAPACITY;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return SXH_ERR_RUNTIME;
    } catch (...) {
        set_last_error("unknown error");
        return SXH_ERR_RUNTIME;
    }
}

// Owning device allocation.
template <class T>
struct DevBuf {
    T* p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    explicit DevBuf(size_t count) { alloc(count); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), n(o.n) { o.p = nullptr; o.n = 0; }
    DevBuf& operator=(DevBuf&& o) noexcept {
        if (this != &o) { release(); p = o.p; n = o.n; o.p = nullptr; o.n = 0; }
        return *this;
    }
    ~DevBuf() { release(); }
    void alloc(size_t count) {
        release();
        n = count;
        if (count) SXH_HIP(hipMalloc(reinterpret_cast<void**>(&p), std::max<size_t>(count * sizeof(T), 16)));
    }
    void ensure(size_t count) {
        if (count > n) alloc(count);
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    size_t bytes() const { return n * sizeof(T); }
};

template <class T>
DevBuf<T> upload(const T* host, size_t count, hipStream_t s) {
    DevBuf<T> d(count);
    if (count && host) SXH_HIP(hipMemcpyAsync(d.p, host, count * sizeof(T), hipMemcpyHostToDevice, s));
    return d;
}
template <class T>
DevBuf<T> zeros(size_t count, hipStream_t s) {
    DevBuf<T> d(count);
    if (count) SXH_HIP(hipMemsetAsync(d.p, 0, count * sizeof(T), s));
    return d;
}
template <class T>
void download(T* host, const DevBuf<T>& d, size_t count, hipStream_t s) {
    if (count && host) SXH_HIP(hipMemcpyAsync(host, d.p, count * sizeof(T), hipMemcpyDeviceToHost, s));
}

// ---- validators (Validate.h) -----------------------------------------------------------------
inline void validate_adam(const sxh_adam_inputs& in, const char* what) {
    if (!in.param || !in.grad || !in.exp_avg || !in.exp_avg_sq) invalid(what, "null tensor");
    if (in.n_elems < 0 || in.n_gauss <= 0 || in.n_elems % in.n_gauss != 0)
        invalid(what, "n_elems must be a positive multiple of n_gauss");
}

inline void validate_projection(const sxh_projection_inputs& in, const char* what) {
    if (in.camera_model != 0)
        throw std::runtime_error(std::string(what) + ": only PINHOLE (camera_model=0) supported in Phase 1");
    if (!in.means || !in.viewmats || !in.Ks) invalid(what, "null means/viewmats/Ks");
    if (!in.covars && (!in.quats || !in.scales)) invalid(what, "need covars (6-triu) or quats+scales");
    if (in.N < 0 || in.C < 0) invalid(what, "negative N or C");
    if (in.C * in.N > INT32_MAX) invalid(what, "C*N must fit in int32");
}

inline void validate_projection_grads(const sxh_projection_grads_in& g, const char* what) {
    if (!g.radii || !g.conics || !g.v_means2d || !g.v_depths || !g.v_conics)
        invalid(what, "null radii/conics/v_means2d/v_depths/v_conics");
    if (g.v_compensations && !g.compensations)
        invalid(what, "v_compensations requires compensations (fwd output)");
}

inline void validate_sh(const sxh_sh_inputs& in, const char* what) {
    if (!in.dirs || !in.coeffs) invalid(what, "null dirs/coeffs");
    if (in.B < 0 || in.N < 0) invalid(what, "negative B or N");
    if (in.K < 1 || in.D == 0) invalid(what, "K and D must be positive");
    if (in.degrees_to_use > 4) invalid(what, "degrees_to_use must be 0..4");
    const int64_t bands = static_cast<int64_t>(in.degrees_to_use) + 1;
    if (bands * bands > in.K) invalid(what, "(degrees_to_use+1)^2 must be <= K");
    if (in.B * in.N > INT32_MAX || in.N * in.K * in.D > INT32_MAX) invalid(what, "sizes must fit in int32");
}

inline void validate_isect(const sxh_isect_inputs& in, const char* what) {
    if (!in.means2d || !in.radii || !in.depths) invalid(what, "null means2d/radii/depths");
    if ((in.conics != nullptr) != (in.opacities != nullptr))
        invalid(what, "conics and opacities must be given together (AccuTile) or both null (AABB)");
    if (in.I < 0 || in.N < 0) invalid(what, "negative I or N");
    if (in.tile_size == 0 || in.tile_width == 0 || in.tile_height == 0)
        invalid(what, "tile_size/tile_width/tile_height must be positive");
    const uint32_t tile_n_bits = sx::bits_for_count(static_cast<int64_t>(in.tile_width) * in.tile_height);
    const uint32_t image_n_bits = sx::bits_for_count(in.I);
    if (image_n_bits + tile_n_bits > 32) invalid(what, "image_n_bits + tile_n_bits must be <= 32");
    if (in.N > 0 && in.I > INT32_MAX / in.N) invalid(what, "I*N must fit in int32 (flatten_ids)");
}

inline void validate_sort(const sxh_sort_inputs& in, const char* what) {
    if (in.n < 0) invalid(what, "negative n");
    if (in.n > 0 && (!in.keys || !in.values)) invalid(what, "null keys/values");
    if (in.n > INT32_MAX) invalid(what, "n must fit in int32 (flatten_ids/GPU params)");
    if (in.key_n_bits < 1 || in.key_n_bits > 64) invalid(what, "key_n_bits must be 1..64");
}

inline void validate_offsets(const sxh_offset_inputs& in, const char* what) {
    if (in.n_isects < 0) invalid(what, "negative n_isects");
    if (in.n_isects > 0 && !in.isect_ids) invalid(what, "null isect_ids");
    if (in.I < 0) invalid(what, "negative I");
    if (in.n_isects > 0 && in.I == 0) invalid(what, "n_isects > 0 requires I > 0 (keys encode image ids)");
    if (in.tile_width == 0 || in.tile_height == 0) invalid(what, "tile_width/tile_height must be positive");
    const int64_t n_tiles = static_cast<int64_t>(in.tile_width) * in.tile_height;
    if (sx::bits_for_count(in.I) + sx::bits_for_count(n_tiles) > 32)
        invalid(what, "image_n_bits + tile_n_bits must be <= 32");
    if (in.n_isects > INT32_MAX) invalid(what, "n_isects must fit in int32 (offsets values)");
    if (in.I > 0 && n_tiles > INT32_MAX / in.I) invalid(what, "I*n_tiles must fit in int32 (offsets table)");
}

inline void validate_raster(const sxh_raster_inputs& in, const char* what) {
    if (!in.means2d || !in.conics || !in.colors || !in.opacities || !in.isect_offsets)
        invalid(what, "null means2d/conics/colors/opacities/isect_offsets");
    if (in.n_isects > 0 && !in.flatten_ids) invalid(what, "null flatten_ids");
    if (in.I < 0 || in.N < 0 || in.n_isects < 0) invalid(what, "negative I/N/n_isects");
    if (in.n_isects > 0 && in.N == 0) invalid(what, "n_isects > 0 requires N > 0 (flatten_ids reference gaussians)");
    if (in.tile_size != 16) invalid(what, "tile_size must be 16 (Phase 1 rasterize instantiation)");
    if (in.image_width == 0 || in.image_height == 0) invalid(what, "image_width/image_height must be positive");
    if (in.tile_width == 0 || in.tile_height == 0) invalid(what, "tile_width/tile_height must be positive");
    if (static_cast<uint64_t>(in.tile_width) * in.tile_size < in.image_width ||
        static_cast<uint64_t>(in.tile_height) * in.tile_size < in.image_height)
        invalid(what, "tile grid must cover the image");
    if (in.n_isects > INT32_MAX) invalid(what, "n_isects must fit in int32 (last_ids)");
    const int64_t n_tiles = static_cast<int64_t>(in.tile_width) * in.tile_height;
    if (in.I > 0 && n_tiles > INT32_MAX / in.I) invalid(what, "I*n_tiles must fit in int32 (offsets table)");
}

inline void validate_raster_grads(const sxh_raster_grads_in& g, const char* what) {
    if (!g.render_alphas || !g.last_ids) invalid(what, "null render_alphas/last_ids (fwd outputs)");
    if (!g.v_render_colors || !g.v_render_alphas) invalid(what, "null v_render_colors/v_render_alphas");
}

inline uint32_t validate_n_isects_readback(int64_t n_isects, const char* what) {
    if (n_isects < 0) invalid(what, "negative n_isects (prefix scan readback)");
    if (n_isects > INT32_MAX) invalid(what, "n_isects must fit in int32 (offsets/last_ids — host-path parity)");
    return static_cast<uint32_t>(n_isects);
}

inline void validate_rng(const sxh_rng_inputs& in, const char* what) {
    if (in.count < 0) invalid(what, "negative count");
    if (in.count > static_cast<int64_t>(UINT32_MAX)) invalid(what, "count must fit in uint32 (RngParams.count)");
}

inline void validate_relocation(const sxh_relocation_inputs& in, const char* what) {
    if (!in.opacities || !in.scales || !in.ratios || !in.binoms) invalid(what, "null opacities/scales/ratios/binoms");
    if (in.N < 0) invalid(what, "negative N");
    if (in.n_max < 1) invalid(what, "n_max must be >= 1");
    if (in.N > static_cast<int64_t>(UINT32_MAX)) invalid(what, "N exceeds uint32 (RelocParams.N)");
}

inline void validate_ssim(const sxh_ssim_inputs& in, const char* what) {
    if (!in.img1 || !in.img2) invalid(what, "null img1/img2");
    if (in.I <= 0 || in.C <= 0) invalid(what, "I and C must be positive (ssim mean undefined on empty batch)");
    if (in.H < 11 || in.W < 11) invalid(what, "H and W must be >= 11 (valid map would be empty)");
    if (in.H > UINT32_MAX || in.W > UINT32_MAX) invalid(what, "H/W exceed uint32 (SsimParams)");
    if (in.I > static_cast<int64_t>(UINT32_MAX) / in.C) invalid(what, "I*C exceeds uint32 (dispatch grid z)");
}

inline void validate_ssim_grads(const sxh_ssim_grads_in& g, const char* what) {
    if (!g.coeff_mu || !g.coeff_sigma || !g.coeff_cross)
        invalid(what, "null coeff maps (run ssim_fwd with need_coeffs=true)");
}

inline void validate_perturb(const sxh_perturb_inputs& in, const char* what) {
    if (!in.positions || !in.quats || !in.scales_log || !in.opacities_logit || !in.noise)
        invalid(what, "null positions/quats/scales_log/opacities_logit/noise");
    if (in.N < 0) invalid(what, "negative N");
    if (in.N > static_cast<int64_t>(UINT32_MAX)) invalid(what, "N exceeds uint32 (MCMCPerturbCUDA.cu:79)");
}

} // namespace sxh

// The backend object behind the opaque C handle.
struct sxh_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string name;
    uint32_t* pinned_word = nullptr;  // a pinned host word for status readbacks of the allocation-free calls
};

namespace sxh {
// Resolves the allocation-free entry points' scratch array on `device` (the current device).
void noalloc_init(int device);
}  // namespace sxh
