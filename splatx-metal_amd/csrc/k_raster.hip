// k_raster.hip — tile rasterizer forward and backward for gfx950.
//
// Contracts: rasterize_to_pixels_3dgs_fwd/bwd (Rasterize3DGSFwd.metal:57-204,
// Rasterize3DGSBwd.metal:70-298). One 256-thread workgroup (4 waves of 64) per 16x16 tile, one
// thread per pixel. Splat records (3 x float4) are staged through LDS in batches of 256.
// Forward: front-to-back compositing with the exclusive T <= 1e-4 stop, per-pixel arithmetic in
// the CPU reference's order (CpuKernels.cpp:821-849) and the deterministic exp of sx_fmath.h, so
// colors/alphas/last_ids are bit-identical to the CPU oracle; the workgroup exits as soon as all
// its pixels are done.
// Backward: back-to-front walk recovering T by division, per-wave reduction of the nine gradient
// components through cross-lane shuffles, one set of float atomics per wave and Gaussian.
#include <hip/hip_runtime.h>

#include "sx_dev.h"
#include "sx_kernels.h"

namespace sxk {
namespace {

constexpr int kThreads = 256;

struct PixelEval {
    float vis, alpha, sigma;
    bool valid;
};

// eval_gaussian_weight (KernelCommon.h:75-96 contract; CpuKernels.cpp:753-760 forms)
__device__ __forceinline__ PixelEval eval_weight(float ca, float cb, float cc, float dx, float dy, float opac) {
    PixelEval e;
    e.sigma = 0.5f * (ca * dx * dx + cc * dy * dy) + cb * dx * dy;
    e.vis = sxm::expf_fast(-e.sigma);
    const float oa = opac * e.vis;
    e.alpha = sxd::smin(sx::kMaxAlpha, oa);
    e.valid = !(e.sigma < 0.f || e.alpha < sx::kAlphaThreshold);
    return e;
}

__global__ void __launch_bounds__(kThreads) k_raster_fwd(RasterArgs a, float* __restrict__ out_rgb,
                                                         float* __restrict__ out_alpha, int32_t* __restrict__ out_last) {
    __shared__ float4 s_xyo[kThreads];
    __shared__ float4 s_con[kThreads];
    __shared__ float4 s_rgb[kThreads];
    const int n_tiles = a.tile_width * a.tile_height;
    const int img = blockIdx.x / n_tiles;
    const int tile = blockIdx.x % n_tiles;
    const int tx = tile % a.tile_width, ty = tile / a.tile_width;
    const int tid = threadIdx.x;
    const int px_i = tx * 16 + (tid & 15), py_i = ty * 16 + (tid >> 4);
    const bool inside = px_i < a.width && py_i < a.height;
    const size_t pix = (size_t)img * a.height * a.width + (size_t)py_i * a.width + px_i;
    const float* bg = a.backgrounds ? a.backgrounds + img * 3 : nullptr;
    if (a.masks && a.masks[(size_t)img * n_tiles + tile] == 0) {  // uniform per workgroup
        if (inside) {
#pragma unroll
            for (int k = 0; k < 3; k++) out_rgb[pix * 3 + k] = bg ? bg[k] : 0.f;
            out_alpha[pix] = 0.f;
            out_last[pix] = 0;
        }
        return;
    }
    const int32_t* offs = a.offsets + (size_t)img * n_tiles;
    const int32_t range_start = offs[tile];
    const int32_t range_end = (img == a.I - 1 && tile == n_tiles - 1) ? a.n_isects : offs[tile + 1];
    const float px = static_cast<float>(px_i) + 0.5f, py = static_cast<float>(py_i) + 0.5f;
    float T = 1.0f;
    int32_t cur = 0;
    float r0 = 0.f, r1 = 0.f, r2 = 0.f;
    bool done = !inside;
    for (int32_t bstart = range_start; bstart < range_end; bstart += kThreads) {
        if (__syncthreads_count(done) == kThreads) break;  // also the barrier before LDS reuse
        const int32_t idx = bstart + tid;
        if (idx < range_end) {
            const int32_t g = a.flatten_ids[idx];
            s_xyo[tid] = a.splats[(size_t)g * 3];
            s_con[tid] = a.splats[(size_t)g * 3 + 1];
            s_rgb[tid] = a.splats[(size_t)g * 3 + 2];
        }
        __syncthreads();
        const int cnt = min(kThreads, range_end - bstart);
        if (!done) {
            for (int t = 0; t < cnt; t++) {
                const float4 xyo = s_xyo[t];
                const float4 con = s_con[t];
                const PixelEval e = eval_weight(con.x, con.y, con.z, xyo.x - px, xyo.y - py, xyo.z);
                if (!e.valid) continue;
                const float next_T = T * (1.0f - e.alpha);
                if (next_T <= sx::kTransmittanceThreshold) {
                    done = true;
                    break;
                }
                const float w = e.alpha * T;
                const float4 c = s_rgb[t];
                r0 = __builtin_fmaf(c.x, w, r0);
                r1 = __builtin_fmaf(c.y, w, r1);
                r2 = __builtin_fmaf(c.z, w, r2);
                cur = bstart + t;
                T = next_T;
            }
        }
    }
    if (!inside) return;
    out_alpha[pix] = 1.0f - T;
    out_rgb[pix * 3] = bg ? __builtin_fmaf(T, bg[0], r0) : r0;
    out_rgb[pix * 3 + 1] = bg ? __builtin_fmaf(T, bg[1], r1) : r1;
    out_rgb[pix * 3 + 2] = bg ? __builtin_fmaf(T, bg[2], r2) : r2;
    out_last[pix] = cur;
}

__global__ void __launch_bounds__(kThreads) k_raster_bwd(RasterArgs a, const float* __restrict__ ralpha,
                                                         const int32_t* __restrict__ last_ids,
                                                         const float* __restrict__ v_rc, const float* __restrict__ v_ra,
                                                         RasterBwdGrads g) {
    __shared__ float4 s_xyo[kThreads];
    __shared__ float4 s_con[kThreads];
    __shared__ float4 s_rgb[kThreads];
    __shared__ int32_t s_id[kThreads];
    const int n_tiles = a.tile_width * a.tile_height;
    const int img = blockIdx.x / n_tiles;
    const int tile = blockIdx.x % n_tiles;
    if (a.masks && a.masks[(size_t)img * n_tiles + tile] == 0) return;  // uniform
    const int tx = tile % a.tile_width, ty = tile / a.tile_width;
    const int tid = threadIdx.x;
    const int px_i = tx * 16 + (tid & 15), py_i = ty * 16 + (tid >> 4);
    const bool inside = px_i < a.width && py_i < a.height;
    const size_t pix = inside ? (size_t)img * a.height * a.width + (size_t)py_i * a.width + px_i
                              : (size_t)img * a.height * a.width;
    const int32_t* offs = a.offsets + (size_t)img * n_tiles;
    const int32_t range_start = offs[tile];
    const int32_t range_end = (img == a.I - 1 && tile == n_tiles - 1) ? a.n_isects : offs[tile + 1];
    const float* bg = a.backgrounds ? a.backgrounds + img * 3 : nullptr;
    const float px = static_cast<float>(px_i) + 0.5f, py = static_cast<float>(py_i) + 0.5f;
    const float T_final = 1.0f - ralpha[pix];
    float T = T_final;
    float b0 = 0.f, b1 = 0.f, b2 = 0.f;
    const int32_t bin_final = inside ? last_ids[pix] : -1;
    const float vc0 = v_rc[pix * 3], vc1 = v_rc[pix * 3 + 1], vc2 = v_rc[pix * 3 + 2];
    const float va = v_ra[pix];
    const float bg_dot = bg ? (bg[0] * vc0 + bg[1] * vc1 + bg[2] * vc2) : 0.f;
    const int32_t wave_bin_final = sxd::wave_max_i(bin_final);
    const bool absgrad = g.v_means2d_abs != nullptr;
    const int32_t num = range_end - range_start;
    const int num_batches = (num + kThreads - 1) / kThreads;
    for (int b = 0; b < num_batches; b++) {
        __syncthreads();
        const int32_t batch_end = range_end - 1 - kThreads * b;
        const int32_t batch_size = min(kThreads, batch_end + 1 - range_start);
        const int32_t idx = batch_end - tid;
        if (idx >= range_start) {
            const int32_t gid = a.flatten_ids[idx];
            s_id[tid] = gid;
            s_xyo[tid] = a.splats[(size_t)gid * 3];
            s_con[tid] = a.splats[(size_t)gid * 3 + 1];
            s_rgb[tid] = a.splats[(size_t)gid * 3 + 2];
        }
        __syncthreads();
        for (int t = max(0, batch_end - wave_bin_final); t < batch_size; t++) {
            bool valid = inside && (batch_end - t) <= bin_final;
            float4 xyo = make_float4(0.f, 0.f, 0.f, 0.f), con = xyo;
            PixelEval e{0.f, 0.f, 0.f, false};
            float dx = 0.f, dy = 0.f;
            if (valid) {
                xyo = s_xyo[t];
                con = s_con[t];
                dx = xyo.x - px;
                dy = xyo.y - py;
                e = eval_weight(con.x, con.y, con.z, dx, dy, xyo.z);
                valid = e.valid;
            }
            if (!__any(valid)) continue;  // wave-uniform
            float g_r = 0.f, g_g = 0.f, g_b = 0.f, g_ca = 0.f, g_cb = 0.f, g_cc = 0.f, g_x = 0.f, g_y = 0.f,
                  g_o = 0.f, g_ax = 0.f, g_ay = 0.f;
            if (valid) {
                const float ra = 1.0f / sxd::smax(sx::kMinOneMinusAlpha, 1.0f - e.alpha);
                T *= ra;
                const float fac = e.alpha * T;
                const float4 c = s_rgb[t];
                g_r = fac * vc0;
                g_g = fac * vc1;
                g_b = fac * vc2;
                float v_alpha = (c.x * T - b0 * ra) * vc0 + (c.y * T - b1 * ra) * vc1 + (c.z * T - b2 * ra) * vc2;
                v_alpha += T_final * ra * va;
                if (bg) v_alpha += -T_final * ra * bg_dot;
                const float opac = xyo.z;
                if (opac * e.vis <= sx::kMaxAlpha) {
                    const float v_sigma = -opac * e.vis * v_alpha;
                    g_ca = 0.5f * v_sigma * dx * dx;
                    g_cb = v_sigma * dx * dy;
                    g_cc = 0.5f * v_sigma * dy * dy;
                    g_x = v_sigma * (con.x * dx + con.y * dy);
                    g_y = v_sigma * (con.y * dx + con.z * dy);
                    g_ax = fabsf(g_x);
                    g_ay = fabsf(g_y);
                    g_o = e.vis * v_alpha;
                }
                b0 += c.x * fac;
                b1 += c.y * fac;
                b2 += c.z * fac;
            }
            g_r = sxd::wave_sum(g_r);
            g_g = sxd::wave_sum(g_g);
            g_b = sxd::wave_sum(g_b);
            g_ca = sxd::wave_sum(g_ca);
            g_cb = sxd::wave_sum(g_cb);
            g_cc = sxd::wave_sum(g_cc);
            g_x = sxd::wave_sum(g_x);
            g_y = sxd::wave_sum(g_y);
            g_o = sxd::wave_sum(g_o);
            if (absgrad) {
                g_ax = sxd::wave_sum(g_ax);
                g_ay = sxd::wave_sum(g_ay);
            }
            if (sxd::lane_id() == 0 && g.packed) {
                float* rec = reinterpret_cast<float*>(g.packed + (size_t)s_id[t] * 3);
                atomicAdd(&rec[0], g_x);
                atomicAdd(&rec[1], g_y);
                atomicAdd(&rec[2], g_o);
                atomicAdd(&rec[4], g_ca);
                atomicAdd(&rec[5], g_cb);
                atomicAdd(&rec[6], g_cc);
                atomicAdd(&rec[8], g_r);
                atomicAdd(&rec[9], g_g);
                atomicAdd(&rec[10], g_b);
            } else if (sxd::lane_id() == 0) {
                const int32_t gid = s_id[t];
                atomicAdd(&g.v_colors[(size_t)gid * 3], g_r);
                atomicAdd(&g.v_colors[(size_t)gid * 3 + 1], g_g);
                atomicAdd(&g.v_colors[(size_t)gid * 3 + 2], g_b);
                atomicAdd(&g.v_conics[(size_t)gid * 3], g_ca);
                atomicAdd(&g.v_conics[(size_t)gid * 3 + 1], g_cb);
                atomicAdd(&g.v_conics[(size_t)gid * 3 + 2], g_cc);
                atomicAdd(&g.v_means2d[(size_t)gid * 2], g_x);
                atomicAdd(&g.v_means2d[(size_t)gid * 2 + 1], g_y);
                atomicAdd(&g.v_opacities[gid], g_o);
                if (absgrad) {
                    atomicAdd(&g.v_means2d_abs[(size_t)gid * 2], g_ax);
                    atomicAdd(&g.v_means2d_abs[(size_t)gid * 2 + 1], g_ay);
                }
            }
        }
    }
}

} // namespace

void raster_fwd(const RasterArgs& a, float* rgb, float* alpha, int32_t* last, hipStream_t s) {
    const int blocks = a.I * a.tile_width * a.tile_height;
    if (blocks <= 0) return;
    hipLaunchKernelGGL(k_raster_fwd, dim3(blocks), dim3(kThreads), 0, s, a, rgb, alpha, last);
}

void raster_bwd(const RasterArgs& a, const float* ralpha, const int32_t* last_ids, const float* v_rc,
                const float* v_ra, const RasterBwdGrads& g, hipStream_t s) {
    const int blocks = a.I * a.tile_width * a.tile_height;
    if (blocks <= 0 || a.n_isects <= 0) return;
    hipLaunchKernelGGL(k_raster_bwd, dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids, v_rc, v_ra, g);
}

} // namespace sxk
