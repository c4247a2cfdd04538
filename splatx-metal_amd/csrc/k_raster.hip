// k_raster.hip — tile rasterizer forward and backward for gfx950.
//
// Contracts: rasterize_to_pixels_3dgs_fwd/bwd (Rasterize3DGSFwd.metal:57-204,
// Rasterize3DGSBwd.metal:70-298). One 256-thread workgroup (4 waves of 64) per 16x16 tile, one
// thread per pixel. Splat records (3 x float4) are staged through LDS in batches of 256.
// Forward: front-to-back compositing with the exclusive T <= 1e-4 stop, per-pixel arithmetic in
// the CPU reference's order (CpuKernels.cpp:821-849) and the deterministic exp of sx_fmath.h, so
// colors/alphas/last_ids are bit-identical to the CPU oracle; the workgroup exits as soon as all
// its pixels are done.
// Backward: back-to-front walk recovering T by division; the nine gradient components of each
// (Gaussian, wave) are summed over the wave with DPP row operations, the four waves of the tile are
// combined in LDS once per batch, and one set of float atomics per (tile, Gaussian) is issued.
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

__device__ __forceinline__ float sigma_of(float ca, float cb, float cc, float dx, float dy) {
    return 0.5f * (ca * dx * dx + cc * dy * dy) + cb * dx * dy;
}

// Largest sigma for which opacity * exp(-sigma) can still reach the 1/255 alpha threshold, plus a
// 0.01 margin: any pair with sigma above it is invalid in the exact evaluation too (its alpha is at
// most e^-0.01/255), so skipping its exp leaves every result bit-identical.
__device__ __forceinline__ float sigma_cutoff(float opac) { return __logf(opac * 255.0f) + 0.01f; }

__global__ void __launch_bounds__(kThreads) k_raster_fwd(RasterArgs a, float* __restrict__ out_rgb,
                                                         float* __restrict__ out_alpha, int32_t* __restrict__ out_last) {
    __shared__ float4 s_xyo[kThreads];  // {x, y, opacity, sigma cutoff}
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
            float4 xyo = a.splats[(size_t)g * 3];
            xyo.w = sigma_cutoff(xyo.z);
            s_xyo[tid] = xyo;
            s_con[tid] = a.splats[(size_t)g * 3 + 1];
            s_rgb[tid] = a.splats[(size_t)g * 3 + 2];
        }
        __syncthreads();
        const int cnt = min(kThreads, range_end - bstart);
        if (!done) {
            for (int t = 0; t < cnt; t++) {
                const float4 xyo = s_xyo[t];
                const float4 con = s_con[t];
                const float dx = xyo.x - px, dy = xyo.y - py;
                const float sigma = sigma_of(con.x, con.y, con.z, dx, dy);
                if (sigma > xyo.w) continue;  // provably below the alpha threshold
                const PixelEval e = eval_weight(con.x, con.y, con.z, dx, dy, xyo.z);
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

// ---- 64-lane sums through DPP (gfx9 data-parallel primitives) -----------------------------------
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
// Sum over the wave; the total is exact in lane 63 (other lanes hold partial sums).
__device__ __forceinline__ float wave_sum_lane63(float v) {
    v += dpp_f<0xB1, 0xF>(v);   // quad_perm(1,0,3,2): pairs
    v += dpp_f<0x4E, 0xF>(v);   // quad_perm(2,3,0,1): quads
    v += dpp_f<0x141, 0xF>(v);  // row_half_mirror: 8 lanes
    v += dpp_f<0x140, 0xF>(v);  // row_mirror: 16-lane row
    v += dpp_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

constexpr int kGrads = 9;  // v_xy(2), v_opacity, v_conic(3), v_rgb(3)

template <bool ABSGRAD>
__global__ void __launch_bounds__(kThreads) k_raster_bwd(RasterArgs a, const float* __restrict__ ralpha,
                                                         const int32_t* __restrict__ last_ids,
                                                         const float* __restrict__ v_rc, const float* __restrict__ v_ra,
                                                         RasterBwdGrads g) {
    constexpr int NV = ABSGRAD ? kGrads + 2 : kGrads;
    __shared__ float4 s_xyo[kThreads];  // {x, y, opacity, sigma cutoff}
    __shared__ float4 s_con[kThreads];
    __shared__ float4 s_rgb[kThreads];
    __shared__ int32_t s_id[kThreads];
    __shared__ float s_part[kThreads / 64][NV][kThreads];  // per-wave sums, Gaussian-minor
    const int n_tiles = a.tile_width * a.tile_height;
    const int img = blockIdx.x / n_tiles;
    const int tile = blockIdx.x % n_tiles;
    if (a.masks && a.masks[(size_t)img * n_tiles + tile] == 0) return;  // uniform
    const int tx = tile % a.tile_width, ty = tile / a.tile_width;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const bool lane63 = (tid & 63) == 63;
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
            float4 xyo = a.splats[(size_t)gid * 3];
            xyo.w = sigma_cutoff(xyo.z);
            s_xyo[tid] = xyo;
            s_con[tid] = a.splats[(size_t)gid * 3 + 1];
            s_rgb[tid] = a.splats[(size_t)gid * 3 + 2];
        }
#pragma unroll
        for (int w = 0; w < kThreads / 64; w++)
#pragma unroll
            for (int k = 0; k < NV; k++) s_part[w][k][tid] = 0.f;
        __syncthreads();
        for (int t = max(0, batch_end - wave_bin_final); t < batch_size; t++) {
            const float4 xyo = s_xyo[t];
            const float4 con = s_con[t];
            const float dx = xyo.x - px, dy = xyo.y - py;
            const float sigma = sigma_of(con.x, con.y, con.z, dx, dy);
            bool valid = inside && (batch_end - t) <= bin_final && !(sigma > xyo.w);
            if (!__any(valid)) continue;  // wave-uniform, before any exp
            float g_r = 0.f, g_g = 0.f, g_b = 0.f, g_ca = 0.f, g_cb = 0.f, g_cc = 0.f, g_x = 0.f, g_y = 0.f,
                  g_o = 0.f, g_ax = 0.f, g_ay = 0.f;
            if (valid) {
                const PixelEval e = eval_weight(con.x, con.y, con.z, dx, dy, xyo.z);
                if (e.valid) {
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
                        if (ABSGRAD) {
                            g_ax = fabsf(g_x);
                            g_ay = fabsf(g_y);
                        }
                        g_o = e.vis * v_alpha;
                    }
                    b0 += c.x * fac;
                    b1 += c.y * fac;
                    b2 += c.z * fac;
                }
            }
            const float s0 = wave_sum_lane63(g_x), s1 = wave_sum_lane63(g_y), s2 = wave_sum_lane63(g_o);
            const float s3 = wave_sum_lane63(g_ca), s4 = wave_sum_lane63(g_cb), s5 = wave_sum_lane63(g_cc);
            const float s6 = wave_sum_lane63(g_r), s7 = wave_sum_lane63(g_g), s8 = wave_sum_lane63(g_b);
            float s9 = 0.f, s10 = 0.f;
            if (ABSGRAD) {
                s9 = wave_sum_lane63(g_ax);
                s10 = wave_sum_lane63(g_ay);
            }
            if (lane63) {
                float* p = &s_part[wave][0][t];
                p[0 * kThreads] = s0; p[1 * kThreads] = s1; p[2 * kThreads] = s2;
                p[3 * kThreads] = s3; p[4 * kThreads] = s4; p[5 * kThreads] = s5;
                p[6 * kThreads] = s6; p[7 * kThreads] = s7; p[8 * kThreads] = s8;
                if (ABSGRAD) {
                    p[9 * kThreads] = s9;
                    p[10 * kThreads] = s10;
                }
            }
        }
        __syncthreads();
        // one thread per Gaussian of the batch: combine the four waves, then one atomic per component
        if (tid < batch_size) {
            float v[NV];
            bool any = false;
#pragma unroll
            for (int k = 0; k < NV; k++) {
                v[k] = s_part[0][k][tid] + s_part[1][k][tid] + s_part[2][k][tid] + s_part[3][k][tid];
                any |= v[k] != 0.f;
            }
            if (any) {
                const int32_t gid = s_id[tid];
                if (g.packed) {
                    float* rec = reinterpret_cast<float*>(g.packed + (size_t)gid * 3);
                    atomicAdd(&rec[0], v[0]);
                    atomicAdd(&rec[1], v[1]);
                    atomicAdd(&rec[2], v[2]);
                    atomicAdd(&rec[4], v[3]);
                    atomicAdd(&rec[5], v[4]);
                    atomicAdd(&rec[6], v[5]);
                    atomicAdd(&rec[8], v[6]);
                    atomicAdd(&rec[9], v[7]);
                    atomicAdd(&rec[10], v[8]);
                } else {
                    atomicAdd(&g.v_means2d[(size_t)gid * 2], v[0]);
                    atomicAdd(&g.v_means2d[(size_t)gid * 2 + 1], v[1]);
                    atomicAdd(&g.v_opacities[gid], v[2]);
                    atomicAdd(&g.v_conics[(size_t)gid * 3], v[3]);
                    atomicAdd(&g.v_conics[(size_t)gid * 3 + 1], v[4]);
                    atomicAdd(&g.v_conics[(size_t)gid * 3 + 2], v[5]);
                    atomicAdd(&g.v_colors[(size_t)gid * 3], v[6]);
                    atomicAdd(&g.v_colors[(size_t)gid * 3 + 1], v[7]);
                    atomicAdd(&g.v_colors[(size_t)gid * 3 + 2], v[8]);
                    if (ABSGRAD) {
                        atomicAdd(&g.v_means2d_abs[(size_t)gid * 2], v[9]);
                        atomicAdd(&g.v_means2d_abs[(size_t)gid * 2 + 1], v[10]);
                    }
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
    if (g.v_means2d_abs)
        hipLaunchKernelGGL(k_raster_bwd<true>, dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids, v_rc, v_ra, g);
    else
        hipLaunchKernelGGL(k_raster_bwd<false>, dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids, v_rc, v_ra, g);
}

} // namespace sxk
