// k_raster.hip — tile rasterizer forward and backward for gfx950.
//
// Contracts: rasterize_to_pixels_3dgs_fwd/bwd (Rasterize3DGSFwd.metal:57-204,
// Rasterize3DGSBwd.metal:70-298). One 256-thread workgroup (4 waves of 64) per 16x16 tile, one
// thread per pixel. Splat records (3 x float4) are staged through LDS in batches of 256.
// Forward: front-to-back compositing with the exclusive T <= 1e-4 stop, per-pixel arithmetic in
// the CPU reference's order (CpuKernels.cpp:821-849) and the deterministic exp of sx_fmath.h, so
// colors/alphas/last_ids are bit-identical to the CPU oracle; the workgroup exits as soon as all
// its pixels are done.
// Backward: back-to-front walk recovering T by division. Contributing Gaussians are taken four at a
// time; their nine gradient components are summed over the wave with one transposed reduction
// (gfx950 v_permlane32_swap / v_permlane16_swap folds, then DPP within 16-lane rows), the four waves
// of the tile add their sums into LDS, and one set of float atomics per (tile, Gaussian) is issued
// after each batch.
#include <hip/hip_runtime.h>

#include "sx_dev.h"
#include "sx_kernels.h"

namespace sxk {
namespace {

constexpr int kThreads = 256;

// sxm::expf_fast(-sigma) without its range branches: identical for sigma in [0, 86] (no overflow,
// no subnormal scaling). exp_neg: `cut` is the Gaussian's sigma cutoff, wave-uniform, and only an
// opacity above ~1e35 pushes it past that range, in which case the general function is used.
__device__ __forceinline__ float exp_neg_poly(float sigma) {
    const float x = -sigma;
    const float kf = __builtin_rintf(x * 1.44269502f);
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);
    r = __builtin_fmaf(kf, -1.42860677e-06f, r);
    float p = 2.48015873e-05f;
    p = __builtin_fmaf(p, r, 1.98412698e-04f);
    p = __builtin_fmaf(p, r, 1.38888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int k = static_cast<int>(kf);
    return p * __uint_as_float(static_cast<uint32_t>(k + 127) << 23);
}

__device__ __forceinline__ float exp_neg(float sigma, float cut) {
    const float cut_u = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(cut)));  // uniform branch
    if (__builtin_expect(cut_u > 86.0f, 0)) return sxm::expf_fast(-sigma);
    return exp_neg_poly(sigma);
}

__device__ __forceinline__ float sigma_of(float ca, float cb, float cc, float dx, float dy) {
    return 0.5f * (ca * dx * dx + cc * dy * dy) + cb * dx * dy;
}

// Largest sigma for which opacity * exp(-sigma) can still reach the 1/255 alpha threshold, plus a
// 0.01 margin: any pair with sigma above it is invalid in the exact evaluation too (its alpha is at
// most e^-0.01/255), so skipping its exp leaves every result bit-identical.
__device__ __forceinline__ float sigma_cutoff(float opac) { return __logf(opac * 255.0f) + 0.01f; }

// Which of the tile's four waves (pixel rows y0 + 4w .. y0 + 4w + 3) the Gaussian's cutoff set
// {sigma <= cut} can reach: for a positive-definite conic the set's y half-extent is
// sqrt(2 cut a / det). Conservative: the extent gets a relative and an absolute margin far above
// float rounding of sigma, and every degenerate, nearly degenerate or non-finite case keeps all
// four waves.
__device__ __forceinline__ uint32_t wave_rows_mask(float4 xyo, float4 con, int y0) {
    const float a = con.x, b = con.y, c = con.z, cut = xyo.w;
    if (cut == -__builtin_inff()) return 0u;  // opacity 0: no pixel passes
    const float det = a * c - b * b;
    const bool finite = __builtin_isfinite(a) && __builtin_isfinite(b) && __builtin_isfinite(c) &&
                        __builtin_isfinite(cut) && __builtin_fabsf(xyo.x) < 1e18f && __builtin_fabsf(xyo.y) < 1e18f;
    if (!finite || !(a > 0.f) || !(det > 1e-4f * a * c)) return 0xFu;
    if (cut < 0.f) return 0u;  // sigma >= 0 everywhere for a positive-definite conic
    const float ry = __builtin_sqrtf(2.0f * cut * a / det) * 1.001f + 0.01f;
    const float lo = xyo.y - ry, hi = xyo.y + ry;
    uint32_t m = 0u;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const float r0 = static_cast<float>(y0 + 4 * w) + 0.5f, r1 = r0 + 3.0f;
        if (hi >= r0 && lo <= r1) m |= 1u << w;
    }
    return m;
}

// Per-wave Gaussian lists of a batch: s_list[w][0 .. s_len[w]) = the batch-local indices t (in
// increasing order) whose mask has bit w. All 256 threads call it; thread t passes Gaussian t's mask
// (0 for slots past the batch). Ends with a barrier.
__device__ __forceinline__ void build_wave_lists(uint32_t m, uint8_t (*s_list)[kThreads], int (*s_wc)[4],
                                                 int* s_len) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int pos[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const unsigned long long bal = __ballot((m >> w) & 1u);
        pos[w] = __popcll(bal & below);
        if (lane == 0) s_wc[w][wave] = __popcll(bal);
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 4; w++) {
        int off = 0;
#pragma unroll
        for (int sw = 0; sw < 4; sw++) off += sw < wave ? s_wc[w][sw] : 0;
        if ((m >> w) & 1u) s_list[w][off + pos[w]] = static_cast<uint8_t>(tid);
        if (tid == 0) s_len[w] = s_wc[w][0] + s_wc[w][1] + s_wc[w][2] + s_wc[w][3];
    }
    __syncthreads();
}

template <bool STATS>
__global__ void __launch_bounds__(kThreads) k_raster_fwd(RasterArgs a, float* __restrict__ out_rgb,
                                                         float* __restrict__ out_alpha, int32_t* __restrict__ out_last) {
    __shared__ float4 s_xyo[kThreads];  // {x, y, opacity, sigma cutoff}
    __shared__ float4 s_con[kThreads];
    __shared__ float4 s_rgb[kThreads];
    __shared__ uint8_t s_list[4][kThreads];
    __shared__ int s_wc[4][4];
    __shared__ int s_len[4];
    const int n_tiles = a.tile_width * a.tile_height;
    const int img = blockIdx.x / n_tiles;
    const int tile = a.tile_order ? a.tile_order[blockIdx.x % n_tiles] : static_cast<int>(blockIdx.x % n_tiles);
    const int tx = tile % a.tile_width, ty = tile / a.tile_width;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
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
    const int32_t range_end = (img == a.I - 1 && tile == n_tiles - 1)
                                  ? (a.n_isects_dev ? static_cast<int32_t>(*a.n_isects_dev) : a.n_isects)
                                  : offs[tile + 1];
    const float px = static_cast<float>(px_i) + 0.5f, py = static_cast<float>(py_i) + 0.5f;
    float T = 1.0f;
    int32_t cur = 0;
    float r0 = 0.f, r1 = 0.f, r2 = 0.f;
    bool done = !inside;
    unsigned long long st_entries = 0, st_taken = 0;  // STATS only (wave-uniform)
    for (int32_t bstart = range_start; bstart < range_end; bstart += kThreads) {
        if (__syncthreads_count(done) == kThreads) break;  // also the barrier before LDS reuse
        const int32_t idx = bstart + tid;
        uint32_t wm = 0u;
        if (idx < range_end) {
            const int32_t g = a.flatten_ids[idx];
            float4 xyo = a.splats[(size_t)g * 3];
            xyo.w = sigma_cutoff(xyo.z);
            const float4 con = a.splats[(size_t)g * 3 + 1];
            s_xyo[tid] = xyo;
            s_con[tid] = con;
            s_rgb[tid] = a.splats[(size_t)g * 3 + 2];
            wm = wave_rows_mask(xyo, con, ty * 16);
        }
        build_wave_lists(wm, s_list, s_wc, s_len);
        // the wave walks its list together (index and count are wave-uniform); a lane takes a pair
        // through selects rather than branches, and stops taking pairs once its T is spent
        const int len = __builtin_amdgcn_readfirstlane(s_len[wave]);
        for (int j = 0; j < len; j++) {
            if (__all(done)) break;  // uniform
            if (STATS) st_entries++;
            const int t = __builtin_amdgcn_readfirstlane(s_list[wave][j]);
            const float4 xyo = s_xyo[t];
            const float4 con = s_con[t];
            const float dx = xyo.x - px, dy = xyo.y - py;
            const float sigma = sigma_of(con.x, con.y, con.z, dx, dy);
            bool take = !done && !(sigma > xyo.w);  // past the cutoff: provably below the alpha threshold
            if (!__any(take)) continue;             // uniform: no lane of the wave needs the exponential
            const float vis = exp_neg(sigma, xyo.w);
            const float alpha = sxd::smin(sx::kMaxAlpha, xyo.z * vis);
            take = take && !(sigma < 0.f) && !(alpha < sx::kAlphaThreshold);
            const float next_T = T * (1.0f - alpha);
            const bool spent = take && next_T <= sx::kTransmittanceThreshold;
            done = done || spent;
            take = take && !spent;
            const float w = alpha * T;
            const float4 c = s_rgb[t];
            r0 = take ? __builtin_fmaf(c.x, w, r0) : r0;
            r1 = take ? __builtin_fmaf(c.y, w, r1) : r1;
            r2 = take ? __builtin_fmaf(c.z, w, r2) : r2;
            cur = take ? bstart + t : cur;
            T = take ? next_T : T;
            if (STATS) st_taken += __popcll(__ballot(take));
        }
    }
    if (STATS && (tid & 63) == 0) {
        atomicAdd(&a.stats[kStatFwdEntries], st_entries);
        atomicAdd(&a.stats[kStatFwdTaken], st_taken);
    }
    if (!inside) return;
    out_alpha[pix] = 1.0f - T;
    out_rgb[pix * 3] = bg ? __builtin_fmaf(T, bg[0], r0) : r0;
    out_rgb[pix * 3 + 1] = bg ? __builtin_fmaf(T, bg[1], r1) : r1;
    out_rgb[pix * 3 + 2] = bg ? __builtin_fmaf(T, bg[2], r2) : r2;
    out_last[pix] = cur;
}

// ---- wave reductions -----------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over each 16-lane row; every lane of the row ends with the row total.
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm(1,0,3,2): pairs
    v += dpp_f<0x4E>(v);   // quad_perm(2,3,0,1): quads
    v += dpp_f<0x141>(v);  // row_half_mirror: 8 lanes
    v += dpp_f<0x140>(v);  // row_mirror: the 16-lane row
    return v;
}
// v_permlane32_swap exchanges lanes 32-63 of `a` with lanes 0-31 of `b`; the sum of the two results
// holds a's 32-lane half sums in lanes 0-31 and b's in lanes 32-63.
__device__ __forceinline__ float fold32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// v_permlane16_swap exchanges the odd 16-lane rows of `a` with the even rows of `b`; after the sum,
// row 0 holds a's row-0 + row-1 partials, row 1 b's, row 2 a's rows 2 + 3, row 3 b's.
__device__ __forceinline__ float fold16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Four per-lane values (one per Gaussian slot A..D) reduced over the 64 lanes in 10 instructions: the
// result's row 0 holds the total of A, row 1 of C, row 2 of B, row 3 of D (every lane of the row).
__device__ __forceinline__ float wave_sum4(float a, float b, float c, float d) {
    return row_sum16(fold16(fold32(a, b), fold32(c, d)));
}

constexpr int kGrads = 9;  // v_xy(2), v_opacity, v_conic(3), v_rgb(3)

template <bool ABSGRAD, bool STATS>
__global__ void __launch_bounds__(kThreads) k_raster_bwd(RasterArgs a, const float* __restrict__ ralpha,
                                                         const int32_t* __restrict__ last_ids,
                                                         const float* __restrict__ v_rc, const float* __restrict__ v_ra,
                                                         RasterBwdGrads g) {
    constexpr int NV = ABSGRAD ? kGrads + 2 : kGrads;
    __shared__ float4 s_xyo[kThreads];  // {x, y, opacity, sigma cutoff}
    __shared__ float4 s_con[kThreads];
    __shared__ float4 s_rgb[kThreads];
    __shared__ int32_t s_id[kThreads];
    __shared__ float4 s_part4[NV * kThreads / 4];  // per-tile sums [k][t], the four waves add into it
    __shared__ __align__(16) uint8_t s_list[4][kThreads];
    __shared__ int s_wc[4][4];
    __shared__ int s_len[4];
    __shared__ int32_t s_wbf[4];  // each wave's last contributing intersection
    float* s_part = reinterpret_cast<float*>(s_part4);
    const int n_tiles = a.tile_width * a.tile_height;
    const int img = blockIdx.x / n_tiles;
    const int tile = a.tile_order ? a.tile_order[blockIdx.x % n_tiles] : static_cast<int>(blockIdx.x % n_tiles);
    if (a.masks && a.masks[(size_t)img * n_tiles + tile] == 0) return;  // uniform
    const int tx = tile % a.tile_width, ty = tile / a.tile_width;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int px_i = tx * 16 + (tid & 15), py_i = ty * 16 + (tid >> 4);
    const bool inside = px_i < a.width && py_i < a.height;
    const size_t pix = inside ? (size_t)img * a.height * a.width + (size_t)py_i * a.width + px_i
                              : (size_t)img * a.height * a.width;
    const int32_t* offs = a.offsets + (size_t)img * n_tiles;
    const int32_t range_start = offs[tile];
    const int32_t range_end = (img == a.I - 1 && tile == n_tiles - 1)
                                  ? (a.n_isects_dev ? static_cast<int32_t>(*a.n_isects_dev) : a.n_isects)
                                  : offs[tile + 1];
    const float* bg = a.backgrounds ? a.backgrounds + img * 3 : nullptr;
    const float px = static_cast<float>(px_i) + 0.5f, py = static_cast<float>(py_i) + 0.5f;
    const float T_final = 1.0f - ralpha[pix];
    float T = T_final;
    float bdot = 0.f;  // <accumulated back colour, v_render> (the back-sum dotted with v_render)
    const int32_t bin_final = inside ? last_ids[pix] : -1;  // -1: no pair of an outside pixel is valid
    const float vc0 = v_rc[pix * 3], vc1 = v_rc[pix * 3 + 1], vc2 = v_rc[pix * 3 + 2];
    const float va = v_ra[pix];
    const float bg_dot = bg ? (bg[0] * vc0 + bg[1] * vc1 + bg[2] * vc2) : 0.f;
    const float tva = T_final * (va - bg_dot);  // the alpha and background terms of every v_alpha, over ra
    const int32_t wave_bin_final = sxd::wave_max_i(bin_final);
    if (lane == 0) s_wbf[wave] = wave_bin_final;
    __syncthreads();
    // the walk starts at the tile's last contributing intersection: everything behind it (most of
    // a dense tile's list, once its pixels saturate) has no pixel to contribute to
    const int32_t tile_end = min(range_end, max(max(s_wbf[0], s_wbf[1]), max(s_wbf[2], s_wbf[3])) + 1);
    const int32_t num = max(0, tile_end - range_start);
    const int num_batches = (num + kThreads - 1) / kThreads;
    // row r of a wave_sum4 result belongs to slot A=0, C=2, B=1, D=3 for r = 0..3
    const int row = lane >> 4;
    const int row_slot = row == 0 ? 0 : row == 1 ? 2 : row == 2 ? 1 : 3;
    // STATS only (wave-uniform)
    unsigned long long st_chunks = 0, st_entries = 0, st_empty = 0, st_cut = 0, st_contrib = 0;
    for (int b = 0; b < num_batches; b++) {
        __syncthreads();
        const int32_t batch_end = tile_end - 1 - kThreads * b;
        const int32_t batch_size = min(kThreads, batch_end + 1 - range_start);
        const int32_t idx = batch_end - tid;
        uint32_t wm = 0u;
        if (idx >= range_start) {
            const int32_t gid = a.flatten_ids[idx];
            s_id[tid] = gid;
            float4 xyo = a.splats[(size_t)gid * 3];
            xyo.w = sigma_cutoff(xyo.z);
            float4 con = a.splats[(size_t)gid * 3 + 1];
            float4 rgb = a.splats[(size_t)gid * 3 + 2];
            // the sigmas at which the two alpha decisions turn: opacity * e^-sigma = 1/255 and = 0.99
            // (approximate; only used to find the pairs close to them)
            con.w = __logf(xyo.z * (1.0f / sx::kMaxAlpha));
            rgb.w = __logf(xyo.z * 255.0f);
            s_xyo[tid] = xyo;
            s_con[tid] = con;
            s_rgb[tid] = rgb;
            // waves whose rows the cutoff set can reach, less those whose every pixel stopped before it
            wm = wave_rows_mask(xyo, con, ty * 16);
#pragma unroll
            for (int w = 0; w < 4; w++)
                if (idx > s_wbf[w]) wm &= ~(1u << w);
        }
#pragma unroll
        for (int j = tid; j < NV * kThreads / 4; j += kThreads) s_part4[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        build_wave_lists(wm, s_list, s_wc, s_len);

        // This wave's Gaussians back to front, four at a time: the four list entries come in one
        // LDS read and their records in one burst, the four pairs' exponentials are independent,
        // only T and the back-sum run through them in order. A pair that does not contribute (or a
        // slot past the list) gets alpha = 0, so T (times 1/(1 - 0) = 1), the back-sum and every
        // gradient term are left unchanged / zero.
        const int len = s_len[wave];
        const uint32_t* list4 = reinterpret_cast<const uint32_t*>(s_list[wave]);
        const int t_min = batch_end - bin_final;  // slots t >= t_min are at or before the lane's last contributor
        for (int j = 0; j < len; j += 4) {
            const uint32_t packed = list4[j >> 2];
            int ts[4], tc[4];
            float4 xyo[4], con[4], rgb[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                ts[k] = j + k < len ? static_cast<int>((packed >> (8 * k)) & 0xFFu) : -1;
                tc[k] = ts[k] < 0 ? 0 : ts[k];
                xyo[k] = s_xyo[tc[k]];
                con[k] = s_con[tc[k]];
                rgb[k] = s_rgb[tc[k]];
            }
            // one wave-uniform choice of exponential for the chunk: the branch-free polynomial unless
            // some cutoff exceeds its range (opacity above ~1e35)
            const float cmax = sxd::smax(sxd::smax(xyo[0].w, xyo[1].w), sxd::smax(xyo[2].w, xyo[3].w));
            const bool general = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(cmax))) > 86.0f;
            float gv[4][NV];
            float alpha[4], vis[4], dxs[4], dys[4], sig[4], e[4];
            bool valid[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                dxs[k] = xyo[k].x - px;
                dys[k] = xyo[k].y - py;
                sig[k] = sigma_of(con[k].x, con[k].y, con[k].z, dxs[k], dys[k]);
                valid[k] = (ts[k] >= 0) & (tc[k] >= t_min) & !(sig[k] > xyo[k].w);  // bitwise: no branches
            }
            const bool any_valid = __any(valid[0] | valid[1] | valid[2] | valid[3]);
            if (STATS) {
                st_chunks++;
                st_entries += min(4, len - j);
                st_empty += any_valid ? 0 : 1;
#pragma unroll
                for (int k = 0; k < 4; k++) st_cut += __popcll(__ballot(valid[k]));
            }
            // no lane has a pair inside the cutoff: every alpha would be 0, leaving T, the back-sum and
            // the gradients as they are
            if (!any_valid) continue;  // uniform
            // The exponential's value only enters gradients (compared at a relative tolerance), so the
            // hardware exp2 serves (relative error below 1.2e-7 (1 + 1.5 sigma): the rounded argument,
            // log2(e) in float, one ulp of v_exp_f32), but the two decisions taken on it — alpha at
            // least 1/255, and opacity * exp at most the 0.99 clamp — must be the forward's. Where a lane
            // lies within 2^-12 in sigma of either turning point, the chunk takes the forward's
            // exponential instead (the points themselves are approximate to ~1e-6).
            bool exact = general;
            if (!exact) {
                bool near = false;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    e[k] = __builtin_amdgcn_exp2f(-sig[k] * 1.44269504f);
                    const bool n1 = __builtin_fabsf(sig[k] - rgb[k].w) < 0x1p-12f;
                    const bool n2 = __builtin_fabsf(sig[k] - con[k].w) < 0x1p-12f;
                    near = near | (valid[k] & (n1 | n2));
                }
                exact = __any(near);
            }
            if (__builtin_expect(exact, 0)) {
                if (general) {
#pragma unroll
                    for (int k = 0; k < 4; k++) e[k] = sxm::expf_fast(-sig[k]);
                } else {
#pragma unroll
                    for (int k = 0; k < 4; k++) e[k] = exp_neg_poly(sig[k]);
                }
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float vis_raw = e[k];
                const float oa = xyo[k].z * vis_raw;
                const float alpha_raw = sxd::smin(sx::kMaxAlpha, oa);
                const bool ok = valid[k] & !((sig[k] < 0.f) | (alpha_raw < sx::kAlphaThreshold));
                alpha[k] = ok ? alpha_raw : 0.0f;
                vis[k] = (ok & (oa <= sx::kMaxAlpha)) ? vis_raw : 0.0f;  // clamped alpha: no sigma/opacity terms
                if (STATS) st_contrib += __popcll(__ballot(ok));
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                // hardware reciprocal (1 ulp; exact for 1): the backward is compared at a relative
                // tolerance, and an IEEE division costs ~10 instructions per pair
                const float ra = __builtin_amdgcn_rcpf(sxd::smax(sx::kMinOneMinusAlpha, 1.0f - alpha[k]));
                T *= ra;
                const float fac = alpha[k] * T;
                gv[k][6] = fac * vc0;
                gv[k][7] = fac * vc1;
                gv[k][8] = fac * vc2;
                // v_alpha = sum_c (c_c T - b_c ra) vc_c + T_final ra (va - <bg, vc>), with the back-sum
                // kept as its dot product with v_render (fused multiply-adds: gradient algebra only)
                const float cvc = __builtin_fmaf(rgb[k].x, vc0, __builtin_fmaf(rgb[k].y, vc1, rgb[k].z * vc2));
                const float v_alpha = __builtin_fmaf(T, cvc, ra * (tva - bdot));
                const float v_sigma = -xyo[k].z * vis[k] * v_alpha;
                const float dx = dxs[k], dy = dys[k];
                const float vdx = v_sigma * dx, vdy = v_sigma * dy;
                if (ABSGRAD) {  // per-pixel 2D gradients are needed for their absolute values
                    gv[k][0] = __builtin_fmaf(con[k].x, vdx, con[k].y * vdy);
                    gv[k][1] = __builtin_fmaf(con[k].y, vdx, con[k].z * vdy);
                    gv[k][3] = 0.5f * vdx * dx;
                    gv[k][5] = 0.5f * vdy * dy;
                    gv[k][9] = fabsf(gv[k][0]);
                    gv[k][10] = fabsf(gv[k][1]);
                } else {  // moments: the conic and the halves are applied once per splat at the flush
                    gv[k][0] = vdx;
                    gv[k][1] = vdy;
                    gv[k][3] = vdx * dx;
                    gv[k][5] = vdy * dy;
                }
                gv[k][4] = vdx * dy;
                gv[k][2] = vis[k] * v_alpha;
                bdot = __builtin_fmaf(fac, cvc, bdot);
            }
            const int t_row = ts[row_slot];
            const bool writer = (lane & 15) == 0 && t_row >= 0;
            float* dst = s_part + (t_row < 0 ? 0 : t_row);
#pragma unroll
            for (int k = 0; k < NV; k++) {
                const float v = wave_sum4(gv[0][k], gv[1][k], gv[2][k], gv[3][k]);
                if (writer) atomicAdd(&dst[k * kThreads], v);  // LDS add: the four waves of the tile
            }
        }
        __syncthreads();
        // one thread per Gaussian of the batch: one global atomic per gradient component
        if (tid < batch_size) {
            float v[NV];
            bool any = false;
#pragma unroll
            for (int k = 0; k < NV; k++) {
                v[k] = s_part[k * kThreads + tid];
                any |= v[k] != 0.f;
            }
            if (!ABSGRAD) {  // sum_p v_sigma (a dx + b dy, b dx + c dy) and the halves of dx^2, dy^2
                const float4 cn = s_con[tid];
                const float sdx = v[0], sdy = v[1];
                v[0] = __builtin_fmaf(cn.x, sdx, cn.y * sdy);
                v[1] = __builtin_fmaf(cn.y, sdx, cn.z * sdy);
                v[3] *= 0.5f;
                v[5] *= 0.5f;
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
    if (STATS && lane == 0) {
        atomicAdd(&a.stats[kStatBwdChunks], st_chunks);
        atomicAdd(&a.stats[kStatBwdEntries], st_entries);
        atomicAdd(&a.stats[kStatBwdEmptyChunks], st_empty);
        atomicAdd(&a.stats[kStatBwdInCutoff], st_cut);
        atomicAdd(&a.stats[kStatBwdContrib], st_contrib);
    }
}

} // namespace

namespace {
// Counting sort of the tiles by descending intersection count (256 buckets of width w, w the
// smallest power of two with max_count < 256 w), one workgroup. Most tiles share a few buckets, so a
// wave's lanes with the same bucket are grouped (one ballot per bucket bit) and one leader lane adds
// the group's size: the LDS adds then never collide within a wave. The order within a bucket is
// arbitrary (the order is only the rasterisers' schedule).
__device__ __forceinline__ uint64_t same_byte_lanes(uint32_t b, bool valid) {
    uint64_t match = __ballot(valid);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const bool bit = (b >> k) & 1u;
        const uint64_t bal = __ballot(bit);
        match &= bit ? bal : ~bal;
    }
    return match;
}

__global__ void __launch_bounds__(1024) k_tile_order(const int32_t* __restrict__ offsets, int n_tiles,
                                                     int64_t n_isects, int32_t* __restrict__ order,
                                                     const int64_t* __restrict__ n_isects_dev) {
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_max;
    if (n_isects_dev) n_isects = *n_isects_dev;
    const int t0 = threadIdx.x, lane = t0 & 63;
    if (t0 < 256) s_hist[t0] = 0;
    if (t0 == 0) s_max = 0;
    __syncthreads();
    auto count_of = [&](int t) -> uint32_t {
        const int64_t e = t + 1 < n_tiles ? offsets[t + 1] : n_isects;
        return static_cast<uint32_t>(e - offsets[t]);
    };
    uint32_t mx = 0;
    for (int t = t0; t < n_tiles; t += 1024) mx = max(mx, count_of(t));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), o, 64)));
    if (lane == 0) atomicMax(&s_max, mx);
    __syncthreads();
    int shift = 0;
    while ((s_max >> shift) >= 256u) shift++;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    // rounds are uniform over the workgroup (every thread runs ceil(n_tiles / 1024) of them)
    for (int t1 = 0; t1 < n_tiles; t1 += 1024) {
        const int t = t1 + t0;
        const bool valid = t < n_tiles;
        const uint32_t b = valid ? 255u - (count_of(t) >> shift) : 0u;
        const uint64_t m = same_byte_lanes(b, valid);
        if (valid && (m & below) == 0) atomicAdd(&s_hist[b], static_cast<uint32_t>(__popcll(m)));
    }
    __syncthreads();
    if (t0 == 0) {  // exclusive prefix over 256 buckets
        uint32_t run = 0;
        for (int b = 0; b < 256; b++) {
            const uint32_t c = s_hist[b];
            s_hist[b] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int t1 = 0; t1 < n_tiles; t1 += 1024) {
        const int t = t1 + t0;
        const bool valid = t < n_tiles;
        const uint32_t b = valid ? 255u - (count_of(t) >> shift) : 0u;
        const uint64_t m = same_byte_lanes(b, valid);
        const int leader = m ? static_cast<int>(__builtin_ctzll(m)) : 0;
        uint32_t base = 0;
        if (valid && lane == leader) base = atomicAdd(&s_hist[b], static_cast<uint32_t>(__popcll(m)));
        base = static_cast<uint32_t>(__shfl(static_cast<int>(base), leader, 64));
        if (valid) order[base + static_cast<uint32_t>(__popcll(m & below))] = t;
    }
}
}  // namespace

void raster_tile_order(const int32_t* offsets, int n_tiles, int64_t n_isects, int32_t* order, hipStream_t s,
                       const int64_t* n_isects_dev) {
    if (n_tiles <= 0) return;
    hipLaunchKernelGGL(k_tile_order, dim3(1), dim3(1024), 0, s, offsets, n_tiles, n_isects, order, n_isects_dev);
}

void raster_fwd(const RasterArgs& a, float* rgb, float* alpha, int32_t* last, hipStream_t s) {
    const int blocks = a.I * a.tile_width * a.tile_height;
    if (blocks <= 0) return;
    if (a.stats)
        hipLaunchKernelGGL(k_raster_fwd<true>, dim3(blocks), dim3(kThreads), 0, s, a, rgb, alpha, last);
    else
        hipLaunchKernelGGL(k_raster_fwd<false>, dim3(blocks), dim3(kThreads), 0, s, a, rgb, alpha, last);
}

void raster_bwd(const RasterArgs& a, const float* ralpha, const int32_t* last_ids, const float* v_rc,
                const float* v_ra, const RasterBwdGrads& g, hipStream_t s) {
    const int blocks = a.I * a.tile_width * a.tile_height;
    if (blocks <= 0 || (!a.n_isects_dev && a.n_isects <= 0)) return;
    if (g.v_means2d_abs)  // the per-op entry's absgrad (never counted)
        hipLaunchKernelGGL((k_raster_bwd<true, false>), dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids, v_rc,
                           v_ra, g);
    else if (a.stats)
        hipLaunchKernelGGL((k_raster_bwd<false, true>), dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids, v_rc,
                           v_ra, g);
    else
        hipLaunchKernelGGL((k_raster_bwd<false, false>), dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids, v_rc,
                           v_ra, g);
}

} // namespace sxk
