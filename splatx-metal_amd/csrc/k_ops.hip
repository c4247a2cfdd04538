// k_ops.hip — gfx950 kernels of the per-op verification surface: Adam, projection fwd/bwd, SH
// fwd/bwd, tile intersection count/emit, int64 scan, tile offsets, splat packing, Philox RNG,
// MCMC relocation and perturbation. Forward math reproduces the CPU reference op order (see
// sx_dev.h); each kernel cites the reference kernel whose contract it implements.
#include <hip/hip_runtime.h>

#include "sx_dev.h"
#include "sx_kernels.h"
#include "sx_philox.h"
#include "sx_dev_bwd.h"

namespace sxk {
using namespace sxd;
namespace {

constexpr int kBlock = 256;
inline int grid_for(int64_t n, int per = kBlock) { return static_cast<int>((n + per - 1) / per); }

// ------------------------------------------------------------------------------------------------
// fused_adam — AdamMCMC.metal:20-46 contract; CpuKernels.cpp:127-144 expression forms.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) k_adam(float* __restrict__ param, const float* __restrict__ grad,
                                                 float* __restrict__ m, float* __restrict__ v,
                                                 const uint8_t* __restrict__ valid, int64_t n, int64_t D,
                                                 float lr, float b1, float b2, float eps) {
    for (int64_t p = blockIdx.x * (int64_t)kBlock + threadIdx.x; p < n; p += (int64_t)gridDim.x * kBlock) {
        if (valid && valid[p / D] == 0) continue;
        const float g = grad[p];
        float mm = m[p], vv = v[p];
        mm = b1 * mm + (1.0f - b1) * g;
        vv = b2 * vv + (1.0f - b2) * g * g;
        const float step = -lr * mm / (__builtin_sqrtf(vv) + eps);
        param[p] += step;
        m[p] = mm;
        v[p] = vv;
    }
}

// ------------------------------------------------------------------------------------------------
// projection fwd — ProjectionEWA.metal:62-180 contract (one thread per (camera, Gaussian)).
// Culled slots write radii = 0 only.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) k_proj_fwd(ProjArgs a, int32_t* __restrict__ radii,
                                                     float* __restrict__ means2d, float* __restrict__ depths,
                                                     float* __restrict__ conics, float* __restrict__ comps) {
    const int64_t idx = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    if (idx >= (int64_t)a.C * a.N) return;
    const int cid = static_cast<int>(idx / a.N);
    const int gid = static_cast<int>(idx % a.N);
    const sxd::Cam cam = sxd::make_cam(a.viewmats + cid * 16, a.Ks + cid * 9, a.width, a.height);
    float Cw[9];
    if (a.covars) {
        const float* cv = a.covars + (size_t)gid * 6;
        Cw[0] = cv[0]; Cw[1] = cv[1]; Cw[2] = cv[2];
        Cw[3] = cv[1]; Cw[4] = cv[3]; Cw[5] = cv[4];
        Cw[6] = cv[2]; Cw[7] = cv[4]; Cw[8] = cv[5];
    } else {
        float q[4] = {a.quats[gid * 4], a.quats[gid * 4 + 1], a.quats[gid * 4 + 2], a.quats[gid * 4 + 3]};
        float s[3] = {a.scales[gid * 3], a.scales[gid * 3 + 1], a.scales[gid * 3 + 2]};
        sxd::quat_scale_to_covar_ref(q, s, Cw);
    }
    sxd::ProjCfg cfg{a.eps2d, a.near_plane, a.far_plane, a.radius_clip, a.calc_comp, a.opacities != nullptr};
    const float mw[3] = {a.means[gid * 3], a.means[gid * 3 + 1], a.means[gid * 3 + 2]};
    const sxd::ProjOut o = sxd::project_one(cam, mw, Cw, a.opacities ? a.opacities[gid] : 1.0f, cfg);
    radii[idx * 2] = o.alive ? o.rx : 0;
    radii[idx * 2 + 1] = o.alive ? o.ry : 0;
    if (!o.alive) return;
    means2d[idx * 2] = o.m2x;
    means2d[idx * 2 + 1] = o.m2y;
    depths[idx] = o.depth;
    conics[idx * 3] = o.ca;
    conics[idx * 3 + 1] = o.cb;
    conics[idx * 3 + 2] = o.cc;
    if (a.calc_comp) comps[idx] = o.comp;
}

// ------------------------------------------------------------------------------------------------
// projection bwd — the VJP of ProjectionEWA.metal:186-560 (inverse, add_blur, persp_proj,
// world->camera, quat/scale->covariance), rematerializing the forward. Dead lanes take part in
// the wave reduction of v_viewmats with zero contributions.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) k_proj_bwd(ProjArgs a, ProjBwdArgs g, float* v_means, float* v_covars,
                                                     float* v_quats, float* v_scales, float* v_view) {
    const int64_t CN = (int64_t)a.C * a.N;
    const int64_t idx0 = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    const bool in_grid = idx0 < CN;
    const int64_t gi = in_grid ? idx0 : 0;
    const int cid = static_cast<int>(gi / a.N);
    const int gid = static_cast<int>(gi % a.N);
    const bool alive = in_grid && g.radii[gi * 2] > 0 && g.radii[gi * 2 + 1] > 0;
    ProjGrad pg;
#pragma unroll
    for (int i = 0; i < 9; i++) { pg.vR[i] = 0.f; pg.vcov[i] = 0.f; }
#pragma unroll
    for (int i = 0; i < 3; i++) { pg.vt[i] = 0.f; pg.vmean[i] = 0.f; }
    float vq[4] = {0.f, 0.f, 0.f, 0.f}, vs[3] = {0.f, 0.f, 0.f};
    float q[4] = {1.f, 0.f, 0.f, 0.f}, s3[3] = {0.f, 0.f, 0.f};
    if (alive) {
        const sxd::Cam cam = sxd::make_cam(a.viewmats + cid * 16, a.Ks + cid * 9, a.width, a.height);
        float Cw[9];
        if (a.covars) {
            const float* cv = a.covars + (size_t)gid * 6;
            Cw[0] = cv[0]; Cw[1] = cv[1]; Cw[2] = cv[2];
            Cw[3] = cv[1]; Cw[4] = cv[3]; Cw[5] = cv[4];
            Cw[6] = cv[2]; Cw[7] = cv[4]; Cw[8] = cv[5];
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) q[k] = a.quats[gid * 4 + k];
#pragma unroll
            for (int k = 0; k < 3; k++) s3[k] = a.scales[gid * 3 + k];
            sxd::quat_scale_to_covar_ref(q, s3, Cw);
        }
        const float mw[3] = {a.means[gid * 3], a.means[gid * 3 + 1], a.means[gid * 3 + 2]};
        const bool has_comp = g.v_comps != nullptr;
        proj_vjp_one(cam, mw, Cw, g.conics[gi * 3], g.conics[gi * 3 + 1], g.conics[gi * 3 + 2],
                     g.v_means2d[gi * 2], g.v_means2d[gi * 2 + 1], g.v_depths[gi], g.v_conics[gi * 3],
                     g.v_conics[gi * 3 + 1], g.v_conics[gi * 3 + 2], has_comp, has_comp ? g.comps[gi] : 0.f,
                     has_comp ? g.v_comps[gi] : 0.f, a.eps2d, pg);
        if (!a.covars) quat_scale_vjp(q, s3, pg.vcov, vq, vs);
    }
    const bool single = a.C == 1;
    if (alive) {
        if (single) {
#pragma unroll
            for (int k = 0; k < 3; k++) v_means[gid * 3 + k] = pg.vmean[k];
            if (a.covars) {
                float* o = v_covars + (size_t)gid * 6;
                o[0] = pg.vcov[0]; o[1] = pg.vcov[1] + pg.vcov[3]; o[2] = pg.vcov[2] + pg.vcov[6];
                o[3] = pg.vcov[4]; o[4] = pg.vcov[5] + pg.vcov[7]; o[5] = pg.vcov[8];
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) v_quats[gid * 4 + k] = vq[k];
#pragma unroll
                for (int k = 0; k < 3; k++) v_scales[gid * 3 + k] = vs[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 3; k++) atomicAdd(&v_means[gid * 3 + k], pg.vmean[k]);
            if (a.covars) {
                float* o = v_covars + (size_t)gid * 6;
                atomicAdd(&o[0], pg.vcov[0]); atomicAdd(&o[1], pg.vcov[1] + pg.vcov[3]);
                atomicAdd(&o[2], pg.vcov[2] + pg.vcov[6]); atomicAdd(&o[3], pg.vcov[4]);
                atomicAdd(&o[4], pg.vcov[5] + pg.vcov[7]); atomicAdd(&o[5], pg.vcov[8]);
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) atomicAdd(&v_quats[gid * 4 + k], vq[k]);
#pragma unroll
                for (int k = 0; k < 3; k++) atomicAdd(&v_scales[gid * 3 + k], vs[k]);
            }
        }
    }
    if (g.viewmats_grad) {
        const int c0 = __shfl(cid, 0, 64);
        const bool uniform = __all(cid == c0);
        if (uniform) {
#pragma unroll
            for (int i = 0; i < 3; i++) {
#pragma unroll
                for (int j = 0; j < 3; j++) {
                    const float r = sxd::wave_sum(pg.vR[i * 3 + j]);
                    if (sxd::lane_id() == 0) atomicAdd(&v_view[c0 * 16 + i * 4 + j], r);
                }
                const float tv = sxd::wave_sum(pg.vt[i]);
                if (sxd::lane_id() == 0) atomicAdd(&v_view[c0 * 16 + i * 4 + 3], tv);
            }
        } else if (alive) {
            for (int i = 0; i < 3; i++) {
                for (int j = 0; j < 3; j++) atomicAdd(&v_view[cid * 16 + i * 4 + j], pg.vR[i * 3 + j]);
                atomicAdd(&v_view[cid * 16 + i * 4 + 3], pg.vt[i]);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// SH fwd/bwd — SphericalHarmonics.metal:399-446 contracts; one thread per element, all channels.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) k_sh_fwd(const float* __restrict__ dirs, const float* __restrict__ coeffs,
                                                   const uint8_t* __restrict__ masks, uint32_t degree, int BN, int N,
                                                   int K, int D, float* __restrict__ colors) {
    const int elem = blockIdx.x * kBlock + threadIdx.x;
    if (elem >= BN) return;
    if (masks && masks[elem] == 0) return;
    const int gid = elem % N;
    const float* cf = coeffs + (size_t)gid * K * D;
    const float dx = dirs[elem * 3], dy = dirs[elem * 3 + 1], dz = dirs[elem * 3 + 2];
    for (int c = 0; c < D; c++)
        colors[(size_t)elem * D + c] = sxd::sh_color(degree, dx, dy, dz, [&](int k) { return cf[k * D + c]; });
}

// DEG is the degree used (compile time, so the basis stays in registers)
template <int DEG>
__global__ void __launch_bounds__(kBlock) k_sh_bwd(const float* __restrict__ dirs, const float* __restrict__ coeffs,
                                                   const uint8_t* __restrict__ masks, int BN, int N,
                                                   int K, int D, const float* __restrict__ v_colors,
                                                   float* __restrict__ v_coeffs, float* __restrict__ v_dirs,
                                                   int atomic_coeffs) {
    constexpr uint32_t degree = DEG;
    const int elem = blockIdx.x * kBlock + threadIdx.x;
    if (elem >= BN) return;
    if (masks && masks[elem] == 0) return;
    const int gid = elem % N;
    const float* cf = coeffs + (size_t)gid * K * D;
    float* vcf = v_coeffs + (size_t)gid * K * D;
    sxd::ShBasis b;
    sxd::sh_basis(degree, dirs[elem * 3], dirs[elem * 3 + 1], dirs[elem * 3 + 2], b);
    constexpr int nb = (DEG + 1) * (DEG + 1);
    float vx = 0.f, vy = 0.f, vz = 0.f;
    for (int c = 0; c < D; c++) {
        const float vc = v_colors[(size_t)elem * D + c];
#pragma unroll
        for (int k = 0; k < nb; k++) {
            const float val = b.Y[k] * vc;
            if (atomic_coeffs) atomicAdd(&vcf[k * D + c], val);
            else vcf[k * D + c] = val;
            const float co = cf[k * D + c];
            vx += vc * (b.dX[k] * co);
            vy += vc * (b.dY[k] * co);
            vz += vc * (b.dZ[k] * co);
        }
    }
    if (v_dirs && degree >= 1) {
        float o[3];
        sxd::sh_dir_vjp(b, vx, vy, vz, o);
        v_dirs[elem * 3] = o[0];
        v_dirs[elem * 3 + 1] = o[1];
        v_dirs[elem * 3 + 2] = o[2];
    }
}

// ------------------------------------------------------------------------------------------------
// isect count / emit — IntersectTile.metal:225-298 contracts (one thread per (image, Gaussian));
// keys iid << (32 + tile_bits) | tile << 32 | f32bits(depth), written into [cum[i-1], cum[i]).
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) k_isect_count(IsectArgs a, int32_t* __restrict__ tiles) {
    const int64_t idx = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    if (idx >= (int64_t)a.I * a.N) return;
    const float rx = static_cast<float>(a.radii[idx * 2]);
    const float ry = static_cast<float>(a.radii[idx * 2 + 1]);
    int32_t cnt = 0;
    if (rx > 0.f && ry > 0.f) {
        const float mx = a.means2d[idx * 2], my = a.means2d[idx * 2 + 1];
        const float ts = static_cast<float>(a.tile_size);
        if (a.conics) {
            cnt = static_cast<int32_t>(sxd::accutile<false>(a.conics[idx * 3], a.conics[idx * 3 + 1],
                                                            a.conics[idx * 3 + 2], a.opacities[idx], mx, my, ts,
                                                            a.tile_width, a.tile_height, [](int32_t) {}));
        } else {
            const sxd::TileRect r = sxd::aabb_rect(mx, my, rx, ry, ts, a.tile_width, a.tile_height);
            cnt = (r.max_y - r.min_y) * (r.max_x - r.min_x);
        }
    }
    tiles[idx] = cnt;
}

__global__ void __launch_bounds__(kBlock) k_isect_emit(IsectArgs a, const int64_t* __restrict__ cum,
                                                       uint64_t* __restrict__ keys, int32_t* __restrict__ vals) {
    const int64_t idx = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    if (idx >= (int64_t)a.I * a.N) return;
    const float rx = static_cast<float>(a.radii[idx * 2]);
    const float ry = static_cast<float>(a.radii[idx * 2 + 1]);
    if (!(rx > 0.f && ry > 0.f)) return;
    const int64_t iid = idx / a.N;
    const uint64_t iid_enc = static_cast<uint64_t>(iid) << (32 + a.tile_n_bits);
    const uint64_t depth_enc = static_cast<uint64_t>(sxm::bits_of(a.depths[idx]));
    int64_t cur = idx == 0 ? 0 : cum[idx - 1];
    const int32_t flat = static_cast<int32_t>(idx);
    const float mx = a.means2d[idx * 2], my = a.means2d[idx * 2 + 1];
    const float ts = static_cast<float>(a.tile_size);
    auto emit = [&](int32_t tile) {
        keys[cur] = iid_enc | (static_cast<uint64_t>(static_cast<uint32_t>(tile)) << 32) | depth_enc;
        vals[cur] = flat;
        ++cur;
    };
    if (a.conics) {
        sxd::accutile<true>(a.conics[idx * 3], a.conics[idx * 3 + 1], a.conics[idx * 3 + 2], a.opacities[idx], mx,
                            my, ts, a.tile_width, a.tile_height, emit);
    } else {
        const sxd::TileRect r = sxd::aabb_rect(mx, my, rx, ry, ts, a.tile_width, a.tile_height);
        for (int32_t i = r.min_y; i < r.max_y; i++)
            for (int32_t j = r.min_x; j < r.max_x; j++) emit(i * a.tile_width + j);
    }
}

// ------------------------------------------------------------------------------------------------
// int32 -> int64 inclusive scan in two launches (block sums; then each block adds the sum of the
// blocks before it, read directly, and scans its own tile). No inter-block waiting.
// ------------------------------------------------------------------------------------------------
constexpr int kScanItems = 16;
constexpr int kScanTile = kBlock * kScanItems;  // 4096

__device__ inline int64_t block_exclusive_scan_i64(int64_t v, int64_t* s_wave, int64_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int64_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int64_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) s_wave[wave] = x;
    __syncthreads();
    int64_t wave_prefix = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kBlock / 64; w++) {
        if (w < wave) wave_prefix += s_wave[w];
        tot += s_wave[w];
    }
    __syncthreads();
    if (total) *total = tot;
    return wave_prefix + x - v;
}

__global__ void __launch_bounds__(kBlock) k_scan_sums(const int32_t* __restrict__ in,
                                                      const int32_t* __restrict__ gather, int64_t n,
                                                      int64_t* __restrict__ sums, const int64_t* __restrict__ n_dev) {
    __shared__ int64_t s_wave[kBlock / 64];
    if (n_dev) n = *n_dev;
    const int64_t base = blockIdx.x * (int64_t)kScanTile;
    int64_t acc = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; i++) {
        const int64_t idx = base + i * kBlock + threadIdx.x;
        if (idx < n) acc += in[gather ? static_cast<int64_t>(gather[idx]) : idx];
    }
    int64_t tot = 0;
    block_exclusive_scan_i64(acc, s_wave, &tot);
    if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

__global__ void __launch_bounds__(kBlock) k_scan_tiles(const int32_t* __restrict__ in,
                                                       const int32_t* __restrict__ gather, int64_t n,
                                                       const int64_t* __restrict__ sums, int64_t* __restrict__ out,
                                                       const int64_t* __restrict__ n_dev) {
    __shared__ int64_t s_wave[kBlock / 64];
    __shared__ int64_t s_prefix;
    if (n_dev) n = *n_dev;
    // prefix of the preceding blocks
    int64_t p = 0;
    for (int b = threadIdx.x; b < static_cast<int>(blockIdx.x); b += kBlock) p += sums[b];
    int64_t ptot = 0;
    block_exclusive_scan_i64(p, s_wave, &ptot);
    if (threadIdx.x == 0) s_prefix = ptot;
    __syncthreads();
    // blocked arrangement: thread t owns items [t*16, t*16+16) of the tile
    const int64_t base = blockIdx.x * (int64_t)kScanTile + (int64_t)threadIdx.x * kScanItems;
    int32_t v[kScanItems];
    int64_t acc = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; i++) {
        v[i] = (base + i < n) ? in[gather ? static_cast<int64_t>(gather[base + i]) : base + i] : 0;
        acc += v[i];
    }
    int64_t run = block_exclusive_scan_i64(acc, s_wave, nullptr) + s_prefix;
#pragma unroll
    for (int i = 0; i < kScanItems; i++) {
        run += v[i];
        if (base + i < n) out[base + i] = run;
    }
}

// ------------------------------------------------------------------------------------------------
// offset encode — IntersectTile.metal:310-335 contract (one thread per sorted intersection).
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) k_offsets(const uint64_t* __restrict__ keys, int64_t n, int64_t total,
                                                    int n_tiles, uint32_t tile_n_bits, int32_t* __restrict__ off,
                                                    uint32_t key_shift) {
    const int64_t idx = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    if (idx >= n) return;
    const uint64_t tile_mask = (static_cast<uint64_t>(1) << tile_n_bits) - 1;
    auto flat_tile = [&](uint64_t key) {
        const uint64_t id = key >> key_shift;
        return static_cast<int64_t>(id >> tile_n_bits) * n_tiles + static_cast<int64_t>(id & tile_mask);
    };
    const int64_t cur = flat_tile(keys[idx]);
    if (idx == 0)
        for (int64_t i = 0; i <= cur; i++) off[i] = 0;
    if (idx == n - 1)
        for (int64_t i = cur + 1; i < total; i++) off[i] = static_cast<int32_t>(n);
    if (idx > 0) {
        if ((keys[idx - 1] >> key_shift) == (keys[idx] >> key_shift)) return;
        const int64_t prev = flat_tile(keys[idx - 1]);
        for (int64_t i = prev + 1; i <= cur; i++) off[i] = static_cast<int32_t>(idx);
    }
}

__global__ void __launch_bounds__(kBlock) k_pack(const float* __restrict__ m2, const float* __restrict__ cn,
                                                 const float* __restrict__ col, const float* __restrict__ op, int n,
                                                 float4* __restrict__ sp) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    sp[i * 3] = make_float4(m2[i * 2], m2[i * 2 + 1], op[i], 0.f);
    sp[i * 3 + 1] = make_float4(cn[i * 3], cn[i * 3 + 1], cn[i * 3 + 2], 0.f);
    sp[i * 3 + 2] = make_float4(col[i * 3], col[i * 3 + 1], col[i * 3 + 2], 0.f);
}

// ------------------------------------------------------------------------------------------------
// RNG / MCMC — Rng.metal:19-47, AdamMCMC.metal:63-140 contracts.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kBlock) k_philox(uint64_t seed, uint64_t offset, int64_t count,
                                                   uint32_t* __restrict__ out) {
    const int64_t t = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    if (t * 4 >= count) return;
    const sx::Philox4 r = sx::philox4x32_10(static_cast<uint32_t>(t), static_cast<uint32_t>(offset),
                                            static_cast<uint32_t>(offset >> 32), 0u, static_cast<uint32_t>(seed),
                                            static_cast<uint32_t>(seed >> 32));
    for (int j = 0; j < 4 && t * 4 + j < count; j++) out[t * 4 + j] = r.v[j];
}

__global__ void __launch_bounds__(kBlock) k_normal(uint64_t seed, uint64_t offset, int64_t count,
                                                   float* __restrict__ out) {
    const int64_t t = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    if (t * 4 >= count) return;
    float z[4];
    sx::philox_normals4(static_cast<uint32_t>(t), seed, offset, z);
    for (int j = 0; j < 4 && t * 4 + j < count; j++) out[t * 4 + j] = z[j];
}

__global__ void __launch_bounds__(kBlock) k_relocation(const float* __restrict__ opac, const float* __restrict__ sc,
                                                       const int32_t* __restrict__ ratios,
                                                       const float* __restrict__ binoms, int N, int n_max,
                                                       float min_opacity, float* __restrict__ new_op,
                                                       float* __restrict__ new_sc) {
    const int idx = blockIdx.x * kBlock + threadIdx.x;
    if (idx >= N) return;
    float coeff;
    new_op[idx] = relocation_one(opac[idx], ratios[idx], binoms, n_max, min_opacity, &coeff);
    for (int i = 0; i < 3; i++) new_sc[idx * 3 + i] = coeff * sc[idx * 3 + i];
}

} // namespace

namespace {
__global__ void __launch_bounds__(kBlock) k_perturb(float* __restrict__ positions, const float* __restrict__ quats,
                                                    const float* __restrict__ slog, const float* __restrict__ logits,
                                                    const float* __restrict__ noise, int N, float noise_scale,
                                                    float tt, float kk) {
    const int idx = blockIdx.x * kBlock + threadIdx.x;
    if (idx >= N) return;
    perturb_one(positions + idx * 3, quats + idx * 4, slog + idx * 3, logits[idx], noise + idx * 3, noise_scale,
                tt, kk);
}
} // namespace

// ---- launchers -------------------------------------------------------------------------------
void adam(float* param, const float* grad, float* m, float* v, const uint8_t* valid, int64_t n, int64_t D,
          float lr, float b1, float b2, float eps, hipStream_t s) {
    if (n <= 0) return;
    const int grid = static_cast<int>(std::min<int64_t>(grid_for(n), 65536));
    hipLaunchKernelGGL(k_adam, dim3(grid), dim3(kBlock), 0, s, param, grad, m, v, valid, n, D, lr, b1, b2, eps);
}

void projection_fwd(const ProjArgs& a, int32_t* radii, float* means2d, float* depths, float* conics, float* comps,
                    hipStream_t s) {
    const int64_t n = (int64_t)a.C * a.N;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_proj_fwd, dim3(grid_for(n)), dim3(kBlock), 0, s, a, radii, means2d, depths, conics, comps);
}

void projection_bwd(const ProjArgs& a, const ProjBwdArgs& g, float* v_means, float* v_covars, float* v_quats,
                    float* v_scales, float* v_viewmats, hipStream_t s) {
    const int64_t n = (int64_t)a.C * a.N;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_proj_bwd, dim3(grid_for(n)), dim3(kBlock), 0, s, a, g, v_means, v_covars, v_quats,
                       v_scales, v_viewmats);
}

void sh_fwd(const float* dirs, const float* coeffs, const uint8_t* masks, uint32_t degree, int B, int N, int K,
            int D, float* colors, hipStream_t s) {
    const int BN = B * N;
    if (BN <= 0) return;
    hipLaunchKernelGGL(k_sh_fwd, dim3(grid_for(BN)), dim3(kBlock), 0, s, dirs, coeffs, masks, degree, BN, N, K, D,
                       colors);
}

void sh_bwd(const float* dirs, const float* coeffs, const uint8_t* masks, uint32_t degree, int B, int N, int K,
            int D, const float* v_colors, float* v_coeffs, float* v_dirs, hipStream_t s) {
    const int BN = B * N;
    if (BN <= 0) return;
    const dim3 grid(grid_for(BN)), block(kBlock);
    const int at = B > 1 ? 1 : 0;
    switch (degree) {
        case 0: hipLaunchKernelGGL(k_sh_bwd<0>, grid, block, 0, s, dirs, coeffs, masks, BN, N, K, D, v_colors, v_coeffs, v_dirs, at); break;
        case 1: hipLaunchKernelGGL(k_sh_bwd<1>, grid, block, 0, s, dirs, coeffs, masks, BN, N, K, D, v_colors, v_coeffs, v_dirs, at); break;
        case 2: hipLaunchKernelGGL(k_sh_bwd<2>, grid, block, 0, s, dirs, coeffs, masks, BN, N, K, D, v_colors, v_coeffs, v_dirs, at); break;
        case 3: hipLaunchKernelGGL(k_sh_bwd<3>, grid, block, 0, s, dirs, coeffs, masks, BN, N, K, D, v_colors, v_coeffs, v_dirs, at); break;
        default: hipLaunchKernelGGL(k_sh_bwd<4>, grid, block, 0, s, dirs, coeffs, masks, BN, N, K, D, v_colors, v_coeffs, v_dirs, at); break;
    }
}

void isect_count(const IsectArgs& a, int32_t* tiles, hipStream_t s) {
    const int64_t n = (int64_t)a.I * a.N;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_isect_count, dim3(grid_for(n)), dim3(kBlock), 0, s, a, tiles);
}

void isect_emit(const IsectArgs& a, const int64_t* cum, uint64_t* keys, int32_t* vals, hipStream_t s) {
    const int64_t n = (int64_t)a.I * a.N;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_isect_emit, dim3(grid_for(n)), dim3(kBlock), 0, s, a, cum, keys, vals);
}

size_t scan_scratch_bytes(int64_t n) { return sizeof(int64_t) * (size_t)std::max<int64_t>(1, grid_for(n, kScanTile)); }

void scan_i32_i64(const int32_t* in, int64_t* out, int64_t n, void* scratch, hipStream_t s, const int32_t* gather,
                  const int64_t* n_dev) {
    if (n <= 0) return;
    const int nb = grid_for(n, kScanTile);
    int64_t* sums = static_cast<int64_t*>(scratch);
    hipLaunchKernelGGL(k_scan_sums, dim3(nb), dim3(kBlock), 0, s, in, gather, n, sums, n_dev);
    hipLaunchKernelGGL(k_scan_tiles, dim3(nb), dim3(kBlock), 0, s, in, gather, n, sums, out, n_dev);
}

void offset_encode(const uint64_t* keys, int64_t n, int I, int n_tiles, uint32_t tile_n_bits, int32_t* off,
                   hipStream_t s, uint32_t key_shift) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_offsets, dim3(grid_for(n)), dim3(kBlock), 0, s, keys, n, (int64_t)I * n_tiles, n_tiles,
                       tile_n_bits, off, key_shift);
}

void pack_splats(const float* m2, const float* cn, const float* col, const float* op, int n, float4* sp,
                 hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_pack, dim3(grid_for(n)), dim3(kBlock), 0, s, m2, cn, col, op, n, sp);
}

void rng_philox_u32(uint64_t seed, uint64_t offset, int64_t count, uint32_t* out, hipStream_t s) {
    if (count <= 0) return;
    hipLaunchKernelGGL(k_philox, dim3(grid_for((count + 3) / 4)), dim3(kBlock), 0, s, seed, offset, count, out);
}

void rng_normal_f32(uint64_t seed, uint64_t offset, int64_t count, float* out, hipStream_t s) {
    if (count <= 0) return;
    hipLaunchKernelGGL(k_normal, dim3(grid_for((count + 3) / 4)), dim3(kBlock), 0, s, seed, offset, count, out);
}

void mcmc_relocation(const float* opac, const float* scales, const int32_t* ratios, const float* binoms, int N,
                     int n_max, float min_opacity, float* new_op, float* new_sc, hipStream_t s) {
    if (N <= 0) return;
    hipLaunchKernelGGL(k_relocation, dim3(grid_for(N)), dim3(kBlock), 0, s, opac, scales, ratios, binoms, N, n_max,
                       min_opacity, new_op, new_sc);
}

void mcmc_perturb(float* positions, const float* quats, const float* slog, const float* logits, const float* noise,
                  int N, float noise_scale, float t, float k, hipStream_t s) {
    if (N <= 0) return;
    hipLaunchKernelGGL(k_perturb, dim3(grid_for(N)), dim3(kBlock), 0, s, positions, quats, slog, logits, noise, N,
                       noise_scale, t, k);
}

} // namespace sxk
