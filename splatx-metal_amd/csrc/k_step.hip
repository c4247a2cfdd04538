// k_step.hip — fused kernels of the device-resident training step (gfx950).
//
// The reference step (MetalBackend.cpp:1696-2264) runs ~95 launches; here the per-Gaussian work
// is two kernels, which a training step runs as one launch per step (the previous step's
// postprocess fused with this step's preprocess, k_postprocess<NC, true>):
//   preprocess  = train_exp + train_sigmoid + projection fwd + AA product + prep_sh + SH fwd (reading
//                 sh0/shN directly, no coeffs assembly) + SH post-op + isect count, and the zeroing
//                 of this Gaussian's gradient record;
//   postprocess = relu mask + SH bwd + AA chain + projection bwd + v_means += v_dirs + activation
//                 chains + regularization + fused Adam of all six groups + (MCMC) Philox normals and
//                 position perturbation of the updated parameters.
// Each reproduces the reference's per-op formulas in the same order as the per-op kernels, so the
// forward is bit-identical to the CPU oracle's host-path step.
#include <hip/hip_runtime.h>

#include <stdexcept>

#include "sx_dev_bwd.h"
#include "sx_loss.h"
#include "sx_philox.h"
#include "sx_step.h"

namespace sxk {
namespace {

constexpr int kBlock = 256;
inline int grid_for(int64_t n, int per = kBlock) { return static_cast<int>((n + per - 1) / per); }

__device__ __forceinline__ void campos_of(const float* vm, float* cp) {
    // campos = -R^T t (Trainer.cpp:753-756)
#pragma unroll
    for (int i = 0; i < 3; i++) cp[i] = -(vm[0 * 4 + i] * vm[0 * 4 + 3] + vm[1 * 4 + i] * vm[1 * 4 + 3] +
                                          vm[2 * 4 + i] * vm[2 * 4 + 3]);
}

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + sxm::expf_(-x)); }

// Adam of one element whose parameter and moments were already loaded (CpuKernels.cpp:127-144 arithmetic);
// returns the updated parameter
// One Adam step of one element; a row that is not `live` (culled: the reference's valid mask skips
// it) writes its values back unchanged, so that a wave stores whole lines of every column.
// The postprocess streams the arena once per step: 708 B per visible row read and written, more than
// the last-level cache holds at a million rows. Nontemporal loads and stores keep that stream from
// evicting what the next kernels and the next step's preprocess read again (measured: postprocess
// 0.31 -> 0.28 ms and preprocess 0.13 -> 0.09 ms at config 3, postprocess 1.02 -> 0.87 ms at config 4).
__device__ __forceinline__ float ld_stream(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream(float* p, float v) { __builtin_nontemporal_store(v, p); }

__device__ __forceinline__ float adam_update(float* __restrict__ p, float* __restrict__ m, float* __restrict__ v,
                                             size_t idx, float p0, float mm, float vv, float g, float lr, float b1,
                                             float b2, float eps, bool live) {
    const float mn = b1 * mm + (1.0f - b1) * g;
    const float vn = b2 * vv + (1.0f - b2) * g * g;
    const float p1 = p0 + -lr * mn / (__builtin_sqrtf(vn) + eps);
    st_stream(&p[idx], live ? p1 : p0);
    st_stream(&m[idx], live ? mn : mm);
    st_stream(&v[idx], live ? vn : vv);
    return live ? p1 : p0;
}


// The preprocess of row i from its parameters (means, quaternion, log scales, logit): projection, colour
// and tile count; stores the splat record and the radii, returns the tile count (0 for a row that is not
// visible; vis = visible). co: the row's SH coefficients when co_ready, else loaded here for a visible
// row (NC = the arena's coefficient count, 1, 4, 9 or 16, a compile-time bound that keeps them in
// registers).
template <int NC>
__device__ __forceinline__ int32_t preprocess_row(const StepConst& c, const Arena& A, int i, const float (&mw)[3],
                                                  const float (&q)[4], const float (&sl)[3], float logit,
                                                  float (&co)[NC][3], bool co_ready, float4* splats, int32_t* radii,
                                                  bool& vis) {
    const size_t R = static_cast<size_t>(A.rows);
    const float s[3] = {sxm::expf_(sl[0]), sxm::expf_(sl[1]), sxm::expf_(sl[2])};
    const float opac = sigmoid_ref(logit);
    float Cw[9];
    sxd::quat_scale_to_covar_ref(q, s, Cw);
    const sxd::Cam cam = sxd::make_cam(c.vm, c.K, c.width, c.height);
    const sxd::ProjCfg cfg{c.eps2d, c.near_plane, c.far_plane, c.radius_clip, c.aa, 1};
    const sxd::ProjOut o = sxd::project_one(cam, mw, Cw, opac, cfg);
    radii[2 * i] = o.alive ? o.rx : 0;
    radii[2 * i + 1] = o.alive ? o.ry : 0;
    int32_t cnt = 0;
    vis = o.alive;
    if (o.alive) {
        const float op_used = c.aa ? opac * o.comp : opac;
        float cp[3];
        campos_of(c.vm, cp);
        const float dx = mw[0] - cp[0], dy = mw[1] - cp[1], dz = mw[2] - cp[2];
        float col[3];
        uint32_t meta = 1u;
        const int nb = (static_cast<int>(c.degree) + 1) * (static_cast<int>(c.degree) + 1);
        if (!co_ready) {
#pragma unroll
            for (int k = 0; k < NC; k++)
#pragma unroll
                for (int ch = 0; ch < 3; ch++)
                    co[k][ch] = k >= nb ? 0.0f : k == 0 ? A.p[4][ch * R + i] : A.p[5][((k - 1) * 3 + ch) * R + i];
        }
#pragma unroll
        for (int ch = 0; ch < 3; ch++) {
            const float raw = sxd::sh_color(c.degree, dx, dy, dz, [&](int k) { return co[k][ch]; });
            const float pre = raw + 0.5f;
            if (pre > 0.0f) meta |= 2u << ch;
            col[ch] = (pre < 0.0f) ? 0.0f : pre;
        }
        if (c.accutile) {
            cnt = static_cast<int32_t>(sxd::accutile<false>(o.ca, o.cb, o.cc, op_used, o.m2x, o.m2y, 16.0f,
                                                            c.tile_width, c.tile_height, [](int32_t) {}));
        } else {
            const sxd::TileRect r = sxd::aabb_rect(o.m2x, o.m2y, static_cast<float>(o.rx),
                                                   static_cast<float>(o.ry), 16.0f, c.tile_width, c.tile_height);
            cnt = (r.max_y - r.min_y) * (r.max_x - r.min_x);
        }
        splats[3 * (size_t)i] = make_float4(o.m2x, o.m2y, op_used, o.depth);
        splats[3 * (size_t)i + 1] = make_float4(o.ca, o.cb, o.cc, o.comp);
        splats[3 * (size_t)i + 2] = make_float4(col[0], col[1], col[2], __uint_as_float(meta));
    } else {
        splats[3 * (size_t)i + 2] = make_float4(0.f, 0.f, 0.f, __uint_as_float(0u));
    }
    return cnt;
}

// The end of a preprocess workgroup (every thread calls it): the step's clears by the first thread of
// the grid, and the block's visible count, tile count and count of Gaussians with tiles (plain stores;
// a single global counter would serialize every wave).
__device__ __forceinline__ void preprocess_block_end(bool vis, uint32_t n_tiles_sum, uint32_t* vis_part,
                                                     const StepClear& clr) {
    __shared__ uint32_t s_vis[kBlock / 64], s_isect[kBlock / 64], s_emit[kBlock / 64];
    if (clr.stamp && blockIdx.x == 0 && threadIdx.x == 0) {
        if (clr.long_prev) *clr.long_prev = *clr.long_count;
        *clr.long_count = 0;
        const uint32_t next = *clr.stamp + 1u;
        *clr.stamp = next ? next : 1u;  // never 0: zeroed entries hold 0
    }
    const unsigned long long bal = __ballot(vis);
    const unsigned long long bal_emit = __ballot(n_tiles_sum > 0u);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        n_tiles_sum += static_cast<uint32_t>(__shfl_xor(static_cast<int>(n_tiles_sum), o, 64));
    if (sxd::lane_id() == 0) {
        s_vis[threadIdx.x >> 6] = static_cast<uint32_t>(__popcll(bal));
        s_isect[threadIdx.x >> 6] = n_tiles_sum;
        s_emit[threadIdx.x >> 6] = static_cast<uint32_t>(__popcll(bal_emit));
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0, isect = 0u, emit = 0u;
#pragma unroll
        for (int w = 0; w < kBlock / 64; w++) {
            t += s_vis[w];
            isect += s_isect[w];
            emit += s_emit[w];
        }
        reinterpret_cast<uint4*>(vis_part)[blockIdx.x] = make_uint4(t, isect, emit, 0u);
    }
}

template <int NC>
__global__ void __launch_bounds__(kBlock) k_preprocess(StepConst c, Arena A, float4* __restrict__ splats,
                                                       int32_t* __restrict__ radii, int32_t* __restrict__ tiles,
                                                       uint32_t* __restrict__ vis_part, StepClear clr) {
    uint32_t n_tiles_sum = 0;  // this lane's tile count; summed per block
    const int i = blockIdx.x * kBlock + threadIdx.x;
    bool vis = false;
    if (i < c.count) {
        const size_t R = static_cast<size_t>(A.rows);
        const float mw[3] = {A.p[0][i], A.p[0][R + i], A.p[0][2 * R + i]};
        const float q[4] = {A.p[1][i], A.p[1][R + i], A.p[1][2 * R + i], A.p[1][3 * R + i]};
        const float sl[3] = {A.p[2][i], A.p[2][R + i], A.p[2][2 * R + i]};
        float co[NC][3];
        const int32_t cnt = preprocess_row<NC>(c, A, i, mw, q, sl, A.p[3][i], co, false, splats, radii, vis);
        tiles[i] = cnt;
        n_tiles_sum = static_cast<uint32_t>(cnt);
        if (clr.touched) clr.touched[i] = 0;
    }
    preprocess_block_end(vis, n_tiles_sum, vis_part, clr);
}

// With the arena in spatial order (row_int[o] = the internal row of original row o): the tile counts in
// original order (tiles_o[o], read by the compaction in sequence) and the per-block counts again, over
// blocks of 256 original rows, so that the compaction below runs in the original order. The visible
// count of block b stays the preprocess's (only its total is read).
__global__ void __launch_bounds__(kBlock) k_orig_block_counts(const int32_t* __restrict__ row_int, int count,
                                                              const int32_t* __restrict__ tiles,
                                                              int32_t* __restrict__ tiles_o,
                                                              uint32_t* __restrict__ vis_part) {
    __shared__ uint32_t s_t[kBlock / 64], s_e[kBlock / 64];
    const int o = blockIdx.x * kBlock + threadIdx.x;
    uint32_t t = 0u;
    if (o < count) {
        t = static_cast<uint32_t>(tiles[row_int[o]]);
        tiles_o[o] = static_cast<int32_t>(t);
    }
    const unsigned long long bal = __ballot(t > 0u);
    uint32_t sum = t;
#pragma unroll
    for (int k = 32; k > 0; k >>= 1) sum += static_cast<uint32_t>(__shfl_xor(static_cast<int>(sum), k, 64));
    if (sxd::lane_id() == 0) {
        s_t[threadIdx.x >> 6] = sum;
        s_e[threadIdx.x >> 6] = static_cast<uint32_t>(__popcll(bal));
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t isect = 0u, emit = 0u;
#pragma unroll
        for (int w = 0; w < kBlock / 64; w++) {
            isect += s_t[w];
            emit += s_e[w];
        }
        uint4* vp = reinterpret_cast<uint4*>(vis_part) + blockIdx.x;
        const uint32_t vis = vp->x;  // the preprocess's (internal block b)
        *vp = make_uint4(vis, isect, emit, 0u);
    }
}

// One workgroup over the preprocess blocks' {visible, tiles, Gaussians with tiles} counts: the totals
// (out = {u64 visible, u64 intersections, u64 Gaussians with tiles, u64 intersections, u64 overflow})
// and, per block b, the intersections and the Gaussians with tiles of the blocks before it (base[2 b],
// base[2 b + 1]). When the intersections exceed `cap` (the buffers' capacity) the step's later kernels
// must not run: overflow = 1 and out[2] = out[3] = 0, the counts they read, so that every one of them
// finds nothing to do (out[1] keeps the true total for the host).
constexpr int kScanBlock = 1024;
constexpr int kScanPer = 4;  // consecutive blocks per thread and chunk
__global__ void __launch_bounds__(kScanBlock) k_block_scan(const uint4* __restrict__ part, int n,
                                                           unsigned long long* __restrict__ out,
                                                           unsigned long long* __restrict__ base,
                                                           unsigned long long cap,
                                                           unsigned long long* __restrict__ host,
                                                           unsigned long long seq) {
    __shared__ unsigned long long s_i[kScanBlock / 64], s_e[kScanBlock / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    unsigned long long vis = 0, carry_i = 0, carry_e = 0;
    for (int b0 = 0; b0 < n; b0 += kScanBlock * kScanPer) {  // uniform
        const int bt = b0 + tid * kScanPer;
        uint4 v[kScanPer];
        unsigned long long si = 0, se = 0;  // the thread's sums
#pragma unroll
        for (int k = 0; k < kScanPer; k++) {
            v[k] = bt + k < n ? part[bt + k] : make_uint4(0u, 0u, 0u, 0u);
            vis += v[k].x;
            si += v[k].y;
            se += v[k].z;
        }
        unsigned long long xi = si, xe = se;  // inclusive scans over the wave
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const unsigned long long yi = __shfl_up(xi, o, 64), ye = __shfl_up(xe, o, 64);
            if (lane >= o) {
                xi += yi;
                xe += ye;
            }
        }
        if (lane == 63) {
            s_i[wave] = xi;
            s_e[wave] = xe;
        }
        __syncthreads();
        unsigned long long pi = carry_i + xi - si, pe = carry_e + xe - se, ti = 0, te = 0;
#pragma unroll
        for (int w = 0; w < kScanBlock / 64; w++) {
            if (w < wave) {
                pi += s_i[w];
                pe += s_e[w];
            }
            ti += s_i[w];
            te += s_e[w];
        }
#pragma unroll
        for (int k = 0; k < kScanPer; k++) {
            if (bt + k < n) {
                base[2 * (size_t)(bt + k)] = pi;
                base[2 * (size_t)(bt + k) + 1] = pe;
            }
            pi += v[k].y;
            pe += v[k].z;
        }
        carry_i += ti;
        carry_e += te;
        __syncthreads();  // s_i / s_e are rewritten by the next chunk
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) vis += __shfl_xor(vis, o, 64);
    if (lane == 0) s_i[wave] = vis;
    __syncthreads();
    if (tid == 0) {
        unsigned long long v = 0;
        for (int w = 0; w < kScanBlock / 64; w++) v += s_i[w];
        const bool ovf = carry_i > cap;
        out[0] = v;
        out[1] = carry_i;
        out[2] = ovf ? 0ull : carry_e;
        out[3] = ovf ? 0ull : carry_i;
        out[4] = ovf ? 1ull : 0ull;
        if (host) {
            store_host(&host[0], v);
            store_host(&host[1], carry_i);
            // the launch's sequence number last: a host that sees it sees the counts
            __hip_atomic_store(&host[4], seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

// The Gaussians with tiles, in index order, compacted: position j = base[2 b + 1] + (its rank among
// block b's) gets list[j] = the Gaussian and (cum set) cum[j] = the inclusive sum of the tile counts
// up to it (base[2 b] + the block's running sum): the emit ranges of the index-first order, and the
// list the depth-first order sorts. row_int (the arena in spatial order): i runs over original rows,
// the list holds internal rows.
__global__ void __launch_bounds__(kBlock) k_emit_compact(const int32_t* __restrict__ tiles, int count,
                                                         const unsigned long long* __restrict__ base,
                                                         int32_t* __restrict__ list, int64_t* __restrict__ cum,
                                                         const int32_t* __restrict__ row_int) {
    __shared__ uint32_t s_n[kBlock / 64], s_t[kBlock / 64];
    const int i = blockIdx.x * kBlock + threadIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = (row_int && i < count) ? row_int[i] : i;  // (with row_int, `tiles` is in original order)
    const uint32_t t = i < count ? static_cast<uint32_t>(tiles[i]) : 0u;
    const unsigned long long bal = __ballot(t > 0u);
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u));
    uint32_t incl = t;  // the block's tile counts are 32-bit (256 Gaussians x at most 2^23 tiles)
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), o, 64));
        if (lane >= o) incl += y;
    }
    if (lane == 63) {
        s_n[wave] = static_cast<uint32_t>(__popcll(bal));
        s_t[wave] = incl;
    }
    __syncthreads();
    uint32_t pn = 0, pt = 0;
#pragma unroll
    for (int w = 0; w < kBlock / 64; w++)
        if (w < wave) {
            pn += s_n[w];
            pt += s_t[w];
        }
    if (t > 0u) {
        const unsigned long long j = base[2 * (size_t)blockIdx.x + 1] + pn + rank;
        list[j] = g;
        if (cum) cum[j] = static_cast<int64_t>(base[2 * (size_t)blockIdx.x] + pt + incl);
    }
}

// Depth-first intersection order. The reference's (tile << depth_bits | depth) keys, sorted stably
// over emit order (Gaussian index, then the Gaussian's own tile order), put each tile's entries in
// (depth, index) order. Here the Gaussians that emit are sorted stably by depth once (a few million
// 32-bit keys), then emit only their tile ids in that order, and a stable sort on the tile bits
// alone finishes the job: within a tile the order is the depth order, ties by index — the same
// permutation, for two radix passes over the intersections instead of five or six.

// depth sort keys of the Gaussians with tiles (list[j], j below *n_list): the depth's float bits (a
// visible depth is positive, so its bits order as the depths do); values = Gaussian index
__global__ void __launch_bounds__(kBlock) k_depth_keys(StepConst c, const float4* __restrict__ splats,
                                                       const int32_t* __restrict__ list,
                                                       const unsigned long long* __restrict__ n_list,
                                                       uint32_t* __restrict__ keys, int32_t* __restrict__ vals) {
    const int j = blockIdx.x * kBlock + threadIdx.x;
    if (j >= c.count || static_cast<unsigned long long>(j) >= *n_list) return;
    const int g = list[j];
    keys[j] = __float_as_uint(splats[3 * (size_t)g].w);
    vals[j] = g;
}

// Thread per position j of the depth order (of the index order when order is null): Gaussian g =
// order[j] owns the output range [cum[j-1], cum[j]) and fills it with its tile ids in the
// reference's emit order, value g. A wave
// works as a queue over the lines of its 64 Gaussians: each lane sets up its own Gaussian's sweep
// (kept in LDS) and counts its lines; the wave then takes the lines of all 64 Gaussians 64 at a
// time, lane l evaluating one line (its cuts are a function of the line alone), and writes the
// chunk's tiles with lane e on entry e — consecutive lanes on consecutive addresses. Tile counts are
// heavy-tailed, and no lane waits on the largest Gaussian of its wave, nor idles through a Gaussian
// of a few lines. A Gaussian of at most kEmitLaneMax tiles is written by its own lane instead (cheaper
// than a queue round for a handful of tiles).
constexpr int kEmitLaneMax = 16;
__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(v, o, 64);
        if (lane >= o) v += y;
    }
    return v;
}

// The last index l of a nondecreasing 64-entry array with a[l] <= x (a[0] <= x).
__device__ __forceinline__ int last_le64(const int* a, int x) {
    int l = 0;
#pragma unroll
    for (int step = 32; step > 0; step >>= 1)
        if (a[l + step] <= x) l += step;
    return l;
}

// Per wave: each Gaussian slot's sweep (the AccuSweep fields the cuts and spans read; with AABB
// tiles, the row range and the column range) and its output range, then the current chunk's lines.
struct EmitWave {
    float4 geo0[64];  // A, B, C, disc
    float4 geo1[64];  // t, p.x, p.y, bbox_max.x
    float4 geo2[64];  // bbox_min.x, bbox_min.y, bbox_max.y, bbox_argmin.y
    float4 geo3[64];  // bbox_argmax.y, rect_min_x (u of the first line), rect_min_y, rect_max_y (bits)
    int is_y[64];
    int line0[65];    // exclusive scan of the slots' line counts
    int g[64];
    uint32_t dbits[64];  // the Gaussian's depth bits (for the per-entry depths of index-first emits)
    long long out0[64], end[64], first[64];  // output range; wave entry index of the slot's first line
    int estart[65];   // the chunk's lines: exclusive scan of their tile counts
    int4 lin0[64];    // output position of the line's first tile (lo, hi), first tile id, id stride
    int4 lin1[64];    // Gaussian, end of its output range (lo, hi), depth bits
};

// Upper cut of sweep line u: the cut at the line's far edge (u + 1) ts while that edge is <= bbox_max.x,
// else the last such cut of the sweep, else the start value (the sweep's carried state, per line).
__device__ __forceinline__ sxd::F2 line_upper_cut(const sxd::AccuSweep& sw, int u) {
    const float e = static_cast<float>(u + 1) * 16.0f;
    if (e <= sw.bbox_max.x) return sxd::accutile_cut(sw, e);
    const float k = __builtin_floorf(sw.bbox_max.x * 0.0625f);  // the last edge index k with 16 k <= bbox_max.x
    if (k >= static_cast<float>(sw.rect_min_x + 1)) return sxd::accutile_cut(sw, k * 16.0f);
    return sxd::accutile_start(sw);
}

// COMPACT (index order): the workgroup takes the 256 rows of preprocess block b instead of 256 emit
// positions, and compacts them first as k_emit_compact does (tiles: the rows' tile counts, base: the block
// scan's bases), writing the list and the offsets (list, cum_out) for the later kernels; a lane's
// Gaussian is then its own row, its output range known without reading them back.
template <class K, bool COMPACT>
__global__ void __launch_bounds__(kBlock) k_emit_sorted(StepConst c, const float4* __restrict__ splats,
                                                        const int32_t* __restrict__ radii,
                                                        const int32_t* __restrict__ order,
                                                        const int64_t* __restrict__ cum, K* __restrict__ keys,
                                                        int32_t* __restrict__ vals, uint32_t* __restrict__ edepth,
                                                        const unsigned long long* __restrict__ n_pos,
                                                        const int32_t* __restrict__ tiles,
                                                        const unsigned long long* __restrict__ base,
                                                        int32_t* __restrict__ list, int64_t* __restrict__ cum_out) {
    __shared__ EmitWave s_w[kBlock / 64];
    const int j = blockIdx.x * kBlock + threadIdx.x;
    const int lane = threadIdx.x & 63;
    EmitWave& W = s_w[threadIdx.x >> 6];
    const int tw = c.tile_width;
    // this lane's Gaussian: its sweep and line count
    int64_t my0 = 0, cnt = 0;
    int g = 0, n_lines = 0;
    uint32_t dbits = 0;
    sxd::AccuSweep sw = {};
    bool have = false;
    if constexpr (COMPACT) {
        __shared__ uint32_t s_n[kBlock / 64], s_t[kBlock / 64];
        const int wave = threadIdx.x >> 6;
        const uint32_t t = j < c.count ? static_cast<uint32_t>(tiles[j]) : 0u;
        const unsigned long long bal = __ballot(t > 0u);
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u));
        uint32_t incl = t;  // the block's tile counts are 32-bit (256 Gaussians x at most 2^23 tiles)
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), o, 64));
            if (lane >= o) incl += y;
        }
        if (lane == 63) {
            s_n[wave] = static_cast<uint32_t>(__popcll(bal));
            s_t[wave] = incl;
        }
        __syncthreads();
        uint32_t pn = 0, pt = 0;
#pragma unroll
        for (int w = 0; w < kBlock / 64; w++)
            if (w < wave) {
                pn += s_n[w];
                pt += s_t[w];
            }
        const unsigned long long jj = base[2 * (size_t)blockIdx.x + 1] + pn + rank;
        if (t > 0u && jj < *n_pos) {  // (n_pos reads 0 after an overflow: nothing is written)
            const int64_t end = static_cast<int64_t>(base[2 * (size_t)blockIdx.x] + pt + incl);
            list[jj] = j;
            cum_out[jj] = end;
            my0 = end - t;
            cnt = t;
            g = j;
            have = true;
        }
    } else if (j < c.count && static_cast<unsigned long long>(j) < *n_pos) {
        my0 = j == 0 ? 0 : cum[j - 1];
        cnt = cum[j] - my0;
        g = cnt > 0 && order ? order[j] : j;
        have = true;
    }
    if (have) {
        if (cnt > 0 && cnt <= kEmitLaneMax) {
            const float4 s0 = splats[3 * (size_t)g];
            dbits = __float_as_uint(s0.w);
            int64_t cur = my0;
            const int64_t end = my0 + cnt;
            auto line = [&](int32_t u, int32_t vmin, int32_t vmax, bool row_major) {
                for (int32_t v = vmin; v < vmax && cur < end; ++v, ++cur) {
                    keys[cur] = static_cast<K>(row_major ? u * tw + v : v * tw + u);
                    vals[cur] = g;
                    if (edepth) edepth[cur] = dbits;
                }
                return true;
            };
            if (c.accutile) {
                const float4 s1 = splats[3 * (size_t)g + 1];
                sxd::accutile_lines(s1.x, s1.y, s1.z, s0.z, s0.x, s0.y, 16.0f, tw, c.tile_height, line);
            } else {
                const sxd::TileRect r = sxd::aabb_rect(s0.x, s0.y, static_cast<float>(radii[2 * g]),
                                                       static_cast<float>(radii[2 * g + 1]), 16.0f, tw, c.tile_height);
                for (int32_t y = r.min_y; y < r.max_y; y++) line(y, r.min_x, r.max_x, true);
            }
        } else if (cnt > 0) {
            const float4 s0 = splats[3 * (size_t)g];
            dbits = __float_as_uint(s0.w);
            if (c.accutile) {
                const float4 s1 = splats[3 * (size_t)g + 1];
                if (sxd::accutile_setup(s1.x, s1.y, s1.z, s0.z, s0.x, s0.y, 16.0f, tw, c.tile_height, sw))
                    n_lines = sw.rect_max_x - sw.rect_min_x;
            } else {
                const sxd::TileRect r = sxd::aabb_rect(s0.x, s0.y, static_cast<float>(radii[2 * g]),
                                                       static_cast<float>(radii[2 * g + 1]), 16.0f, tw, c.tile_height);
                sw.rect_min_x = r.min_y;  // lines are tile rows
                sw.rect_min_y = r.min_x;
                sw.rect_max_y = r.max_x;
                sw.isY = true;
                n_lines = r.max_x > r.min_x ? r.max_y - r.min_y : 0;
            }
        }
    }
    W.geo0[lane] = make_float4(sw.A, sw.B, sw.C, sw.disc);
    W.geo1[lane] = make_float4(sw.t, sw.p.x, sw.p.y, sw.bbox_max.x);
    W.geo2[lane] = make_float4(sw.bbox_min.x, sw.bbox_min.y, sw.bbox_max.y, sw.bbox_argmin.y);
    W.geo3[lane] = make_float4(sw.bbox_argmax.y, __int_as_float(sw.rect_min_x), __int_as_float(sw.rect_min_y),
                               __int_as_float(sw.rect_max_y));
    W.is_y[lane] = sw.isY ? 1 : 0;
    W.g[lane] = g;
    W.dbits[lane] = dbits;
    W.out0[lane] = my0;
    W.end[lane] = my0 + cnt;
    const int lincl = wave_incl_scan(n_lines);
    W.line0[lane] = lincl - n_lines;
    const int total_lines = __shfl(lincl, 63, 64);
    if (lane == 63) W.line0[64] = total_lines;
    __builtin_amdgcn_wave_barrier();
    int64_t ebase = 0;  // wave entry index of the chunk's first tile
    for (int q0 = 0; q0 < total_lines; q0 += 64) {  // uniform
        const int q = q0 + lane;
        const bool live = q < total_lines;
        int k = 0, len = 0, key0 = 0, stride = 1;
        if (live) {
            k = last_le64(W.line0, q);
            const float4 g3 = W.geo3[k];
            const int u = __float_as_int(g3.y) + (q - W.line0[k]);
            const int rmin_y = __float_as_int(g3.z), rmax_y = __float_as_int(g3.w);
            int vmin = rmin_y, vmax = rmax_y;
            const bool is_y = W.is_y[k] != 0;
            if (c.accutile) {
                const float4 g0 = W.geo0[k], g1 = W.geo1[k], g2 = W.geo2[k];
                sxd::AccuSweep ls;
                ls.A = g0.x; ls.B = g0.y; ls.C = g0.z; ls.disc = g0.w;
                ls.t = g1.x; ls.p = {g1.y, g1.z};
                ls.bbox_max = {g1.w, g2.z};
                ls.bbox_min = {g2.x, g2.y};
                ls.bbox_argmin = {0.f, g2.w};
                ls.bbox_argmax = {0.f, g3.x};
                ls.rect_min_x = __float_as_int(g3.y);
                ls.rect_min_y = rmin_y;
                ls.rect_max_y = rmax_y;
                ls.rect_max_x = 0;  // not read by the cuts or spans
                ls.isY = is_y;
                const float min_line = static_cast<float>(u) * 16.0f;
                const float max_line = min_line + 16.0f;
                sxd::F2 lo;
                if (u == ls.rect_min_x)
                    lo = ls.bbox_min.x <= min_line ? sxd::accutile_cut(ls, min_line) : sxd::accutile_start(ls);
                else
                    lo = line_upper_cut(ls, u - 1);
                const sxd::F2 hi = line_upper_cut(ls, u);
                sxd::accutile_span(ls, min_line, max_line, lo, hi, 16.0f, vmin, vmax);
            }
            len = vmax > vmin ? vmax - vmin : 0;
            key0 = is_y ? u * tw + vmin : vmin * tw + u;
            stride = is_y ? 1 : tw;
        }
        const int eincl = wave_incl_scan(len);
        const int estart = eincl - len;
        const int chunk_total = __shfl(eincl, 63, 64);
        if (live && q == W.line0[k]) W.first[k] = ebase + estart;
        W.estart[lane] = live ? estart : chunk_total;
        __builtin_amdgcn_wave_barrier();
        if (live) {
            const long long lbase = W.out0[k] + (ebase + estart - W.first[k]);
            const long long lend = W.end[k];
            W.lin0[lane] = make_int4(static_cast<int>(lbase), static_cast<int>(lbase >> 32), key0, stride);
            W.lin1[lane] = make_int4(W.g[k], static_cast<int>(lend), static_cast<int>(lend >> 32),
                                     static_cast<int>(W.dbits[k]));
        }
        __builtin_amdgcn_wave_barrier();
        for (int e = lane; e < chunk_total; e += 64) {
            const int l = last_le64(W.estart, e);
            const int4 a = W.lin0[l], b = W.lin1[l];
            const int i = e - W.estart[l];
            const int64_t pos = ((static_cast<int64_t>(a.y) << 32) | static_cast<uint32_t>(a.x)) + i;
            const int64_t end = (static_cast<int64_t>(b.z) << 32) | static_cast<uint32_t>(b.y);
            if (pos < end) {
                keys[pos] = static_cast<K>(a.z + i * a.w);
                vals[pos] = b.x;
                if (edepth) edepth[pos] = static_cast<uint32_t>(b.w);
            }
        }
        __builtin_amdgcn_wave_barrier();  // every lane is done with this chunk's lines
        ebase += chunk_total;
    }
}

// offsets[t] = first position of tile t in the sorted tile ids (lower bound; n for trailing empty
// tiles) — the isect_offset_encode contract for one image. Two ways: a binary search per tile (cost
// independent of n), or a pass over the ids in which position i writes the tiles t with
// ids[i-1] < t <= ids[i] (ids[-1] = -1, ids[n] = n_tiles), every offset once (a few MB read, no
// dependent loads: faster up to some tens of millions of ids).
constexpr int kOffPer = 8;  // positions per thread of the pass
template <class K>
__global__ void __launch_bounds__(kBlock) k_tile_offsets_pass(const K* __restrict__ keys, int64_t n, int n_tiles,
                                                              int32_t* __restrict__ off,
                                                              const int64_t* __restrict__ n_dev) {
    if (n_dev) n = *n_dev;
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * kOffPer;
    if (i0 > n) return;
    int prev = i0 == 0 ? -1 : static_cast<int>(keys[i0 - 1]);
#pragma unroll
    for (int k = 0; k < kOffPer; k++) {
        const int64_t i = i0 + k;
        if (i > n) break;
        const int cur = i == n ? n_tiles : static_cast<int>(keys[i]);
        for (int t = prev + 1; t <= cur && t < n_tiles; t++) off[t] = static_cast<int32_t>(i);
        prev = cur;
    }
}

template <class K>
__global__ void __launch_bounds__(kBlock) k_tile_offsets(const K* __restrict__ keys, int64_t n, int n_tiles,
                                                         int32_t* __restrict__ off, const int64_t* __restrict__ n_dev) {
    const int t = blockIdx.x * kBlock + threadIdx.x;
    if (t >= n_tiles) return;
    if (n_dev) n = *n_dev;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = lo + ((hi - lo) >> 1);
        if (static_cast<int>(keys[mid]) < t) lo = mid + 1;
        else hi = mid;
    }
    off[t] = static_cast<int32_t>(lo);
}

// The parameter update of a training step (constants c; NC = the arena's SH coefficient count, 1, 4, 9 or
// 16, a compile-time bound so that the SH basis and its partials stay in registers), per row: relu mask,
// SH backward fused with the Adam of sh0/shN, AA chain, projection backward, gradient chains and
// regularisers, Adam of the geometry; then, with c.inject_noise, the MCMC position noise. The arena is
// left as it was when the step overflowed its buffers and runs again (skip), or when the tile sort gave
// up (sort_err: its lists, and every gradient rasterised from them, are wrong; the host reports the
// error).
// FUSED: the next step's preprocess too (constants cn, the same rows), from the row's updated values
// still in registers instead of a second read of the arena — the same results as this update followed
// by k_preprocess; the row's touched flag (read by the update) is then cleared for the new step when
// clr.touched is set.
template <int NC, bool FUSED>
__global__ void __launch_bounds__(kBlock) k_postprocess(StepConst c, Arena A, float4* splats,
                                                        const float4* __restrict__ grads, uint8_t* touched,
                                                        const unsigned long long* __restrict__ skip,
                                                        const uint32_t* __restrict__ sort_err, StepConst cn,
                                                        int32_t* __restrict__ radii, int32_t* __restrict__ tiles,
                                                        uint32_t* __restrict__ vis_part, StepClear clr,
                                                        const int32_t* __restrict__ row_orig) {
    const bool apply = !(skip && *skip) && !(sort_err && *sort_err);  // uniform
    if (!FUSED && !apply) return;
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (!FUSED && i >= c.count) return;
    const bool row = i < c.count;
    const size_t R = static_cast<size_t>(A.rows);
    const uint32_t meta = row ? __float_as_uint(splats[3 * (size_t)i + 2].w) : 0u;
    const bool live = meta & 1u;
    // A wave with a visible row takes its culled rows along (loaded and stored back unchanged): the
    // columns are SoA, so skipping them would leave every line partially written (a read-modify-write
    // in the memory system). A wave of culled rows with no noise has nothing to read or write.
    const bool wave_live = __any(live);
    if (!FUSED && !wave_live && !c.inject_noise) return;
    float mw[3], q[4], sl[3], logit = 0.f;
    if (row) {
        mw[0] = ld_stream(&A.p[0][i]);
        mw[1] = ld_stream(&A.p[0][R + i]);
        mw[2] = ld_stream(&A.p[0][2 * R + i]);
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = ld_stream(&A.p[1][k * R + i]);
#pragma unroll
        for (int k = 0; k < 3; k++) sl[k] = ld_stream(&A.p[2][k * R + i]);
        logit = ld_stream(&A.p[3][i]);
    }
    float co[NC][3];  // FUSED: the updated SH coefficients when co_ready
    bool co_ready = false;
    if (row && apply && wave_live) {
        // rows no tile reached have no gradient record this step: zeros
        // (a branch around the loads: as selects between a load and a zero vector, the compiler can turn
        // them into one load through a select of two pointers, one to a zero vector in scratch memory)
        float4 g0 = make_float4(0.f, 0.f, 0.f, 0.f), g1 = g0, g2 = g0;
        if (live && touched[i]) {
            g0 = grads[3 * (size_t)i];
            g1 = grads[3 * (size_t)i + 1];
            g2 = grads[3 * (size_t)i + 2];
        }
        const float4 s1 = splats[3 * (size_t)i + 1];
        // relu mask (train_relu_mask_apply)
        const float vrgb[3] = {(meta & 2u) ? g2.x : 0.0f, (meta & 4u) ? g2.y : 0.0f, (meta & 8u) ? g2.z : 0.0f};
        // moments of means, quats, scales and opacity, requested now and used at the end
        float m0[3], v0[3], m1[4], v1[4], m2[3], v2[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            m0[k] = ld_stream(&A.m[0][k * R + i]);
            v0[k] = ld_stream(&A.v[0][k * R + i]);
            m2[k] = ld_stream(&A.m[2][k * R + i]);
            v2[k] = ld_stream(&A.v[2][k * R + i]);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            m1[k] = ld_stream(&A.m[1][k * R + i]);
            v1[k] = ld_stream(&A.v[1][k * R + i]);
        }
        const float m3 = ld_stream(&A.m[3][i]), v3 = ld_stream(&A.v[3][i]);
        // SH backward fused with Adam of sh0 / shN. Loads are issued in bursts (all coefficients,
        // then the moments chunk by chunk) so that a wave has many requests in flight instead of one
        // load-update-store round trip per coefficient.
        float cp[3];
        campos_of(c.vm, cp);
        sxd::ShBasis b;
        sxd::sh_basis(c.degree, mw[0] - cp[0], mw[1] - cp[1], mw[2] - cp[2], b);
        const int nb = (static_cast<int>(c.degree) + 1) * (static_cast<int>(c.degree) + 1);
#pragma unroll
        for (int k = 0; k < NC; k++)
#pragma unroll
            for (int ch = 0; ch < 3; ch++)
                co[k][ch] = k == 0 ? ld_stream(&A.p[4][(size_t)ch * R + i])
                                   : ld_stream(&A.p[5][(size_t)((k - 1) * 3 + ch) * R + i]);
        float vx = 0.f, vy = 0.f, vz = 0.f;
#pragma unroll
        for (int k = 0; k < NC; k++)
#pragma unroll
            for (int ch = 0; ch < 3; ch++)
                if (k < nb) {
                    vx += vrgb[ch] * (b.dX[k] * co[k][ch]);
                    vy += vrgb[ch] * (b.dY[k] * co[k][ch]);
                    vz += vrgb[ch] * (b.dZ[k] * co[k][ch]);
                }
        constexpr int KC = NC < 4 ? NC : 4;  // coefficients per moment burst
#pragma unroll
        for (int k0 = 0; k0 < NC; k0 += KC) {
            float mm[KC][3], vv[KC][3];
#pragma unroll
            for (int dk = 0; dk < KC; dk++)
#pragma unroll
                for (int ch = 0; ch < 3; ch++) {
                    const int k = k0 + dk;
                    if (k >= NC) continue;  // last chunk of NC = 9 is partial
                    const int grp = k == 0 ? 4 : 5;
                    const size_t idx = (k == 0 ? (size_t)ch : (size_t)((k - 1) * 3 + ch)) * R + i;
                    mm[dk][ch] = ld_stream(&A.m[grp][idx]);
                    vv[dk][ch] = ld_stream(&A.v[grp][idx]);
                }
#pragma unroll
            for (int dk = 0; dk < KC; dk++)
#pragma unroll
                for (int ch = 0; ch < 3; ch++) {
                    const int k = k0 + dk;
                    if (k >= NC) continue;
                    const int grp = k == 0 ? 4 : 5;
                    const size_t idx = (k == 0 ? (size_t)ch : (size_t)((k - 1) * 3 + ch)) * R + i;
                    const float g = k < nb ? b.Y[k] * vrgb[ch] : 0.0f;
                    co[k][ch] = adam_update(A.p[grp], A.m[grp], A.v[grp], idx, co[k][ch], mm[dk][ch], vv[dk][ch], g,
                                            c.lr[grp], c.b1, c.b2, c.eps, live);
                }
        }
        float vdir[3] = {0.f, 0.f, 0.f};
        if (c.degree >= 1) sxd::sh_dir_vjp(b, vx, vy, vz, vdir);
        // AA chain (train_aa_chain) and projection backward
        const float opac = sigmoid_ref(logit);
        float v_op = g0.z, v_comp = 0.f;
        if (c.aa) {
            v_comp = v_op * opac;
            v_op = v_op * s1.w;
        }
        const float s[3] = {sxm::expf_(sl[0]), sxm::expf_(sl[1]), sxm::expf_(sl[2])};
        float Cw[9];
        sxd::quat_scale_to_covar_ref(q, s, Cw);
        const sxd::Cam cam = sxd::make_cam(c.vm, c.K, c.width, c.height);
        sxd::ProjGrad pg;
        sxd::proj_vjp_one(cam, mw, Cw, s1.x, s1.y, s1.z, g0.x, g0.y, 0.f, g1.x, g1.y, g1.z, c.aa != 0, s1.w, v_comp,
                          c.eps2d, pg);
        float vq[4], vs[3];
        sxd::quat_scale_vjp(q, s, pg.vcov, vq, vs);
        // chains (train_add_inplace, train_scale_grad_chain, train_opacity_grad_chain)
        float vm_[3];
#pragma unroll
        for (int k = 0; k < 3; k++) vm_[k] = pg.vmean[k] + vdir[k];
        float vsl[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            float v = vs[k] * s[k];
            if (c.scale_reg_w > 0.0f) v += c.scale_reg_w * s[k];
            vsl[k] = v;
        }
        float vlog = v_op * (opac * (1.0f - opac));
        if (c.opacity_reg_w > 0.0f) vlog += c.opacity_reg_w * opac * (1.0f - opac);
        // Adam of means, quats, scales, opacities (the updated values stay in registers for the noise
        // step and the next preprocess)
#pragma unroll
        for (int k = 0; k < 3; k++)
            mw[k] = adam_update(A.p[0], A.m[0], A.v[0], k * R + i, mw[k], m0[k], v0[k], vm_[k], c.lr[0], c.b1, c.b2,
                                c.eps, live);
#pragma unroll
        for (int k = 0; k < 4; k++)
            q[k] = adam_update(A.p[1], A.m[1], A.v[1], k * R + i, q[k], m1[k], v1[k], vq[k], c.lr[1], c.b1, c.b2, c.eps,
                               live);
#pragma unroll
        for (int k = 0; k < 3; k++)
            sl[k] = adam_update(A.p[2], A.m[2], A.v[2], k * R + i, sl[k], m2[k], v2[k], vsl[k], c.lr[2], c.b1, c.b2,
                                c.eps, live);
        logit = adam_update(A.p[3], A.m[3], A.v[3], i, logit, m3, v3, vlog, c.lr[3], c.b1, c.b2, c.eps, live);
        co_ready = true;
    }
    if (row && apply && c.inject_noise) {
        // normals 3i..3i+2 of the Philox stream (seed, offset), i the original row: blocks t = n / 4
        const uint32_t n0 = 3u * static_cast<uint32_t>(row_orig ? row_orig[i] : i);
        const uint32_t t0 = n0 >> 2, t1 = (n0 + 2u) >> 2;
        float z0[4], z1[4];
        sx::philox_normals4(t0, c.noise_seed, c.noise_offset, z0);
        if (t1 != t0) sx::philox_normals4(t1, c.noise_seed, c.noise_offset, z1);
        float nz[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const uint32_t n = n0 + k;
            const uint32_t t = n >> 2;
            const uint32_t j = n & 3u;  // register selects (a dynamic array index would go to scratch)
            const float a = j == 0 ? z0[0] : j == 1 ? z0[1] : j == 2 ? z0[2] : z0[3];
            const float b = j == 0 ? z1[0] : j == 1 ? z1[1] : j == 2 ? z1[2] : z1[3];
            nz[k] = (t == t0) ? a : b;
        }
        sxd::perturb_one(mw, q, sl, logit, nz, c.noise_scale, 0.005f, 100.0f);
#pragma unroll
        for (int k = 0; k < 3; k++) A.p[0][k * R + i] = mw[k];
    }
    if constexpr (FUSED) {
        uint32_t n_tiles_sum = 0;
        bool vis = false;
        if (row) {
            const int32_t cnt = preprocess_row<NC>(cn, A, i, mw, q, sl, logit, co, co_ready, splats, radii, vis);
            tiles[i] = cnt;
            n_tiles_sum = static_cast<uint32_t>(cnt);
            if (clr.touched) touched[i] = 0;
        }
        preprocess_block_end(vis, n_tiles_sum, vis_part, clr);
    }
}

__global__ void __launch_bounds__(kBlock) k_l1(const float* __restrict__ render, const float* __restrict__ gt, int64_t n,
                                               float g, float* __restrict__ v, double* __restrict__ partials) {
    __shared__ double s_red[kBlock];
    double acc = 0.0;
    for (int64_t k = blockIdx.x * (int64_t)kBlock + threadIdx.x; k < n; k += (int64_t)gridDim.x * kBlock) {
        const float d = render[k] - gt[k];
        acc += fabs(static_cast<double>(d));
        v[k] = d > 0.0f ? g : (d < 0.0f ? -g : 0.0f);
    }
    s_red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = kBlock / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) s_red[threadIdx.x] += s_red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) partials[blockIdx.x] = s_red[0];
}


__global__ void k_set_word(uint32_t* word, uint32_t value) { *word = value; }

__global__ void k_step_readback(StepReadback rb) {
    store_host(&rb.host[0], 0u);
    store_host(&rb.host[1], *rb.sort_err);
    store_host(&rb.host[2], *rb.max_tile);
    store_host(&rb.host[3], 0u);
    __hip_atomic_store(rb.seq_host, rb.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void __launch_bounds__(kBlock) k_aos_to_soa(const float* __restrict__ aos, float* __restrict__ soa, int rows,
                                                       int dim, int stride) {
    const int64_t k = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    if (k >= (int64_t)rows * dim) return;
    const int r = static_cast<int>(k / dim), d = static_cast<int>(k % dim);
    soa[(size_t)d * stride + r] = aos[k];
}

__global__ void __launch_bounds__(kBlock) k_soa_to_aos(const float* __restrict__ soa, float* __restrict__ aos, int rows,
                                                       int dim, int stride) {
    const int64_t k = blockIdx.x * (int64_t)kBlock + threadIdx.x;
    if (k >= (int64_t)rows * dim) return;
    const int r = static_cast<int>(k / dim), d = static_cast<int>(k % dim);
    aos[k] = soa[(size_t)d * stride + r];
}

} // namespace

void step_preprocess(const StepConst& c, const Arena& A, float4* splats, int32_t* radii, int32_t* tiles,
                     uint32_t* vis_part, unsigned long long* n_visible, unsigned long long* block_base,
                     unsigned long long isect_cap, unsigned long long* host_counts, unsigned long long seq,
                     const StepClear& clr, hipStream_t s, const int32_t* row_int, int32_t* tiles_o) {
    if (c.count <= 0) return;
    const dim3 grid(grid_for(c.count)), block(kBlock);
    switch (c.n_coeffs) {
        case 1: hipLaunchKernelGGL(k_preprocess<1>, grid, block, 0, s, c, A, splats, radii, tiles, vis_part, clr); break;
        case 4: hipLaunchKernelGGL(k_preprocess<4>, grid, block, 0, s, c, A, splats, radii, tiles, vis_part, clr); break;
        case 9: hipLaunchKernelGGL(k_preprocess<9>, grid, block, 0, s, c, A, splats, radii, tiles, vis_part, clr); break;
        case 16: hipLaunchKernelGGL(k_preprocess<16>, grid, block, 0, s, c, A, splats, radii, tiles, vis_part, clr); break;
        default: throw std::invalid_argument("preprocess: SH coefficient count must be 1, 4, 9 or 16");
    }
    if (row_int)  // the tile counts and the block counts in original order
        hipLaunchKernelGGL(k_orig_block_counts, grid, block, 0, s, row_int, c.count, tiles, tiles_o, vis_part);
    hipLaunchKernelGGL(k_block_scan, dim3(1), dim3(kScanBlock), 0, s, reinterpret_cast<const uint4*>(vis_part),
                       static_cast<int>(grid.x), n_visible, block_base, isect_cap, host_counts, seq);
}

void step_emit_compact(const StepConst& c, const int32_t* tiles, const unsigned long long* block_base, int32_t* list,
                       int64_t* cum, hipStream_t s, const int32_t* row_int) {
    if (c.count <= 0) return;
    hipLaunchKernelGGL(k_emit_compact, dim3(grid_for(c.count)), dim3(kBlock), 0, s, tiles, c.count, block_base, list,
                       cum, row_int);
}

int step_preprocess_blocks(int64_t count) { return grid_for(count); }

void step_depth_keys(const StepConst& c, const float4* splats, const int32_t* list, const unsigned long long* n_list,
                     uint32_t* keys, int32_t* vals, hipStream_t s) {
    if (c.count <= 0) return;
    hipLaunchKernelGGL(k_depth_keys, dim3(grid_for(c.count)), dim3(kBlock), 0, s, c, splats, list, n_list, keys,
                       vals);
}

void step_emit_sorted(const StepConst& c, const float4* splats, const int32_t* radii, const int32_t* order,
                      const int64_t* cum, const unsigned long long* n_pos, uint16_t* keys, int32_t* vals,
                      hipStream_t s, uint32_t* edepth) {
    if (c.count <= 0) return;
    hipLaunchKernelGGL((k_emit_sorted<uint16_t, false>), dim3(grid_for(c.count)), dim3(kBlock), 0, s, c, splats, radii,
                       order, cum, keys, vals, edepth, n_pos, nullptr, nullptr, nullptr, nullptr);
}

void step_emit_sorted(const StepConst& c, const float4* splats, const int32_t* radii, const int32_t* order,
                      const int64_t* cum, const unsigned long long* n_pos, uint32_t* keys, int32_t* vals,
                      hipStream_t s, uint32_t* edepth) {
    if (c.count <= 0) return;
    hipLaunchKernelGGL((k_emit_sorted<uint32_t, false>), dim3(grid_for(c.count)), dim3(kBlock), 0, s, c, splats, radii,
                       order, cum, keys, vals, edepth, n_pos, nullptr, nullptr, nullptr, nullptr);
}

template <class K>
static void launch_emit_compact_sorted(const StepConst& c, const float4* splats, const int32_t* radii,
                                       const int32_t* tiles, const unsigned long long* block_base, int32_t* list,
                                       int64_t* cum, const unsigned long long* n_pos, K* keys, int32_t* vals,
                                       hipStream_t s, uint32_t* edepth) {
    if (c.count <= 0) return;
    hipLaunchKernelGGL((k_emit_sorted<K, true>), dim3(grid_for(c.count)), dim3(kBlock), 0, s, c, splats, radii,
                       nullptr, nullptr, keys, vals, edepth, n_pos, tiles, block_base, list, cum);
}

void step_emit_compact_sorted(const StepConst& c, const float4* splats, const int32_t* radii, const int32_t* tiles,
                              const unsigned long long* block_base, int32_t* list, int64_t* cum,
                              const unsigned long long* n_pos, uint16_t* keys, int32_t* vals, hipStream_t s,
                              uint32_t* edepth) {
    launch_emit_compact_sorted(c, splats, radii, tiles, block_base, list, cum, n_pos, keys, vals, s, edepth);
}

void step_emit_compact_sorted(const StepConst& c, const float4* splats, const int32_t* radii, const int32_t* tiles,
                              const unsigned long long* block_base, int32_t* list, int64_t* cum,
                              const unsigned long long* n_pos, uint32_t* keys, int32_t* vals, hipStream_t s,
                              uint32_t* edepth) {
    launch_emit_compact_sorted(c, splats, radii, tiles, block_base, list, cum, n_pos, keys, vals, s, edepth);
}

// n (the count, or with n_dev its upper bound) picks the way: the pass up to 2^25 ids
constexpr int64_t kOffPassMax = int64_t{1} << 25;
template <class K>
static void launch_tile_offsets(const K* keys, int64_t n, int n_tiles, int32_t* offsets, hipStream_t s,
                                const int64_t* n_dev) {
    if (n_tiles <= 0) return;
    if (n <= kOffPassMax) {
        const int64_t threads = n / kOffPer + 1;  // positions 0..n
        hipLaunchKernelGGL(k_tile_offsets_pass<K>, dim3(grid_for(threads)), dim3(kBlock), 0, s, keys, n, n_tiles,
                           offsets, n_dev);
    } else {
        hipLaunchKernelGGL(k_tile_offsets<K>, dim3(grid_for(n_tiles)), dim3(kBlock), 0, s, keys, n, n_tiles, offsets,
                           n_dev);
    }
}

void step_tile_offsets(const uint16_t* keys, int64_t n, int n_tiles, int32_t* offsets, hipStream_t s,
                       const int64_t* n_dev) {
    launch_tile_offsets(keys, n, n_tiles, offsets, s, n_dev);
}

void step_tile_offsets(const uint32_t* keys, int64_t n, int n_tiles, int32_t* offsets, hipStream_t s,
                       const int64_t* n_dev) {
    launch_tile_offsets(keys, n, n_tiles, offsets, s, n_dev);
}

void step_update_preprocess(const StepConst& cu, const StepConst& c, const Arena& A, float4* splats, const float4* grads,
                            uint8_t* touched, const unsigned long long* skip, const uint32_t* sort_err, int32_t* radii,
                            int32_t* tiles, uint32_t* vis_part, unsigned long long* n_visible,
                            unsigned long long* block_base, unsigned long long isect_cap, unsigned long long* host_counts,
                            unsigned long long seq, const StepClear& clr, hipStream_t s, const int32_t* row_orig,
                            const int32_t* row_int, int32_t* tiles_o) {
    if (c.count <= 0) return;
    if (cu.count != c.count || cu.n_coeffs != c.n_coeffs)
        throw std::invalid_argument("update_preprocess: both steps must cover the same rows");
    if (clr.touched && clr.touched != touched)
        throw std::invalid_argument("update_preprocess: the touched flags cleared must be the ones read");
    const dim3 grid(grid_for(c.count)), block(kBlock);
#define SX_UPD(NC)                                                                                              \
    hipLaunchKernelGGL((k_postprocess<NC, true>), grid, block, 0, s, cu, A, splats, grads, touched, skip, sort_err, c, \
                       radii, tiles, vis_part, clr, row_orig)
    switch (c.n_coeffs) {
        case 1: SX_UPD(1); break;
        case 4: SX_UPD(4); break;
        case 9: SX_UPD(9); break;
        case 16: SX_UPD(16); break;
        default: throw std::invalid_argument("update_preprocess: SH coefficient count must be 1, 4, 9 or 16");
    }
#undef SX_UPD
    if (row_int)  // the tile counts and the block counts in original order
        hipLaunchKernelGGL(k_orig_block_counts, grid, block, 0, s, row_int, c.count, tiles, tiles_o, vis_part);
    hipLaunchKernelGGL(k_block_scan, dim3(1), dim3(kScanBlock), 0, s, reinterpret_cast<const uint4*>(vis_part),
                       static_cast<int>(grid.x), n_visible, block_base, isect_cap, host_counts, seq);
}

void step_postprocess(const StepConst& c, const Arena& A, const float4* splats, const float4* grads,
                      const uint8_t* touched, hipStream_t s, const unsigned long long* skip,
                      const uint32_t* sort_err, const int32_t* row_orig) {
    if (c.count <= 0) return;
    const dim3 grid(grid_for(c.count)), block(kBlock);
    // (the splat records and touched flags are only read: the launch shares the fused variant's signature)
    float4* sp = const_cast<float4*>(splats);
    uint8_t* tch = const_cast<uint8_t*>(touched);
#define SX_PP(NC)                                                                                                \
    hipLaunchKernelGGL((k_postprocess<NC, false>), grid, block, 0, s, c, A, sp, grads, tch, skip, sort_err, c, \
                       nullptr, nullptr, nullptr, StepClear{}, row_orig)
    switch (c.n_coeffs) {
        case 1: SX_PP(1); break;
        case 4: SX_PP(4); break;
        case 9: SX_PP(9); break;
        case 16: SX_PP(16); break;
        default: throw std::invalid_argument("postprocess: SH coefficient count must be 1, 4, 9 or 16");
    }
#undef SX_PP
}

int step_l1_blocks(int64_t n) { return static_cast<int>(std::min<int64_t>(1024, grid_for(n))); }

void step_l1_grad(const float* render, const float* gt, int64_t n, float* v_render, double* partials, int n_blocks,
                  hipStream_t s) {
    const float g = 1.0f / static_cast<float>(n);
    hipLaunchKernelGGL(k_l1, dim3(n_blocks), dim3(kBlock), 0, s, render, gt, n, g, v_render, partials);
}

void step_set_word(uint32_t* word, uint32_t value, hipStream_t s) {
    hipLaunchKernelGGL(k_set_word, dim3(1), dim3(1), 0, s, word, value);
}

void step_readback(const StepReadback& rb, hipStream_t s) {
    if (!rb.host) return;
    hipLaunchKernelGGL(k_step_readback, dim3(1), dim3(1), 0, s, rb);
}

void aos_to_soa(const float* aos, float* soa, int rows, int dim, int stride, hipStream_t s) {
    const int64_t n = (int64_t)rows * dim;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_aos_to_soa, dim3(grid_for(n)), dim3(kBlock), 0, s, aos, soa, rows, dim, stride);
}

void soa_to_aos(const float* soa, float* aos, int rows, int dim, int stride, hipStream_t s) {
    const int64_t n = (int64_t)rows * dim;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_soa_to_aos, dim3(grid_for(n)), dim3(kBlock), 0, s, soa, aos, rows, dim, stride);
}

} // namespace sxk
