// k_raster.hip — tile rasterizer forward and backward for gfx950.
//
// Contracts: rasterize_to_pixels_3dgs_fwd/bwd (Rasterize3DGSFwd.metal:57-204,
// Rasterize3DGSBwd.metal:70-298). One 256-thread workgroup (4 waves of 64) per 16x16 tile, one
// thread per pixel. Splat records (3 x float4) are staged through LDS in batches of 256.
//
// Block groups: the tile is sixteen 4x4 pixel blocks. Wave w covers the 8x8 quadrant
// (w & 1, w >> 1); its lanes form four 16-lane groups, one block each (lane l: group l >> 4, pixel
// l & 15 at (l & 3, (l >> 2) & 3) of the block). Per batch each block gets the list of the batch's
// splats whose cutoff set can reach it, in depth order, and the four groups of a wave walk their own
// lists in lockstep: a group reads its own splat from LDS, so a wave evaluates four splats against
// the 16 pixels each can reach instead of one splat against a 64-pixel strip (the splats are small:
// most of a strip's lanes would sit outside their cutoff).
// Forward: front-to-back compositing with the exclusive T <= 1e-4 stop, per-pixel arithmetic in
// the CPU reference's order (CpuKernels.cpp:821-849) and the deterministic exp of sx_fmath.h, so
// colors/alphas/last_ids are bit-identical to the CPU oracle; two list entries per iteration; the
// workgroup exits as soon as all its pixels are done.
// Backward: back-to-front walk recovering T by division, four list entries per group at a time;
// a group sums its four splats' nine gradient components over its 16 lanes with one transposed
// reduction (8 DPP instructions per component) and stores the sums in an LDS entry buffer; per
// segment (a run of batch slots in which no block's list passes the buffer's 32 entries) the threads of
// each slot add its entries over the blocks it reached and store the (tile, Gaussian) totals at the
// slot's emit position (plain stores), which the gather then adds per Gaussian in a fixed order. The
// per-op entry point adds them with float atomics.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "sx_dev.h"
#include "sx_kernels.h"
#include "sx_loss.h"
#include "sx_order.h"

namespace sxk {
namespace {

constexpr int kThreads = 256;
constexpr int kBlocks = 16;  // 4x4 pixel blocks of a tile
#ifndef SX_BWD_SEG
#define SX_BWD_SEG 32
#endif
// backward segment: at most this many entries per block list between flushes (the entry buffer's row:
// 32 gives 36 KB of LDS, 4 workgroups per CU)
constexpr int kBwdSeg = SX_BWD_SEG;

// sxm::expf_fast(-sigma) without its range branches: identical for sigma in [0, 86] (no overflow,
// no subnormal scaling). Only an opacity above ~1e35 pushes a cutoff past that range; the callers
// then take the general function for the whole batch of splats.
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
    // p * 2^k with k in [-125, 0]: the product is a normal float, so scaling the exponent (v_ldexp_f32)
    // gives the same bits as multiplying by 2^k, in one instruction instead of three
    return __builtin_amdgcn_ldexpf(p, static_cast<int>(kf));
}

__device__ __forceinline__ float sigma_of(float ca, float cb, float cc, float dx, float dy) {
    return 0.5f * (ca * dx * dx + cc * dy * dy) + cb * dx * dy;
}

// Largest sigma for which opacity * exp(-sigma) can still reach the 1/255 alpha threshold, plus a
// 0.01 margin: any pair with sigma above it is invalid in the exact evaluation too (its alpha is at
// most e^-0.01/255), so skipping its exp leaves every result bit-identical.
constexpr float kCutoffMargin = 0.01f;
__device__ __forceinline__ float sigma_cutoff(float opac) { return __logf(opac * 255.0f) + kCutoffMargin; }

// The block of lane `lane` in wave `wave` (bit index by * 4 + bx of a block mask).
__device__ __forceinline__ int block_of(int wave, int lane) {
    const int q = lane >> 4;
    return (2 * (wave >> 1) + (q >> 1)) * 4 + 2 * (wave & 1) + (q & 1);
}

// Which of the tile's sixteen 4x4 blocks the Gaussian's cutoff set {sigma <= cut} can reach (bit
// by * 4 + bx). First the set's bounding box (half-extents rx = sqrt(2 cut c / det) in x and
// ry = sqrt(2 cut a / det) in y for a positive-definite conic) against each block's rectangle of pixel
// centres; then, per block row, the set's exact x-range within the row's band of pixel-centre rows:
// for an offset v = y - my the set spans dx in [-(b/a) v -+ sqrt(2 cut a - det v^2) / a]; over the band
// [v0, v1] the right end is largest at the set's rightmost point (v = -(b/c) rx, where it is rx) when
// that lies in the band, else at an end of the band (it is concave in v), and the left end mirrors it.
// A block is kept when both tests reach it: a splat's bounding box holds ~20 % more blocks than the
// set itself reaches at the benchmark scenes, whose list entries and lane pairs this saves. Conservative:
// the extents get a relative and an absolute margin far above the rounding of these float expressions
// and of the rasterisers' sigma, and every degenerate, nearly degenerate or non-finite case keeps all
// sixteen blocks.
__device__ __forceinline__ uint32_t block_mask(float4 xyo, float4 con, float x0, float y0) {
    const float a = con.x, b = con.y, c = con.z, cut = xyo.w;
    if (cut == -__builtin_inff()) return 0u;  // opacity 0: no pixel passes
    const float det = a * c - b * b;
    const bool finite = __builtin_isfinite(a) && __builtin_isfinite(b) && __builtin_isfinite(c) &&
                        __builtin_isfinite(cut) && __builtin_fabsf(xyo.x) < 1e18f && __builtin_fabsf(xyo.y) < 1e18f;
    if (!finite || !(a > 0.f) || !(det > 1e-4f * a * c)) return 0xFFFFu;
    if (cut < 0.f) return 0u;  // sigma >= 0 everywhere for a positive-definite conic
    const float k2 = 2.0f * cut;
    const float idet = __builtin_amdgcn_rcpf(det);
    const float rx0 = __builtin_amdgcn_sqrtf(k2 * c * idet), ry0 = __builtin_amdgcn_sqrtf(k2 * a * idet);
    const float rx = rx0 * 1.001f + 0.01f, ry = ry0 * 1.001f + 0.01f;
    const float mg = rx0 * 0.001f + 0.01f;  // margin of the per-row x-ranges
    const float inva = __builtin_amdgcn_rcpf(a), ba = b * inva, ak2 = a * k2;
    const float dyr = -(b * __builtin_amdgcn_rcpf(c)) * rx0;  // the rightmost point's offset; the leftmost: -dyr
    uint32_t cols = 0u, m = 0u;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float bx0 = x0 + static_cast<float>(4 * k) + 0.5f;
        if (xyo.x + rx >= bx0 && xyo.x - rx <= bx0 + 3.0f) cols |= 1u << k;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {  // block row k
        const float u0 = y0 + static_cast<float>(4 * k) + 0.5f - xyo.y;
        const float v0 = __builtin_fmaxf(u0, -ry), v1 = __builtin_fminf(u0 + 3.0f, ry);
        const float s0 = __builtin_amdgcn_sqrtf(__builtin_fmaxf(0.f, ak2 - det * v0 * v0)) * inva;
        const float s1 = __builtin_amdgcn_sqrtf(__builtin_fmaxf(0.f, ak2 - det * v1 * v1)) * inva;
        const float c0 = -ba * v0, c1 = -ba * v1;
        const float xmax = xyo.x + ((v0 <= dyr && dyr <= v1) ? rx0 : __builtin_fmaxf(c0 + s0, c1 + s1)) + mg;
        const float xmin = xyo.x + ((v0 <= -dyr && -dyr <= v1) ? -rx0 : __builtin_fminf(c0 - s0, c1 - s1)) - mg;
        uint32_t rc = 0u;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float bx0 = x0 + static_cast<float>(4 * j) + 0.5f;
            if (xmax >= bx0 && xmin <= bx0 + 3.0f) rc |= 1u << j;
        }
        if (v0 <= v1) m |= (rc & cols) << (4 * k);  // an empty band: no block of this row
    }
    return m;
}

// Rows of the forward's block lists: a batch's slots plus the padding to a whole chunk of four.
constexpr int kListRow = kThreads + 4;
// LDS byte offset of the record that no pixel reaches (slot kThreads of the record arrays).
constexpr uint32_t kPadRecord = kThreads * sizeof(float4);

// Per-block Gaussian lists of a batch: s_list[bl][0 .. s_len[bl]) = the LDS byte offsets (slot * 16) of
// the batch-local slots t (in increasing order) whose mask has bit bl, padded to a multiple of four
// entries with kPadRecord. All 256 threads call it; thread t passes Gaussian t's mask (0 for slots past
// the batch). Ends with a barrier. Each block's ballot is taken once; lane bl < 16 then holds the
// block's offset for the wave (the counts of the waves before it), and a lane's place among the wave's
// lanes with the bit is its count of them below it (mbcnt).
__device__ __forceinline__ void build_block_lists(uint32_t m, uint16_t (*s_list)[kListRow], int (*s_bc)[4],
                                                  int* s_len) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    unsigned long long bal[kBlocks];
    int cnt = 0;  // lane bl < 16: the wave's count for block bl
#pragma unroll
    for (int bl = 0; bl < kBlocks; bl++) {
        bal[bl] = __ballot((m >> bl) & 1u);
        cnt = lane == bl ? __popcll(bal[bl]) : cnt;
    }
    if (lane < kBlocks) s_bc[lane][wave] = cnt;
    __syncthreads();
    int off = 0;  // lane bl < 16: where the wave's entries of block bl start
    if (lane < kBlocks) {
        const int4 c = *reinterpret_cast<const int4*>(s_bc[lane]);
        off = (wave > 0 ? c.x : 0) + (wave > 1 ? c.y : 0) + (wave > 2 ? c.z : 0);
        if (wave == 0) {  // the list's length and padding
            const int len = c.x + c.y + c.z + c.w;
            s_len[lane] = len;
            for (int q = len; q < ((len + 3) & ~3); q++) s_list[lane][q] = static_cast<uint16_t>(kPadRecord);
        }
    }
#pragma unroll
    for (int bl = 0; bl < kBlocks; bl++) {
        const int base = __builtin_amdgcn_readlane(off, bl);
        const int rank = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal[bl] >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal[bl]), 0u)));
        if ((m >> bl) & 1u) s_list[bl][base + rank] = static_cast<uint16_t>(tid * sizeof(float4));
    }
    __syncthreads();
}

// The longest of the four block lists of wave `wave` (wave-uniform).
__device__ __forceinline__ int wave_list_max(const int* s_len, int wave) {
    const int b0 = block_of(wave, 0), b1 = block_of(wave, 16), b2 = block_of(wave, 32), b3 = block_of(wave, 48);
    return max(max(s_len[b0], s_len[b1]), max(s_len[b2], s_len[b3]));
}

template <bool STATS>
__global__ void __launch_bounds__(kThreads) k_raster_fwd(RasterArgs a, float* __restrict__ out_rgb,
                                                         float* __restrict__ out_alpha, int32_t* __restrict__ out_last) {
    // the batch's records, then (slot kThreads) one that no pixel reaches: cutoff -inf, the lists' padding
    __shared__ float4 s_xyo[kThreads + 1];  // {x, y, opacity, sigma cutoff}
    __shared__ float4 s_con[kThreads + 1];
    __shared__ float4 s_rgb[kThreads + 1];
    __shared__ __align__(16) uint16_t s_list[kBlocks][kListRow];
    __shared__ __align__(16) int s_bc[kBlocks][4];
    __shared__ int s_len[kBlocks];
    __shared__ unsigned long long s_gen[kThreads / 64];  // per wave: the batch's splats past the polynomial's range
    const int n_tiles = a.tile_width * a.tile_height;
    const int img = blockIdx.x / n_tiles;
    const int tile = a.tile_order ? a.tile_order[blockIdx.x % n_tiles] : static_cast<int>(blockIdx.x % n_tiles);
    const int tx = tile % a.tile_width, ty = tile / a.tile_width;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int bl = block_of(wave, lane);
    const int px_i = tx * 16 + 4 * (bl & 3) + (lane & 3), py_i = ty * 16 + 4 * (bl >> 2) + ((lane >> 2) & 3);
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
    unsigned long long st_iters = 0, st_entries = 0, st_taken = 0;  // STATS only (wave-uniform)
    int32_t loaded_end = range_end;  // the end of the entries loaded (and their block masks stored)
    if (tid == 0) {  // (published by the first batch's barriers)
        s_xyo[kThreads] = make_float4(0.f, 0.f, 0.f, -__builtin_inff());
        s_con[kThreads] = make_float4(0.f, 0.f, 0.f, 0.f);
        s_rgb[kThreads] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int32_t bstart = range_start; bstart < range_end; bstart += kThreads) {
        if (__syncthreads_count(done) == kThreads) {  // also the barrier before LDS reuse
            loaded_end = bstart;
            break;
        }
        const int32_t idx = bstart + tid;
        uint32_t bm = 0u;
        bool big = false;
        if (idx < range_end) {
            const int32_t f = a.flatten_ids[idx];
            const int32_t g = a.id_of ? a.id_of[f] : f;
            float4 xyo = a.splats[(size_t)g * 3];
            xyo.w = sigma_cutoff(xyo.z);
            const float4 con = a.splats[(size_t)g * 3 + 1];
            s_xyo[tid] = xyo;
            s_con[tid] = con;
            s_rgb[tid] = a.splats[(size_t)g * 3 + 2];
            bm = block_mask(xyo, con, static_cast<float>(tx * 16), static_cast<float>(ty * 16));
            if (a.block_masks) a.block_masks[idx] = static_cast<uint16_t>(bm);
            big = bm != 0u && xyo.w > 86.0f;
        }
        {
            const unsigned long long gb = __ballot(big);
            if (lane == 0) s_gen[wave] = gb;
        }
        build_block_lists(bm, s_list, s_bc, s_len);  // (its barriers publish s_gen too)
        // one choice of exponential for the batch: the branch-free polynomial unless some splat's cutoff
        // exceeds its range (opacity above ~1e35)
        const bool general = (s_gen[0] | s_gen[1] | s_gen[2] | s_gen[3]) != 0ull;
        // the groups walk their lists together (the iteration count is the wave's longest list); a
        // lane takes a pair through selects rather than branches, and stops once its T is spent
        const int len = s_len[bl];
        const int n_it = __builtin_amdgcn_readfirstlane(wave_list_max(s_len, wave));
        const uint2* const list4 = reinterpret_cast<const uint2*>(s_list[bl]);
        const char* const lds_xyo = reinterpret_cast<const char*>(s_xyo);
        const char* const lds_con = reinterpret_cast<const char*>(s_con);
        const char* const lds_rgb = reinterpret_cast<const char*>(s_rgb);
        // one list entry composited into the lane's pixel: opacity * exp(-sigma) = oe
        auto composite = [&](bool in, float sg, float oe, int off, int32_t id) {
            const float alpha = sxd::smin(sx::kMaxAlpha, oe);
            bool take = in && !done && !(sg < 0.f) && !(alpha < sx::kAlphaThreshold);
            const float next_T = T * (1.0f - alpha);
            const bool spent = take && next_T <= sx::kTransmittanceThreshold;
            done = done || spent;
            take = take && !spent;
            const float w = alpha * T;
            const float4 c = *reinterpret_cast<const float4*>(lds_rgb + off);
            r0 = take ? __builtin_fmaf(c.x, w, r0) : r0;
            r1 = take ? __builtin_fmaf(c.y, w, r1) : r1;
            r2 = take ? __builtin_fmaf(c.z, w, r2) : r2;
            cur = take ? id : cur;
            T = take ? next_T : T;
            if (STATS) st_taken += __popcll(__ballot(take));
        };
        // four list entries per iteration (their record offsets in one LDS read): their sigmas and
        // exponentials are independent, only T and the colour sums run through them in order. The
        // iteration loop is compiled once per exponential (the choice is the batch's), so no entry tests it.
        auto walk = [&](auto general_exp) {
            for (int j = 0; j < n_it; j += 4) {
                if (__all(done)) break;  // uniform
                // a chunk past the group's list (the list is padded to whole chunks) reads the padding record
                const uint2 pk4 = list4[j >> 2];
                const uint2 pk = j < len ? pk4 : make_uint2(kPadRecord * 0x10001u, kPadRecord * 0x10001u);
                const int off[4] = {static_cast<int>(pk.x & 0xFFFFu), static_cast<int>(pk.x >> 16),
                                    static_cast<int>(pk.y & 0xFFFFu), static_cast<int>(pk.y >> 16)};
                float4 xyo[4];
                float sg[4];
                bool in[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    xyo[k] = *reinterpret_cast<const float4*>(lds_xyo + off[k]);
                    const float4 con = *reinterpret_cast<const float4*>(lds_con + off[k]);
                    sg[k] = sigma_of(con.x, con.y, con.z, xyo[k].x - px, xyo[k].y - py);
                    in[k] = !done & !(sg[k] > xyo[k].w);  // (the padding record's cutoff is -inf)
                }
                if (STATS) {
                    st_iters += min(4, n_it - j);
#pragma unroll
                    for (int k = 0; k < 4; k++) st_entries += __popcll(__ballot((lane & 15) == 0 && j + k < len));
                }
                if (!__any(in[0] | in[1] | in[2] | in[3])) continue;  // uniform
                float vis[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if constexpr (decltype(general_exp)::value) vis[k] = sxm::expf_fast(-sg[k]);
                    else vis[k] = exp_neg_poly(sg[k]);
                }
                // front to back: a lane that stopped at an entry takes nothing more
#pragma unroll
                for (int k = 0; k < 4; k++)
                    composite(in[k], sg[k], xyo[k].z * vis[k], off[k], bstart + (off[k] >> 4));
            }
        };
        if (general)
            walk(std::true_type{});
        else
            walk(std::false_type{});
    }
    // every pixel's last contributor lies in a loaded batch, before loaded_end: the backward's walk
    // stays inside the stored masks
    if (a.block_masks && tid == 0) a.mask_end[(size_t)img * n_tiles + tile] = loaded_end;
    if (STATS && lane == 0) {
        atomicAdd(&a.stats[kStatFwdIters], st_iters);
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

// ---- group reductions ------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// Maximum over each 16-lane row (every lane of the row ends with it).
__device__ __forceinline__ int row_max16(int v) {
    v = max(v, dpp_i<0xB1>(v));   // quad_perm(1,0,3,2)
    v = max(v, dpp_i<0x4E>(v));   // quad_perm(2,3,0,1)
    v = max(v, dpp_i<0x141>(v));  // row_half_mirror
    v = max(v, dpp_i<0x140>(v));  // row_mirror
    return v;
}
// Minimum over each 16-lane row (every lane of the row ends with it).
__device__ __forceinline__ int row_min16(int v) {
    v = min(v, dpp_i<0xB1>(v));
    v = min(v, dpp_i<0x4E>(v));
    v = min(v, dpp_i<0x141>(v));
    v = min(v, dpp_i<0x140>(v));
    return v;
}
// Four per-lane values (one per list slot A..D of the group) summed over each 16-lane group in 8
// instructions. Stage 1 pairs lane r with r ^ 8 (row_ror:8): lanes 0-7 sum A, lanes 8-15 sum B (C
// and D likewise); stage 2 pairs r with its mirror in the 8-lane half (row_half_mirror): quads 0 and
// 2 sum the stage-1 A / B, quads 1 and 3 the C / D; the quad sums finish it. The result: quad 0 holds
// the group total of A, quad 1 of C, quad 2 of B, quad 3 of D (every lane of the quad). Each stage
// writes its two halves with two DPP adds whose bank masks (4-lane banks of the 16-lane row) select
// the lanes, so no select instruction picks the operands. The outputs are early-clobber (the second
// add of a pair still reads the inputs); the s_nop covers the DPP read of a just-written VGPR.
__device__ __forceinline__ float group_sum4(float a, float b, float c, float d) {
    float s1, t1, v;
    asm volatile(
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %2, %2 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
        "v_add_f32_dpp %0, %3, %3 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
        "v_add_f32_dpp %1, %4, %4 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
        "v_add_f32_dpp %1, %5, %5 row_ror:8 row_mask:0xf bank_mask:0xc"
        : "=&v"(s1), "=&v"(t1)
        : "v"(a), "v"(b), "v"(c), "v"(d));
    asm volatile(
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
        "v_add_f32_dpp %0, %2, %2 row_half_mirror row_mask:0xf bank_mask:0xa"
        : "=&v"(v)
        : "v"(s1), "v"(t1));
    // the quad sums, in place (a DPP source reads the VGPR before the add writes it); each reads the
    // value the previous instruction wrote, hence the s_nop
    asm volatile(
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf"
        : "+v"(v));
    return v;
}

constexpr int kGrads = 9;  // v_xy(2), v_opacity, v_conic(3), v_rgb(3)
// log(255 * 0.99): from the sigma where alpha turns 1/255 to the sigma where it reaches the 0.99 clamp
constexpr float kLogAlphaSpan = 5.53121185f;

// The address of gradient component k of Gaussian gid: the packed record (x, y, opacity, - | conic
// a, b, c, - | r, g, b, -) or the per-op arrays.
__device__ __forceinline__ float* grad_slot(const RasterBwdGrads& g, int32_t gid, int k) {
    if (g.packed) {
        static constexpr int kRec[9] = {0, 1, 2, 4, 5, 6, 8, 9, 10};
        return reinterpret_cast<float*>(g.packed + (size_t)gid * 3) + kRec[k];
    }
    switch (k) {
        case 0: return &g.v_means2d[(size_t)gid * 2];
        case 1: return &g.v_means2d[(size_t)gid * 2 + 1];
        case 2: return &g.v_opacities[gid];
        case 3: return &g.v_conics[(size_t)gid * 3];
        case 4: return &g.v_conics[(size_t)gid * 3 + 1];
        case 5: return &g.v_conics[(size_t)gid * 3 + 2];
        case 6: return &g.v_colors[(size_t)gid * 3];
        case 7: return &g.v_colors[(size_t)gid * 3 + 1];
        case 8: return &g.v_colors[(size_t)gid * 3 + 2];
        case 9: return &g.v_means2d_abs[(size_t)gid * 2];
        default: return &g.v_means2d_abs[(size_t)gid * 2 + 1];
    }
}

// The position of the n-th (1-based) set bit of w, for 1 <= n <= popcount(w): a binary descent over
// the halves, quarters, ... of the word (uniform work, no loop over the bits).
__device__ __forceinline__ int nth_set_bit(unsigned long long w, int n) {
    int pos = 0;
    uint32_t x = static_cast<uint32_t>(w);
    int c = __popc(x);
    if (n > c) { n -= c; x = static_cast<uint32_t>(w >> 32); pos = 32; }
    c = __popc(x & 0xFFFFu);
    if (n > c) { n -= c; x >>= 16; pos += 16; }
    c = __popc(x & 0xFFu);
    if (n > c) { n -= c; x >>= 8; pos += 8; }
    c = __popc(x & 0xFu);
    if (n > c) { n -= c; x >>= 4; pos += 4; }
    c = __popc(x & 0x3u);
    if (n > c) { n -= c; x >>= 2; pos += 2; }
    return pos + (n > static_cast<int>(x & 1u) ? 1 : 0);
}

// The slot of the (seg + 1)-th set bit at or after slot s0 (uniform) of a 256-bit slot mask, kThreads if
// there is none: where a block's list from s0 on would pass seg entries. It is the (r + seg + 1)-th set
// bit of the whole mask, r the set bits before s0, so one descent over the word that holds it finds it.
__device__ __forceinline__ int seg_limit(const unsigned long long* w4, int s0, int seg) {
    const unsigned long long w0 = w4[0], w1 = w4[1], w2 = w4[2], w3 = w4[3];
    const int p1 = __popcll(w0), p2 = p1 + __popcll(w1), p3 = p2 + __popcll(w2), p4 = p3 + __popcll(w3);
    const int i0 = s0 >> 6;
    const unsigned long long ws = i0 == 0 ? w0 : i0 == 1 ? w1 : i0 == 2 ? w2 : w3;
    const int before = (i0 == 0 ? 0 : i0 == 1 ? p1 : i0 == 2 ? p2 : p3) + __popcll(ws & ((1ull << (s0 & 63)) - 1ull));
    const int need = before + seg + 1;
    if (need > p4) return kThreads;
    const int i = need <= p1 ? 0 : need <= p2 ? 1 : need <= p3 ? 2 : 3;
    const unsigned long long w = i == 0 ? w0 : i == 1 ? w1 : i == 2 ? w2 : w3;
    return 64 * i + nth_set_bit(w, need - (i == 0 ? 0 : i == 1 ? p1 : i == 2 ? p2 : p3));
}

// Position of entry e of block bl in its row of the backward's entry buffer: rotated by 0, 4, 8 or 12
// by the block's place in its 2x2 quadrant, so that the 16 writers of a chunk (the four blocks of a wave,
// four consecutive entries each; entries of 10 or 12 words, written as pairs of words) use different
// LDS banks.
__device__ __forceinline__ int ent_rot(int e, int bl, int seg) {
    return (e + 4 * ((bl & 1) + 2 * ((bl >> 2) & 1))) & (seg - 1);
}

template <bool ABSGRAD, bool STATS, int kSeg>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 8))) k_raster_bwd(RasterArgs a, const float* __restrict__ ralpha,
                                                         const int32_t* __restrict__ last_ids,
                                                         const float* __restrict__ v_rc, const float* __restrict__ v_ra,
                                                         RasterBwdGrads g) {
    constexpr int NV = ABSGRAD ? kGrads + 2 : kGrads;
    // A segment: a run of batch slots in which no block's list holds more than kSeg entries (the
    // capacity of its entry buffer); its per-entry sums are flushed before the next.
    static_assert(kSeg == 32 || kSeg == 64, "entry buffer rows of 32 or 64 words");
    // the batch's records, and after them one record that no pixel reaches (slot kThreads: turning
    // point -inf, so its sigma fails the cutoff), which pads the block lists to whole chunks
    __shared__ float4 s_xyo[kThreads + 1];  // {x, y, opacity, sigma where alpha turns 1/255}
    __shared__ float4 s_con[kThreads + 1];  // {a, b, c, Gaussian id (int bits)}
    __shared__ float4 s_rgb[kThreads + 1];  // {r, g, b, flatten_ids entry (int bits)}
    // per-entry gradient sums of the current segment: [block][position in the block's list, rotated by
    // ent_rot][component], an entry's components contiguous (written and read as pairs of words)
    constexpr int kEntWords = (NV + 2) & ~1;
    __shared__ __align__(16) float s_ent[kBlocks][kSeg][kEntWords];
    __shared__ unsigned long long s_bits[kBlocks][4];  // [block][wave]: the wave's batch slots that reach the block
    // the block's list of the current segment as byte offsets of the slots' records (slot * 16), padded to
    // kSeg entries with the record no pixel reaches
    __shared__ __align__(8) uint16_t s_seg[kBlocks][kSeg];
    __shared__ uint8_t s_epos[kThreads][kBlocks];     // [slot][block]: the slot's entry in the block's row
    __shared__ uint16_t s_bm[kThreads];               // each batch slot's block mask
    __shared__ int32_t s_bbf[kBlocks];                // each block's last contributing intersection
    __shared__ unsigned long long s_gen[4];           // per wave: the batch's splats past the polynomial's range
    const int n_tiles = a.tile_width * a.tile_height;
    const int img = blockIdx.x / n_tiles;
    const int tile = a.tile_order ? a.tile_order[blockIdx.x % n_tiles] : static_cast<int>(blockIdx.x % n_tiles);
    if (a.masks && a.masks[(size_t)img * n_tiles + tile] == 0) return;  // uniform
    const int tx = tile % a.tile_width, ty = tile / a.tile_width;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15;  // lane within its group
    const int bl = block_of(wave, lane);
    const int px_i = tx * 16 + 4 * (bl & 3) + (r & 3), py_i = ty * 16 + 4 * (bl >> 2) + (r >> 2);
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
    const int32_t block_bin_final = row_max16(bin_final);
    const uint32_t stamp = g.part ? *g.stamp : 0u;  // the step's stamp for `part` entries
    if (r == 0) s_bbf[bl] = block_bin_final;
    if (tid == 0) {
        s_xyo[kThreads] = make_float4(0.f, 0.f, 0.f, -__builtin_inff());
        s_con[kThreads] = make_float4(0.f, 0.f, 0.f, 0.f);
        s_rgb[kThreads] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    // the walk starts at the tile's last contributing intersection: everything behind it (most of
    // a dense tile's list, once its pixels saturate) has no pixel to contribute to
    int32_t tile_bf = s_bbf[0];
#pragma unroll
    for (int k = 1; k < kBlocks; k++) tile_bf = max(tile_bf, s_bbf[k]);
    const int32_t tile_end = min(range_end, tile_bf + 1);
    const int32_t num = max(0, tile_end - range_start);
    // the forward stored the masks of [range_start, mask_end), which holds [range_start, tile_end): the
    // forward loads whole batches until every pixel is done, and tile_end - 1 is some pixel's last
    // contributor. An entry past mask_end would take the computed mask.
    const int32_t mask_end = a.block_masks ? a.mask_end[(size_t)img * n_tiles + tile] : range_start;
    const int num_batches = (num + kThreads - 1) / kThreads;
    // a group's reduction leaves slot A in lane 0, B in 8, C in 4, D in 12: those lanes store them
    const int wslot = (r == 0) ? 0 : (r == 8) ? 1 : (r == 4) ? 2 : (r == 12) ? 3 : -1;
    // STATS only (wave-uniform)
    unsigned long long st_chunks = 0, st_entries = 0, st_empty = 0, st_cut = 0, st_contrib = 0;
    for (int b = 0; b < num_batches; b++) {
        __syncthreads();  // the previous batch's flush has read the records
        const int32_t batch_end = tile_end - 1 - kThreads * b;
        const int32_t batch_size = min(kThreads, batch_end + 1 - range_start);
        const int32_t idx = batch_end - tid;
        uint32_t bm = 0u;
        bool big = false;
        if (idx >= range_start) {
            const int32_t f = a.flatten_ids[idx];  // the Gaussian, or its emit position (id_of)
            const int32_t gid = a.id_of ? a.id_of[f] : f;
            float4 xyo = a.splats[(size_t)gid * 3];
            xyo.w = sigma_cutoff(xyo.z);
            float4 con = a.splats[(size_t)gid * 3 + 1];
            float4 rgb = a.splats[(size_t)gid * 3 + 2];
            // blocks the cutoff set can reach (the forward's, when it kept them), less those whose every
            // pixel stopped before it
            bm = idx < mask_end ? static_cast<uint32_t>(a.block_masks[idx])
                                : block_mask(xyo, con, static_cast<float>(tx * 16), static_cast<float>(ty * 16));
#pragma unroll
            for (int k = 0; k < kBlocks; k++)
                if (idx > s_bbf[k]) bm &= ~(1u << k);
            big = bm != 0u && xyo.w > 86.0f;
            xyo.w -= kCutoffMargin;  // the walk keeps the turning point: sigma - it decides cutoff and nearness
            con.w = __int_as_float(gid);
            rgb.w = __int_as_float(f);
            s_xyo[tid] = xyo;
            s_con[tid] = con;
            s_rgb[tid] = rgb;
        }
        s_bm[tid] = static_cast<uint16_t>(bm);
#pragma unroll
        for (int k = 0; k < kBlocks; k++) {
            const unsigned long long bal = __ballot((bm >> k) & 1u);
            if (lane == 0) s_bits[k][wave] = bal;
        }
        {
            const unsigned long long gb = __ballot(big);
            if (lane == 0) s_gen[wave] = gb;
        }
        __syncthreads();
        // one choice of exponential for the batch: the branch-free polynomial (or the hardware exp2 with
        // the checks below) unless some splat's cutoff exceeds its range (opacity above ~1e35)
        const bool general = (s_gen[0] | s_gen[1] | s_gen[2] | s_gen[3]) != 0ull;

        const int t_min = batch_end - bin_final;  // slots t >= t_min are at or before the lane's last contributor
        // the same bound on the list's record offsets (slot * 16; the padding record at kThreads * 16 passes
        // it whenever any slot does, and fails the cutoff)
        const int tmin16 = t_min * static_cast<int>(sizeof(float4));
        // The batch's slots are walked in segments [s0, s1), each ending before the slot of the entry
        // with which some block's list would pass kSeg entries; so the lists are as long as the entry
        // buffer allows whatever the slots' density (fixed 32-slot segments left ~6 entries per list,
        // and half of the four groups' lockstep chunks past their lists). Every wave derives the same
        // bounds from the block masks.
        const unsigned long long w_bl[4] = {s_bits[bl][0], s_bits[bl][1], s_bits[bl][2], s_bits[bl][3]};
        for (int s0 = 0; s0 < batch_size;) {  // uniform
            // lane k < 16 (lanes 16-63 repeat them): the slot of block k's (kSeg + 1)-th entry from s0 (none:
            // kThreads); s1 = the least
            const int lim = row_min16(seg_limit(s_bits[lane & (kBlocks - 1)], s0, kSeg));
            // (lim >= s0 + kSeg for every block, so s1 > s0; the max only makes progress explicit)
            const int s1 = max(s0 + 1, min(static_cast<int>(batch_size), __builtin_amdgcn_readfirstlane(lim)));
            // this group's list of the segment: lane r places the set slots among slots [16 r, 16 r + 16)
            unsigned long long wr[4];
            int cnt = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int lo = min(max(s0 - 64 * i, 0), 64), hi = min(max(s1 - 64 * i, 0), 64);
                const unsigned long long mhi = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
                const unsigned long long mlo = lo >= 64 ? ~0ull : ((1ull << lo) - 1ull);
                wr[i] = w_bl[i] & mhi & ~mlo;
                cnt += __popcll(wr[i]);
            }
            {
                // lane r takes the segment's slots [a, a + span): the span is at most 16, so its bits lie in
                // one or two words
                const int span = (s1 - s0 + 15) >> 4;
                const int a0 = s0 + r * span;
                const int a = min(a0, s1), e = min(a0 + span, s1);
                const int ia = a >> 6, ib = (e - 1) >> 6;
                const unsigned long long wa = ia == 0 ? wr[0] : ia == 1 ? wr[1] : ia == 2 ? wr[2] : wr[3];
                const unsigned long long wb = ib == 0 ? wr[0] : ib == 1 ? wr[1] : ib == 2 ? wr[2] : wr[3];
                int pos = __popcll(wa & ((1ull << (a & 63)) - 1ull));
#pragma unroll
                for (int k = 0; k < 3; k++) pos += k < ia ? __popcll(wr[k]) : 0;
                // the span's bits, from slot a on: the rest of word ia, then the start of word ib
                uint32_t bits = 0u;
                if (e > a) {
                    const unsigned long long lo = wa >> (a & 63);
                    const unsigned long long hi = (ib != ia) ? (wb << (64 - (a & 63))) : 0ull;
                    bits = static_cast<uint32_t>(lo | hi) & ((1u << (e - a)) - 1u);
                }
                while (bits) {  // at most kSeg entries over the group (the segment's bound)
                    const int slot = a + __builtin_ctz(bits);
                    bits &= bits - 1u;
                    if (pos < kSeg) {  // always (the bound); kept so that no write can leave the row
                        s_seg[bl][pos] = static_cast<uint16_t>(slot * sizeof(float4));
                        s_epos[slot][bl] = static_cast<uint8_t>(ent_rot(pos, bl, kSeg));
                    }
                    pos++;
                }
                // the rest of the row: the record no pixel reaches (positions past the list, disjoint from
                // the ones written above)
                static_assert(kSeg == 32 || kSeg == 64, "two or four pad positions per lane");
#pragma unroll
                for (int q = r; q < kSeg; q += 16)
                    if (q >= cnt) s_seg[bl][q] = static_cast<uint16_t>(kThreads * sizeof(float4));
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the group's lanes read what the others wrote
            int lmax = cnt;  // the longest of the wave's four lists (cnt is uniform within a group)
            lmax = max(lmax, __shfl_xor(lmax, 16, 64));
            lmax = max(lmax, __shfl_xor(lmax, 32, 64));
            const int n4 = (__builtin_amdgcn_readfirstlane(lmax) + 3) >> 2;
            const uint2* seg8 = reinterpret_cast<const uint2*>(s_seg[bl]);
            const char* const lds_xyo = reinterpret_cast<const char*>(s_xyo);
            const char* const lds_con = reinterpret_cast<const char*>(s_con);
            const char* const lds_rgb = reinterpret_cast<const char*>(s_rgb);
            // The group's Gaussians back to front, four at a time: the four list entries (record offsets)
            // come in one LDS read and their records in one burst, the four pairs' exponentials are
            // independent, only T and the back-sum run through them in order. A pair that does not
            // contribute (or a position past the list, which holds the record no pixel reaches) gets
            // alpha = 0, so T (times 1/(1 - 0) = 1), the back-sum and every gradient term are left
            // unchanged / zero.
            for (int j4 = 0; j4 < n4; j4++) {
                const int j = 4 * j4;
                const uint2 pk = seg8[j4];
                const int off[4] = {static_cast<int>(pk.x & 0xFFFFu), static_cast<int>(pk.x >> 16),
                                    static_cast<int>(pk.y & 0xFFFFu), static_cast<int>(pk.y >> 16)};
                float4 xyo[4], con[4], rgb[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    xyo[k] = *reinterpret_cast<const float4*>(lds_xyo + off[k]);
                    con[k] = *reinterpret_cast<const float4*>(lds_con + off[k]);
                    rgb[k] = *reinterpret_cast<const float4*>(lds_rgb + off[k]);
                }
                // the lane storing a slot's sums, and where: the slot's position in the block's list
                const int e_w = wslot >= 0 && j + wslot < cnt ? j + wslot : -1;
                float gv[4][NV];
                float alpha[4], vis[4], dxs[4], dys[4], sig[4], d1[4], e[4];
                bool valid[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    dxs[k] = xyo[k].x - px;
                    dys[k] = xyo[k].y - py;
                    // the forward's sigma expression, bit for bit: the decisions below must be the forward's
                    sig[k] = sigma_of(con[k].x, con[k].y, con[k].z, dxs[k], dys[k]);
                    d1[k] = sig[k] - xyo[k].w;  // sigma less the turning point (alpha = 1/255 there)
                    // at or before the lane's last contributor (slot >= t_min), and inside the cutoff
                    valid[k] = (off[k] >= tmin16) & !(d1[k] > kCutoffMargin);  // bitwise: no branches
                }
                const bool any_valid = __any(valid[0] | valid[1] | valid[2] | valid[3]);
                if (STATS) {
                    st_chunks++;
                    st_empty += any_valid ? 0 : 1;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        st_entries += __popcll(__ballot(r == 0 && j + k < cnt));
                        st_cut += __popcll(__ballot(valid[k]));
                    }
                }
                if (!any_valid) {  // uniform: every alpha 0, T, the back-sum and the gradients unchanged
                    if (e_w >= 0) {
                        float* ent = s_ent[bl][ent_rot(e_w, bl, kSeg)];
#pragma unroll
                        for (int k = 0; k < NV; k += 2) {
                            if (k + 1 < NV)
                                *reinterpret_cast<float2*>(ent + k) = make_float2(0.f, 0.f);
                            else
                                ent[k] = 0.f;
                        }
                    }
                    continue;
                }
                // The exponential's value only enters gradients (compared at a relative tolerance), so the
                // hardware exp2 serves (relative error below 1.2e-7 (1 + 1.5 sigma): the rounded argument,
                // log2(e) in float, one ulp of v_exp_f32), but the decisions taken on it — alpha at least
                // 1/255, opacity * exp at most the 0.99 clamp, and sigma not negative — must be the
                // forward's. Where a valid lane lies within 2^-12 in sigma of either turning point (alpha =
                // 1/255 at d1 = 0, alpha = 0.99 at d1 = -log(255 * 0.99); both approximate to ~1e-6 and
                // only used to find the pairs close to them) or has sigma below 2^-12, the chunk takes the
                // forward's exponential and sign test instead.
                bool exact = general;
                if (!exact) {
                    bool near = false;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        e[k] = __builtin_amdgcn_exp2f(-sig[k] * 1.44269504f);
                        const float m = __builtin_fminf(
                            __builtin_fminf(__builtin_fabsf(d1[k]), __builtin_fabsf(d1[k] + kLogAlphaSpan)), sig[k]);
                        near = near | (valid[k] & (m < 0x1p-12f));
                    }
                    exact = __any(near);
                }
                if (__builtin_expect(exact, 0)) {
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        e[k] = general ? sxm::expf_fast(-sig[k]) : exp_neg_poly(sig[k]);
                        valid[k] = valid[k] & !(sig[k] < 0.f);  // (the fast path has no valid lane below 2^-12)
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float vis_raw = e[k];
                    const float oa = xyo[k].z * vis_raw;
                    const float alpha_raw = sxd::smin(sx::kMaxAlpha, oa);
                    const bool ok = valid[k] & !(alpha_raw < sx::kAlphaThreshold);
                    alpha[k] = ok ? alpha_raw : 0.0f;
                    vis[k] = (ok & (oa <= sx::kMaxAlpha)) ? vis_raw : 0.0f;  // clamped alpha: no sigma/opacity terms
                    if (STATS) st_contrib += __popcll(__ballot(ok));
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    // hardware reciprocal (1 ulp; exact for 1): the backward is compared at a relative
                    // tolerance, and an IEEE division costs ~10 instructions per pair. alpha is 0 or in
                    // [1/255, 0.99], so 1 - alpha >= 0.01 needs no floor.
                    const float ra = __builtin_amdgcn_rcpf(1.0f - alpha[k]);
                    T *= ra;
                    const float fac = alpha[k] * T;
                    gv[k][6] = fac * vc0;
                    gv[k][7] = fac * vc1;
                    gv[k][8] = fac * vc2;
                    // v_alpha = sum_c (c_c T - b_c ra) vc_c + T_final ra (va - <bg, vc>), with the back-sum
                    // kept as its dot product with v_render (fused multiply-adds: gradient algebra only)
                    const float cvc = __builtin_fmaf(rgb[k].x, vc0, __builtin_fmaf(rgb[k].y, vc1, rgb[k].z * vc2));
                    const float v_alpha = __builtin_fmaf(T, cvc, ra * (tva - bdot));
                    const float dx = dxs[k], dy = dys[k];
                    const float gw = vis[k] * v_alpha;  // v_opacity's term; v_sigma = -opacity * gw
                    gv[k][2] = gw;
                    if (ABSGRAD) {  // per-pixel 2D gradients are needed for their absolute values
                        const float v_sigma = -xyo[k].z * vis[k] * v_alpha;
                        const float vdx = v_sigma * dx, vdy = v_sigma * dy;
                        gv[k][0] = __builtin_fmaf(con[k].x, vdx, con[k].y * vdy);
                        gv[k][1] = __builtin_fmaf(con[k].y, vdx, con[k].z * vdy);
                        gv[k][3] = 0.5f * vdx * dx;
                        gv[k][4] = vdx * dy;
                        gv[k][5] = 0.5f * vdy * dy;
                        gv[k][9] = fabsf(gv[k][0]);
                        gv[k][10] = fabsf(gv[k][1]);
                    } else {  // moments of gw: the conic, -opacity and the halves are applied once per splat
                        const float wdx = gw * dx, wdy = gw * dy;  // at the flush
                        gv[k][0] = wdx;
                        gv[k][1] = wdy;
                        gv[k][3] = wdx * dx;
                        gv[k][4] = wdx * dy;
                        gv[k][5] = wdy * dy;
                    }
                    bdot = __builtin_fmaf(fac, cvc, bdot);
                }
                float sv[NV];
#pragma unroll
                for (int k = 0; k < NV; k++) sv[k] = group_sum4(gv[0][k], gv[1][k], gv[2][k], gv[3][k]);
                if (e_w >= 0) {  // plain stores: one writer per (block, entry)
                    float* ent = s_ent[bl][ent_rot(e_w, bl, kSeg)];
#pragma unroll
                    for (int k = 0; k < NV; k += 2) {
                        if (k + 1 < NV)
                            *reinterpret_cast<float2*>(ent + k) = make_float2(sv[k], sv[k + 1]);
                        else
                            ent[k] = sv[k];
                    }
                }
            }
            __syncthreads();
            // the segment's totals: thread t sums slot s0 + t's entries over the blocks it reaches, all
            // components at once (s1 - s0 <= kThreads). (Components shared out over 2, 3, 4 or 8 threads
            // per slot measured slower: each thread walks the slot's blocks again; so did slots dealt to
            // the four waves in turn, which spreads the same issue over four waves instead of one or two.)
            if (tid < s1 - s0) {
                const int slot = s0 + tid;
                uint32_t m = static_cast<uint32_t>(s_bm[slot]);
                if (m) {
                    float v[NV];
#pragma unroll
                    for (int k = 0; k < NV; k++) v[k] = 0.f;
                    while (m) {
                        const int b2 = __builtin_ctz(m);
                        m &= m - 1u;
                        const float* ent = s_ent[b2][s_epos[slot][b2]];  // the slot's entry in the block's row
#pragma unroll
                        for (int k = 0; k < NV; k += 2) {
                            if (k + 1 < NV) {
                                const float2 x = *reinterpret_cast<const float2*>(ent + k);
                                v[k] += x.x;
                                v[k + 1] += x.y;
                            } else {
                                v[k] += ent[k];
                            }
                        }
                    }
                    if (!ABSGRAD) {
                        // sum_p gw (a dx + b dy, b dx + c dy); the moments of gw times -opacity are those of
                        // v_sigma, and dx^2, dy^2 take a half
                        const float4 cn = s_con[slot];
                        const float sdx = v[0], sdy = v[1];
                        const float nop = -s_xyo[slot].z;
                        v[0] = __builtin_fmaf(cn.x, sdx, cn.y * sdy) * nop;
                        v[1] = __builtin_fmaf(cn.y, sdx, cn.z * sdy) * nop;
                        v[3] *= 0.5f * nop;
                        v[4] *= nop;
                        v[5] *= 0.5f * nop;
                    }
                    const int32_t f = __float_as_int(s_rgb[slot].w);
                    if (g.part) {  // plain stores at the emit position; the gather sums them in a fixed order
                        float4* dst = reinterpret_cast<float4*>(g.part + (size_t)f * kPartStride);
                        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
                        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
                        dst[2] = make_float4(v[8], __uint_as_float(stamp), 0.f, 0.f);  // the entry is this step's
                        g.touched[__float_as_int(s_con[slot].w)] = 1;  // the Gaussian has entries to gather
                    } else {
#pragma unroll
                        for (int k = 0; k < NV; k++)
                            if (v[k] != 0.f) atomicAdd(grad_slot(g, f, k), v[k]);
                    }
                }
            }
            __syncthreads();  // the next segment overwrites the entries and the group lists
            s0 = s1;
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
constexpr int kLongRange = 64;  // gather: longer entry ranges are reduced by a whole wave

// the backward's new stamp (never 0: zeroed entries hold 0), the rows' touched flags and the gather's
// long-range queue count
__global__ void __launch_bounds__(kThreads) k_bwd_begin(uint32_t* __restrict__ stamp, uint8_t* __restrict__ touched,
                                                        int rows, int32_t* __restrict__ long_count) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *long_count = 0;
        const uint32_t next = *stamp + 1u;
        *stamp = next ? next : 1u;
    }
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) touched[i] = 0;
}

// entry p of `part` as three aligned float4 loads: the 9 sums, and whether its stamp is `stamp`
__device__ __forceinline__ bool load_entry(const float* __restrict__ part, int32_t p, uint32_t stamp, float* e) {
    const float4* a = reinterpret_cast<const float4*>(part + (size_t)p * kPartStride);
    const float4 x = a[0], y = a[1], z = a[2];
    e[0] = x.x; e[1] = x.y; e[2] = x.z; e[3] = x.w;
    e[4] = y.x; e[5] = y.y; e[6] = y.z; e[7] = y.w;
    e[8] = z.x;
    return __float_as_uint(z.y) == stamp;
}

__device__ __forceinline__ void store_grad_record(float4* grads, size_t g, const float* v) {
    grads[3 * g] = make_float4(v[0], v[1], v[2], 0.f);
    grads[3 * g + 1] = make_float4(v[3], v[4], v[5], 0.f);
    grads[3 * g + 2] = make_float4(v[6], v[7], v[8], 0.f);
}

// One range [p0, p1) of `part` reduced by a whole wave: 64 entries per round (lane l takes entry
// base + l when it carries the stamp), each round's values added in a fixed tree (DPP within rows, then
// across rows) and the rounds in order; every lane ends with the sums.
__device__ __forceinline__ void reduce_long_range(const float* __restrict__ part, int32_t p0, int32_t p1,
                                                  uint32_t stamp, float* v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < kPartFloats; k++) v[k] = 0.f;
    for (int32_t base = p0; base < p1; base += 64) {
        const int32_t p = base + lane;
        float x[kPartFloats];
        const bool on = load_entry(part, min(p, p1 - 1), stamp, x) & (p < p1);
#pragma unroll
        for (int k = 0; k < kPartFloats; k++) {
            float y = on ? x[k] : 0.f;
            y += dpp_f<0xB1>(y);   // quad_perm(1,0,3,2)
            y += dpp_f<0x4E>(y);   // quad_perm(2,3,0,1)
            y += dpp_f<0x141>(y);  // row_half_mirror
            y += dpp_f<0x140>(y);  // row_mirror: the 16-lane row total
            y += __shfl_xor(y, 16, 64);
            y += __shfl_xor(y, 32, 64);
            v[k] += y;
        }
    }
}

constexpr int kGatherWave = 64;    // lanes of a gather workgroup (one wave)
constexpr int kGatherStage = 256;  // entries staged in LDS per round

// One wave per `npos` (32 or 64) consecutive positions j of the emit order, for Gaussian order[j] (lane l
// takes position l; lanes past npos only stage entries): the sums of its
// (tile, Gaussian) entries, which the emit placed at [cum[j-1], cum[j]), in emit order (its tiles in
// the order the intersection emit visits them), into its gradient record {v_x, v_y, v_opacity, 0 |
// v_conic a, b, c, 0 | v_r, v_g, v_b, 0}. The wave's ranges lie back to back in `part`, so the wave
// stages them in LDS with loads of consecutive entries (a lane per entry) and each lane then adds its
// own range from there, in order. Entries without this step's stamp (tiles that never reached the
// Gaussian) are staged as zeros: an added +0 leaves every partial sum as it was (a sum that starts at
// +0 never becomes -0). A Gaussian with no stamped entry (exactly the untouched ones) stages nothing
// and gets no record: the postprocess reads zeros for it. Touched ranges longer than kLongRange are
// either queued for k_gather_long (the queue's order does not matter: each range is reduced on its
// own) or, with inline_long, reduced by the wave itself after its short ranges, one after another,
// and only counted in *long_count; both reduce a range the same way (the same sums, bit for bit).
// Inline suits steps with few long ranges (it saves the second launch); many of them, one after
// another per wave, are far slower than the queue's wave per range.
__global__ void __launch_bounds__(kGatherWave) k_gather_grads(int count, const int32_t* __restrict__ order,
                                                              const int64_t* __restrict__ cum,
                                                              const float* __restrict__ part,
                                                              const uint32_t* __restrict__ stamp_p,
                                                              const uint8_t* __restrict__ touched,
                                                              float4* __restrict__ grads,
                                                              int32_t* __restrict__ long_list,
                                                              int32_t* __restrict__ long_count,
                                                              const int64_t* __restrict__ count_dev,
                                                              int inline_long, int npos, StepLoss L) {
    // the first workgroup (one wave) also reduces the step's loss, before its ranges (L.out null: none)
    if (L.out && blockIdx.x == 0) loss_final_wave(L);
    __shared__ float s_rec[kGatherStage][kPartFloats];  // odd row stride: lanes on different rows, different banks
    __shared__ int32_t s_off[kGatherWave];              // each lane's first staged entry
    __shared__ int32_t s_src[kGatherWave];              // each lane's first entry in `part`
    const int lane = threadIdx.x;
    const int j = blockIdx.x * npos + lane;
    const int n_pos = count_dev ? static_cast<int>(*count_dev) : count;
    const uint32_t stamp = *stamp_p;
    int32_t p0 = 0, p1 = 0, n = 0;
    int g = 0;
    bool is_long = false;
    if (lane < npos && j < n_pos) {
        p1 = static_cast<int32_t>(cum[j]);
        p0 = j > 0 ? static_cast<int32_t>(cum[j - 1]) : 0;
        g = order ? order[j] : j;
        if (p1 > p0 && touched[g] != 0) {  // an untouched range has no stamped entry
            if (p1 - p0 > kLongRange) {
                const int32_t q = atomicAdd(long_count, 1);
                if (inline_long)
                    is_long = true;
                else
                    long_list[q] = j;
            } else {
                n = p1 - p0;
            }
        }
    }
    // exclusive scan of the staged lengths over the wave
    int incl = n;
#pragma unroll
    for (int o = 1; o < kGatherWave; o <<= 1) {
        const int y = __shfl_up(incl, o, kGatherWave);
        if (lane >= o) incl += y;
    }
    const int off = incl - n;
    const int total = __shfl(incl, kGatherWave - 1, kGatherWave);
    if (total > 0) {  // uniform
    s_off[lane] = off;
    s_src[lane] = p0;
    __syncthreads();
    float v[kPartFloats];
#pragma unroll
    for (int k = 0; k < kPartFloats; k++) v[k] = 0.f;
    for (int base = 0; base < total; base += kGatherStage) {  // uniform
        const int cnt = min(kGatherStage, total - base);
        // the round's entries, kGatherStage / kGatherWave per lane, loaded together (the lanes past the
        // round's end load its last entry again) and then staged
        constexpr int kPerLane = kGatherStage / kGatherWave;
        float e[kPerLane][kPartFloats];
        bool on[kPerLane];
#pragma unroll
        for (int u = 0; u < kPerLane; u++) {
            // the staged entry's owner: the last lane whose first staged entry is at or before it (lanes
            // that stage nothing share the next lane's offset, and the search passes over them)
            const int k = base + min(lane + u * kGatherWave, cnt - 1);
            int lo = 0;
#pragma unroll
            for (int step = kGatherWave / 2; step > 0; step >>= 1)
                if (s_off[lo + step] <= k) lo += step;
            on[u] = load_entry(part, s_src[lo] + (k - s_off[lo]), stamp, e[u]);
        }
#pragma unroll
        for (int u = 0; u < kPerLane; u++) {
            const int i = lane + u * kGatherWave;
            if (i < cnt)
#pragma unroll
                for (int c = 0; c < kPartFloats; c++) s_rec[i][c] = on[u] ? e[u][c] : 0.f;
        }
        __syncthreads();
        const int a = max(off, base), b = min(off + n, base + cnt);
        for (int k = a; k < b; k++)
#pragma unroll
            for (int c = 0; c < kPartFloats; c++) v[c] += s_rec[k - base][c];
        __syncthreads();  // the next round restages
    }
    if (n > 0) store_grad_record(grads, static_cast<size_t>(g), v);
    }
    // inline: the wave's long ranges, as k_gather_long reduces them
    for (unsigned long long lm = __ballot(is_long); lm; lm &= lm - 1) {  // uniform
        const int L = static_cast<int>(__builtin_ctzll(lm));
        const int32_t q0 = __shfl(p0, L, kGatherWave), q1 = __shfl(p1, L, kGatherWave);
        const int gl = __shfl(g, L, kGatherWave);  // (every lane takes part in the shuffles)
        float acc[kPartFloats];
        reduce_long_range(part, q0, q1, stamp, acc);
        if (lane == 0) store_grad_record(grads, static_cast<size_t>(gl), acc);
    }
}

// The queued long ranges, one wave each, 64 entries per round (lane l takes entry base + l when it
// carries the stamp); each round's 64 values are added in a fixed tree (DPP within rows, then across
// rows) and the rounds in order.
__global__ void __launch_bounds__(kThreads) k_gather_long(const int32_t* __restrict__ order,
                                                          const int64_t* __restrict__ cum,
                                                          const float* __restrict__ part,
                                                          const uint32_t* __restrict__ stamp_p,
                                                          float4* __restrict__ grads,
                                                          const int32_t* __restrict__ long_list,
                                                          const int32_t* __restrict__ long_count) {
    const int lane = threadIdx.x & 63;
    const int n_long = *long_count;
    const uint32_t stamp = *stamp_p;
    const int n_waves = gridDim.x * (kThreads / 64);
    for (int q = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); q < n_long; q += n_waves) {  // wave-uniform
        const int j = long_list[q];
        const int32_t p1 = static_cast<int32_t>(cum[j]);
        const int32_t p0 = j > 0 ? static_cast<int32_t>(cum[j - 1]) : 0;
        float v[kPartFloats];
        reduce_long_range(part, p0, p1, stamp, v);
        if (lane == 0) store_grad_record(grads, static_cast<size_t>(order ? order[j] : j), v);
    }
}
}  // namespace

void raster_bwd_begin(uint32_t* stamp, uint8_t* touched, int rows, int32_t* long_count, hipStream_t s) {
    const int blocks = std::min(std::max((rows + kThreads - 1) / kThreads, 1), 4096);
    hipLaunchKernelGGL(k_bwd_begin, dim3(blocks), dim3(kThreads), 0, s, stamp, touched, rows, long_count);
}

void raster_gather_grads(int count, const int32_t* order, const int64_t* cum, const float* part, const uint32_t* stamp,
                         const uint8_t* touched, float4* grads, int32_t* long_list, int32_t* long_count,
                         hipStream_t s, const int64_t* count_dev, bool inline_long, const StepLoss* loss,
                         int positions_per_wave) {
    if (count <= 0) return;
    if (positions_per_wave != 32 && positions_per_wave != 64)
        throw std::invalid_argument("raster_gather_grads: positions_per_wave must be 32 or 64");
    hipLaunchKernelGGL(k_gather_grads, dim3((count + positions_per_wave - 1) / positions_per_wave), dim3(kGatherWave),
                       0, s, count, order, cum, part, stamp, touched, grads, long_list, long_count, count_dev,
                       inline_long ? 1 : 0, positions_per_wave, loss ? *loss : StepLoss{});
    if (!inline_long)
        hipLaunchKernelGGL(k_gather_long, dim3(1024), dim3(kThreads), 0, s, order, cum, part, stamp, grads,
                           long_list, long_count);
}

namespace {
// Counting sort of the tiles by descending intersection count (256 buckets of width w, w the
// smallest power of two with max_count < 256 w), one workgroup. Most tiles share a few buckets, so a
// wave's lanes with the same bucket are grouped (one ballot per bucket bit) and one leader lane adds
// the group's size: the LDS adds then never collide within a wave. The order within a bucket is
// arbitrary (the order is only the rasterisers' schedule).
// One workgroup of 1024 threads: the order, and the largest count into *max_count when given.
__global__ void __launch_bounds__(1024) k_tile_order(const int32_t* __restrict__ offsets, int n_tiles,
                                                     int64_t n_isects, int32_t* __restrict__ order,
                                                     const int64_t* __restrict__ n_isects_dev,
                                                     uint32_t* __restrict__ max_count) {
    __shared__ OrderScratch sc;
    if (n_isects_dev) n_isects = *n_isects_dev;
    tile_order_block<1024, 8>(offsets, n_tiles, n_isects, order, max_count, &sc);  // 8192 tiles from registers
}
}  // namespace

void raster_tile_order(const int32_t* offsets, int n_tiles, int64_t n_isects, int32_t* order, hipStream_t s,
                       const int64_t* n_isects_dev, uint32_t* max_count) {
    if (n_tiles <= 0) return;
    hipLaunchKernelGGL(k_tile_order, dim3(1), dim3(1024), 0, s, offsets, n_tiles, n_isects, order, n_isects_dev,
                       max_count);
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
        hipLaunchKernelGGL((k_raster_bwd<true, false, kBwdSeg>), dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids,
                           v_rc, v_ra, g);
    else if (a.stats)
        hipLaunchKernelGGL((k_raster_bwd<false, true, kBwdSeg>), dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids,
                           v_rc, v_ra, g);
    else
        hipLaunchKernelGGL((k_raster_bwd<false, false, kBwdSeg>), dim3(blocks), dim3(kThreads), 0, s, a, ralpha, last_ids,
                           v_rc, v_ra, g);
}

} // namespace sxk
