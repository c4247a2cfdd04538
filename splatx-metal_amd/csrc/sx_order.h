// sx_order.h — the rasterisers' tile order, heaviest tile first, worked out by one workgroup.
//
// The order only schedules the per-tile workgroups of the rasterisers (each tile's results are the same
// in any order); the heaviest tiles first keep a few long ones from running alone at the end of a
// launch. It is a counting sort of the tiles on 256 buckets of count >> shift, shift the least that
// brings the largest count below 256, so any counts give a permutation of [0, n_tiles).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sxk {

// LDS of one workgroup's tile order
struct OrderScratch {
    uint32_t hist[256];
    uint32_t wtot[4];
    uint32_t max;
};

// The lanes of the wave whose byte b equals this lane's (among the valid lanes).
__device__ __forceinline__ uint64_t order_same_byte_lanes(uint32_t b, bool valid) {
    uint64_t match = __ballot(valid);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const bool bit = (b >> k) & 1u;
        const uint64_t bal = __ballot(bit);
        match &= bit ? bal : ~bal;
    }
    return match;
}

// The order by one workgroup of NT threads (a multiple of 64, at least 256), from the tile counts (tile
// t's: offsets[t + 1] - offsets[t], the last tile's up to n_isects): each thread keeps its first KEEP
// counts in registers for the later passes (further ones are read again). Every thread of the workgroup
// calls it; the largest count goes to *max_count when given.
template <int NT, int KEEP>
__device__ void tile_order_block(const int32_t* __restrict__ offsets, int n_tiles, int64_t n_isects,
                                 int32_t* __restrict__ order, uint32_t* __restrict__ max_count, OrderScratch* sc) {
    static_assert(NT % 64 == 0 && NT >= 256, "whole waves, and at least one thread per bucket");
    const int t0 = threadIdx.x, lane = t0 & 63;
    auto count_of = [&](int t) -> uint32_t {
        const int64_t e = t + 1 < n_tiles ? offsets[t + 1] : n_isects;
        return static_cast<uint32_t>(e - offsets[t]);
    };
    if (t0 < 256) sc->hist[t0] = 0;
    if (t0 == 0) sc->max = 0;
    __syncthreads();
    uint32_t kept[KEEP];
    uint32_t mx = 0;
#pragma unroll
    for (int r = 0; r < KEEP; r++) {
        const int t = t0 + NT * r;
        kept[r] = t < n_tiles ? count_of(t) : 0u;
        mx = max(mx, kept[r]);
    }
    for (int t = t0 + NT * KEEP; t < n_tiles; t += NT) mx = max(mx, count_of(t));
    auto count_at = [&](int r, int t) -> uint32_t { return r < KEEP ? kept[r] : count_of(t); };
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), o, 64)));
    if (lane == 0) atomicMax(&sc->max, mx);
    __syncthreads();
    mx = sc->max;
    int shift = 0;
    while ((mx >> shift) >= 256u) shift++;
    if (max_count && t0 == 0) *max_count = mx;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    // rounds are uniform over the workgroup (every thread runs ceil(n_tiles / NT) of them)
    for (int t1 = 0, r = 0; t1 < n_tiles; t1 += NT, r++) {
        const int t = t1 + t0;
        const bool valid = t < n_tiles;
        const uint32_t b = valid ? 255u - (count_at(r, t) >> shift) : 0u;
        const uint64_t m = order_same_byte_lanes(b, valid);
        if (valid && (m & below) == 0) atomicAdd(&sc->hist[b], static_cast<uint32_t>(__popcll(m)));
    }
    __syncthreads();
    // exclusive prefix over the 256 buckets: waves 0-3 scan them, then add the lower waves' totals
    uint32_t hc = 0, hx = 0;
    if (t0 < 256) {  // whole waves
        hc = sc->hist[t0];
        hx = hc;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = static_cast<uint32_t>(__shfl_up(static_cast<int>(hx), o, 64));
            if (lane >= o) hx += y;
        }
        if (lane == 63) sc->wtot[t0 >> 6] = hx;
    }
    __syncthreads();
    if (t0 < 256) {
        uint32_t pre = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) pre += w < (t0 >> 6) ? sc->wtot[w] : 0u;
        sc->hist[t0] = pre + hx - hc;
    }
    __syncthreads();
    for (int t1 = 0, r = 0; t1 < n_tiles; t1 += NT, r++) {
        const int t = t1 + t0;
        const bool valid = t < n_tiles;
        const uint32_t b = valid ? 255u - (count_at(r, t) >> shift) : 0u;
        const uint64_t m = order_same_byte_lanes(b, valid);
        const int leader = m ? static_cast<int>(__builtin_ctzll(m)) : 0;
        uint32_t base = 0;
        if (valid && lane == leader) base = atomicAdd(&sc->hist[b], static_cast<uint32_t>(__popcll(m)));
        base = static_cast<uint32_t>(__shfl(static_cast<int>(base), leader, 64));
        if (valid) order[base + static_cast<uint32_t>(__popcll(m & below))] = t;
    }
}

}  // namespace sxk
