// k_sort.hip — stable LSD radix sort of (u64 key, i32 value) pairs for gfx950.
//
// Contract: KernelBackend.h:130-148 / sort_isect (ascending unsigned key, stable, only bits
// [0, key_bits) significant). Design: 8-bit digits, so a 45-bit isect key needs 6 passes (the
// reference's 4-bit digits need 12). Each pass is three launches with no inter-workgroup waiting:
//   1. per-tile digit histogram (LDS counters)        -> hist[digit][tile]
//   2. exclusive scan of hist in digit-major order     -> global start of (digit, tile)
//   3. stable scatter: each 64-lane wave ranks its keys per digit with 8 ballots (lanes with an
//      identical digit form one match mask), waves are ordered through LDS counts, rounds keep
//      input order, so equal digits keep their relative order.
#include <hip/hip_runtime.h>

#include "sx_kernels.h"

namespace sxk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRounds = 16;
constexpr int kTile = kThreads * kRounds;  // 4096 keys per workgroup
constexpr int kBins = 256;

__global__ void __launch_bounds__(kThreads) k_hist(const uint64_t* __restrict__ keys, int64_t n, int shift,
                                                   uint32_t* __restrict__ hist, int n_tiles) {
    __shared__ uint32_t h[kBins];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kTile;
#pragma unroll 4
    for (int r = 0; r < kRounds; r++) {
        const int64_t idx = base + r * kThreads + threadIdx.x;
        if (idx < n) atomicAdd(&h[(keys[idx] >> shift) & 0xFF], 1u);
    }
    __syncthreads();
    hist[(size_t)threadIdx.x * n_tiles + blockIdx.x] = h[threadIdx.x];
}

// Exclusive scan of a u32 array in two launches (block sums, then per-block prefix + local scan).
constexpr int kScanItems = 16;
constexpr int kScanTile = kThreads * kScanItems;

__device__ inline uint32_t block_excl_scan_u32(uint32_t v, uint32_t* s_wave, uint32_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) s_wave[wave] = x;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        if (w < wave) pre += s_wave[w];
        tot += s_wave[w];
    }
    __syncthreads();
    if (total) *total = tot;
    return pre + x - v;
}

__global__ void __launch_bounds__(kThreads) k_u32_sums(const uint32_t* __restrict__ in, int64_t n,
                                                       uint32_t* __restrict__ sums) {
    __shared__ uint32_t s_wave[kWaves];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    uint32_t acc = 0;
    for (int i = 0; i < kScanItems; i++) {
        const int64_t idx = base + i * kThreads + threadIdx.x;
        if (idx < n) acc += in[idx];
    }
    uint32_t tot = 0;
    block_excl_scan_u32(acc, s_wave, &tot);
    if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

__global__ void __launch_bounds__(kThreads) k_u32_scan(uint32_t* __restrict__ data, int64_t n,
                                                       const uint32_t* __restrict__ sums) {
    __shared__ uint32_t s_wave[kWaves];
    __shared__ uint32_t s_prefix;
    uint32_t p = 0;
    for (int b = threadIdx.x; b < static_cast<int>(blockIdx.x); b += kThreads) p += sums[b];
    uint32_t ptot = 0;
    block_excl_scan_u32(p, s_wave, &ptot);
    if (threadIdx.x == 0) s_prefix = ptot;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    uint32_t v[kScanItems];
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; i++) {
        v[i] = (base + i < n) ? data[base + i] : 0u;
        acc += v[i];
    }
    uint32_t run = block_excl_scan_u32(acc, s_wave, nullptr) + s_prefix;
#pragma unroll
    for (int i = 0; i < kScanItems; i++) {
        if (base + i < n) data[base + i] = run;
        run += v[i];
    }
}

__global__ void __launch_bounds__(kThreads) k_scatter(const uint64_t* __restrict__ kin, const int32_t* __restrict__ vin,
                                                      uint64_t* __restrict__ kout, int32_t* __restrict__ vout,
                                                      int64_t n, int shift, const uint32_t* __restrict__ hist,
                                                      int n_tiles) {
    __shared__ uint32_t s_off[kBins];
    __shared__ uint32_t s_cnt[kWaves][kBins];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    s_off[tid] = hist[(size_t)tid * n_tiles + blockIdx.x];
    const uint64_t lanes_below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int64_t base = (int64_t)blockIdx.x * kTile;
    for (int r = 0; r < kRounds; r++) {
        const int64_t round_base = base + r * kThreads;
        if (round_base >= n) break;  // uniform across the workgroup
#pragma unroll
        for (int w = 0; w < kWaves; w++) s_cnt[w][tid] = 0;
        __syncthreads();
        const int64_t idx = round_base + tid;
        const bool valid = idx < n;
        const uint64_t key = valid ? kin[idx] : 0ull;
        const int32_t val = valid ? vin[idx] : 0;
        const uint32_t digit = static_cast<uint32_t>((key >> shift) & 0xFF);
        uint64_t match = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const bool bit = (digit >> b) & 1u;
            const uint64_t bal = __ballot(bit);
            match &= bit ? bal : ~bal;
        }
        const uint32_t rank = static_cast<uint32_t>(__popcll(match & lanes_below));
        if (valid && rank == 0) s_cnt[wave][digit] = static_cast<uint32_t>(__popcll(match));
        __syncthreads();
        if (valid) {
            uint32_t pos = s_off[digit] + rank;
            for (int w = 0; w < wave; w++) pos += s_cnt[w][digit];
            kout[pos] = key;
            vout[pos] = val;
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int w = 0; w < kWaves; w++) add += s_cnt[w][tid];
        s_off[tid] += add;
        __syncthreads();
    }
}

int tiles_for(int64_t n) { return static_cast<int>((n + kTile - 1) / kTile); }

} // namespace

size_t sort_scratch_bytes(int64_t n) {
    const int64_t tiles = std::max<int64_t>(1, tiles_for(n));
    const int64_t hist = tiles * kBins;
    const int64_t sums = (hist + kScanTile - 1) / kScanTile;
    return sizeof(uint32_t) * static_cast<size_t>(hist + sums + 64);
}

int radix_sort(uint64_t* keys_a, int32_t* vals_a, uint64_t* keys_b, int32_t* vals_b, int64_t n, uint32_t key_bits,
               void* scratch, hipStream_t s) {
    if (n <= 0 || key_bits == 0) return 0;
    const int tiles = tiles_for(n);
    uint32_t* hist = static_cast<uint32_t*>(scratch);
    const int64_t hist_n = (int64_t)tiles * kBins;
    uint32_t* sums = hist + hist_n;
    const int scan_blocks = static_cast<int>((hist_n + kScanTile - 1) / kScanTile);
    const int passes = static_cast<int>((key_bits + 7) / 8);
    uint64_t* kin = keys_a;
    int32_t* vin = vals_a;
    uint64_t* kout = keys_b;
    int32_t* vout = vals_b;
    for (int p = 0; p < passes; p++) {
        const int shift = 8 * p;
        hipLaunchKernelGGL(k_hist, dim3(tiles), dim3(kThreads), 0, s, kin, n, shift, hist, tiles);
        hipLaunchKernelGGL(k_u32_sums, dim3(scan_blocks), dim3(kThreads), 0, s, hist, hist_n, sums);
        hipLaunchKernelGGL(k_u32_scan, dim3(scan_blocks), dim3(kThreads), 0, s, hist, hist_n, sums);
        hipLaunchKernelGGL(k_scatter, dim3(tiles), dim3(kThreads), 0, s, kin, vin, kout, vout, n, shift, hist,
                           tiles);
        std::swap(kin, kout);
        std::swap(vin, vout);
    }
    return (passes & 1) ? 1 : 0;
}

} // namespace sxk
