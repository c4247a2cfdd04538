// k_sort.hip — stable LSD radix sort of (key, i32 value) pairs for gfx950, keys u64 (the isect
// keys of sort_isect), u32 (depths) or u16 (tile ids).
//
// Contract: KernelBackend.h:130-148 / sort_isect (ascending unsigned key, stable, only bits
// [0, key_bits) significant). Design: digits of at most 8 bits, the key bits spread evenly over the
// fewest passes, so a 45-bit isect key needs 6 passes (the reference's 4-bit digits need 12) and a
// 13-bit tile id two passes (6 then 7 bits; 7 then 6 in onesweep). Below 16 tiles of 4096 keys the passes run onesweep (see
// k_os_pass): the digit histograms of all passes come from one read of the keys, and each pass is one
// launch whose tiles chain their digit prefixes by look-back. From 16 tiles (and below 2^30 keys) on
// each pass counts its tiles' digits, scans the count matrix and scatters with the same pass kernel,
// without the chain (see k_rs_count). The fallback at 2^30 keys and above is three launches per pass
// with no inter-workgroup waiting:
//   1. per-tile digit histogram (LDS counters)        -> hist[digit][tile], plus the digit totals
//   2. one workgroup per digit scans its row of hist   -> global start of (digit, tile)
//   3. stable scatter: each 64-lane wave ranks the keys of its quarter of the tile per digit with 8
//      ballots (lanes with an identical digit form one match mask) and per-wave LDS offsets, so
//      equal digits keep their relative order; the tile is reordered in LDS first so that the
//      global writes of each digit's run are contiguous.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdexcept>
#include <type_traits>

#include "sx_kernels.h"
#include "sx_order.h"

namespace sxk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRounds = 16;
constexpr int kTile = kThreads * kRounds;  // 4096 keys per workgroup
constexpr int kBins = 256;
constexpr int kMaxPassesOs = 8;
constexpr int kXcds = 8;  // XCDs of an MI355X (workgroups are dealt to them round-robin)

// Pass p of a sort on bits [0, key_bits) with digits of `dbits` bits covers bits [p dbits, p dbits +
// width), the last pass only what is left of key_bits (bits above key_bits never count).
__host__ __device__ inline uint32_t digit_mask(int p, int dbits, uint32_t key_bits) {
    const int width = min(dbits, static_cast<int>(key_bits) - p * dbits);
    return (1u << width) - 1u;
}

// Lanes of the wave whose 8-bit digit equals this lane's (among lanes where `valid`), from 8 ballots.
__device__ __forceinline__ uint64_t digit_match(uint32_t digit, bool valid) {
    uint64_t match = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const bool bit = (digit >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        match &= bit ? bal : ~bal;
    }
    return match;
}

// Per-tile digit histogram -> hist[digit][tile]; the tile's counts are also added to the pass's
// digit totals (zeroed by k_zero_totals before the first pass). Equal digits of a wave are counted
// by one leader lane (match masks), so concentrated digits cost no LDS atomic contention.
template <class K>
__global__ void __launch_bounds__(kThreads) k_hist(const K* __restrict__ keys, int64_t n, int shift, uint32_t mask,
                                                   uint32_t* __restrict__ hist, int n_tiles,
                                                   uint32_t* __restrict__ totals) {
    __shared__ uint32_t h[kBins];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kTile;
    const int lane = threadIdx.x & 63;
    const uint64_t lanes_below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    K key[kRounds];
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
        const int64_t idx = base + r * kThreads + threadIdx.x;
        key[r] = idx < n ? keys[idx] : K(0);
    }
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
        const bool valid = base + r * kThreads + threadIdx.x < n;
        const uint32_t d = static_cast<uint32_t>(key[r] >> shift) & mask;
        const uint64_t match = digit_match(d, valid);
        if (valid && (match & lanes_below) == 0) atomicAdd(&h[d], static_cast<uint32_t>(__popcll(match)));
    }
    __syncthreads();
    const uint32_t c = h[threadIdx.x];
    hist[(size_t)threadIdx.x * n_tiles + blockIdx.x] = c;
    if (c) atomicAdd(&totals[threadIdx.x], c);
}

__global__ void __launch_bounds__(kThreads) k_zero_totals(uint32_t* __restrict__ totals, int n,
                                                          uint32_t* __restrict__ err) {
    for (int i = threadIdx.x; i < n; i += kThreads) totals[i] = 0;
    if (err && threadIdx.x == 0) *err = 0u;
}

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

// One workgroup per digit d: hist[d][t] <- (keys of digits < d) + (keys of digit d in tiles < t),
// the global output start of tile t's run of digit d.
__global__ void __launch_bounds__(kThreads) k_scan_digit(uint32_t* __restrict__ hist, int n_tiles,
                                                         const uint32_t* __restrict__ totals) {
    __shared__ uint32_t s_wave[kWaves];
    const int d = blockIdx.x, tid = threadIdx.x;
    uint32_t all = 0;
    const uint32_t before = block_excl_scan_u32(totals[tid], s_wave, &all);
    __shared__ uint32_t s_base;
    if (tid == d) s_base = before;
    __syncthreads();
    uint32_t carry = s_base;
    uint32_t* row = hist + (size_t)d * n_tiles;
    constexpr int kItems = 4;
    for (int c0 = 0; c0 < n_tiles; c0 += kThreads * kItems) {
        const int i0 = c0 + tid * kItems;
        uint32_t v[kItems], sum = 0;
#pragma unroll
        for (int j = 0; j < kItems; j++) {
            v[j] = i0 + j < n_tiles ? row[i0 + j] : 0u;
            sum += v[j];
        }
        uint32_t chunk = 0;
        uint32_t run = block_excl_scan_u32(sum, s_wave, &chunk) + carry;
#pragma unroll
        for (int j = 0; j < kItems; j++) {
            if (i0 + j < n_tiles) row[i0 + j] = run;
            run += v[j];
        }
        carry += chunk;
    }
}

// Stable scatter of one tile of 4096 keys. Wave w owns the contiguous quarter [1024 w, 1024 w + 1024)
// of the tile and walks it in 16 rounds of 64 keys; ranks among equal digits come from 64-lane
// match masks (8 ballots), so within the tile the order is (wave, round, lane) = input order. The
// tile is reordered by digit in LDS and then written out run by run: consecutive threads store
// consecutive addresses of one digit's output range.
template <class K>
__global__ void __launch_bounds__(kThreads) k_scatter(const K* __restrict__ kin, const int32_t* __restrict__ vin,
                                                      K* __restrict__ kout, int32_t* __restrict__ vout,
                                                      int64_t n, int shift, uint32_t mask, const uint32_t* __restrict__ hist,
                                                      int n_tiles) {
    constexpr int kPerWave = kTile / kWaves;  // 1024
    __shared__ K s_k[kTile];
    __shared__ int32_t s_v[kTile];
    __shared__ uint32_t s_gstart[kBins];  // global start of this tile's run of each digit
    __shared__ uint32_t s_lstart[kBins];  // local (in-tile) start of each digit's run
    __shared__ uint32_t s_woff[kWaves][kBins];  // per wave: next local slot of each digit
    __shared__ uint32_t s_wave[kWaves];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int64_t base = (int64_t)blockIdx.x * kTile;
    const int tile_n = static_cast<int>(min<int64_t>(kTile, n - base));
    s_gstart[tid] = hist[(size_t)tid * n_tiles + blockIdx.x];
#pragma unroll
    for (int w = 0; w < kWaves; w++) s_woff[w][tid] = 0;
    __syncthreads();
    K key[kRounds];
    int32_t val[kRounds];
    if (vin) {  // uniform; null values: the input index
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            const int i = wave * kPerWave + r * 64 + lane;
            key[r] = i < tile_n ? kin[base + i] : K(0);
            val[r] = i < tile_n ? vin[base + i] : 0;
        }
    } else {
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            const int i = wave * kPerWave + r * 64 + lane;
            key[r] = i < tile_n ? kin[base + i] : K(0);
            val[r] = i < tile_n ? static_cast<int32_t>(base + i) : 0;
        }
    }
    // per-wave digit histograms: one leader lane per distinct digit of a round; the ranks among
    // equal digits (and the leaders' counts) are kept for the placement below
    const uint64_t lanes_below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint8_t rank[kRounds];
    uint8_t cnt[kRounds];  // 0 unless this lane leads its digit group (then popcount - 1, fits 0..63)
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
        const bool valid = wave * kPerWave + r * 64 + lane < tile_n;
        const uint32_t d = static_cast<uint32_t>(key[r] >> shift) & mask;
        const uint64_t match = digit_match(d, valid);
        rank[r] = static_cast<uint8_t>(__popcll(match & lanes_below));
        cnt[r] = 0;
        if (valid && rank[r] == 0) {
            const uint32_t c = static_cast<uint32_t>(__popcll(match));
            cnt[r] = static_cast<uint8_t>(c - 1);
            s_woff[wave][d] += c;  // only this wave writes its row, one leader per digit
        }
    }
    __syncthreads();
    {
        // thread = digit: the digit's in-tile start, then each wave's start inside the digit's run
        uint32_t c[kWaves], tot = 0;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            c[w] = s_woff[w][tid];
            tot += c[w];
        }
        uint32_t all = 0;
        uint32_t run = block_excl_scan_u32(tot, s_wave, &all);
        s_lstart[tid] = run;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            s_woff[w][tid] = run;
            run += c[w];
        }
    }
    __syncthreads();
    uint32_t* woff = s_woff[wave];
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
        if (wave * kPerWave + r * 64 >= tile_n) break;  // uniform within the wave
        const bool valid = wave * kPerWave + r * 64 + lane < tile_n;
        const uint32_t digit = static_cast<uint32_t>(key[r] >> shift) & mask;
        if (valid) {
            const uint32_t pos = woff[digit] + rank[r];
            s_k[pos] = key[r];
            s_v[pos] = val[r];
        }
        __builtin_amdgcn_wave_barrier();  // every lane has read woff[] before it is advanced
        if (valid && rank[r] == 0) woff[digit] += static_cast<uint32_t>(cnt[r]) + 1u;
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    for (int p = tid; p < tile_n; p += kThreads) {
        const K k = s_k[p];
        const uint32_t d = static_cast<uint32_t>(k >> shift) & mask;
        const uint32_t g = s_gstart[d] + (static_cast<uint32_t>(p) - s_lstart[d]);
        kout[g] = k;
        vout[g] = s_v[p];
    }
}

// ---- onesweep: one launch per pass (digit histograms of every pass from one read up front) ----
// Tile t of a pass publishes its digit counts to status[t][d] as soon as it has ranked its keys
// (flag AGG), then looks back over its predecessors' words, adding counts until it meets an
// inclusive prefix (flag INC), and publishes its own inclusive prefix. Tiles take their index from
// an atomic counter in the order they start, so every tile a tile waits on has already started and
// publishes without waiting itself: the look-back always ends. A bounded spin turns a broken
// invariant into an error flag instead of a hang.
constexpr uint32_t kFlagAgg = 1u << 30;
constexpr uint32_t kFlagInc = 2u << 30;
constexpr uint32_t kValMask = (1u << 30) - 1u;
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr int kLook = 8;  // predecessor words per lane and look-back round trip
// A pass with 2^w < 256 digit values gives each digit G = min(256 / 2^w, kLookLanes) adjacent lanes
// for its look-back, so a round trip reads G * kLook predecessors: the chain of inclusive prefixes
// then advances G times faster, which is what bounds a pass over many tiles.
constexpr int kLookLanes = 16;

__device__ __forceinline__ uint32_t ld_status(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_status(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Digit histograms of passes [0, passes) -> totals[p][d]; clears the first pass's status words and
// the per-pass tile counters. Grid-stride over 4096-key chunks. A wave whose 64 digits agree (the
// tile bits of neighbouring keys) adds once; otherwise each lane adds 1 (spread digits, few
// collisions): cheaper than match masks here, where no ranks are needed.
template <class K>
__global__ void __launch_bounds__(kThreads) k_os_hist(const K* __restrict__ keys, int64_t n, int passes, int dbits, uint32_t key_bits,
                                                      uint32_t* __restrict__ totals, uint32_t* __restrict__ status0,
                                                      int64_t status_words, uint32_t* __restrict__ counters,
                                                      const int64_t* __restrict__ n_dev) {
    __shared__ uint32_t h[kMaxPassesOs][kBins];
    if (n_dev) {
        n = *n_dev;
        status_words = (n + kTile - 1) / kTile * kBins;
    }
    for (int p = 0; p < kMaxPassesOs; p++) h[p][threadIdx.x] = 0;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < status_words; i += (int64_t)gridDim.x * kThreads)
        status0[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x < kMaxPassesOs) counters[threadIdx.x] = 0u;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int64_t chunks = (n + kTile - 1) / kTile;
    for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const int64_t base = c * kTile;
        K key[kRounds];  // the whole chunk in flight before any counting
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            const int64_t idx = base + r * kThreads + threadIdx.x;
            key[r] = idx < n ? keys[idx] : K(0);
        }
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            const bool valid = base + r * kThreads + threadIdx.x < n;
            for (int p = 0; p < passes; p++) {
                const uint32_t d = static_cast<uint32_t>(key[r] >> (dbits * p)) & digit_mask(p, dbits, key_bits);
                const uint32_t d0 = __builtin_amdgcn_readfirstlane(d);
                if (__all(valid && d == d0)) {  // one digit for the whole wave: one add
                    if (lane == 0) atomicAdd(&h[p][d0], 64u);
                } else if (valid) {
                    atomicAdd(&h[p][d], 1u);  // spread digits: lanes mostly hit distinct counters
                }
            }
        }
    }
    __syncthreads();
    for (int p = 0; p < passes; p++) {
        const uint32_t v = h[p][threadIdx.x];
        if (v) atomicAdd(&totals[p * kBins + threadIdx.x], v);
    }
}

// The same digit totals for keys of at most kFullBits significant bits: one LDS counter per key
// value (2^key_bits of them, dynamic LDS), one add per key, then each pass's digit totals are sums
// of those counters. With few digit values (a 13-bit tile id sorts as 128 + 64 bins) a wave's 64
// random keys would collide on the same digit counter and serialize; over 8192 key counters they
// rarely do, and there is one add per key instead of one per pass.
constexpr uint32_t kFullBits = 14;
// blocks of the histogram kernels: each adds its digit counts to the same few totals, and adds to one
// address serialize, so the grid is kept near the CU count (grid-stride over the chunks)
constexpr int kHistBlocks = 512;
template <class K>
__global__ void __launch_bounds__(kThreads) k_os_hist_full(const K* __restrict__ keys, int64_t n, int passes, int dbits,
                                                           uint32_t key_bits, uint32_t* __restrict__ totals,
                                                           uint32_t* __restrict__ status0, int64_t status_words,
                                                           uint32_t* __restrict__ counters, const int64_t* __restrict__ n_dev) {
    extern __shared__ uint32_t hf[];
    __shared__ uint32_t s_dig[kBins];
    if (n_dev) {
        n = *n_dev;
        status_words = (n + kTile - 1) / kTile * kBins;
    }
    const uint32_t nb = 1u << key_bits;
    for (uint32_t i = threadIdx.x; i < nb; i += kThreads) hf[i] = 0;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < status_words; i += (int64_t)gridDim.x * kThreads)
        status0[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x < kMaxPassesOs) counters[threadIdx.x] = 0u;
    __syncthreads();
    const uint32_t kmask = nb - 1u;
    const int64_t chunks = (n + kTile - 1) / kTile;
    for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const int64_t base = c * kTile;
        K key[kRounds];
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            const int64_t idx = base + r * kThreads + threadIdx.x;
            key[r] = idx < n ? keys[idx] : K(0);
        }
#pragma unroll
        for (int r = 0; r < kRounds; r++)
            if (base + r * kThreads + threadIdx.x < n) atomicAdd(&hf[static_cast<uint32_t>(key[r]) & kmask], 1u);
    }
    __syncthreads();
    // pass p, digit d (width w at shift s) counts the key values (hi << (s + w)) | (d << s) | lo, i.e.
    // the j-th of its 2^(key_bits - w) counters is j = hi 2^s + lo; the 256 threads split the digits'
    // counters evenly and add their partial sums to the totals
    for (int p = 0; p < passes; p++) {
        const int s = dbits * p;
        const uint32_t dm = digit_mask(p, dbits, key_bits);
        const int w = __popc(dm);
        const uint32_t per_digit = nb >> w;                        // counters per digit
        const uint32_t tpd = kThreads >> w;                        // threads per digit (w <= 8)
        const uint32_t d = threadIdx.x >> (8 - w);                 // this thread's digit
        const uint32_t span = per_digit / tpd ? per_digit / tpd : 1u;
        const uint32_t j0 = (threadIdx.x & (tpd - 1)) * span;
        uint32_t acc = 0;
        if (j0 < per_digit)
            for (uint32_t j = j0; j < j0 + span && j < per_digit; j++)
                acc += hf[((j >> s) << (s + w)) | (d << s) | (j & ((1u << s) - 1u))];
        // one global add per digit and block: the totals are few addresses that every block adds to,
        // and adds to one address serialize
        s_dig[threadIdx.x] = 0;
        __syncthreads();
        if (acc) atomicAdd(&s_dig[d], acc);
        __syncthreads();
        if (threadIdx.x <= dm && s_dig[threadIdx.x]) atomicAdd(&totals[p * kBins + threadIdx.x], s_dig[threadIdx.x]);
        __syncthreads();
    }
}

// totals[p][d] -> base[p][d] = keys of digits < d (exclusive scan per pass); totals left as is
__global__ void __launch_bounds__(kThreads) k_os_scan(const uint32_t* __restrict__ totals, int passes,
                                                      uint32_t* __restrict__ base) {
    __shared__ uint32_t s_wave[kWaves];
    for (int p = 0; p < passes; p++) {
        uint32_t all = 0;
        base[p * kBins + threadIdx.x] = block_excl_scan_u32(totals[p * kBins + threadIdx.x], s_wave, &all);
    }
}

// Lanes of the wave (among `valid_mask`) whose digit, the low NB bits of x, equals this lane's: one
// ballot per bit, each lane collecting the lanes that differ from it in that bit. Per bit: v_bfe_i32
// (the bit as 0 or ~0; written as asm, as the compiler otherwise makes a shift pair of it), the ballot's
// compare, and mis |= ballot ^ bit as one v_bitop3 per half (truth table 0xF6: src0 | (src1 ^ src2)).
template <int B, int NB>
__device__ __forceinline__ void digit_mismatch(uint32_t x, uint32_t& mis_lo, uint32_t& mis_hi) {
    if constexpr (B < NB) {
        uint32_t m;
        asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(m) : "v"(x), "n"(B));
        const uint64_t bal = __ballot(m != 0u);
        mis_lo = __builtin_amdgcn_bitop3_b32(mis_lo, static_cast<uint32_t>(bal), m, 0xf6);
        mis_hi = __builtin_amdgcn_bitop3_b32(mis_hi, static_cast<uint32_t>(bal >> 32), m, 0xf6);
        digit_mismatch<B + 1, NB>(x, mis_lo, mis_hi);
    }
}
template <int NB>
__device__ __forceinline__ uint64_t digit_match_bits(uint32_t x, uint64_t valid_mask) {
    uint32_t mis_lo = 0u, mis_hi = 0u;
    digit_mismatch<0, NB>(x, mis_lo, mis_hi);
    return valid_mask & ~((static_cast<uint64_t>(mis_hi) << 32) | mis_lo);
}

// Set bits of `mask` in the lanes below this one.
__device__ __forceinline__ uint32_t lanes_below_count(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// ---- reduce-then-scan: the pass's prefixes without a chain between tiles ------------------------
// For sorts of many tiles the onesweep pass is bound by its look-back: a tile waits until its
// predecessors' inclusive prefixes have been published, which advance at a fixed rate along the chain.
// Instead each pass counts the digits of every tile (k_rs_count, digit-major: cnt[d][tile]), scans the
// whole count matrix once (the exclusive prefix of entry (d, tile) is where the tile's run of digit d
// starts in the output: all keys of smaller digits, then those of digit d in earlier tiles), and the
// pass kernel places its keys with these starts. Counts fit u32: a pass sorts fewer than 2^30 keys.
constexpr int kScanChunk = kThreads * 16;  // elements per workgroup of the count-matrix scan

// Digit counts of tile blockIdx.x -> cnt[d * n_tiles + tile] for d <= mask. Every workgroup of the grid
// writes its counts (zeros for a tile past the device count), so the scanned matrix is complete. A
// thread takes 16 consecutive keys (16-B loads) and adds each run of equal digits once: neighbouring
// keys often share the high digits (the tiles of one Gaussian along a row), and the lanes of a wave,
// 16 keys apart, rarely hit the same counter at once.
// err (optional): the sort's error word, zeroed by workgroup 0 (a sort that starts with this pass).
template <class K>
__global__ void __launch_bounds__(kThreads) k_rs_count(const K* __restrict__ keys, int64_t n, int shift, uint32_t mask,
                                                       uint32_t* __restrict__ cnt, int n_tiles,
                                                       const int64_t* __restrict__ n_dev, uint32_t* __restrict__ err) {
    static_assert(kRounds * sizeof(K) % 16 == 0, "a thread's keys are whole 16-B vectors");
    __shared__ uint32_t h[kBins];
    if (err && blockIdx.x == 0 && threadIdx.x == 0) *err = 0u;
    // tiles dealt XCD by XCD, as in k_os_pass (a grid of kXcds * ceil(n_tiles / kXcds)): a digit's counts
    // of consecutive tiles are neighbouring words of the matrix, and their partial lines then merge in
    // one L2
    const int per = (n_tiles + kXcds - 1) / kXcds;
    const int tile = static_cast<int>(blockIdx.x % kXcds) * per + static_cast<int>(blockIdx.x / kXcds);
    if (tile >= n_tiles) return;  // uniform
    if (n_dev) n = *n_dev;
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t i0 = (int64_t)tile * kTile + (int64_t)threadIdx.x * kRounds;
    K key[kRounds];
    if (i0 + kRounds <= n) {  // the tile is 16-B aligned (4096 keys), and so is each thread's part
        constexpr int kVec = kRounds * sizeof(K) / 16;
        uint4 w[kVec];
#pragma unroll
        for (int q = 0; q < kVec; q++) w[q] = reinterpret_cast<const uint4*>(keys + i0)[q];
        __builtin_memcpy(key, w, sizeof(key));
    } else {
#pragma unroll
        for (int r = 0; r < kRounds; r++) key[r] = i0 + r < n ? keys[i0 + r] : K(0);
    }
    const int valid = static_cast<int>(min<int64_t>(kRounds, max<int64_t>(0, n - i0)));  // keys of the thread
    uint32_t run_d = static_cast<uint32_t>(key[0] >> shift) & mask, run_n = 0;
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
        const uint32_t d = static_cast<uint32_t>(key[r] >> shift) & mask;
        if (r < valid) {
            if (d != run_d) {
                if (run_n) atomicAdd(&h[run_d], run_n);
                run_d = d;
                run_n = 0;
            }
            run_n++;
        }
    }
    if (run_n) atomicAdd(&h[run_d], run_n);
    __syncthreads();
    if (threadIdx.x <= mask) cnt[(size_t)threadIdx.x * n_tiles + tile] = h[threadIdx.x];
}

// Exclusive scan of v[0, len) in place, in two launches: chunk sums, then the scan of each chunk
// from its prefix, which each workgroup of the second adds up from the chunk sums before it (a few
// thousand words at most: cheaper than a launch that scans them first). v starts 64-B aligned (16-B
// loads).
__global__ void __launch_bounds__(kThreads) k_rs_reduce(const uint32_t* __restrict__ v, int64_t len,
                                                        uint32_t* __restrict__ sums) {
    __shared__ uint32_t s_wave[kWaves];
    const int64_t base = (int64_t)blockIdx.x * kScanChunk;
    uint32_t acc = 0;
    if (base + kScanChunk <= len) {  // four coalesced 16-B loads per thread
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 w = reinterpret_cast<const uint4*>(v + base)[q * kThreads + threadIdx.x];
            acc += w.x + w.y + w.z + w.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int64_t k = base + i * kThreads + threadIdx.x;
            acc += k < len ? v[k] : 0u;
        }
    }
    uint32_t all = 0;
    block_excl_scan_u32(acc, s_wave, &all);
    if (threadIdx.x == 0) sums[blockIdx.x] = all;
}

__global__ void __launch_bounds__(kThreads) k_rs_down(uint32_t* __restrict__ v, int64_t len,
                                                      const uint32_t* __restrict__ sums) {
    __shared__ uint32_t s_wave[kWaves];
    const int64_t i0 = (int64_t)blockIdx.x * kScanChunk + threadIdx.x * 16;  // 16 consecutive per thread
    uint32_t x[16], acc = 0;
    if (i0 + 16 <= len) {  // four 16-B loads
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 w = reinterpret_cast<const uint4*>(v + i0)[q];
            x[4 * q] = w.x;
            x[4 * q + 1] = w.y;
            x[4 * q + 2] = w.z;
            x[4 * q + 3] = w.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) x[i] = i0 + i < len ? v[i0 + i] : 0u;
    }
#pragma unroll
    for (int i = 0; i < 16; i++) acc += x[i];
    uint32_t pre = 0;  // the chunks before this one
    for (int c = threadIdx.x; c < static_cast<int>(blockIdx.x); c += kThreads) pre += sums[c];
    uint32_t all = 0;
    (void)block_excl_scan_u32(pre, s_wave, &all);  // (its closing barrier frees s_wave)
    const uint32_t chunk_base = all;
    uint32_t run = block_excl_scan_u32(acc, s_wave, &all) + chunk_base;
    uint32_t y[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        y[i] = run;
        run += x[i];
    }
    if (i0 + 16 <= len) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            reinterpret_cast<uint4*>(v + i0)[q] = make_uint4(y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (i0 + i < len) v[i0 + i] = y[i];
    }
}

// NB = the digit's width in bits (mask = 2^NB - 1). CHAIN: the onesweep pass (tile index from the
// counter, prefixes by look-back); otherwise tile = blockIdx.x and the tile's run of digit d starts at
// starts[d * n_tiles + tile] (the scanned count matrix of the reduce-then-scan path).
// X: each key also carries a u32 second value, read from xin at the key's input position and written to
// xout at its output position (null pointers when X is false). IDX: vin is null, and each key's value is
// its input position.
template <class K, int NB, bool CHAIN, bool X, bool IDX>
__global__ void __launch_bounds__(kThreads) k_os_pass(const K* __restrict__ kin, const int32_t* __restrict__ vin,
                                                      K* __restrict__ kout, int32_t* __restrict__ vout,
                                                      int64_t n, int shift, uint32_t mask, const uint32_t* __restrict__ digit_base,
                                                      uint32_t* __restrict__ status, uint32_t* __restrict__ status_next,
                                                      uint32_t* __restrict__ counter, uint32_t* __restrict__ err,
                                                      const int64_t* __restrict__ n_dev,
                                                      const uint32_t* __restrict__ starts, int n_tiles,
                                                      const uint32_t* __restrict__ xin, uint32_t* __restrict__ xout) {
    constexpr int kPerWave = kTile / kWaves;  // 1024
    __shared__ K s_k[kTile];
    // IDX (no input values: each key's value is its input position): no value registers, and the LDS
    // reorder moves the keys' 16-bit positions in the tile (83 VGPRs and 22 KB instead of 97 and 30 KB:
    // 5 waves per SIMD instead of 4)
    __shared__ typename std::conditional<IDX, uint16_t, int32_t>::type s_v[kTile];
    __shared__ uint32_t s_x[X ? kTile : 1];
    __shared__ uint32_t s_gstart[kBins];  // global start of this tile's run of each digit, minus its local start
    __shared__ uint32_t s_lstart[kBins];
    __shared__ uint32_t s_woff[kWaves][kBins];
    __shared__ uint32_t s_wave[kWaves];
    __shared__ uint32_t s_cnt[kBins];  // this tile's count of each digit
    __shared__ uint32_t s_tile;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    if (n_dev) {  // the grid is sized for a capacity: exactly one workgroup per tile of keys takes a tile
        n = *n_dev;
        if (CHAIN && static_cast<int64_t>(blockIdx.x) * kTile >= n) return;  // uniform
    }
    // CHAIN: one tile, from the counter. Otherwise one tile below the (device) key count, by the
    // workgroup's index.
    const int64_t n_work = (n + kTile - 1) / kTile;
    // XCD-aware tile order: the GPU deals workgroups to its kXcds XCDs round-robin (workgroup b to XCD
    // b % kXcds, each XCD taking its share in order), so tile (b % kXcds) * per + b / kXcds gives every XCD
    // a contiguous range of tiles. The runs of one digit that consecutive tiles write sit next to each
    // other in the output: written from the same L2, their partial lines merge before they leave it. The
    // grid has kXcds * ceil(tiles / kXcds) workgroups; the ones past the device count leave.
    // (Fewer workgroups per CU, or each looping over several tiles, measured slower.)
    const int64_t per = (n_work + kXcds - 1) / kXcds;
    {
        const int64_t k = blockIdx.x;
        const int64_t t = CHAIN ? 0 : (k % kXcds) * per + k / kXcds;
        if (!CHAIN && (k >= per * kXcds || t >= n_work)) return;  // uniform
        if (CHAIN && tid == 0) s_tile = atomicAdd(counter, 1u);
#pragma unroll
        for (int w = 0; w < kWaves; w++) s_woff[w][tid] = 0;
        __syncthreads();
        const uint32_t tile = CHAIN ? s_tile : static_cast<uint32_t>(t);
        // the tile's digit starts are requested now, so their latency overlaps the loads and the ranking
        const uint32_t my_start = (!CHAIN && tid <= mask) ? starts[(size_t)tid * n_tiles + tile] : 0u;
        const int64_t base = (int64_t)tile * kTile;
        const int tile_n = static_cast<int>(min<int64_t>(kTile, n - base));
        K key[kRounds];
        int32_t val[IDX ? 1 : kRounds];
        uint32_t xv[X ? kRounds : 1];
        if (X) {
#pragma unroll
            for (int r = 0; r < kRounds; r++) {
                const int i = wave * kPerWave + r * 64 + lane;
                xv[r] = i < tile_n ? xin[base + i] : 0u;
            }
        }
        // null values: the input index. The (uniform) choice is taken once around straight-line loads: a
        // choice per round compiles to a wait for every load before the next is issued.
        if (tile_n == kTile) {  // uniform
            if (vin) {
#pragma unroll
                for (int r = 0; r < kRounds; r++) {
                    const int i = wave * kPerWave + r * 64 + lane;
                    key[r] = kin[base + i];
                    val[r] = vin[base + i];
                }
            } else {
#pragma unroll
                for (int r = 0; r < kRounds; r++) {
                    const int i = wave * kPerWave + r * 64 + lane;
                    key[r] = kin[base + i];
                    if (!IDX) val[r] = static_cast<int32_t>(base + i);
                }
            }
        } else if (vin) {
#pragma unroll
            for (int r = 0; r < kRounds; r++) {
                const int i = wave * kPerWave + r * 64 + lane;
                key[r] = i < tile_n ? kin[base + i] : K(0);
                val[r] = i < tile_n ? vin[base + i] : 0;
            }
        } else {
#pragma unroll
            for (int r = 0; r < kRounds; r++) {
                const int i = wave * kPerWave + r * 64 + lane;
                key[r] = i < tile_n ? kin[base + i] : K(0);
                if (!IDX) val[r] = i < tile_n ? static_cast<int32_t>(base + i) : 0;
            }
        }
        // per-wave digit counts, rounds in order; off[r] = the key's place among the wave's keys of its
        // digit (keys of earlier rounds, then lanes below it with the same digit). All lanes read the
        // digit's running count before one leader lane per digit group advances it.
        uint32_t off[kRounds];
        uint32_t* woff = s_woff[wave];
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            const bool valid = wave * kPerWave + r * 64 + lane < tile_n;
            const uint32_t x = static_cast<uint32_t>(key[r] >> shift);
            const uint32_t d = x & mask;
            const uint64_t match = digit_match_bits<NB>(x, __ballot(valid));
            const uint32_t rank = lanes_below_count(match);
            const uint32_t prior = valid ? woff[d] : 0u;
            __builtin_amdgcn_wave_barrier();
            if (valid && rank == 0u) woff[d] = prior + static_cast<uint32_t>(__popcll(match));
            __builtin_amdgcn_wave_barrier();
            off[r] = prior + rank;
        }
        __syncthreads();
        uint32_t tile_count;
        {
            uint32_t c[kWaves], tot = 0;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                c[w] = s_woff[w][tid];
                tot += c[w];
            }
            tile_count = tot;
            uint32_t all = 0;
            uint32_t run = block_excl_scan_u32(tot, s_wave, &all);
            s_lstart[tid] = run;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                s_woff[w][tid] = run;
                run += c[w];
            }
        }
        // publish this tile's digit counts now; the look-back for the prefixes of the tiles before it
        // waits until the tile has been reordered in LDS, which gives them time to finish theirs
        if (CHAIN) st_status(status + (size_t)tile * kBins + tid, (tile == 0 ? kFlagInc : kFlagAgg) | tile_count);
        s_cnt[tid] = tile_count;
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            if (wave * kPerWave + r * 64 >= tile_n) break;  // uniform within the wave
            if (wave * kPerWave + r * 64 + lane < tile_n) {
                const uint32_t pos = woff[static_cast<uint32_t>(key[r] >> shift) & mask] + off[r];
                s_k[pos] = key[r];
                s_v[pos] = IDX ? static_cast<uint16_t>(wave * kPerWave + r * 64 + lane) : val[IDX ? 0 : r];
                if (X) s_x[pos] = xv[r];
            }
        }
        __syncthreads();
        // look back: the G lanes of digit d read kLook predecessors' words each per round trip, lane s
        // the s-th run of kLook below j, newest first; the group adds counts up to the newest inclusive
        // prefix among them, or up to the newest word not yet published and retries from there
        const int bins = static_cast<int>(mask) + 1;
        const int G = min(kThreads / bins, kLookLanes);  // a power of two dividing 64
        if (!CHAIN) {
            if (tid < bins) s_gstart[tid] = my_start - s_lstart[tid];
        } else if (tile == 0) {
            s_gstart[tid] = digit_base[tid] - s_lstart[tid];
        } else if (tid < bins * G) {
            const int d = tid / G, sub = tid & (G - 1);
            const int gbase = lane & ~(G - 1);
            const uint64_t gmask = (G == 64 ? ~0ull : ((1ull << G) - 1ull)) << gbase;
            uint32_t excl = 0;
            int64_t j = (int64_t)tile - 1;
            uint32_t spins = 0;
            for (;;) {  // the group's lanes take every branch together
                const int64_t top = j - (int64_t)sub * kLook;
                uint32_t w[kLook];
#pragma unroll
                for (int q = 0; q < kLook; q++)
                    w[q] = top - q >= 0 ? ld_status(status + (size_t)(top - q) * kBins + d) : kFlagInc;
                uint32_t part = 0;
                int stop = 0, at = kLook;  // stop: 1 = met an inclusive prefix, 2 = met an unpublished word at q = at
#pragma unroll
                for (int q = 0; q < kLook; q++) {
                    if (stop == 0) {
                        const uint32_t f = w[q] & ~kValMask;
                        if (f == 0u) {
                            stop = 2;
                            at = q;
                        } else {
                            part += w[q] & kValMask;
                            if (f == kFlagInc) stop = 1;
                        }
                    }
                }
                uint32_t scan = part;  // inclusive over the group's lanes
                for (int o = 1; o < G; o <<= 1) {
                    const uint32_t y = __shfl_up(scan, o, 64);
                    if (sub >= o) scan += y;
                }
                const uint64_t stops = __ballot(stop != 0) & gmask;
                const int first = stops ? static_cast<int>(__builtin_ctzll(stops)) - gbase : G - 1;
                excl += __shfl(scan, gbase + first, 64);
                if (!stops) {
                    j -= (int64_t)G * kLook;
                    continue;
                }
                if (__shfl(stop, gbase + first, 64) == 1) break;
                const int64_t adv = (int64_t)first * kLook + __shfl(at, gbase + first, 64);
                j -= adv;
                if (adv == 0) {
                    if (++spins > kSpinLimit) {
                        atomicOr(err, 1u);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            if (sub == 0) {
                st_status(status + (size_t)tile * kBins + d, kFlagInc | (excl + s_cnt[d]));
                s_gstart[d] = digit_base[d] + excl - s_lstart[d];
            }
        }
        if (CHAIN && status_next) status_next[(size_t)tile * kBins + tid] = 0u;
        __syncthreads();
        const uint32_t n32 = static_cast<uint32_t>(n);  // onesweep runs below 2^30 keys
        for (int p = tid; p < tile_n; p += kThreads) {
            const K k = s_k[p];
            const uint32_t g = s_gstart[static_cast<uint32_t>(k >> shift) & mask] + static_cast<uint32_t>(p);
            if (g < n32) {  // always, unless the look-back gave up (err set): then no write lands out of range
                kout[g] = k;
                vout[g] = IDX ? static_cast<int32_t>(base + s_v[p]) : static_cast<int32_t>(s_v[p]);
                if (X) xout[g] = s_x[p];
            }
        }
    }
}

int tiles_for(int64_t n) { return static_cast<int>((n + kTile - 1) / kTile); }

// One onesweep pass over the digit of `mask`'s width at `shift`.
template <class K, bool CHAIN, bool X = false>
void launch_os_pass(int tiles, hipStream_t s, const K* kin, const int32_t* vin, K* kout, int32_t* vout, int64_t n,
                    int shift, uint32_t mask, const uint32_t* digit_base, uint32_t* status, uint32_t* status_next,
                    uint32_t* counter, uint32_t* err, const int64_t* n_dev, const uint32_t* starts = nullptr,
                    const uint32_t* xin = nullptr, uint32_t* xout = nullptr) {
#define SX_OS_PASS(NB)                                                                                          \
    do {                                                                                                        \
        if (vin)                                                                                                \
            hipLaunchKernelGGL((k_os_pass<K, NB, CHAIN, X, false>),                                             \
                               dim3(CHAIN ? tiles : (tiles + kXcds - 1) / kXcds * kXcds), dim3(kThreads), 0, s, \
                               kin, vin, kout, vout, n, shift, mask, digit_base, status, status_next, counter,  \
                               err, n_dev, starts, tiles, xin, xout);                                           \
        else                                                                                                    \
            hipLaunchKernelGGL((k_os_pass<K, NB, CHAIN, X, true>),                                              \
                               dim3(CHAIN ? tiles : (tiles + kXcds - 1) / kXcds * kXcds), dim3(kThreads), 0, s, \
                               kin, vin, kout, vout, n, shift, mask, digit_base, status, status_next, counter,  \
                               err, n_dev, starts, tiles, xin, xout);                                           \
    } while (0)
    switch (__builtin_popcount(mask)) {
        case 1: SX_OS_PASS(1); break;
        case 2: SX_OS_PASS(2); break;
        case 3: SX_OS_PASS(3); break;
        case 4: SX_OS_PASS(4); break;
        case 5: SX_OS_PASS(5); break;
        case 6: SX_OS_PASS(6); break;
        case 7: SX_OS_PASS(7); break;
        default: SX_OS_PASS(8); break;
    }
#undef SX_OS_PASS
}

// x_dst[i] = x_src[pos[i]] (grid-stride)
__global__ void __launch_bounds__(kThreads) k_gather_x(const int32_t* __restrict__ pos, const uint32_t* __restrict__ x_src,
                                                       uint32_t* __restrict__ x_dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        x_dst[i] = x_src[pos[i]];
}
__global__ void __launch_bounds__(kThreads) k_copy_u32(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst,
                                                       int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        dst[i] = src[i];
}

constexpr int kMaxPasses = 8;
// From this many 4096-key tiles on (64 Ki keys) a pass takes its prefixes from a scan of the tiles'
// digit counts instead of the look-back chain: the counting read costs less than the chain's waits
// (measured at 143 to 40,557 tiles: config 2's 0.58 M-key tile sort 44.7 -> 39.4 us; the two-launch
// count scan made the difference at the small sizes).
constexpr int kRtsMinTiles = 16;
// scratch layout: a fixed header (digit totals and bases of up to 8 passes, the per-pass tile
// counters, the error word) and then two tiles x 256 word buffers (the three-launch path's
// histogram, or the onesweep status words of alternate passes)
constexpr int kHeaderWords = 2 * kMaxPasses * kBins + 64;
static_assert(kHeaderWords * sizeof(uint32_t) % 64 == 0, "the count matrix after the header is 64-B aligned");

// The passes read `src` first and then alternate between the two sides: pass p writes side[p & 1],
// pass p > 0 reads side[(p - 1) & 1]. src may be side[1] (the sort then works in place over two
// buffers). n_dev: when set, the key count is read on the device from *n_dev (at most n, the capacity
// the grids are sized for), so the launches do not depend on it (a captured graph can replay them).
// Returns the number of passes, or -1 when nothing was launched because n_dev asks for the
// three-launch path. src_x (optional; then side_x too): a u32 second value per key that travels with it
// through the passes like the values (pass p writes side_x[p & 1]); the three-launch path, whose
// scatter does not carry it, gathers it once after the sort through the values, which must then be
// the input positions (src_v null).
// no_wait: reduce-then-scan at every size below 2^30 keys (no workgroup ever waits on another, so the
// sort cannot give up; the onesweep passes below 16 tiles wait on their predecessors with a bounded
// spin and set the error word if it runs out).
template <class K>
int radix_sort_t(const K* src_k, const int32_t* src_v, K* const side_k[2], int32_t* const side_v[2], int64_t n,
                 uint32_t key_bits, void* scratch, bool clear_err, hipStream_t s, const int64_t* n_dev,
                 const uint32_t* src_x = nullptr, uint32_t* const* side_x = nullptr, bool no_wait = false) {
    uint32_t* totals = static_cast<uint32_t*>(scratch);
    uint32_t* bases = totals + kMaxPasses * kBins;
    uint32_t* counters = bases + kMaxPasses * kBins;
    uint32_t* err = counters + kMaxPasses;
    key_bits = std::min<uint32_t>(key_bits, 8 * sizeof(K));
    // fewest 8-bit-or-narrower passes, the bits spread evenly over them (longer runs per digit in each
    // tile's writes than 8 + 5 for a 13-bit tile id); the onesweep passes take the wider digits first
    // (7 + 6), the reduce-then-scan passes the narrower ones (6 + 7, below)
    const int passes = static_cast<int>((key_bits + 7) / 8);
    const int dbits = passes ? static_cast<int>((key_bits + passes - 1) / passes) : 0;
    if (n <= 0 || passes == 0) {
        if (clear_err) hipLaunchKernelGGL(k_zero_totals, dim3(1), dim3(kThreads), 0, s, totals, 0, err);
        return 0;
    }
    if (n_dev && n >= (int64_t{1} << 30)) return -1;  // the three-launch path sizes its grids by the count
    const int tiles = std::max(1, tiles_for(n));
    const int64_t hist_n = (int64_t)tiles * kBins;
    uint32_t* hist = totals + kHeaderWords;
    uint32_t* status_b = hist + hist_n;
    const K* kin = src_k;
    const int32_t* vin = src_v;
    if (n < (int64_t{1} << 30) && (tiles >= kRtsMinTiles || no_wait)) {  // reduce-then-scan (see k_rs_count)
        // (the digit totals are not used here; the first count kernel clears the error word)
        uint32_t* cnt = hist;       // (mask + 1) x tiles counts, then their starts
        uint32_t* sums = status_b;  // the scan's chunk sums
        // narrower digits first: the first pass, over keys in the emit's order, has every digit in each
        // tile and so the shortest runs to write (config 5's 166 M tile ids: 1.026 -> 1.015 ms for the sort)
        const int narrow = static_cast<int>(key_bits) / passes, wide_from = passes - static_cast<int>(key_bits) % passes;
        for (int p = 0; p < passes; p++) {
            const int shift = p * narrow + std::max(0, p - wide_from);
            const uint32_t mask = (1u << (narrow + (p >= wide_from ? 1 : 0))) - 1u;
            const int64_t len = static_cast<int64_t>(mask + 1) * tiles;
            const int chunks = static_cast<int>((len + kScanChunk - 1) / kScanChunk);
            hipLaunchKernelGGL(k_rs_count<K>, dim3((tiles + kXcds - 1) / kXcds * kXcds), dim3(kThreads), 0, s, kin, n,
                               shift, mask, cnt, tiles, n_dev, (p == 0 && clear_err) ? err : nullptr);
            // (one workgroup scanning a small matrix in one launch measured slower than these)
            hipLaunchKernelGGL(k_rs_reduce, dim3(chunks), dim3(kThreads), 0, s, cnt, len, sums);
            hipLaunchKernelGGL(k_rs_down, dim3(chunks), dim3(kThreads), 0, s, cnt, len, sums);
            if (src_x)
                launch_os_pass<K, false, true>(tiles, s, kin, vin, side_k[p & 1], side_v[p & 1], n, shift, mask,
                                               nullptr, nullptr, nullptr, nullptr, err, n_dev, cnt,
                                               p == 0 ? src_x : side_x[(p - 1) & 1], side_x[p & 1]);
            else
                launch_os_pass<K, false>(tiles, s, kin, vin, side_k[p & 1], side_v[p & 1], n, shift, mask, nullptr,
                                         nullptr, nullptr, nullptr, err, n_dev, cnt);
            kin = side_k[p & 1];
            vin = side_v[p & 1];
        }
        return passes;
    }
    hipLaunchKernelGGL(k_zero_totals, dim3(1), dim3(kThreads), 0, s, totals, passes * kBins,
                       clear_err ? err : nullptr);
    if (n < (int64_t{1} << 30)) {  // onesweep: counts and prefixes fit the 30-bit status words
        const int hist_blocks = std::min(tiles, kHistBlocks);
        if (key_bits <= kFullBits)
            hipLaunchKernelGGL(k_os_hist_full<K>, dim3(hist_blocks), dim3(kThreads), sizeof(uint32_t) << key_bits, s,
                               kin, n, passes, dbits, key_bits, totals, hist, hist_n, counters, n_dev);
        else
            hipLaunchKernelGGL(k_os_hist<K>, dim3(hist_blocks), dim3(kThreads), 0, s, kin, n, passes, dbits,
                               key_bits, totals, hist, hist_n, counters, n_dev);
        hipLaunchKernelGGL(k_os_scan, dim3(1), dim3(kThreads), 0, s, totals, passes, bases);
        uint32_t* st[2] = {hist, status_b};
        for (int p = 0; p < passes; p++) {
            uint32_t* next = p + 1 < passes ? st[(p + 1) & 1] : nullptr;
            if (src_x)
                launch_os_pass<K, true, true>(tiles, s, kin, vin, side_k[p & 1], side_v[p & 1], n, dbits * p,
                                              digit_mask(p, dbits, key_bits), bases + p * kBins, st[p & 1], next,
                                              counters + p, err, n_dev, nullptr,
                                              p == 0 ? src_x : side_x[(p - 1) & 1], side_x[p & 1]);
            else
                launch_os_pass<K, true>(tiles, s, kin, vin, side_k[p & 1], side_v[p & 1], n, dbits * p,
                                        digit_mask(p, dbits, key_bits), bases + p * kBins, st[p & 1], next,
                                        counters + p, err, n_dev);
            kin = side_k[p & 1];
            vin = side_v[p & 1];
        }
        return passes;
    }
    for (int p = 0; p < passes; p++) {
        const int shift = dbits * p;
        const uint32_t mask = digit_mask(p, dbits, key_bits);
        hipLaunchKernelGGL(k_hist<K>, dim3(tiles), dim3(kThreads), 0, s, kin, n, shift, mask, hist, tiles,
                           totals + p * kBins);
        hipLaunchKernelGGL(k_scan_digit, dim3(kBins), dim3(kThreads), 0, s, hist, tiles, totals + p * kBins);
        hipLaunchKernelGGL(k_scatter<K>, dim3(tiles), dim3(kThreads), 0, s, kin, vin, side_k[p & 1], side_v[p & 1],
                           n, shift, mask, hist, tiles);
        kin = side_k[p & 1];
        vin = side_v[p & 1];
    }
    if (src_x) {
        // the sorted values are the input positions: the second values follow them by a gather, into the
        // side the passes would have left them in (through side[0] when that is the input itself)
        const int blocks = static_cast<int>(std::min<int64_t>((n + kThreads - 1) / kThreads, int64_t{1} << 20));
        uint32_t* const dst = side_x[(passes - 1) & 1];
        if (dst != src_x) {
            hipLaunchKernelGGL(k_gather_x, dim3(blocks), dim3(kThreads), 0, s, vin, src_x, dst, n);
        } else {
            hipLaunchKernelGGL(k_gather_x, dim3(blocks), dim3(kThreads), 0, s, vin, src_x, side_x[0], n);
            hipLaunchKernelGGL(k_copy_u32, dim3(blocks), dim3(kThreads), 0, s, side_x[0], dst, n);
        }
    }
    return passes;
}

// In place over two buffers: a -> b -> a -> ...; the result is in a after an even pass count. With
// index_values the first pass takes each key's input position as its value (vals_a is not read).
template <class K>
int radix_sort_ab(K* keys_a, int32_t* vals_a, K* keys_b, int32_t* vals_b, int64_t n, uint32_t key_bits,
                  void* scratch, bool clear_err, hipStream_t s, const int64_t* n_dev, bool index_values = false,
                  uint32_t* x_a = nullptr, uint32_t* x_b = nullptr, bool no_wait = false) {
    K* const sk[2] = {keys_b, keys_a};
    int32_t* const sv[2] = {vals_b, vals_a};
    uint32_t* const sx[2] = {x_b, x_a};
    const int passes = radix_sort_t<K>(keys_a, index_values ? nullptr : vals_a, sk, sv, n, key_bits, scratch,
                                       clear_err, s, n_dev, x_a, x_a ? sx : nullptr, no_wait);
    return passes < 0 ? -1 : (passes & 1);
}

// ---- the depth order within each tile (index-first intersections) --------------------------------
// When the Gaussians emit in index order, a stable sort on the tile ids leaves each tile's entries in
// index order; sorting them stably by the depth bits of their Gaussians (which the emit stored per
// entry) then gives the order of the reference's (tile | depth) keys: depth, ties by index. One
// workgroup per tile. A tile of at most 2048 entries is sorted in LDS by 8-bit LSD passes, wave w
// holding the w-th quarter of the list (in whole 64-key rounds) in registers and ranking with match
// masks as the onesweep pass does; bytes on which every key of the tile agrees are skipped. A larger
// tile runs the same passes through global scratch, 2048 keys at a time in list order.
__device__ __forceinline__ uint32_t wave_and_u32(uint32_t x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x &= static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), o, 64));
    return x;
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), o, 64));
    return x;
}

// The bits in which the keys of the workgroup differ (AND and OR of each thread's `a` / `o`).
__device__ __forceinline__ uint32_t block_key_diff(uint32_t a, uint32_t o, uint32_t* s_and, uint32_t* s_or) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    a = wave_and_u32(a);
    o = wave_or_u32(o);
    if (lane == 0) {
        s_and[wave] = a;
        s_or[wave] = o;
    }
    __syncthreads();
    uint32_t A = ~0u, O = 0u;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        A &= s_and[w];
        O |= s_or[w];
    }
    return A ^ O;
}

// Ranks the wave's keys (rounds r < R, key index wave_base + 64 r + lane below `count`) by the byte at
// `shift`: off[r] = the key's place among the wave's keys of that digit (earlier rounds, then lower
// lanes); woff receives the wave's digit counts (zeroed by the caller).
template <int RMAX>
__device__ __forceinline__ void wave_rank_byte(const uint32_t* key, int R, int wave_base, int count, int shift,
                                               uint32_t* woff, uint32_t* off) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int r = 0; r < RMAX; r++) {
        if (r >= R) break;  // uniform
        const bool valid = wave_base + r * 64 + lane < count;
        const uint32_t x = key[r] >> shift;
        const uint32_t d = x & 255u;
        const uint64_t match = digit_match_bits<8>(x, __ballot(valid));
        const uint32_t rank = lanes_below_count(match);
        const uint32_t prior = valid ? woff[d] : 0u;
        __builtin_amdgcn_wave_barrier();
        if (valid && rank == 0u) woff[d] = prior + static_cast<uint32_t>(__popcll(match));
        __builtin_amdgcn_wave_barrier();
        off[r] = prior + rank;
    }
}

// thread = digit: the waves' counts of digit tid become their first output places, from `base` on;
// returns base + the digit's count
__device__ __forceinline__ uint32_t wave_starts(uint32_t (*s_woff)[kBins], uint32_t base) {
    const int tid = threadIdx.x;
    uint32_t run = base;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        const uint32_t c = s_woff[w][tid];
        s_woff[w][tid] = run;
        run += c;
    }
    return run;
}

// equal depths: runs up to this long are put in order in place, a tile with a longer one is sorted again
constexpr int kTieRun = 32;

// The run of keys equal to keys[i] that starts at i when one does (the key before differs, the next one
// equals it): its end, up to i + kTieRun + 1 (a longer run); i otherwise.
__device__ __forceinline__ int32_t tie_run_end(const uint32_t* keys, int32_t i, int32_t n) {
    const uint32_t k = keys[i];
    if ((i > 0 && keys[i - 1] == k) || i + 1 >= n || keys[i + 1] != k) return i;
    int32_t e = i + 2;
    while (e < n && e <= i + kTieRun && keys[e] == k) e++;
    return e;
}

// RMAX: rounds of 64 keys per wave that the kernel holds in registers. One launch takes every tile,
// heaviest first (tile_order): up to kCap = 256 RMAX entries in LDS, larger ones through global
// scratch. RMAX 8 (2048 entries, 12 KB of LDS) measured fastest: a separate launch for the tiles
// past 1024 entries with 16 rounds (twice the LDS) left its few long tiles running alone after
// the small ones, and 4 rounds send more tiles through global scratch. (One wave per small tile, with
// no workgroup barriers, measured slower: its ranking rounds wait on LDS one after another.)
// order_out (optional): workgroup 0 writes the rasterisers' tile order there instead (and the largest
// tile's count into *max_count), beside the sorting workgroups, which then take tile blockIdx.x - 1: the
// per-tile sorts gain nothing from running heaviest first, and the order costs no launch of its own.
// row_orig (optional, with id_of and splats): the lists are in an internal row order whose equal depths
// must go by original row (row_orig[id_of[value]]). After the depth sort, equal depths are runs of
// adjacent entries: a run of up to kTieRun entries is put in that order by the thread at its start (an
// insertion sort in LDS, or in global scratch for the large tiles); a tile with a longer run, or with
// one depth, is sorted again through global scratch, LSD by its original rows' varying bytes, then by
// its depth bytes (an entry's depth is word 3 of its Gaussian's splat record, splats[3 id_of[value]].w,
// the key the emit wrote). One compare per entry for tiles without equal depths. (The occupancy target
// of 7 waves per SIMD, which the LDS allows, keeps the register allocation of the tie work within it:
// without it 75 VGPRs, 6 waves.)
template <int RMAX>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(7)))
k_tile_depth_sort(const int32_t* __restrict__ offsets, int n_tiles, int32_t n_isects, const int64_t* __restrict__ n_dev,
                  const int32_t* __restrict__ tile_order, int32_t* __restrict__ vals,
                  const uint32_t* __restrict__ sdepth, uint32_t* __restrict__ sk0, uint32_t* __restrict__ sk1,
                  int32_t* __restrict__ sv, int32_t* __restrict__ order_out, uint32_t* __restrict__ max_count,
                  const int32_t* __restrict__ id_of, const int32_t* __restrict__ row_orig,
                  const float4* __restrict__ splats) {
    constexpr int kCap = kWaves * 64 * RMAX;
    __shared__ uint32_t s_key[kCap];
    __shared__ int32_t s_val[kCap];
    __shared__ uint32_t s_woff[kWaves][kBins];
    __shared__ uint32_t s_base[kBins];
    __shared__ uint32_t s_wave[kWaves];
    __shared__ uint32_t s_and[kWaves], s_or[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t n_all = n_dev ? static_cast<int32_t>(*n_dev) : n_isects;
    if (order_out && blockIdx.x == 0) {  // uniform
        static_assert(sizeof(OrderScratch) <= sizeof(s_woff), "the order's scratch fits in s_woff");
        tile_order_block<kThreads, 8>(offsets, n_tiles, n_all, order_out, max_count,
                                      reinterpret_cast<OrderScratch*>(&s_woff[0][0]));
        return;
    }
    const int bx = order_out ? static_cast<int>(blockIdx.x) - 1 : static_cast<int>(blockIdx.x);
    const int t = tile_order ? tile_order[bx] : bx;
    const int32_t start = offsets[t];
    const int32_t nt = (t + 1 < n_tiles ? offsets[t + 1] : n_all) - start;
    if (nt <= 1) return;  // uniform
    int32_t* const seg = vals + start;
    const bool by_orig = row_orig != nullptr;
    auto orig_of = [&](int32_t v) -> uint32_t { return static_cast<uint32_t>(row_orig[id_of[v]]); };
    auto depth_of = [&](int32_t v) -> uint32_t { return __float_as_uint(splats[3 * (size_t)id_of[v]].w); };
    // with row_orig, a tile with a run of equal depths longer than kTieRun (or with one depth) is sorted
    // again through global scratch (the large tiles' path): stage 1 by its original rows, stage 2 by its
    // depth bits
    int stage = 0;
    uint32_t key[RMAX];
    int32_t val[RMAX];
    uint32_t off[RMAX];
    if (nt <= kCap) {
        // wave w holds list entries [w Q, w Q + Q), Q a whole number of 64-entry rounds
        const int Q = ((nt + kWaves - 1) / kWaves + 63) & ~63;
        const int R = Q >> 6;
        const int wb = wave * Q;
#pragma unroll
        for (int r = 0; r < RMAX; r++) {
            const int i = wb + r * 64 + lane;
            val[r] = (r < R && i < nt) ? seg[i] : 0;
        }
        const uint32_t* const dk = sdepth + start;
        uint32_t a = ~0u, o = 0u;
#pragma unroll
        for (int r = 0; r < RMAX; r++) {
            const bool valid = r < R && wb + r * 64 + lane < nt;
            key[r] = valid ? dk[wb + r * 64 + lane] : 0u;
            if (valid) {
                a &= key[r];
                o |= key[r];
            }
        }
        const uint32_t diff = block_key_diff(a, o, s_and, s_or);
        if (diff == 0u && !by_orig) return;  // one depth: the index order stands
        if (diff == 0u) stage = 1;  // (one run: by original row alone)
        for (int p = 0; p < 4; p++) {
            const int shift = 8 * p;
            if (((diff >> shift) & 255u) == 0u) continue;  // uniform: every key has this byte
#pragma unroll
            for (int w = 0; w < kWaves; w++) s_woff[w][tid] = 0;
            __syncthreads();
            wave_rank_byte<RMAX>(key, R, wb, nt, shift, s_woff[wave], off);
            __syncthreads();
            {
                uint32_t tot = 0;
#pragma unroll
                for (int w = 0; w < kWaves; w++) tot += s_woff[w][tid];
                uint32_t all = 0;
                (void)wave_starts(s_woff, block_excl_scan_u32(tot, s_wave, &all));
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                if (r < R && wb + r * 64 + lane < nt) {
                    const uint32_t pos = s_woff[wave][(key[r] >> shift) & 255u] + off[r];
                    s_key[pos] = key[r];
                    s_val[pos] = val[r];
                }
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                const int i = wb + r * 64 + lane;
                if (r < R && i < nt) {
                    key[r] = s_key[i];
                    val[r] = s_val[i];
                }
            }
            __syncthreads();
        }
        if (by_orig && stage == 0) {
            // equal depths are adjacent now: each key against the one before it, from the lane below (DPP
            // wave shift) or, for lane 0, the wave's previous round
            int tie = 0;
            uint32_t carry = (wb > 0 && wb <= nt) ? s_key[wb - 1] : 0u;  // the key before the wave's first
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                if (r >= R) break;  // uniform
                const int i = wb + r * 64 + lane;
                const uint32_t prev = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                    static_cast<int>(carry), static_cast<int>(key[r]), 0x138, 0xf, 0xf, false));  // wave_shr:1
                if (i < nt && i > 0) tie |= prev == key[r];
                carry = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key[r]), 63));
            }
            if (__syncthreads_or(tie)) {
                // the runs starting at this thread's entries (s_key holds the sorted keys): lengths, a byte
                // per round
                uint64_t runs = 0;
                int long_run = 0;
#pragma unroll
                for (int r = 0; r < RMAX; r++) {
                    const int i = wb + r * 64 + lane;
                    if (r < R && i < nt) {
                        const int32_t len = tie_run_end(s_key, i, nt) - i;
                        long_run |= len > kTieRun;
                        runs |= static_cast<uint64_t>(len > kTieRun ? 0 : len) << (8 * r);
                    }
                }
                if (__syncthreads_or(long_run)) {
                    stage = 1;  // (the whole tile again, from the values as loaded: any order will do)
                } else {
                    // the thread at a run's start replaces its keys (all equal) with the entries' original
                    // rows and sorts them with the values
#pragma unroll
                    for (int r = 0; r < RMAX; r++) {
                        const int i = wb + r * 64 + lane;
                        const int len = static_cast<int>((runs >> (8 * r)) & 255u);
                        if (len == 0) continue;
                        for (int m = i; m < i + len; m++) s_key[m] = orig_of(s_val[m]);
                        for (int m = i + 1; m < i + len; m++) {
                            const uint32_t km = s_key[m];
                            const int32_t vm = s_val[m];
                            int q = m;
                            for (; q > i && s_key[q - 1] > km; q--) {
                                s_key[q] = s_key[q - 1];
                                s_val[q] = s_val[q - 1];
                            }
                            s_key[q] = km;
                            s_val[q] = vm;
                        }
                    }
                    __syncthreads();
#pragma unroll
                    for (int r = 0; r < RMAX; r++) {
                        const int i = wb + r * 64 + lane;
                        if (r < R && i < nt) val[r] = s_val[i];
                    }
                }
            }
        }
        if (stage == 0) {
#pragma unroll
            for (int r = 0; r < RMAX; r++) {
                const int i = wb + r * 64 + lane;
                if (r < R && i < nt) seg[i] = val[r];
            }
            return;
        }
    }
    {
        // a tile of more than kCap entries (or one sorted again by original row): the keys go to sk0, then
        // each pass moves (key, value) between (sk0, vals) and (sk1, sv) over the tile's range, chunk by
        // chunk in list order
        uint32_t* src_k = sk0 + start;
        int32_t* src_v = seg;
        uint32_t* dst_k = sk1 + start;
        int32_t* dst_v = sv + start;
        uint32_t todo = 0u;
        if (stage == 0) {
            uint32_t a = ~0u, o = 0u;
            for (int32_t i = tid; i < nt; i += kThreads) {
                const uint32_t k = sdepth[start + i];
                sk0[start + i] = k;
                a &= k;
                o |= k;
            }
            todo = block_key_diff(a, o, s_and, s_or);  // (its barrier also orders the sk0 stores)
            if (todo == 0u && by_orig) stage = 1;
        }
        // (chunks of half the LDS path's rounds: this path's registers stay within the LDS path's)
        constexpr int kRG = RMAX / 2 > 0 ? RMAX / 2 : 1;
        constexpr int kChunk = kWaves * 64 * kRG;
        constexpr int kPerWave = kChunk / kWaves;
        for (;;) {
            if (stage > 0) {
                // the keys (scratch) replaced: 1 the entries' original rows, 2 their depth bits again
                uint32_t a = ~0u, o = 0u;
                for (int32_t i = tid; i < nt; i += kThreads) {
                    const uint32_t k = stage == 1 ? orig_of(src_v[i]) : depth_of(src_v[i]);
                    src_k[i] = k;
                    a &= k;
                    o |= k;
                }
                todo = block_key_diff(a, o, s_and, s_or);  // (orders the key stores)
            }
            for (int p = 0; p < 4; p++) {
                const int shift = 8 * p;
                if (((todo >> shift) & 255u) == 0u) continue;  // uniform
                s_base[tid] = 0;
                __syncthreads();
                for (int32_t i = tid; i < nt; i += kThreads) atomicAdd(&s_base[(src_k[i] >> shift) & 255u], 1u);
                __syncthreads();
                {
                    uint32_t all = 0;
                    const uint32_t b = block_excl_scan_u32(s_base[tid], s_wave, &all);
                    s_base[tid] = b;  // every thread has read its own digit's count above
                }
                __syncthreads();
                for (int32_t c0 = 0; c0 < nt; c0 += kChunk) {  // uniform
                    const int cn = static_cast<int>(min<int32_t>(kChunk, nt - c0));
                    const int wb = wave * kPerWave;
#pragma unroll
                    for (int r = 0; r < kRG; r++) {
                        const int i = wb + r * 64 + lane;
                        key[r] = i < cn ? src_k[c0 + i] : 0u;
                        val[r] = i < cn ? src_v[c0 + i] : 0;
                    }
#pragma unroll
                    for (int w = 0; w < kWaves; w++) s_woff[w][tid] = 0;
                    __syncthreads();
                    wave_rank_byte<kRG>(key, kRG, wb, cn, shift, s_woff[wave], off);
                    __syncthreads();
                    s_base[tid] = wave_starts(s_woff, s_base[tid]);
                    __syncthreads();
#pragma unroll
                    for (int r = 0; r < kRG; r++) {
                        if (wb + r * 64 + lane < cn) {
                            const uint32_t pos = s_woff[wave][(key[r] >> shift) & 255u] + off[r];
                            dst_k[pos] = key[r];
                            dst_v[pos] = val[r];
                        }
                    }
                    __syncthreads();  // s_woff is cleared for the next chunk; the next pass reads these stores
                }
                uint32_t* tk = src_k;
                src_k = dst_k;
                dst_k = tk;
                int32_t* tv = src_v;
                src_v = dst_v;
                dst_v = tv;
            }
            if (!by_orig || stage == 2) break;
            if (stage == 1) {
                stage = 2;
                continue;
            }
            // stage 0, as in LDS: runs of up to kTieRun fixed by the thread at their start (the original rows
            // in dst_k, the keys in src_k left for the other threads' run search), longer ones sorted again
            int tie = 0, long_run = 0;
            for (int32_t i = tid; i < nt; i += kThreads) {
                const int32_t len = tie_run_end(src_k, i, nt) - i;
                tie |= len > 0;
                long_run |= len > kTieRun;
            }
            if (__syncthreads_or(long_run)) {
                stage = 1;
                continue;
            }
            if (__syncthreads_or(tie)) {
                for (int32_t i = tid; i < nt; i += kThreads) {
                    const int32_t e = tie_run_end(src_k, i, nt);
                    for (int32_t m = i; m < e; m++) dst_k[m] = orig_of(src_v[m]);
                    for (int32_t m = i + 1; m < e; m++) {
                        const uint32_t km = dst_k[m];
                        const int32_t vm = src_v[m];
                        int32_t q = m;
                        for (; q > i && dst_k[q - 1] > km; q--) {
                            dst_k[q] = dst_k[q - 1];
                            src_v[q] = src_v[q - 1];
                        }
                        dst_k[q] = km;
                        src_v[q] = vm;
                    }
                }
                __syncthreads();  // the copy below reads other threads' runs
            }
            break;
        }
        if (src_v != seg)
            for (int32_t i = tid; i < nt; i += kThreads) seg[i] = src_v[i];
    }
}

} // namespace

size_t sort_scratch_bytes(int64_t n) {
    const int64_t tiles = std::max<int64_t>(1, tiles_for(n));
    return sizeof(uint32_t) * static_cast<size_t>(kHeaderWords + 2 * tiles * kBins);
}

uint32_t* sort_error_flag(void* scratch) {
    return static_cast<uint32_t*>(scratch) + 2 * kMaxPasses * kBins + kMaxPasses;
}

int radix_sort(uint64_t* keys_a, int32_t* vals_a, uint64_t* keys_b, int32_t* vals_b, int64_t n, uint32_t key_bits,
               void* scratch, hipStream_t s, bool clear_err, const int64_t* n_dev) {
    return radix_sort_ab(keys_a, vals_a, keys_b, vals_b, n, key_bits, scratch, clear_err, s, n_dev);
}

int radix_sort(uint32_t* keys_a, int32_t* vals_a, uint32_t* keys_b, int32_t* vals_b, int64_t n, uint32_t key_bits,
               void* scratch, hipStream_t s, bool clear_err, const int64_t* n_dev, bool no_wait) {
    return radix_sort_ab(keys_a, vals_a, keys_b, vals_b, n, key_bits, scratch, clear_err, s, n_dev, false, nullptr,
                         nullptr, no_wait);
}

int radix_sort(uint16_t* keys_a, int32_t* vals_a, uint16_t* keys_b, int32_t* vals_b, int64_t n, uint32_t key_bits,
               void* scratch, hipStream_t s, bool clear_err, const int64_t* n_dev) {
    return radix_sort_ab(keys_a, vals_a, keys_b, vals_b, n, key_bits, scratch, clear_err, s, n_dev);
}

int radix_sort_positions(uint16_t* keys_a, int32_t* vals_a, uint16_t* keys_b, int32_t* vals_b, int64_t n,
                         uint32_t key_bits, void* scratch, hipStream_t s, bool clear_err, const int64_t* n_dev,
                         uint32_t* x_a, uint32_t* x_b, bool no_wait) {
    return radix_sort_ab(keys_a, vals_a, keys_b, vals_b, n, key_bits, scratch, clear_err, s, n_dev, true, x_a, x_b,
                         no_wait);
}

int radix_sort_positions(uint32_t* keys_a, int32_t* vals_a, uint32_t* keys_b, int32_t* vals_b, int64_t n,
                         uint32_t key_bits, void* scratch, hipStream_t s, bool clear_err, const int64_t* n_dev,
                         uint32_t* x_a, uint32_t* x_b, bool no_wait) {
    return radix_sort_ab(keys_a, vals_a, keys_b, vals_b, n, key_bits, scratch, clear_err, s, n_dev, true, x_a, x_b,
                         no_wait);
}

constexpr int kDepthSortRounds = 8;

void tile_depth_sort(const int32_t* offsets, int n_tiles, int64_t n_isects, const int64_t* n_dev,
                     const int32_t* tile_order, int32_t* vals, const uint32_t* sdepth, uint32_t* scratch_k0,
                     uint32_t* scratch_k1, int32_t* scratch_v, hipStream_t s, int32_t* order_out,
                     uint32_t* max_count, const TieOrder* ties) {
    if (n_tiles <= 0 || (!order_out && !n_dev && n_isects <= 1)) return;
    if (ties && (!ties->id_of || !ties->row_orig || !ties->splats))
        throw std::invalid_argument("tile_depth_sort: incomplete tie order arguments");
    hipLaunchKernelGGL(k_tile_depth_sort<kDepthSortRounds>, dim3(n_tiles + (order_out ? 1 : 0)), dim3(kThreads), 0,
                       s, offsets, n_tiles, static_cast<int32_t>(n_isects), n_dev, tile_order, vals, sdepth,
                       scratch_k0, scratch_k1, scratch_v, order_out, max_count, ties ? ties->id_of : nullptr,
                       ties ? ties->row_orig : nullptr, ties ? ties->splats : nullptr);
}

void radix_sort_into(const uint64_t* keys, const int32_t* vals, uint64_t* keys_out, int32_t* vals_out,
                     uint64_t* keys_tmp, int32_t* vals_tmp, int64_t n, uint32_t key_bits, void* scratch,
                     hipStream_t s) {
    const int passes = static_cast<int>((std::min<uint32_t>(key_bits, 64) + 7) / 8);
    // the last pass, passes - 1, writes side[(passes - 1) & 1]: make that side the output
    uint64_t* const sk[2] = {(passes & 1) ? keys_out : keys_tmp, (passes & 1) ? keys_tmp : keys_out};
    int32_t* const sv[2] = {(passes & 1) ? vals_out : vals_tmp, (passes & 1) ? vals_tmp : vals_out};
    (void)radix_sort_t<uint64_t>(keys, vals, sk, sv, n, key_bits, scratch, true, s, nullptr);
}

} // namespace sxk
