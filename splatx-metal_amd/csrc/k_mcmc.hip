// k_mcmc.hip — MCMC refine on the device (gfx950): the host orchestration of Trainer::mcmc_refine
// (Sources/SplatXCore/Trainer.cpp:1273-1435) as kernels over the SoA arena, so a refine no longer
// moves the arena to the host and back.
//
//   k_mc_activate   sigmoid_f32 of every live logit (Trainer.cpp:430, 455-459) + dead flags
//                   (:1288-1291) + NaN detection for the multinomial's weight check (:1205-1206)
//   k_mc_compact    stable dead / alive index lists from an int64 scan of the flags
//   k_cdf_*         the multinomial's running f64 sum (:1202-1208), bit-identical to the
//                   left-to-right accumulation but computed as a scan (see below)
//   k_mc_mt_gen     std::mt19937_64 words: the 312-word twist in LDS, one workgroup
//   k_mc_search     u = (r >> 11) * 2^-53 * acc, upper_bound on the cdf, clamp (:1211-1216),
//                   source index and bincount (:1238-1240)
//   k_mc_reloc      Eq.9 of every draw (the relocation kernel, :1243-1257 inputs) and the back
//                   conversion logit_f32 / log (:1313-1321), into temporaries
//   k_mc_apply      source rows <- the new opacity / scale (duplicated sources write equal values)
//   k_mc_copy_rows  destination row <- updated source row, every parameter group (:1323-1330)
//   k_mc_zero_rows  Adam moments of a row list <- 0 (:1422-1435)
//   k_mc_noise      mcmc_inject_noise (:1400-1418) over the SoA arena
#include <hip/hip_runtime.h>

#include "sx_dev_bwd.h"
#include "sx_philox.h"
#include "sx_step.h"
#include "sx_mcmc.h"

namespace sxk {
namespace {

constexpr int kBlock = 256;
inline int grid_for(int64_t n, int per = kBlock) { return static_cast<int>((n + per - 1) / per); }

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + sxm::expf_(-x)); }

__global__ void __launch_bounds__(kBlock) k_mc_activate(const float* __restrict__ logits, int n, float min_opacity,
                                                        float* __restrict__ op_act, int32_t* __restrict__ dead,
                                                        uint32_t* __restrict__ err) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const float o = sigmoid_ref(logits[i]);
    op_act[i] = o;
    if (dead) dead[i] = (o <= min_opacity) ? 1 : 0;
    if (!(o >= 0.0f)) atomicOr(err, kMcErrWeights);
}

// dead rows in ascending order at [0, n_dead), alive rows in ascending order (the reference's
// push_back order, Trainer.cpp:1290-1291); cum = inclusive scan of the dead flags
__global__ void __launch_bounds__(kBlock) k_mc_compact(const int32_t* __restrict__ dead, const int64_t* __restrict__ cum,
                                                       int n, int32_t* __restrict__ dead_list,
                                                       int32_t* __restrict__ alive_list) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const int64_t c = cum[i];
    if (dead[i]) dead_list[c - 1] = i;
    else alive_list[i - c] = i;
}

// ---- the running f64 sum ----------------------------------------------------------------------
// s_0 = 0, s_i = RN(s_{i-1} + w_i) over float weights w_i >= 0. While s stays in one binade
// [2^E, 2^(E+1)) with ulp u = 2^(E-52), s = a*u for an integer a in [2^52, 2^53) and
// RN(a*u + w) = (a + r)*u, where w = q*u + f (0 <= f < u) and r = q below the half-ulp, q + 1
// above it, and at an exact half the choice that leaves a + r even. So each element is a map on
// the parity of a: non-tie elements add r and flip parity by r's low bit, ties add q or q + 1 and
// leave a even. These maps compose associatively, which makes the left-to-right sum a scan:
//   A  chunk sums (4096 weights per workgroup, any order: only used to predict)
//   B  predicted binade of every chunk from the approximate prefix, or "uncertain" near a power of 2
//   C  per chunk, the composed map of its weights in the predicted binade
//   D  one workgroup walks the chunks in order with the exact running sum: a chunk whose start lies
//      in the predicted binade and whose composed map keeps a < 2^53 advances in O(1); any other
//      chunk (the first, those that cross a binade, wrong predictions) is summed by the whole
//      workgroup element-exactly, restarting after each element that leaves the binade
//   E  per chunk not summed in D, the exact start value + an in-chunk scan of the maps -> cdf.
// The result equals the sequential loop bit for bit whatever the predictions were (D checks them);
// they only decide how many chunks take the slow path (those that cross one of the 20-40 binades).
constexpr int kCdfChunk = 4096;
constexpr int kCdfBlock = 256;
constexpr int kCdfPerT = kCdfChunk / kCdfBlock;  // 16
constexpr int kWalkThreads = 512;
constexpr int kWalkPer = kCdfChunk / kWalkThreads;  // 4
constexpr int kWalkTile = kWalkThreads;  // chunk records staged in LDS at a time (one per thread)
constexpr int kUncertain = -100000;
constexpr uint64_t kSat = 1ull << 62;
constexpr uint64_t kTwo53 = 1ull << 53;
constexpr int64_t kNone = INT64_MAX;

struct ParMap {
    uint64_t d0, d1;  // increment of a for incoming parity 0 / 1 (saturating at 2^62)
    uint32_t o;       // bit b: outgoing parity for incoming parity b
};

__device__ __forceinline__ ParMap pm_identity() { return ParMap{0, 0, 2u}; }

__device__ __forceinline__ uint64_t sat_add(uint64_t a, uint64_t b) {
    const uint64_t s = a + b;  // a, b <= 2^62: no wrap
    return s < kSat ? s : kSat;
}

// first A, then B
__device__ __forceinline__ ParMap pm_compose(const ParMap& A, const ParMap& B) {
    const uint32_t a0 = A.o & 1u, a1 = (A.o >> 1) & 1u;
    ParMap r;
    r.d0 = sat_add(A.d0, a0 ? B.d1 : B.d0);
    r.d1 = sat_add(A.d1, a1 ? B.d1 : B.d0);
    r.o = ((B.o >> a0) & 1u) | (((B.o >> a1) & 1u) << 1);
    return r;
}

// the map of adding weight w in the binade of exponent E
__device__ __forceinline__ ParMap pm_of(float w, int E) {
    const uint32_t b = __float_as_uint(w);
    const uint32_t ex = (b >> 23) & 0xffu, man = b & 0x7fffffu;
    const uint32_t m = ex ? (man | 0x800000u) : man;  // w = m * 2^x
    const int x = ex ? static_cast<int>(ex) - 150 : -149;
    const int k = x - (E - 52);                        // w / u = m * 2^k
    uint64_t q = 0;
    int cls = 0;  // 0: f < u/2, 1: f > u/2, 2: f == u/2
    if (m != 0) {
        if (k >= 0) {
            q = k > 38 ? kSat : (static_cast<uint64_t>(m) << k);
        } else if (-k < 25) {
            const int sh = -k;
            q = m >> sh;
            const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
            cls = rem > half ? 1 : (rem == half ? 2 : 0);
        }  // else 0 < w < u/2: q = 0, below
    }
    ParMap t;
    if (cls == 2) {
        const uint64_t qb = q & 1u;
        t.d0 = q + qb;
        t.d1 = q + 1u - qb;
        t.o = 0u;
    } else {
        const uint64_t r = q + static_cast<uint64_t>(cls);
        t.d0 = t.d1 = r;
        const uint32_t rb = static_cast<uint32_t>(r & 1u);
        t.o = rb | ((rb ^ 1u) << 1);
    }
    return t;
}

__device__ __forceinline__ ParMap pm_shfl_up(const ParMap& v, int delta) {
    ParMap r;
    r.d0 = __shfl_up(v.d0, delta, 64);
    r.d1 = __shfl_up(v.d1, delta, 64);
    r.o = __shfl_up(v.o, delta, 64);
    return r;
}

__device__ __forceinline__ int exponent_of(double s) {
    return static_cast<int>((static_cast<uint64_t>(__double_as_longlong(s)) >> 52) & 0x7ffu) - 1023;
}
__device__ __forceinline__ uint64_t units_of(double s) {  // s / ulp(s) for a normal s
    const uint64_t sb = static_cast<uint64_t>(__double_as_longlong(s));
    return (sb & ((1ull << 52) - 1u)) | (1ull << 52);
}
__device__ __forceinline__ double ulp_of_binade(int E) {
    return __longlong_as_double(static_cast<long long>(static_cast<uint64_t>(E - 52 + 1023) << 52));
}

__device__ __forceinline__ float load_w(const float* __restrict__ w_all, const int32_t* __restrict__ gather,
                                        int64_t i) {
    return w_all[gather ? gather[i] : i];
}

// Ordered exclusive scan of one map per thread over a workgroup of NT threads; returns the
// composition of the maps of all lower threads and sets `all` to the workgroup's total.
template <int NT>
__device__ __forceinline__ ParMap wg_exclusive_scan(ParMap x, ParMap* s_wave, ParMap& all) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const ParMap y = pm_shfl_up(x, off);
        if (lane >= off) x = pm_compose(y, x);
    }
    const ParMap lanes_before = pm_shfl_up(x, 1);
    if (lane == 63) s_wave[wv] = x;
    __syncthreads();
    ParMap pre = pm_identity();
    all = pm_identity();
#pragma unroll
    for (int k = 0; k < NT / 64; k++) {
        if (k < wv) pre = pm_compose(pre, s_wave[k]);
        all = pm_compose(all, s_wave[k]);
    }
    if (lane > 0) pre = pm_compose(pre, lanes_before);
    return pre;
}

// A: chunk sums in f64 (any order) + the NaN check of the multinomial
__global__ void __launch_bounds__(kCdfBlock) k_cdf_chunk_sum(const float* __restrict__ w_all,
                                                             const int32_t* __restrict__ gather, int64_t n,
                                                             double* __restrict__ chunk_sum,
                                                             uint32_t* __restrict__ err) {
    __shared__ double s_red[kCdfBlock / 64];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kCdfChunk;
    double acc = 0.0;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < kCdfPerT; j++) {
        const int64_t i = base + j * kCdfBlock + threadIdx.x;
        if (i < n) {
            const float w = load_w(w_all, gather, i);
            bad |= !(w >= 0.0f);
            acc += static_cast<double>(w);
        }
    }
    if (bad) atomicOr(err, kMcErrWeights);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
#pragma unroll
        for (int k = 0; k < kCdfBlock / 64; k++) t += s_red[k];
        chunk_sum[blockIdx.x] = t;
    }
}

// B: approximate prefix of the chunk sums -> predicted binade of each chunk (kUncertain when the
// chunk's approximate range comes within a relative 2^-20 of a power of two, or starts at 0)
__global__ void __launch_bounds__(kWalkThreads) k_cdf_predict(const double* __restrict__ chunk_sum, int n_chunks,
                                                              int32_t* __restrict__ chunk_E) {
    __shared__ double s_v[kWalkThreads];
    double carry = 0.0;
    for (int tile = 0; tile < n_chunks; tile += kWalkThreads) {
        const int c = tile + static_cast<int>(threadIdx.x);
        const double v = c < n_chunks ? chunk_sum[c] : 0.0;
        s_v[threadIdx.x] = v;
        __syncthreads();
        for (int off = 1; off < kWalkThreads; off <<= 1) {  // inclusive Hillis-Steele scan
            const double y = threadIdx.x >= static_cast<unsigned>(off) ? s_v[threadIdx.x - off] : 0.0;
            __syncthreads();
            s_v[threadIdx.x] += y;
            __syncthreads();
        }
        const double incl = carry + s_v[threadIdx.x];
        const double excl = incl - v;
        if (c < n_chunks) {
            const double lo = excl * (1.0 - 0x1.0p-20), hi = incl * (1.0 + 0x1.0p-20);
            const int Elo = exponent_of(lo), Ehi = exponent_of(hi);
            chunk_E[c] = (excl > 0.0 && Elo == Ehi) ? Elo : kUncertain;
        }
        carry += s_v[kWalkThreads - 1];
        __syncthreads();
    }
}

// C: composed map of each chunk in its predicted binade
__global__ void __launch_bounds__(kCdfBlock) k_cdf_chunk_map(const float* __restrict__ w_all,
                                                             const int32_t* __restrict__ gather, int64_t n,
                                                             const int32_t* __restrict__ chunk_E,
                                                             uint64_t* __restrict__ map_d0,
                                                             uint64_t* __restrict__ map_d1,
                                                             uint32_t* __restrict__ map_o) {
    __shared__ ParMap s_wave[kCdfBlock / 64];
    const int E = chunk_E[blockIdx.x];
    if (E == kUncertain) return;  // uniform over the workgroup
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kCdfChunk + static_cast<int64_t>(threadIdx.x) * kCdfPerT;
    ParMap acc = pm_identity();
#pragma unroll
    for (int j = 0; j < kCdfPerT; j++) {
        const int64_t i = base + j;
        if (i < n) acc = pm_compose(acc, pm_of(load_w(w_all, gather, i), E));
    }
    ParMap all;
    (void)wg_exclusive_scan<kCdfBlock>(acc, s_wave, all);
    if (threadIdx.x == 0) {
        map_d0[blockIdx.x] = all.d0;
        map_d1[blockIdx.x] = all.d1;
        map_o[blockIdx.x] = all.o;
    }
}

// The element-exact sum of [begin, end) by the whole walk workgroup, starting from the exact s;
// writes cdf[begin, end) and returns the sum after end - 1. Uniform call (contains barriers).
__device__ double cdf_range_exact(const float* __restrict__ w_all, const int32_t* __restrict__ gather,
                                  int64_t begin, int64_t end, double s, double* __restrict__ cdf,
                                  ParMap* s_wave, unsigned long long* s_cross, double* s_next) {
    const int t = threadIdx.x;
    int64_t start = begin;
    while (start < end) {
        __syncthreads();
        if (t == 0) *s_cross = static_cast<unsigned long long>(kNone);
        const int64_t base = start + static_cast<int64_t>(t) * kWalkPer;
        float w[kWalkPer];
#pragma unroll
        for (int j = 0; j < kWalkPer; j++) w[j] = base + j < end ? load_w(w_all, gather, base + j) : 0.0f;
        if (s == 0.0) {
            // leading zero weights: the sum stays 0; the first positive weight is the sum itself
            __syncthreads();
            int64_t first = kNone;
#pragma unroll
            for (int j = kWalkPer - 1; j >= 0; j--)
                if (base + j < end && w[j] > 0.0f) first = base + j;
            if (first != kNone) atomicMin(s_cross, static_cast<unsigned long long>(first));
            __syncthreads();
            const int64_t c = static_cast<int64_t>(*s_cross);
#pragma unroll
            for (int j = 0; j < kWalkPer; j++) {
                const int64_t i = base + j;
                if (i < end && i < c) cdf[i] = 0.0;
                if (i == c) {
                    cdf[i] = static_cast<double>(w[j]);
                    *s_next = static_cast<double>(w[j]);
                }
            }
            __syncthreads();
            if (c != kNone) {
                s = *s_next;
                start = c + 1;
            } else {
                start = end;  // every weight of the range is zero; the range covers all threads' loads
            }
            continue;
        }
        const int E = exponent_of(s);
        const uint64_t a0 = units_of(s);
        const uint32_t p0 = static_cast<uint32_t>(a0 & 1u);
        const double u = ulp_of_binade(E);
        ParMap loc[kWalkPer];
        ParMap acc = pm_identity();
#pragma unroll
        for (int j = 0; j < kWalkPer; j++) {
            acc = pm_compose(acc, pm_of(w[j], E));
            loc[j] = acc;
        }
        ParMap all;
        const ParMap pre = wg_exclusive_scan<kWalkThreads>(acc, s_wave, all);
        uint64_t a[kWalkPer];
#pragma unroll
        for (int j = 0; j < kWalkPer; j++) {
            const ParMap T = pm_compose(pre, loc[j]);
            a[j] = a0 + (p0 ? T.d1 : T.d0);
        }
        int64_t first = kNone;
#pragma unroll
        for (int j = kWalkPer - 1; j >= 0; j--)
            if (base + j < end && a[j] >= kTwo53) first = base + j;
        if (first != kNone) atomicMin(s_cross, static_cast<unsigned long long>(first));
        __syncthreads();
        const int64_t c = static_cast<int64_t>(*s_cross);
        const int64_t stop = start + kWalkThreads * kWalkPer < end ? start + kWalkThreads * kWalkPer : end;
#pragma unroll
        for (int j = 0; j < kWalkPer; j++) {
            const int64_t i = base + j;
            if (i < stop && i < c) cdf[i] = static_cast<double>(a[j]) * u;
            if (i == c) {
                // the element that leaves the binade: a plain f64 add on the exact previous sum
                const uint64_t a_prev = j > 0 ? a[j > 0 ? j - 1 : 0] : a0 + (p0 ? pre.d1 : pre.d0);
                const double sc = static_cast<double>(a_prev) * u + static_cast<double>(w[j]);
                cdf[i] = sc;
                *s_next = sc;
            }
        }
        if (c == kNone) {
            s = static_cast<double>(a0 + (p0 ? all.d1 : all.d0)) * u;
            start = stop;
        } else {
            __syncthreads();
            s = *s_next;
            start = c + 1;
        }
    }
    __syncthreads();
    return s;
}

// One element of the segmented scan over a tile of chunk maps: segments are runs of chunks that
// share a predicted binade; `head` is the index of the segment's first chunk.
struct SegMap {
    ParMap m;
    uint32_t flag;  // a segment starts at this element (or within the combined range)
    int head;
};

__device__ __forceinline__ SegMap seg_combine(const SegMap& A, const SegMap& B) {  // A earlier
    const ParMap c = pm_compose(A.m, B.m);
    const bool b = B.flag != 0u;  // selects, not a branch: keeps the struct in registers
    SegMap r;
    r.m.d0 = b ? B.m.d0 : c.d0;
    r.m.d1 = b ? B.m.d1 : c.d1;
    r.m.o = b ? B.m.o : c.o;
    r.flag = A.flag | B.flag;
    r.head = b ? B.head : A.head;
    return r;
}

__device__ __forceinline__ SegMap seg_shfl_up(const SegMap& v, int delta) {
    SegMap r;
    r.m = pm_shfl_up(v.m, delta);
    r.flag = __shfl_up(v.flag, delta, 64);
    r.head = __shfl_up(v.head, delta, 64);
    return r;
}

// D: the ordered walk over the chunks with the exact running sum. Per tile of kWalkTile chunks, a
// segmented scan composes the maps of each run of chunks predicted in one binade; the walk then
// advances a whole run in O(1) when the exact sum at its head lies in that binade and the run's
// total keeps a < 2^53 (so every chunk of it does), writing the runs' chunk start values in
// parallel. Otherwise it goes chunk by chunk, summing element-exactly where a chunk's own map
// cannot be applied.
__global__ void __launch_bounds__(kWalkThreads) k_cdf_walk(const float* __restrict__ w_all,
                                                           const int32_t* __restrict__ gather, int64_t n,
                                                           int n_chunks, const int32_t* __restrict__ chunk_E,
                                                           const uint64_t* __restrict__ map_d0,
                                                           const uint64_t* __restrict__ map_d1,
                                                           const uint32_t* __restrict__ map_o,
                                                           double* __restrict__ chunk_start,
                                                           uint32_t* __restrict__ walked, double* __restrict__ cdf,
                                                           double* __restrict__ total) {
    static_assert(kWalkTile == kWalkThreads, "one chunk record per thread");
    __shared__ int32_t sE[kWalkTile];
    __shared__ uint64_t sd0[kWalkTile], sd1[kWalkTile];  // each chunk's own map (parity-indexed increments)
    __shared__ uint64_t pd0[kWalkTile], pd1[kWalkTile];  // inclusive prefix from the segment head
    __shared__ uint8_t s_head[kWalkTile];
    __shared__ int32_t s_seg_end[kWalkTile];             // at a head: one past the segment's last chunk
    __shared__ SegMap s_segw[kWalkThreads / 64];
    __shared__ ParMap s_wave[kWalkThreads / 64];
    __shared__ unsigned long long s_cross;
    __shared__ double s_next;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    double s = 0.0;  // uniform
    for (int tile = 0; tile < n_chunks; tile += kWalkTile) {
        __syncthreads();
        const int cnt = n_chunks - tile < kWalkTile ? n_chunks - tile : kWalkTile;
        int E = kUncertain;
        ParMap m = pm_identity();
        if (t < cnt) {
            E = chunk_E[tile + t];
            if (E != kUncertain) m = ParMap{map_d0[tile + t], map_d1[tile + t], map_o[tile + t]};
        }
        sE[t] = E;
        sd0[t] = m.d0;
        sd1[t] = m.d1;
        __syncthreads();
        const uint32_t head = (t == 0 || t >= cnt || E == kUncertain || sE[t - 1] == kUncertain || sE[t - 1] != E)
                                  ? 1u : 0u;
        s_head[t] = static_cast<uint8_t>(head);
        SegMap x{m, head, head ? t : -1};
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const SegMap y = seg_shfl_up(x, off);
            if (lane >= off) x = seg_combine(y, x);
        }
        if (lane == 63) s_segw[wv] = x;
        __syncthreads();
        SegMap pre{pm_identity(), 0u, -1};
#pragma unroll
        for (int k = 0; k < kWalkThreads / 64; k++)
            if (k < wv) pre = seg_combine(pre, s_segw[k]);
        const SegMap incl = seg_combine(pre, x);
        pd0[t] = incl.m.d0;
        pd1[t] = incl.m.d1;
        const bool last_of_segment = (t == cnt - 1) || (t + 1 < cnt && s_head[t + 1]);
        if (t < cnt && last_of_segment) s_seg_end[incl.head] = t + 1;
        __syncthreads();
        int k = 0;
        while (k < cnt) {  // uniform
            const int c = tile + k;
            const int Ek = sE[k];
            if (Ek != kUncertain && s > 0.0 && exponent_of(s) == Ek) {
                const uint64_t a0 = units_of(s);
                const bool p1 = (a0 & 1u) != 0;
                const double u = ulp_of_binade(Ek);
                if (s_head[k]) {
                    const int j_end = s_seg_end[k];
                    const uint64_t a_end = a0 + (p1 ? pd1[j_end - 1] : pd0[j_end - 1]);
                    if (a_end < kTwo53) {
                        for (int j = k + t; j < j_end; j += kWalkThreads) {
                            const uint64_t aj = j == k ? a0 : a0 + (p1 ? pd1[j - 1] : pd0[j - 1]);
                            chunk_start[tile + j] = static_cast<double>(aj) * u;
                            walked[tile + j] = 0u;
                        }
                        s = static_cast<double>(a_end) * u;
                        k = j_end;
                        continue;
                    }
                }
                const uint64_t a = a0 + (p1 ? sd1[k] : sd0[k]);
                if (a < kTwo53) {
                    if (t == 0) {
                        chunk_start[c] = s;
                        walked[c] = 0u;
                    }
                    s = static_cast<double>(a) * u;
                    k++;
                    continue;
                }
            }
            if (t == 0) {
                chunk_start[c] = s;
                walked[c] = 1u;
            }
            const int64_t b = static_cast<int64_t>(c) * kCdfChunk;
            const int64_t e = b + kCdfChunk < n ? b + kCdfChunk : n;
            s = cdf_range_exact(w_all, gather, b, e, s, cdf, s_wave, &s_cross, &s_next);
            k++;
        }
    }
    if (t == 0) *total = s;
}

// E: the cdf of every chunk the walk advanced in O(1)
__global__ void __launch_bounds__(kCdfBlock) k_cdf_write(const float* __restrict__ w_all,
                                                         const int32_t* __restrict__ gather, int64_t n,
                                                         const int32_t* __restrict__ chunk_E,
                                                         const double* __restrict__ chunk_start,
                                                         const uint32_t* __restrict__ walked,
                                                         double* __restrict__ cdf) {
    __shared__ ParMap s_wave[kCdfBlock / 64];
    if (walked[blockIdx.x]) return;  // uniform
    const int E = chunk_E[blockIdx.x];
    const double s = chunk_start[blockIdx.x];
    const uint64_t a0 = units_of(s);
    const uint32_t p0 = static_cast<uint32_t>(a0 & 1u);
    const double u = ulp_of_binade(E);
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kCdfChunk + static_cast<int64_t>(threadIdx.x) * kCdfPerT;
    ParMap loc[kCdfPerT];
    ParMap acc = pm_identity();
#pragma unroll
    for (int j = 0; j < kCdfPerT; j++) {
        const int64_t i = base + j;
        if (i < n) acc = pm_compose(acc, pm_of(load_w(w_all, gather, i), E));
        loc[j] = acc;
    }
    ParMap all;
    const ParMap pre = wg_exclusive_scan<kCdfBlock>(acc, s_wave, all);
#pragma unroll
    for (int j = 0; j < kCdfPerT; j++) {
        const int64_t i = base + j;
        if (i < n) {
            const ParMap T = pm_compose(pre, loc[j]);
            cdf[i] = static_cast<double>(a0 + (p0 ? T.d1 : T.d0)) * u;
        }
    }
}

// ---- std::mt19937_64 ----------------------------------------------------------------------------
// Parameters of the standard engine (C++ [rand.predef]): w 64, n 312, m 156, r 31,
// a 0xB5026F5AA96619E9, tempering (u 29, d), (s 17, b), (t 37, c), l 43.
constexpr int kMtN = 312, kMtM = 156;
constexpr uint64_t kMtA = 0xB5026F5AA96619E9ull;
constexpr uint64_t kMtUpper = ~0ull << 31, kMtLower = ~kMtUpper;

__device__ __forceinline__ uint64_t mt_mix(uint64_t hi_src, uint64_t lo_src, uint64_t xm) {
    const uint64_t y = (hi_src & kMtUpper) | (lo_src & kMtLower);
    return xm ^ (y >> 1) ^ ((y & 1u) ? kMtA : 0ull);
}

__device__ __forceinline__ uint64_t mt_temper(uint64_t z) {
    z ^= (z >> 29) & 0x5555555555555555ull;
    z ^= (z << 17) & 0x71D67FFFEDA60000ull;
    z ^= (z << 37) & 0xFFF7EEE000000000ull;
    z ^= z >> 43;
    return z;
}

// The in-place twist in libstdc++'s order (k ascending): words [0,156) read only old words;
// words [156,311) read the new words k-156; word 311 reads the new words 0 and 155.
__device__ void mt_twist(uint64_t* x, int t) {
    uint64_t v = 0;
    if (t < kMtN - kMtM) v = mt_mix(x[t], x[t + 1], x[t + kMtM]);
    __syncthreads();
    if (t < kMtN - kMtM) x[t] = v;
    __syncthreads();
    if (t >= kMtN - kMtM && t < kMtN - 1) v = mt_mix(x[t], x[t + 1], x[t + kMtM - kMtN]);
    __syncthreads();
    if (t >= kMtN - kMtM && t < kMtN - 1) x[t] = v;
    __syncthreads();
    if (t == kMtN - 1) x[t] = mt_mix(x[kMtN - 1], x[0], x[kMtM - 1]);
    __syncthreads();
}

constexpr int kMtThreads = 320;

// state: x[0..311], state[312] = p. Writes the untempered words of the next n_out draws.
__global__ void __launch_bounds__(kMtThreads) k_mc_mt_gen(uint64_t* __restrict__ state, int64_t n_out,
                                                          uint64_t* __restrict__ raw) {
    __shared__ uint64_t x[kMtN];
    const int t = threadIdx.x;
    if (t < kMtN) x[t] = state[t];
    int64_t p = static_cast<int64_t>(state[kMtN]);
    __syncthreads();
    int64_t done = 0;
    while (done < n_out) {
        if (p >= kMtN) {
            mt_twist(x, t);
            p = 0;
        }
        const int64_t left = n_out - done;
        const int64_t avail = (kMtN - p) < left ? (kMtN - p) : left;
        if (t < avail) raw[done + t] = x[p + t];
        done += avail;
        p += avail;
    }
    if (t < kMtN) state[t] = x[t];
    if (t == 0) state[kMtN] = static_cast<uint64_t>(p);
}

// multinomial draw j: u in [0, acc), first index whose running sum exceeds u, clamped to n - 1
__global__ void __launch_bounds__(kBlock) k_mc_search(const uint64_t* __restrict__ raw, int64_t n_draw,
                                                      const double* __restrict__ cdf, int64_t n_w,
                                                      const double* __restrict__ total,
                                                      const int32_t* __restrict__ gather,
                                                      int32_t* __restrict__ sampled, uint32_t* __restrict__ counts) {
    const int64_t j = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (j >= n_draw) return;
    const double acc = *total;
    const double u = static_cast<double>(mt_temper(raw[j]) >> 11) * 0x1.0p-53 * acc;
    int64_t lo = 0, len = n_w;
    while (len > 0) {  // std::upper_bound
        const int64_t half = len >> 1;
        if (!(u < cdf[lo + half])) {
            lo += half + 1;
            len -= half + 1;
        } else {
            len = half;
        }
    }
    const int64_t idx = lo < n_w - 1 ? lo : n_w - 1;
    const int32_t src = gather ? gather[idx] : static_cast<int32_t>(idx);
    sampled[j] = src;
    atomicAdd(&counts[src], 1u);
}

__global__ void __launch_bounds__(kBlock) k_mc_reloc(const int32_t* __restrict__ sampled, int n_draw,
                                                     const uint32_t* __restrict__ counts,
                                                     const float* __restrict__ op_act,
                                                     const float* __restrict__ log_scales, int rows,
                                                     const float* __restrict__ binoms, int n_max, float min_opacity,
                                                     float* __restrict__ new_logit, float* __restrict__ new_log_scale,
                                                     uint32_t* __restrict__ err) {
    const int j = blockIdx.x * kBlock + threadIdx.x;
    if (j >= n_draw) return;
    const int src = sampled[j];
    const int c1 = static_cast<int>(counts[src]) + 1;
    const int ratio = c1 < n_max ? c1 : n_max;
    float coeff;
    const float nop = sxd::relocation_one(op_act[src], ratio, binoms, n_max, min_opacity, &coeff);
    if (!(nop > 0.0f && nop < 1.0f)) atomicOr(err, kMcErrLogit);
    new_logit[j] = sxm::logf_(nop / (1.0f - nop));
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const float ns = coeff * sxm::expf_(log_scales[static_cast<size_t>(k) * rows + src]);
        if (!(ns > 0.0f)) atomicOr(err, kMcErrScale);
        new_log_scale[static_cast<size_t>(j) * 3 + k] = sxm::logf_(ns);
    }
}

__global__ void __launch_bounds__(kBlock) k_mc_apply(const int32_t* __restrict__ sampled, int n_draw,
                                                     const float* __restrict__ new_logit,
                                                     const float* __restrict__ new_log_scale, float* __restrict__ logits,
                                                     float* __restrict__ log_scales, int rows) {
    const int j = blockIdx.x * kBlock + threadIdx.x;
    if (j >= n_draw) return;
    const int src = sampled[j];
    logits[src] = new_logit[j];
#pragma unroll
    for (int k = 0; k < 3; k++) log_scales[static_cast<size_t>(k) * rows + src] = new_log_scale[static_cast<size_t>(j) * 3 + k];
}

struct ColMap {
    float* p[6];
    int dim[6];
    int cols;
};

__device__ __forceinline__ float* col_ptr(const ColMap& cm, int col, int& k) {
    // group of a column by running bounds (selects, no dynamic index into the argument struct)
    const int e0 = cm.dim[0], e1 = e0 + cm.dim[1], e2 = e1 + cm.dim[2], e3 = e2 + cm.dim[3], e4 = e3 + cm.dim[4];
    if (col < e0) { k = col; return cm.p[0]; }
    if (col < e1) { k = col - e0; return cm.p[1]; }
    if (col < e2) { k = col - e1; return cm.p[2]; }
    if (col < e3) { k = col - e2; return cm.p[3]; }
    if (col < e4) { k = col - e3; return cm.p[4]; }
    k = col - e4;
    return cm.p[5];
}

// column-major over (column, row j): consecutive threads touch consecutive destination rows
__global__ void __launch_bounds__(kBlock) k_mc_copy_rows(ColMap cm, int rows, const int32_t* __restrict__ dst_list,
                                                         int dst_base, const int32_t* __restrict__ src_list, int n) {
    const int64_t t = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (t >= static_cast<int64_t>(n) * cm.cols) return;
    const int col = static_cast<int>(t / n), j = static_cast<int>(t - static_cast<int64_t>(col) * n);
    int k;
    float* p = col_ptr(cm, col, k);
    const int dst = dst_list ? dst_list[j] : dst_base + j;
    p[static_cast<size_t>(k) * rows + dst] = p[static_cast<size_t>(k) * rows + src_list[j]];
}

__global__ void __launch_bounds__(kBlock) k_mc_zero_rows(ColMap cm_m, ColMap cm_v, int rows,
                                                         const int32_t* __restrict__ row_list, int row_base, int n) {
    const int64_t t = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (t >= static_cast<int64_t>(n) * cm_m.cols) return;
    const int col = static_cast<int>(t / n), j = static_cast<int>(t - static_cast<int64_t>(col) * n);
    int k;
    float* m = col_ptr(cm_m, col, k);
    float* v = col_ptr(cm_v, col, k);
    const size_t at = static_cast<size_t>(k) * rows + (row_list ? row_list[j] : row_base + j);
    m[at] = 0.0f;
    v[at] = 0.0f;
}

// mcmc_inject_noise over rows [0, n): normals 3i..3i+2 of the Philox stream (seed, offset), then
// the perturbation of CpuKernels.cpp:969-1008 with t = 0.005, k = 100 (the PerturbInputs defaults)
__global__ void __launch_bounds__(kBlock) k_mc_noise(Arena A, int n, uint64_t seed, uint64_t offset,
                                                     float noise_scale) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const size_t R = static_cast<size_t>(A.rows);
    float mw[3], q[4], sl[3];
#pragma unroll
    for (int k = 0; k < 3; k++) mw[k] = A.p[0][k * R + i];
#pragma unroll
    for (int k = 0; k < 4; k++) q[k] = A.p[1][k * R + i];
#pragma unroll
    for (int k = 0; k < 3; k++) sl[k] = A.p[2][k * R + i];
    const float logit = A.p[3][i];
    const uint32_t n0 = 3u * static_cast<uint32_t>(i);
    const uint32_t t0 = n0 >> 2, t1 = (n0 + 2u) >> 2;
    float z0[4], z1[4];
    sx::philox_normals4(t0, seed, offset, z0);
    if (t1 != t0) sx::philox_normals4(t1, seed, offset, z1);
    float nz[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const uint32_t m = n0 + k;
        const uint32_t j = m & 3u;  // register selects (a dynamic array index would go to scratch)
        const float a = j == 0 ? z0[0] : j == 1 ? z0[1] : j == 2 ? z0[2] : z0[3];
        const float b = j == 0 ? z1[0] : j == 1 ? z1[1] : j == 2 ? z1[2] : z1[3];
        nz[k] = ((m >> 2) == t0) ? a : b;
    }
    sxd::perturb_one(mw, q, sl, logit, nz, noise_scale, 0.005f, 100.0f);
#pragma unroll
    for (int k = 0; k < 3; k++) A.p[0][k * R + i] = mw[k];
}

__global__ void __launch_bounds__(kBlock) k_mc_temper(const uint64_t* __restrict__ raw, int64_t n,
                                                      uint64_t* __restrict__ out) {
    const int64_t i = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (i < n) out[i] = mt_temper(raw[i]);
}

__global__ void __launch_bounds__(kBlock) k_fill_u32(uint32_t* __restrict__ p, uint32_t v, int64_t n) {
    const int64_t i = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (i < n) p[i] = v;
}

ColMap col_map(float* const* p, const int* dims) {
    ColMap cm{};
    cm.cols = 0;
    for (int g = 0; g < 6; g++) {
        cm.p[g] = p[g];
        cm.dim[g] = dims[g];
        cm.cols += dims[g];
    }
    return cm;
}

}  // namespace

// ---- launchers -------------------------------------------------------------------------------
void fill_u32(uint32_t* p, uint32_t v, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(n)), dim3(kBlock), 0, s, p, v, n);
}

void mc_activate(const float* logits, int n, float min_opacity, float* op_act, int32_t* dead, uint32_t* err,
                 hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_mc_activate, dim3(grid_for(n)), dim3(kBlock), 0, s, logits, n, min_opacity, op_act, dead, err);
}

void mc_compact(const int32_t* dead, const int64_t* cum, int n, int32_t* dead_list, int32_t* alive_list,
                hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_mc_compact, dim3(grid_for(n)), dim3(kBlock), 0, s, dead, cum, n, dead_list, alive_list);
}

size_t mc_cdf_scratch_bytes(int64_t n) {
    const size_t nc = static_cast<size_t>((n + kCdfChunk - 1) / kCdfChunk);
    return nc * (8 + 4 + 8 + 8 + 4 + 8 + 4) + 256;
}

void mc_cdf(const float* w, const int32_t* gather, int64_t n, double* cdf, double* total, uint32_t* err,
            void* scratch, hipStream_t s) {
    const int nc = static_cast<int>((n + kCdfChunk - 1) / kCdfChunk);
    // scratch layout: 8-byte arrays first, then the 4-byte ones
    double* chunk_sum = static_cast<double*>(scratch);
    double* chunk_start = chunk_sum + nc;
    uint64_t* d0 = reinterpret_cast<uint64_t*>(chunk_start + nc);
    uint64_t* d1 = d0 + nc;
    int32_t* chunk_E = reinterpret_cast<int32_t*>(d1 + nc);
    uint32_t* o = reinterpret_cast<uint32_t*>(chunk_E + nc);
    uint32_t* walked = o + nc;
    if (nc > 0) {
        hipLaunchKernelGGL(k_cdf_chunk_sum, dim3(nc), dim3(kCdfBlock), 0, s, w, gather, n, chunk_sum, err);
        hipLaunchKernelGGL(k_cdf_predict, dim3(1), dim3(kWalkThreads), 0, s, chunk_sum, nc, chunk_E);
        hipLaunchKernelGGL(k_cdf_chunk_map, dim3(nc), dim3(kCdfBlock), 0, s, w, gather, n, chunk_E, d0, d1, o);
    }
    hipLaunchKernelGGL(k_cdf_walk, dim3(1), dim3(kWalkThreads), 0, s, w, gather, n, nc, chunk_E, d0, d1, o,
                       chunk_start, walked, cdf, total);
    if (nc > 0)
        hipLaunchKernelGGL(k_cdf_write, dim3(nc), dim3(kCdfBlock), 0, s, w, gather, n, chunk_E, chunk_start, walked,
                           cdf);
}

void mc_mt_gen(uint64_t* state, int64_t n_out, uint64_t* raw, hipStream_t s) {
    if (n_out <= 0) return;
    hipLaunchKernelGGL(k_mc_mt_gen, dim3(1), dim3(kMtThreads), 0, s, state, n_out, raw);
}

void mc_search(const uint64_t* raw, int64_t n_draw, const double* cdf, int64_t n_w, const double* total,
               const int32_t* gather, int32_t* sampled, uint32_t* counts, hipStream_t s) {
    if (n_draw <= 0) return;
    hipLaunchKernelGGL(k_mc_search, dim3(grid_for(n_draw)), dim3(kBlock), 0, s, raw, n_draw, cdf, n_w, total, gather,
                       sampled, counts);
}

void mc_reloc(const int32_t* sampled, int n_draw, const uint32_t* counts, const float* op_act,
              const float* log_scales, int rows, const float* binoms, int n_max, float min_opacity,
              float* new_logit, float* new_log_scale, uint32_t* err, hipStream_t s) {
    if (n_draw <= 0) return;
    hipLaunchKernelGGL(k_mc_reloc, dim3(grid_for(n_draw)), dim3(kBlock), 0, s, sampled, n_draw, counts, op_act,
                       log_scales, rows, binoms, n_max, min_opacity, new_logit, new_log_scale, err);
}

void mc_apply(const int32_t* sampled, int n_draw, const float* new_logit, const float* new_log_scale, float* logits,
              float* log_scales, int rows, hipStream_t s) {
    if (n_draw <= 0) return;
    hipLaunchKernelGGL(k_mc_apply, dim3(grid_for(n_draw)), dim3(kBlock), 0, s, sampled, n_draw, new_logit,
                       new_log_scale, logits, log_scales, rows);
}

void mc_copy_rows(const Arena& A, const int* dims, const int32_t* dst_list, int dst_base, const int32_t* src_list,
                  int n, hipStream_t s) {
    if (n <= 0) return;
    const ColMap cm = col_map(A.p, dims);
    const int64_t total = static_cast<int64_t>(n) * cm.cols;
    hipLaunchKernelGGL(k_mc_copy_rows, dim3(grid_for(total)), dim3(kBlock), 0, s, cm, A.rows, dst_list, dst_base,
                       src_list, n);
}

void mc_zero_rows(const Arena& A, const int* dims, const int32_t* row_list, int row_base, int n, hipStream_t s) {
    if (n <= 0) return;
    const ColMap cm = col_map(A.m, dims), cv = col_map(A.v, dims);
    const int64_t total = static_cast<int64_t>(n) * cm.cols;
    hipLaunchKernelGGL(k_mc_zero_rows, dim3(grid_for(total)), dim3(kBlock), 0, s, cm, cv, A.rows, row_list, row_base,
                       n);
}

void mc_temper(const uint64_t* raw, int64_t n, uint64_t* out, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_mc_temper, dim3(grid_for(n)), dim3(kBlock), 0, s, raw, n, out);
}

void mc_noise(const Arena& A, int n, uint64_t seed, uint64_t offset, float noise_scale, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_mc_noise, dim3(grid_for(n)), dim3(kBlock), 0, s, A, n, seed, offset, noise_scale);
}

}  // namespace sxk
