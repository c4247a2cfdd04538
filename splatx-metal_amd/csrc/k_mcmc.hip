// k_mcmc.hip — MCMC refine on the device (gfx950): the host orchestration of Trainer::mcmc_refine
// (Sources/SplatXCore/Trainer.cpp:1273-1435) as kernels over the SoA arena, so a refine no longer
// moves the arena to the host and back.
//
//   k_mc_activate   sigmoid_f32 of every live logit (Trainer.cpp:430, 455-459) + dead flags
//                   (:1288-1291) + NaN detection for the multinomial's weight check (:1205-1206)
//   k_mc_compact    stable dead / alive index lists from an int64 scan of the flags
//   k_mc_cdf        the multinomial's running f64 sum (:1202-1208), bit-identical to the
//                   left-to-right accumulation but computed by a whole workgroup (see below)
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
// leave a even. These maps compose associatively, so a workgroup scans 8192 of them at a time;
// the first element whose sum leaves the binade (a >= 2^53) is recomputed with a plain f64 add,
// and the scan restarts after it in the new binade. The result equals the sequential loop bit for
// bit; there are only as many restarts as binades crossed (about 20-40 for millions of weights).
constexpr int kCdfThreads = 1024;
constexpr int kCdfPer = 8;
constexpr int kCdfChunk = kCdfThreads * kCdfPer;
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

__global__ void __launch_bounds__(kCdfThreads) k_mc_cdf(const float* __restrict__ w_all,
                                                        const int32_t* __restrict__ gather, int64_t n,
                                                        double* __restrict__ cdf, double* __restrict__ total,
                                                        uint32_t* __restrict__ err) {
    __shared__ ParMap s_wave[kCdfThreads / 64];
    __shared__ unsigned long long s_cross;
    __shared__ double s_next;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    double s = 0.0;  // running sum before element `start` (uniform)
    int64_t start = 0;
    bool bad = false;
    while (start < n) {
        if (t == 0) s_cross = static_cast<unsigned long long>(kNone);
        const int64_t base = start + static_cast<int64_t>(t) * kCdfPer;
        const int64_t chunk_end = start + kCdfChunk < n ? start + kCdfChunk : n;
        float w[kCdfPer];
#pragma unroll
        for (int j = 0; j < kCdfPer; j++) {
            const int64_t i = base + j;
            w[j] = 0.0f;
            if (i < chunk_end) {
                w[j] = w_all[gather ? gather[i] : i];
                bad |= !(w[j] >= 0.0f);
            }
        }
        if (s == 0.0) {
            // leading zero weights: the sum stays 0; the first positive weight is the sum itself
            __syncthreads();
#pragma unroll
            for (int j = 0; j < kCdfPer; j++)
                if (base + j < chunk_end && w[j] > 0.0f) {
                    atomicMin(&s_cross, static_cast<unsigned long long>(base + j));
                    break;
                }
            __syncthreads();
            const int64_t c = static_cast<int64_t>(s_cross);
#pragma unroll
            for (int j = 0; j < kCdfPer; j++) {
                const int64_t i = base + j;
                if (i < chunk_end && i < c) cdf[i] = 0.0;
                if (i == c) {
                    cdf[i] = static_cast<double>(w[j]);
                    s_next = static_cast<double>(w[j]);
                }
            }
            __syncthreads();
            if (c != kNone) {
                s = s_next;
                start = c + 1;
            } else {
                start = chunk_end;
            }
            __syncthreads();
            continue;
        }
        const uint64_t sb = static_cast<uint64_t>(__double_as_longlong(s));
        const int E = static_cast<int>((sb >> 52) & 0x7ffu) - 1023;
        const uint64_t a0 = (sb & ((1ull << 52) - 1u)) | (1ull << 52);
        const uint32_t p0 = static_cast<uint32_t>(a0 & 1u);
        const double u = __longlong_as_double(static_cast<long long>(static_cast<uint64_t>(E - 52 + 1023) << 52));
        ParMap loc[kCdfPer];
        ParMap acc = pm_identity();
#pragma unroll
        for (int j = 0; j < kCdfPer; j++) {
            acc = pm_compose(acc, pm_of(w[j], E));
            loc[j] = acc;
        }
        ParMap x = acc;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const ParMap y = pm_shfl_up(x, off);
            if (lane >= off) x = pm_compose(y, x);
        }
        if (lane == 63) s_wave[wv] = x;
        const ParMap lanes_before = pm_shfl_up(x, 1);
        __syncthreads();
        ParMap pre = pm_identity();
        for (int k = 0; k < wv; k++) pre = pm_compose(pre, s_wave[k]);
        if (lane > 0) pre = pm_compose(pre, lanes_before);
        uint64_t a[kCdfPer];
#pragma unroll
        for (int j = 0; j < kCdfPer; j++) {
            const ParMap T = pm_compose(pre, loc[j]);
            a[j] = a0 + (p0 ? T.d1 : T.d0);
        }
#pragma unroll
        for (int j = 0; j < kCdfPer; j++)
            if (base + j < chunk_end && a[j] >= kTwo53) {
                atomicMin(&s_cross, static_cast<unsigned long long>(base + j));
                break;
            }
        __syncthreads();
        const int64_t c = static_cast<int64_t>(s_cross);
#pragma unroll
        for (int j = 0; j < kCdfPer; j++) {
            const int64_t i = base + j;
            if (i < chunk_end && i < c) cdf[i] = static_cast<double>(a[j]) * u;
            if (i == c) {
                // the element that leaves the binade: a plain f64 add on the exact previous sum
                const uint64_t a_prev = j > 0 ? a[j > 0 ? j - 1 : 0] : a0 + (p0 ? pre.d1 : pre.d0);
                const double sc = static_cast<double>(a_prev) * u + static_cast<double>(w[j]);
                cdf[i] = sc;
                s_next = sc;
            }
        }
        if (c == kNone) {
            ParMap all = pm_identity();
            for (int k = 0; k < kCdfThreads / 64; k++) all = pm_compose(all, s_wave[k]);
            s = static_cast<double>(a0 + (p0 ? all.d1 : all.d0)) * u;
            start = chunk_end;
        } else {
            __syncthreads();
            s = s_next;
            start = c + 1;
        }
        __syncthreads();
    }
    if (t == 0) *total = s;
    if (bad) atomicOr(err, kMcErrWeights);
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

void mc_cdf(const float* w, const int32_t* gather, int64_t n, double* cdf, double* total, uint32_t* err,
            hipStream_t s) {
    hipLaunchKernelGGL(k_mc_cdf, dim3(1), dim3(kCdfThreads), 0, s, w, gather, n, cdf, total, err);
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
