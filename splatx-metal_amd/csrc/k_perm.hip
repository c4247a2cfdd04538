// k_perm.hip — the arena's spatial row order (gfx950).
//
// The step reads and writes its parameter rows column by column (SoA), and the rows of one cache line
// are 32 consecutive rows. In the caller's order (the reference's) the rows a camera culls are spread
// over every line, so each step streams the whole arena. Kept in the order of a Morton curve over the
// means instead, the culled rows fill whole waves, which the update skips: the executor may hold the
// live rows [0, count) in that order, with the maps between its internal rows and the caller's
// (original) rows. Every result stays the caller's: depth first, the emit runs in original order (so
// the stable depth sort's ties go by original row); index first, it runs in internal order and the
// per-tile depth sort puts equal depths in original-row order; the MCMC noise is drawn by original row,
// and every entry point that exchanges rows with the caller restores the original order first.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sx_step.h"

namespace sxk {
namespace {

constexpr int kBlock = 256;
inline int grid_for(int64_t n) { return static_cast<int>((n + kBlock - 1) / kBlock); }

// Per-block bounding boxes of the means of rows [0, count) (x, y, z columns at stride R): part[6 b ..
// 6 b + 6) = {min x, min y, min z, max x, max y, max z}; non-finite coordinates are left out.
__global__ void __launch_bounds__(kBlock) k_bbox_part(const float* __restrict__ m, size_t R, int count,
                                                      float* __restrict__ part) {
    __shared__ float s[6][kBlock / 64];
    const int i = blockIdx.x * kBlock + threadIdx.x;
    float lo[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
    float hi[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
    if (i < count) {
#pragma unroll
        for (int d = 0; d < 3; d++) {
            const float x = m[d * R + i];
            if (__builtin_isfinite(x)) {
                lo[d] = x;
                hi[d] = x;
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int d = 0; d < 3; d++) {
            lo[d] = fminf(lo[d], __shfl_xor(lo[d], o, 64));
            hi[d] = fmaxf(hi[d], __shfl_xor(hi[d], o, 64));
        }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0)
#pragma unroll
        for (int d = 0; d < 3; d++) {
            s[d][wave] = lo[d];
            s[3 + d][wave] = hi[d];
        }
    __syncthreads();
    if (threadIdx.x < 6) {
        float v = s[threadIdx.x][0];
#pragma unroll
        for (int w = 1; w < kBlock / 64; w++) v = threadIdx.x < 3 ? fminf(v, s[threadIdx.x][w]) : fmaxf(v, s[threadIdx.x][w]);
        part[6 * (size_t)blockIdx.x + threadIdx.x] = v;
    }
}

// One workgroup: the blocks' boxes into bbox[0..6).
__global__ void __launch_bounds__(kBlock) k_bbox_final(const float* __restrict__ part, int nb, float* __restrict__ bbox) {
    __shared__ float s[6][kBlock];
    float lo[3] = {__builtin_inff(), __builtin_inff(), __builtin_inff()};
    float hi[3] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
    for (int b = threadIdx.x; b < nb; b += kBlock)
#pragma unroll
        for (int d = 0; d < 3; d++) {
            lo[d] = fminf(lo[d], part[6 * (size_t)b + d]);
            hi[d] = fmaxf(hi[d], part[6 * (size_t)b + 3 + d]);
        }
#pragma unroll
    for (int d = 0; d < 3; d++) {
        s[d][threadIdx.x] = lo[d];
        s[3 + d][threadIdx.x] = hi[d];
    }
    __syncthreads();
    if (threadIdx.x < 6) {
        float v = s[threadIdx.x][0];
        for (int t = 1; t < kBlock; t++) v = threadIdx.x < 3 ? fminf(v, s[threadIdx.x][t]) : fmaxf(v, s[threadIdx.x][t]);
        bbox[threadIdx.x] = v;
    }
}

// 10 bits of x spread to every third bit
__device__ __forceinline__ uint32_t spread3(uint32_t x) {
    x &= 0x3FFu;
    x = (x | (x << 16)) & 0x030000FFu;
    x = (x | (x << 8)) & 0x0300F00Fu;
    x = (x | (x << 4)) & 0x030C30C3u;
    x = (x | (x << 2)) & 0x09249249u;
    return x;
}

// keys[i] = the 30-bit Morton code of row i's mean in the box (10 bits per axis; non-finite: 0), vals[i] = i
__global__ void __launch_bounds__(kBlock) k_morton(const float* __restrict__ m, size_t R, int count,
                                                   const float* __restrict__ bbox, uint32_t* __restrict__ keys,
                                                   int32_t* __restrict__ vals) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= count) return;
    uint32_t q[3];
#pragma unroll
    for (int d = 0; d < 3; d++) {
        const float lo = bbox[d], ext = bbox[3 + d] - bbox[d];
        const float x = m[d * R + i];
        const float t = ext > 0.f ? (x - lo) / ext : 0.f;  // NaN (non-finite x) fails both compares below
        q[d] = t > 0.f ? static_cast<uint32_t>(fminf(t, 1.0f) * 1023.0f) : 0u;
    }
    keys[i] = spread3(q[0]) | (spread3(q[1]) << 1) | (spread3(q[2]) << 2);
    vals[i] = i;
}

// tmp[d * count + k] = col[d * R + src[k]] for the dim columns of one arena array, rows k < count
__global__ void __launch_bounds__(kBlock) k_gather_rows(const float* __restrict__ col, size_t R, int dim, int count,
                                                        const int32_t* __restrict__ src, float* __restrict__ tmp) {
    const int k = blockIdx.x * kBlock + threadIdx.x;
    if (k >= count) return;
    const size_t r = static_cast<size_t>(src[k]);
    for (int d = 0; d < dim; d++) tmp[(size_t)d * count + k] = col[d * R + r];
}

__global__ void __launch_bounds__(kBlock) k_put_rows(const float* __restrict__ tmp, size_t R, int dim, int count,
                                                     float* __restrict__ col) {
    const int k = blockIdx.x * kBlock + threadIdx.x;
    if (k >= count) return;
    for (int d = 0; d < dim; d++) col[d * R + k] = tmp[(size_t)d * count + k];
}

// the maps of a permutation from the original order: internal row k holds original row src[k]
__global__ void __launch_bounds__(kBlock) k_perm_maps(const int32_t* __restrict__ src, int count,
                                                      int32_t* __restrict__ row_orig, int32_t* __restrict__ row_int) {
    const int k = blockIdx.x * kBlock + threadIdx.x;
    if (k >= count) return;
    const int32_t o = src[k];
    row_orig[k] = o;
    row_int[o] = k;
}

}  // namespace

void arena_morton_keys(const Arena& A, int count, float* scratch, uint32_t* keys, int32_t* vals, hipStream_t s) {
    if (count <= 0) return;
    const int nb = grid_for(count);
    float* part = scratch + 8;  // scratch[0..6): the box
    hipLaunchKernelGGL(k_bbox_part, dim3(nb), dim3(kBlock), 0, s, A.p[0], static_cast<size_t>(A.rows), count, part);
    hipLaunchKernelGGL(k_bbox_final, dim3(1), dim3(kBlock), 0, s, part, nb, scratch);
    hipLaunchKernelGGL(k_morton, dim3(nb), dim3(kBlock), 0, s, A.p[0], static_cast<size_t>(A.rows), count, scratch,
                       keys, vals);
}

size_t arena_morton_scratch_floats(int count) { return 8 + 6 * static_cast<size_t>(grid_for(count)); }

void arena_permute_rows(const Arena& A, const int dims[6], int count, const int32_t* src, float* tmp, hipStream_t s) {
    if (count <= 0) return;
    const size_t R = static_cast<size_t>(A.rows);
    for (int g = 0; g < 6; g++) {
        if (dims[g] == 0) continue;
        float* cols[3] = {A.p[g], A.m[g], A.v[g]};
        for (float* col : cols) {
            hipLaunchKernelGGL(k_gather_rows, dim3(grid_for(count)), dim3(kBlock), 0, s, col, R, dims[g], count, src,
                               tmp);
            hipLaunchKernelGGL(k_put_rows, dim3(grid_for(count)), dim3(kBlock), 0, s, tmp, R, dims[g], count, col);
        }
    }
}

void perm_maps(const int32_t* src, int count, int32_t* row_orig, int32_t* row_int, hipStream_t s) {
    if (count <= 0) return;
    hipLaunchKernelGGL(k_perm_maps, dim3(grid_for(count)), dim3(kBlock), 0, s, src, count, row_orig, row_int);
}

}  // namespace sxk
