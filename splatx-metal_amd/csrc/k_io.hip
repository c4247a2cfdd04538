// k_io.hip — device side of the data formats either side of the step (gfx950): the export filter
// and INRIA PLY row packing (Sources/SplatXCore/PlyIO.cpp semantics, PlyIO.h:20-51), the SXCK
// checkpoint payload packing/unpacking (Checkpoint.h:11-63: fp32 verbatim, fp16 with clamp and the
// sqrt compression of exp_avg_sq, paired zeroing on load), and the RGBA8 quantization of a render
// session frame (TrainC.cpp:1558-1571). All of it reads or writes the SoA arena in place, so only the
// packed bytes cross PCIe.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "sx_io.h"

namespace sxk {
namespace {

constexpr int kBlock = 256;
inline int grid_for(int64_t n, int per = kBlock) { return static_cast<int>((n + per - 1) / per); }

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + sxm::expf_(-x)); }
__device__ __forceinline__ bool finite_f(float x) { return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u; }

// filter_cloud_for_export's predicate per row: every parameter finite, then sigmoid(opacity) >
// min_opacity (strict); counts of the two removal classes (PlyIO.cpp:139-147 classification order)
__global__ void __launch_bounds__(kBlock) k_export_flags(Arena A, Dims6 dims, int count, float min_opacity,
                                                         int32_t* __restrict__ keep,
                                                         unsigned long long* __restrict__ removed) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    bool nonfinite = false, low = false;
    if (i < count) {
        const size_t R = static_cast<size_t>(A.rows);
        bool ok = true;
        for (int g = 0; g < 6; g++)
            for (int k = 0; k < dims.d[g]; k++) ok &= finite_f(A.p[g][k * R + i]);
        nonfinite = !ok;
        low = ok && !(sigmoid_ref(A.p[3][i]) > min_opacity);
        keep[i] = (ok && !low) ? 1 : 0;
    }
    const int n_nonfinite = __syncthreads_count(nonfinite);
    const int n_low = __syncthreads_count(low);
    if (threadIdx.x == 0) {
        if (n_nonfinite) atomicAdd(&removed[0], static_cast<unsigned long long>(n_nonfinite));
        if (n_low) atomicAdd(&removed[1], static_cast<unsigned long long>(n_low));
    }
}

__global__ void __launch_bounds__(kBlock) k_export_list(const int32_t* __restrict__ keep,
                                                        const int64_t* __restrict__ cum, int count,
                                                        int32_t* __restrict__ list) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i < count && keep[i]) list[cum[i] - 1] = i;
}

// One PLY row per kept Gaussian (PlyIO.cpp:36-52 field order): x y z, nx ny nz = 0, f_dc_0..2,
// f_rest channel-major (Kw per channel; coefficients k >= K written 0 — the viewer padding),
// opacity, scale_0..2, rot_0..3. Thread per output float of rows [row0, row0 + rows).
__global__ void __launch_bounds__(kBlock) k_export_pack(Arena A, int K, int Kw, const int32_t* __restrict__ list,
                                                        int64_t row0, int64_t rows, float* __restrict__ out) {
    const int cols = 6 + 3 + 3 * Kw + 1 + 3 + 4;
    const int64_t t = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (t >= rows * cols) return;
    const int64_t j = t / cols;
    const int c = static_cast<int>(t - j * cols);
    const size_t R = static_cast<size_t>(A.rows);
    const size_t i = static_cast<size_t>(list[row0 + j]);
    float v = 0.0f;
    const int rest0 = 9, op = 9 + 3 * Kw;
    if (c < 3) v = A.p[0][c * R + i];
    else if (c < 6) v = 0.0f;
    else if (c < rest0) v = A.p[4][(c - 6) * R + i];
    else if (c < op) {
        const int q = c - rest0, ch = q / Kw, k = q - ch * Kw;
        v = k < K ? A.p[5][(static_cast<size_t>(k) * 3 + ch) * R + i] : 0.0f;
    } else if (c == op) v = A.p[3][i];
    else if (c < op + 4) v = A.p[2][(c - op - 1) * R + i];
    else v = A.p[1][(c - op - 4) * R + i];
    out[t] = v;
}

// IEEE half bits, round to nearest even, finite values clamped to +-65504 first, NaN kept
__device__ __forceinline__ uint16_t half_bits(float x) {
    if (x > 65504.0f) x = 65504.0f;
    else if (x < -65504.0f) x = -65504.0f;
    return __half_as_ushort(__float2half_rn(x));
}

// rows [row0, row0 + rows) of one SoA column group -> row-major [rows, dim] (the file's layout)
__global__ void __launch_bounds__(kBlock) k_ckpt_pack(const float* __restrict__ soa, int R, int dim, int64_t row0,
                                                      int64_t rows, int mode, void* __restrict__ out) {
    const int64_t t = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (t >= rows * dim) return;
    const int64_t r = t / dim;
    const int k = static_cast<int>(t - r * dim);
    const float x = soa[static_cast<size_t>(k) * R + static_cast<size_t>(row0 + r)];
    if (mode == kCkptF32) static_cast<float*>(out)[t] = x;
    else static_cast<uint16_t*>(out)[t] = half_bits(mode == kCkptF16Sqrt ? sqrtf(x) : x);
}

__global__ void __launch_bounds__(kBlock) k_ckpt_unpack(const void* __restrict__ in, int mode, float* __restrict__ soa,
                                                        int R, int dim, int64_t row0, int64_t rows) {
    const int64_t t = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (t >= rows * dim) return;
    const int64_t r = t / dim;
    const int k = static_cast<int>(t - r * dim);
    float x;
    if (mode == kCkptF32) {
        x = static_cast<const float*>(in)[t];
    } else {
        x = __half2float(__ushort_as_half(static_cast<const uint16_t*>(in)[t]));
        if (mode == kCkptF16Sqrt) x = x * x;
    }
    soa[static_cast<size_t>(k) * R + static_cast<size_t>(row0 + r)] = x;
}

// fp16 load: an exp_avg_sq that decoded to 0 zeroes its exp_avg (Checkpoint.cpp read path)
__global__ void __launch_bounds__(kBlock) k_ckpt_pair_zero(float* __restrict__ m, const float* __restrict__ v, int R,
                                                           int dim, int n) {
    const int64_t t = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (t >= static_cast<int64_t>(n) * dim) return;
    const int k = static_cast<int>(t / n), r = static_cast<int>(t - static_cast<int64_t>(k) * n);
    const size_t at = static_cast<size_t>(k) * R + r;
    if (v[at] == 0.0f) m[at] = 0.0f;
}

// rows [n, R) of every column of one SoA group <- 0
__global__ void __launch_bounds__(kBlock) k_zero_tail(float* __restrict__ soa, int R, int dim, int n) {
    const int64_t tail = R - n;
    const int64_t t = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (t >= tail * dim) return;
    const int k = static_cast<int>(t / tail);
    const int64_t r = n + (t - static_cast<int64_t>(k) * tail);
    soa[static_cast<size_t>(k) * R + static_cast<size_t>(r)] = 0.0f;
}

// [H,W,3] f32 -> RGBA8: NaN and v <= 0 -> 0, v > 1 -> 1, round-to-nearest-even of v * 255, alpha 255
__global__ void __launch_bounds__(kBlock) k_rgba8(const float* __restrict__ rgb, int64_t n_px,
                                                  uint32_t* __restrict__ out) {
    const int64_t p = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (p >= n_px) return;
    uint32_t word = 0xff000000u;
#pragma unroll
    for (int c = 0; c < 3; c++) {
        float v = rgb[p * 3 + c];
        if (!(v > 0.0f)) v = 0.0f;
        if (v > 1.0f) v = 1.0f;
        word |= static_cast<uint32_t>(rintf(v * 255.0f)) << (8 * c);
    }
    out[p] = word;
}

// rows list[j], j in [0, n), of one SoA group -> row-major [n, dim] (raw values, the snapshot layout)
__global__ void __launch_bounds__(kBlock) k_gather_rows(const float* __restrict__ soa, int R, int dim,
                                                        const int32_t* __restrict__ list, int64_t n,
                                                        float* __restrict__ out) {
    const int64_t t = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x;
    if (t >= n * dim) return;
    const int64_t j = t / dim;
    const int k = static_cast<int>(t - j * dim);
    out[t] = soa[static_cast<size_t>(k) * R + static_cast<size_t>(list[j])];
}

// partials[b] = f64 sum over block b's grid-stride share of (clamp(a, 0, 1) - b)^2, clamp as
// std::clamp (NaN passes through); a fixed grid, so the host sums the partials in a fixed order
constexpr int kSqBlocks = 512;
__global__ void __launch_bounds__(kBlock) k_sq_err(const float* __restrict__ a, const float* __restrict__ b,
                                                   int64_t n, double* __restrict__ partials) {
    __shared__ double s_red[kBlock];
    double acc = 0.0;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x; i < n;
         i += static_cast<int64_t>(kSqBlocks) * kBlock) {
        float v = a[i];
        v = v < 0.0f ? 0.0f : (1.0f < v ? 1.0f : v);
        const double d = static_cast<double>(v) - static_cast<double>(b[i]);
        acc += d * d;
    }
    s_red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = kBlock / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) s_red[threadIdx.x] += s_red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) partials[blockIdx.x] = s_red[0];
}

}  // namespace

void gather_rows(const float* soa, int R, int dim, const int32_t* list, int64_t n, float* out, hipStream_t s) {
    const int64_t total = n * dim;
    if (total <= 0) return;
    hipLaunchKernelGGL(k_gather_rows, dim3(grid_for(total)), dim3(kBlock), 0, s, soa, R, dim, list, n, out);
}

int sq_err_blocks() { return kSqBlocks; }

void sq_err(const float* a, const float* b, int64_t n, double* partials, hipStream_t s) {
    hipLaunchKernelGGL(k_sq_err, dim3(kSqBlocks), dim3(kBlock), 0, s, a, b, n, partials);
}

void export_flags(const Arena& A, const Dims6& dims, int count, float min_opacity, int32_t* keep,
                  unsigned long long* removed, hipStream_t s) {
    if (count <= 0) return;
    hipLaunchKernelGGL(k_export_flags, dim3(grid_for(count)), dim3(kBlock), 0, s, A, dims, count, min_opacity, keep,
                       removed);
}

void export_list(const int32_t* keep, const int64_t* cum, int count, int32_t* list, hipStream_t s) {
    if (count <= 0) return;
    hipLaunchKernelGGL(k_export_list, dim3(grid_for(count)), dim3(kBlock), 0, s, keep, cum, count, list);
}

int export_row_floats(int Kw) { return 6 + 3 + 3 * Kw + 1 + 3 + 4; }

void export_pack(const Arena& A, int K, int Kw, const int32_t* list, int64_t row0, int64_t rows, float* out,
                 hipStream_t s) {
    const int64_t n = rows * export_row_floats(Kw);
    if (n <= 0) return;
    hipLaunchKernelGGL(k_export_pack, dim3(grid_for(n)), dim3(kBlock), 0, s, A, K, Kw, list, row0, rows, out);
}

void ckpt_pack(const float* soa, int R, int dim, int64_t row0, int64_t rows, int mode, void* out, hipStream_t s) {
    const int64_t n = rows * dim;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_ckpt_pack, dim3(grid_for(n)), dim3(kBlock), 0, s, soa, R, dim, row0, rows, mode, out);
}

void ckpt_unpack(const void* in, int mode, float* soa, int R, int dim, int64_t row0, int64_t rows, hipStream_t s) {
    const int64_t n = rows * dim;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_ckpt_unpack, dim3(grid_for(n)), dim3(kBlock), 0, s, in, mode, soa, R, dim, row0, rows);
}

void ckpt_pair_zero(float* m, const float* v, int R, int dim, int n, hipStream_t s) {
    const int64_t total = static_cast<int64_t>(n) * dim;
    if (total <= 0) return;
    hipLaunchKernelGGL(k_ckpt_pair_zero, dim3(grid_for(total)), dim3(kBlock), 0, s, m, v, R, dim, n);
}

void zero_tail(float* soa, int R, int dim, int n, hipStream_t s) {
    const int64_t total = static_cast<int64_t>(R - n) * dim;
    if (total <= 0) return;
    hipLaunchKernelGGL(k_zero_tail, dim3(grid_for(total)), dim3(kBlock), 0, s, soa, R, dim, n);
}

void rgba8(const float* rgb, int64_t n_px, uint32_t* out, hipStream_t s) {
    if (n_px <= 0) return;
    hipLaunchKernelGGL(k_rgba8, dim3(grid_for(n_px)), dim3(kBlock), 0, s, rgb, n_px, out);
}

}  // namespace sxk
