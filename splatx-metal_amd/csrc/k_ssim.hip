// k_ssim.hip — SSIM forward/backward (11x11 Gaussian window, sigma 1.5, valid padding) for gfx950.
//
// Contracts: ssim_fwd / ssim_bwd (Ssim.metal:66-268). One 16x16 workgroup per output tile and
// channel; the 26x26 apron is staged in LDS, the separable passes run horizontal then vertical with
// fma chains in tap order, exactly the CPU reference's order (CpuKernels.cpp:1036-1103), so the map
// and the coefficient maps are bit-identical to the CPU oracle. The forward also writes one f64
// partial sum of the map per workgroup (reduced deterministically by the caller).
#include <hip/hip_runtime.h>

#include "sx_common.h"
#include "sx_kernels.h"
#include "sx_step.h"

namespace sxk {
namespace {

constexpr int T = 16;
constexpr int A = 26;  // T + 11 - 1
__constant__ float c_taps[11] = SX_SSIM_TAPS;

__device__ inline size_t ihwc(int i, int y, int x, int c, int H, int W, int C) {
    return ((((size_t)i * H + y) * W) + x) * C + c;
}

__global__ void __launch_bounds__(256) k_ssim_fwd(const float* __restrict__ img1, const float* __restrict__ img2, int H,
                                                  int W, int C, int need_coeffs, float* __restrict__ map,
                                                  float* __restrict__ cmu, float* __restrict__ csg,
                                                  float* __restrict__ ccr, double* __restrict__ block_sums) {
    __shared__ float sx[A][A + 1];
    __shared__ float sy[A][A + 1];
    __shared__ float h[5][A][T + 1];
    __shared__ double s_red[256];
    const int mh = H - 10, mw = W - 10;
    const int img = blockIdx.z / C, ch = blockIdx.z % C;
    const int oy = blockIdx.y * T, ox = blockIdx.x * T;
    const int tid = threadIdx.y * T + threadIdx.x;
    for (int k = tid; k < A * A; k += 256) {
        const int ay = k / A, ax = k % A;
        const int y = oy + ay, x = ox + ax;
        float a = 0.f, b = 0.f;
        if (y < H && x < W) {
            const size_t off = ihwc(img, y, x, ch, H, W, C);
            a = img1[off];
            b = img2[off];
        }
        sx[ay][ax] = a;
        sy[ay][ax] = b;
    }
    __syncthreads();
    for (int k = tid; k < A * T; k += 256) {
        const int r = k / T, cx = k % T;
        float m1 = 0.f, m2 = 0.f, e11 = 0.f, e22 = 0.f, e12 = 0.f;
#pragma unroll
        for (int u = 0; u < 11; u++) {
            const float w = c_taps[u];
            const float x = sx[r][cx + u], g = sy[r][cx + u];
            m1 = __builtin_fmaf(w, x, m1);
            m2 = __builtin_fmaf(w, g, m2);
            e11 = __builtin_fmaf(w * x, x, e11);
            e22 = __builtin_fmaf(w * g, g, e22);
            e12 = __builtin_fmaf(w * x, g, e12);
        }
        h[0][r][cx] = m1;
        h[1][r][cx] = m2;
        h[2][r][cx] = e11;
        h[3][r][cx] = e22;
        h[4][r][cx] = e12;
    }
    __syncthreads();
    const int my = oy + threadIdx.y, mx = ox + threadIdx.x;
    double contrib = 0.0;
    if (my < mh && mx < mw) {
        float mu1 = 0.f, mu2 = 0.f, e11 = 0.f, e22 = 0.f, e12 = 0.f;
#pragma unroll
        for (int v = 0; v < 11; v++) {
            const float w = c_taps[v];
            const int r = threadIdx.y + v;
            mu1 = __builtin_fmaf(w, h[0][r][threadIdx.x], mu1);
            mu2 = __builtin_fmaf(w, h[1][r][threadIdx.x], mu2);
            e11 = __builtin_fmaf(w, h[2][r][threadIdx.x], e11);
            e22 = __builtin_fmaf(w, h[3][r][threadIdx.x], e22);
            e12 = __builtin_fmaf(w, h[4][r][threadIdx.x], e12);
        }
        const float sigma1 = __builtin_fmaf(-mu1, mu1, e11);
        const float sigma2 = __builtin_fmaf(-mu2, mu2, e22);
        const float sigma12 = __builtin_fmaf(-mu1, mu2, e12);
        const float A1 = 2.f * mu1 * mu2 + sx::kSsimC1;
        const float B1 = mu1 * mu1 + mu2 * mu2 + sx::kSsimC1;
        const float A2 = 2.f * sigma12 + sx::kSsimC2;
        const float B2 = sigma1 + sigma2 + sx::kSsimC2;
        const float denom = B1 * B2;
        const float S = (A1 * A2) / denom;
        const size_t mo = ihwc(img, my, mx, ch, mh, mw, C);
        map[mo] = S;
        contrib = static_cast<double>(S);
        if (need_coeffs) {
            const float dS_dmu1 = 2.f * (mu2 * A2 / denom - mu1 * S / B1);
            const float dS_dsigma1 = -S / B2;
            const float dS_dsigma12 = 2.f * A1 / denom;
            cmu[mo] = dS_dmu1 - 2.f * mu1 * dS_dsigma1 - mu2 * dS_dsigma12;
            csg[mo] = dS_dsigma1;
            ccr[mo] = dS_dsigma12;
        }
    }
    if (block_sums) {  // fixed-shape tree: deterministic
        s_red[tid] = contrib;
        __syncthreads();
        for (int o = 128; o > 0; o >>= 1) {
            if (tid < o) s_red[tid] += s_red[tid + o];
            __syncthreads();
        }
        if (tid == 0) {
            const size_t bid = ((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
            block_sums[bid] = s_red[0];
        }
    }
}

// Any channel count: one workgroup per (tile, channel).
__global__ void __launch_bounds__(256) k_ssim_bwd(const float* __restrict__ img1, const float* __restrict__ img2,
                                                  const float* __restrict__ cmu, const float* __restrict__ csg,
                                                  const float* __restrict__ ccr, int H, int W, int C, float G,
                                                  float* __restrict__ v_img1) {
    __shared__ float d[3][A][A + 1];
    __shared__ float h[3][A][T + 1];
    const int mh = H - 10, mw = W - 10;
    const int img = blockIdx.z / C, ch = blockIdx.z % C;
    const int oy = blockIdx.y * T, ox = blockIdx.x * T;
    const int tid = threadIdx.y * T + threadIdx.x;
    for (int k = tid; k < A * A; k += 256) {
        const int ay = k / A, ax = k % A;
        const int y = oy + ay - 10, x = ox + ax - 10;
        float a = 0.f, b = 0.f, c = 0.f;
        if (y >= 0 && y < mh && x >= 0 && x < mw) {
            const size_t off = ihwc(img, y, x, ch, mh, mw, C);
            a = cmu[off];
            b = csg[off];
            c = ccr[off];
        }
        d[0][ay][ax] = a;
        d[1][ay][ax] = b;
        d[2][ay][ax] = c;
    }
    __syncthreads();
    for (int k = tid; k < A * T; k += 256) {
        const int r = k / T, cx = k % T;
        float s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int u = 0; u < 11; u++) {
            const float w = c_taps[u];
            s1 = __builtin_fmaf(w, d[0][r][cx + u], s1);
            s2 = __builtin_fmaf(w, d[1][r][cx + u], s2);
            s3 = __builtin_fmaf(w, d[2][r][cx + u], s3);
        }
        h[0][r][cx] = s1;
        h[1][r][cx] = s2;
        h[2][r][cx] = s3;
    }
    __syncthreads();
    const int qy = oy + threadIdx.y, qx = ox + threadIdx.x;
    if (qy < H && qx < W) {
        float c1 = 0.f, c2 = 0.f, c3 = 0.f;
#pragma unroll
        for (int v = 0; v < 11; v++) {
            const float w = c_taps[v];
            const int r = threadIdx.y + v;
            c1 = __builtin_fmaf(w, h[0][r][threadIdx.x], c1);
            c2 = __builtin_fmaf(w, h[1][r][threadIdx.x], c2);
            c3 = __builtin_fmaf(w, h[2][r][threadIdx.x], c3);
        }
        const size_t q = ihwc(img, qy, qx, ch, H, W, C);
        const float x = img1[q], y = img2[q];
        v_img1[q] = G * (c1 + 2.f * x * c2 + y * c3);
    }
}

// Three-channel variants (the training images). The forward: one workgroup per 16x16 tile covers all
// three channels, so every global load and store touches whole interleaved pixels, and each channel's
// passes keep the tap order above (same results), register-blocked by two columns (horizontal) and two
// rows (vertical) with conflict-free LDS strides. The backward: one workgroup per 16 x 32
// tile, the apron of all three channels staged at once (whole pixels again) and the passes run one
// channel after another. The taller tile cuts the horizontal pass's apron rows (42 per 32 outputs
// instead of 26 per 16), and both passes are register-blocked: a horizontal task reads the 14 inputs
// of 4 consecutive columns once, a vertical thread the 12 rows of 2 consecutive outputs. The LDS
// strides keep both passes free of bank conflicts: a horizontal wave takes one column group over 42
// rows (odd row strides 27 and 17), and a half-wave of the vertical pass two row pairs 16 rows apart.
// (The same tiling measured slower for the forward: its 5 sums per tap need 43 KB of LDS per
// workgroup, which leaves 3 workgroups per CU.)
constexpr int C3 = 3;
constexpr int TW3 = 16, TH3 = 32;              // output tile
constexpr int AW3 = TW3 + 10, AH3 = TH3 + 10;  // its apron: 26 x 42
constexpr int SX3 = AW3 + 1;                   // row stride of the staged inputs (odd)
constexpr int SH3 = TW3 + 1;                   // row stride of the horizontal sums (odd)
constexpr int CG3 = 4;                         // columns per horizontal task (wave w: columns 4w..4w+3)
static_assert(TW3 == CG3 * 4 && AH3 <= 64 && TH3 == 32, "one wave per column group, 16 row pairs");

// the vertical pass's thread: column tx, rows 2 rg and 2 rg + 1
__device__ __forceinline__ int vert_rg(int tid) { return (tid >> 5) + 8 * ((tid >> 4) & 1); }

constexpr int SHF = T + 2;  // the forward's row stride of the horizontal sums: 18 (see below)

__global__ void __launch_bounds__(256) k_ssim_fwd3(const float* __restrict__ img1, const float* __restrict__ img2,
                                                   int H, int W, int need_coeffs, float* __restrict__ map,
                                                   float* __restrict__ cmu, float* __restrict__ csg,
                                                   float* __restrict__ ccr, double* __restrict__ block_sums) {
    __shared__ float sx[C3][A][A + 1];
    __shared__ float sy[C3][A][A + 1];
    __shared__ float h[5][A][SHF];
    __shared__ double s_red[256];
    const int mh = H - 10, mw = W - 10;
    const int img = blockIdx.z;
    const int oy = blockIdx.y * T, ox = blockIdx.x * T;
    const int tid = threadIdx.y * T + threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    {
        // every load of the apron issued before the first LDS store: one wait for all of them
        constexpr int kN = A * A * C3, kIt = (kN + 255) / 256;
        float va[kIt], vb[kIt];
#pragma unroll
        for (int it = 0; it < kIt; it++) {
            const int k = tid + 256 * it;
            const int ay = k / (A * C3), rem = k % (A * C3);
            const int ax = rem / C3, c = rem % C3;
            const int y = oy + ay, x = ox + ax;
            va[it] = 0.f;
            vb[it] = 0.f;
            if (k < kN && y < H && x < W) {
                const size_t off = ihwc(img, y, x, c, H, W, C3);
                va[it] = img1[off];
                vb[it] = img2[off];
            }
        }
#pragma unroll
        for (int it = 0; it < kIt; it++) {
            const int k = tid + 256 * it;
            if (k < kN) {
                const int ay = k / (A * C3), rem = k % (A * C3);
                const int ax = rem / C3, c = rem % C3;
                sx[c][ay][ax] = va[it];
                sy[c][ay][ax] = vb[it];
            }
        }
    }
    // Register-blocked passes. Horizontal: a task is one row and two adjacent columns (12 inputs read
    // once); half-wave h of wave w takes column pair 2w + h over the 26 rows (odd input row stride 27:
    // no bank conflicts). Vertical: threads 0..127, column vtx, rows 2 rg and 2 rg + 1 (12 sums read
    // once per quantity); the two 16-lane groups of a half-wave take row pairs 8 rows apart, which the
    // sums' row stride 18 puts 16 banks apart.
    const int hr = lane & 31, hc0 = 4 * wave + 2 * (lane >> 5);
    const bool hor = hr < A;
    const bool vert = tid < 128;
    const int vtx = tid & 15, vrg = ((tid >> 5) & 3) + 4 * ((tid >> 4) & 1);
    const int vmx = ox + vtx;
    float res[2][C3][4];
    double contrib = 0.0;
#pragma unroll
    for (int c = 0; c < C3; c++) {
        __syncthreads();  // loads done / previous channel's vertical pass done with h
        if (hor) {
            float xv[12], gv[12];
#pragma unroll
            for (int i = 0; i < 12; i++) {
                xv[i] = sx[c][hr][hc0 + i];
                gv[i] = sy[c][hr][hc0 + i];
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                float m1 = 0.f, m2 = 0.f, e11 = 0.f, e22 = 0.f, e12 = 0.f;
#pragma unroll
                for (int u = 0; u < 11; u++) {
                    const float w = c_taps[u];
                    const float x = xv[j + u], g = gv[j + u];
                    m1 = __builtin_fmaf(w, x, m1);
                    m2 = __builtin_fmaf(w, g, m2);
                    e11 = __builtin_fmaf(w * x, x, e11);
                    e22 = __builtin_fmaf(w * g, g, e22);
                    e12 = __builtin_fmaf(w * x, g, e12);
                }
                h[0][hr][hc0 + j] = m1;
                h[1][hr][hc0 + j] = m2;
                h[2][hr][hc0 + j] = e11;
                h[3][hr][hc0 + j] = e22;
                h[4][hr][hc0 + j] = e12;
            }
        }
        __syncthreads();
        if (vert) {
            float acc[5][2];
#pragma unroll
            for (int q = 0; q < 5; q++) {
                float hv[12];
#pragma unroll
                for (int v = 0; v < 12; v++) hv[v] = h[q][2 * vrg + v][vtx];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    float t = 0.f;
#pragma unroll
                    for (int v = 0; v < 11; v++) t = __builtin_fmaf(c_taps[v], hv[i + v], t);
                    acc[q][i] = t;
                }
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                res[i][c][0] = res[i][c][1] = res[i][c][2] = res[i][c][3] = 0.f;
                const int my = oy + 2 * vrg + i;
                if (my >= mh || vmx >= mw) continue;
                const float mu1 = acc[0][i], mu2 = acc[1][i], e11 = acc[2][i], e22 = acc[3][i], e12 = acc[4][i];
                const float sigma1 = __builtin_fmaf(-mu1, mu1, e11);
                const float sigma2 = __builtin_fmaf(-mu2, mu2, e22);
                const float sigma12 = __builtin_fmaf(-mu1, mu2, e12);
                const float A1 = 2.f * mu1 * mu2 + sx::kSsimC1;
                const float B1 = mu1 * mu1 + mu2 * mu2 + sx::kSsimC1;
                const float A2 = 2.f * sigma12 + sx::kSsimC2;
                const float B2 = sigma1 + sigma2 + sx::kSsimC2;
                const float denom = B1 * B2;
                const float S = (A1 * A2) / denom;
                contrib += static_cast<double>(S);
                const float dS_dmu1 = 2.f * (mu2 * A2 / denom - mu1 * S / B1);
                const float dS_dsigma1 = -S / B2;
                const float dS_dsigma12 = 2.f * A1 / denom;
                res[i][c][0] = S;
                res[i][c][1] = dS_dmu1 - 2.f * mu1 * dS_dsigma1 - mu2 * dS_dsigma12;
                res[i][c][2] = dS_dsigma1;
                res[i][c][3] = dS_dsigma12;
            }
        }
    }
    if (vert) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int my = oy + 2 * vrg + i;
            if (my >= mh || vmx >= mw) continue;
            const size_t mo = ihwc(img, my, vmx, 0, mh, mw, C3);
#pragma unroll
            for (int c = 0; c < C3; c++) {
                if (map) map[mo + c] = res[i][c][0];
                if (need_coeffs) {
                    cmu[mo + c] = res[i][c][1];
                    csg[mo + c] = res[i][c][2];
                    ccr[mo + c] = res[i][c][3];
                }
            }
        }
    }
    if (block_sums) {  // fixed-shape tree: deterministic
        s_red[tid] = contrib;
        __syncthreads();
        for (int o = 128; o > 0; o >>= 1) {
            if (tid < o) s_red[tid] += s_red[tid + o];
            __syncthreads();
        }
        if (tid == 0) block_sums[((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x] = s_red[0];
    }
}

// FUSE_L1: the resident step's loss gradient — v = w_l1 * sign(x - y) * g_l1 + G*(...), and one
// f64 partial sum of |x - y| per workgroup (TrainStep.metal:143-155 combination, Trainer.cpp:330-345).
template <bool FUSE_L1>
__global__ void __launch_bounds__(256) k_ssim_bwd3(const float* __restrict__ img1, const float* __restrict__ img2,
                                                   const float* __restrict__ cmu, const float* __restrict__ csg,
                                                   const float* __restrict__ ccr, int H, int W, float G,
                                                   float* __restrict__ v_img1, float w_l1, float g_l1,
                                                   double* __restrict__ l1_partials) {
    __shared__ double s_red[256];
    __shared__ float d[3][C3][AH3][SX3];
    __shared__ float h[3][AH3][SH3];
    const int mh = H - 10, mw = W - 10;
    const int img = blockIdx.z;
    const int oy = blockIdx.y * TH3, ox = blockIdx.x * TW3;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tx = tid & 15, rg = vert_rg(tid);
    const int qx = ox + tx;
    {
        // every load of the apron issued before the first LDS store: one wait for all of them
        constexpr int kN = AH3 * AW3 * C3, kIt = (kN + 255) / 256;
        float va[kIt], vb[kIt], ve[kIt];
#pragma unroll
        for (int it = 0; it < kIt; it++) {
            const int k = tid + 256 * it;
            const int ay = k / (AW3 * C3), rem = k - ay * (AW3 * C3);
            const int ax = rem / C3, c = rem - ax * C3;
            const int y = oy + ay - 10, x = ox + ax - 10;
            va[it] = 0.f;
            vb[it] = 0.f;
            ve[it] = 0.f;
            if (k < kN && y >= 0 && y < mh && x >= 0 && x < mw) {
                const size_t off = ihwc(img, y, x, c, mh, mw, C3);
                va[it] = cmu[off];
                vb[it] = csg[off];
                ve[it] = ccr[off];
            }
        }
#pragma unroll
        for (int it = 0; it < kIt; it++) {
            const int k = tid + 256 * it;
            if (k < kN) {
                const int ay = k / (AW3 * C3), rem = k - ay * (AW3 * C3);
                const int ax = rem / C3, c = rem - ax * C3;
                d[0][c][ay][ax] = va[it];
                d[1][c][ay][ax] = vb[it];
                d[2][c][ay][ax] = ve[it];
            }
        }
    }
    // the two output pixels' inputs, all three channels (whole interleaved pixels)
    float xs[2][C3], ys[2][C3], vout[2][C3];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int qy = oy + 2 * rg + i;
        const bool in = qy < H && qx < W;
        const size_t q0 = ihwc(img, in ? qy : 0, in ? qx : 0, 0, H, W, C3);
#pragma unroll
        for (int c = 0; c < C3; c++) {
            xs[i][c] = in ? img1[q0 + c] : 0.f;
            ys[i][c] = in ? img2[q0 + c] : 0.f;
        }
    }
    double l1 = 0.0;
#pragma unroll
    for (int c = 0; c < C3; c++) {
        __syncthreads();  // the staged maps are in; the previous channel's vertical pass is done with h
        if (lane < AH3) {  // horizontal: row `lane`, columns CG3 * wave + j
            const int r = lane, c0 = CG3 * wave;
#pragma unroll
            for (int q = 0; q < 3; q++) {
                float dv[CG3 + 10];
#pragma unroll
                for (int i = 0; i < CG3 + 10; i++) dv[i] = d[q][c][r][c0 + i];
#pragma unroll
                for (int j = 0; j < CG3; j++) {
                    float t = 0.f;
#pragma unroll
                    for (int u = 0; u < 11; u++) t = __builtin_fmaf(c_taps[u], dv[j + u], t);
                    h[q][r][c0 + j] = t;
                }
            }
        }
        __syncthreads();
        float acc[3][2];
#pragma unroll
        for (int q = 0; q < 3; q++) {
            float hv[12];
#pragma unroll
            for (int v = 0; v < 12; v++) hv[v] = h[q][2 * rg + v][tx];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                float t = 0.f;
#pragma unroll
                for (int v = 0; v < 11; v++) t = __builtin_fmaf(c_taps[v], hv[i + v], t);
                acc[q][i] = t;
            }
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int qy = oy + 2 * rg + i;
            const float x = xs[i][c], y = ys[i][c];
            const float c1 = acc[0][i], c2 = acc[1][i], c3 = acc[2][i];
            const float vd = G * (c1 + 2.f * x * c2 + y * c3);
            if (FUSE_L1) {
                const float dd = x - y;
                const float base = dd > 0.0f ? g_l1 : (dd < 0.0f ? -g_l1 : 0.0f);
                vout[i][c] = w_l1 * base + vd;
                if (qy < H && qx < W) l1 += fabs(static_cast<double>(dd));
            } else {
                vout[i][c] = vd;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int qy = oy + 2 * rg + i;
        if (qy >= H || qx >= W) continue;
        const size_t q0 = ihwc(img, qy, qx, 0, H, W, C3);
#pragma unroll
        for (int c = 0; c < C3; c++) v_img1[q0 + c] = vout[i][c];
    }
    if (FUSE_L1) {
        s_red[tid] = l1;
        __syncthreads();
        for (int o = 128; o > 0; o >>= 1) {
            if (tid < o) s_red[tid] += s_red[tid + o];
            __syncthreads();
        }
        if (tid == 0) l1_partials[((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x] = s_red[0];
    }
}

} // namespace

int ssim_fwd_blocks(int I, int H, int W, int C) {
    const int mh = H - 10, mw = W - 10;
    return ((mw + T - 1) / T) * ((mh + T - 1) / T) * I * (C == C3 ? 1 : C);
}

void ssim_fwd(const float* img1, const float* img2, int I, int H, int W, int C, int need_coeffs, float* map,
              float* cmu, float* csg, float* ccr, double* block_sums, hipStream_t s) {
    const int mh = H - 10, mw = W - 10;
    if (mh <= 0 || mw <= 0) return;
    if (C == C3) {
        dim3 grid((mw + T - 1) / T, (mh + T - 1) / T, I);
        hipLaunchKernelGGL(k_ssim_fwd3, grid, dim3(T, T), 0, s, img1, img2, H, W, need_coeffs, map, cmu, csg, ccr,
                           block_sums);
        return;
    }
    dim3 grid((mw + T - 1) / T, (mh + T - 1) / T, I * C);
    hipLaunchKernelGGL(k_ssim_fwd, grid, dim3(T, T), 0, s, img1, img2, H, W, C, need_coeffs, map, cmu, csg, ccr,
                       block_sums);
}

void ssim_bwd(const float* img1, const float* img2, const float* cmu, const float* csg, const float* ccr, int I,
              int H, int W, int C, float G, float* v_img1, hipStream_t s) {
    if (C == C3) {
        dim3 grid((W + TW3 - 1) / TW3, (H + TH3 - 1) / TH3, I);
        hipLaunchKernelGGL(k_ssim_bwd3<false>, grid, dim3(256), 0, s, img1, img2, cmu, csg, ccr, H, W, G, v_img1,
                           0.f, 0.f, nullptr);
        return;
    }
    dim3 grid((W + T - 1) / T, (H + T - 1) / T, I * C);
    hipLaunchKernelGGL(k_ssim_bwd, grid, dim3(T, T), 0, s, img1, img2, cmu, csg, ccr, H, W, C, G, v_img1);
}

int step_ssim_bwd_blocks(int H, int W) { return ((W + TW3 - 1) / TW3) * ((H + TH3 - 1) / TH3); }

void step_ssim_bwd_l1(const float* render, const float* gt, const float* cmu, const float* csg, const float* ccr,
                      int H, int W, float G, float w_l1, float g_l1, float* v_render, double* l1_partials,
                      hipStream_t s) {
    dim3 grid((W + TW3 - 1) / TW3, (H + TH3 - 1) / TH3, 1);
    hipLaunchKernelGGL(k_ssim_bwd3<true>, grid, dim3(256), 0, s, render, gt, cmu, csg, ccr, H, W, G, v_render,
                       w_l1, g_l1, l1_partials);
}

} // namespace sxk
