// sx_dev.h — gfx950 device functions of the 3DGS step (projection, SH, AccuTile/AABB tile sets).
//
// These are the per-Gaussian building blocks shared by the per-op kernels (the verification
// surface) and the fused resident-step kernels. Their floating-point operation order reproduces
// the reference CPU code (Sources/SplatXCore/CpuKernels.cpp, Math.cpp), and everything is compiled
// with -ffp-contract=off and IEEE division/sqrt, so the integer outputs (radii, tile sets, keys)
// and the forward values are bit-identical to the CPU oracle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sx_common.h"
#include "sx_fmath.h"

#define SX_DEV __device__ __forceinline__

namespace sxd {

// std::min / std::max semantics: min(a,b) = (b < a) ? b : a ; max(a,b) = (a < b) ? b : a
SX_DEV float smin(float a, float b) { return (b < a) ? b : a; }
SX_DEV float smax(float a, float b) { return (a < b) ? b : a; }
SX_DEV int32_t imin(int32_t a, int32_t b) { return (b < a) ? b : a; }
SX_DEV int32_t imax(int32_t a, int32_t b) { return (a < b) ? b : a; }

// ---------------------------------------------------------------------------------------------
// Wave (64-lane) helpers
// ---------------------------------------------------------------------------------------------
SX_DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
SX_DEV int32_t wave_max_i(int32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const int32_t u = __shfl_xor(v, o, 64);
        v = u > v ? u : v;
    }
    return v;
}
SX_DEV uint32_t lane_id() { return __lane_id(); }

// ---------------------------------------------------------------------------------------------
// Math.cpp:9-45 — quaternion (w,x,y,z) normalized by division, R row-major, covar = (R S)(R S)^T
// with every 3x3 product accumulated as s = 0; s += a*b.
// ---------------------------------------------------------------------------------------------
SX_DEV void m3mul(const float* a, const float* b, float* c) {
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) {
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 3; k++) s += a[i * 3 + k] * b[k * 3 + j];
            c[i * 3 + j] = s;
        }
}
SX_DEV void m3tr(const float* a, float* t) {
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) t[i * 3 + j] = a[j * 3 + i];
}

SX_DEV void quat_to_rotmat_ref(float w, float x, float y, float z, float* R) {
    const float n = __builtin_sqrtf(w * w + x * x + y * y + z * z);
    if (n > 0.0f) {
        w /= n;
        x /= n;
        y /= n;
        z /= n;
    }
    R[0] = 1.0f - 2.0f * (y * y + z * z);
    R[1] = 2.0f * (x * y - w * z);
    R[2] = 2.0f * (x * z + w * y);
    R[3] = 2.0f * (x * y + w * z);
    R[4] = 1.0f - 2.0f * (x * x + z * z);
    R[5] = 2.0f * (y * z - w * x);
    R[6] = 2.0f * (x * z - w * y);
    R[7] = 2.0f * (y * z + w * x);
    R[8] = 1.0f - 2.0f * (x * x + y * y);
}

SX_DEV void quat_scale_to_covar_ref(const float q[4], const float s[3], float* Cw) {
    float R[9], M[9], Mt[9];
    quat_to_rotmat_ref(q[0], q[1], q[2], q[3], R);
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) M[i * 3 + j] = R[i * 3 + j] * s[j];
    m3tr(M, Mt);
    m3mul(M, Mt, Cw);
}

// ---------------------------------------------------------------------------------------------
// Camera constants of the PINHOLE projection (CpuKernels.cpp:171-184)
// ---------------------------------------------------------------------------------------------
struct Cam {
    float R[9];
    float t[3];
    float fx, fy, cx, cy;
    float lim_x_pos, lim_x_neg, lim_y_pos, lim_y_neg;
    float width, height;
};

SX_DEV Cam make_cam(const float* vm, const float* K, int width, int height) {
    Cam c;
    c.R[0] = vm[0]; c.R[1] = vm[1]; c.R[2] = vm[2];
    c.R[3] = vm[4]; c.R[4] = vm[5]; c.R[5] = vm[6];
    c.R[6] = vm[8]; c.R[7] = vm[9]; c.R[8] = vm[10];
    c.t[0] = vm[3]; c.t[1] = vm[7]; c.t[2] = vm[11];
    c.fx = K[0]; c.fy = K[4]; c.cx = K[2]; c.cy = K[5];
    c.width = static_cast<float>(width);
    c.height = static_cast<float>(height);
    const float tan_fovx = 0.5f * c.width / c.fx;
    const float tan_fovy = 0.5f * c.height / c.fy;
    c.lim_x_pos = (c.width - c.cx) / c.fx + 0.3f * tan_fovx;
    c.lim_x_neg = c.cx / c.fx + 0.3f * tan_fovx;
    c.lim_y_pos = (c.height - c.cy) / c.fy + 0.3f * tan_fovy;
    c.lim_y_neg = c.cy / c.fy + 0.3f * tan_fovy;
    return c;
}

struct ProjOut {
    bool alive;
    int32_t rx, ry;
    float m2x, m2y, depth;
    float ca, cb, cc;
    float comp;
};

struct ProjCfg {
    float eps2d, near_plane, far_plane, radius_clip;
    int calc_comp;
    int has_opac;
};

// projection_ewa_3dgs_fused_fwd for one (camera, Gaussian) — CpuKernels.cpp:186-269.
// `Cw` is the world covariance (row-major 3x3).
SX_DEV ProjOut project_one(const Cam& cam, const float* mw, const float* Cw, float opacity,
                           const ProjCfg& cfg) {
    ProjOut o;
    o.alive = false;
    o.rx = 0;
    o.ry = 0;
    o.comp = 0.0f;
    const float* R = cam.R;
    const float mx = R[0] * mw[0] + R[1] * mw[1] + R[2] * mw[2] + cam.t[0];
    const float my = R[3] * mw[0] + R[4] * mw[1] + R[5] * mw[2] + cam.t[1];
    const float mz = R[6] * mw[0] + R[7] * mw[1] + R[8] * mw[2] + cam.t[2];
    if (mz < cfg.near_plane || mz > cfg.far_plane) return o;

    float RC[9], Rt[9], Cc[9];
    m3mul(R, Cw, RC);
    m3tr(R, Rt);
    m3mul(RC, Rt, Cc);

    const float rz = 1.0f / mz, rz2 = rz * rz;
    const float txc = mz * smin(cam.lim_x_pos, smax(-cam.lim_x_neg, mx * rz));
    const float tyc = mz * smin(cam.lim_y_pos, smax(-cam.lim_y_neg, my * rz));
    const float J00 = cam.fx * rz, J02 = -cam.fx * txc * rz2;
    const float J11 = cam.fy * rz, J12 = -cam.fy * tyc * rz2;
    const float JC00 = J00 * Cc[0] + J02 * Cc[6];
    const float JC01 = J00 * Cc[1] + J02 * Cc[7];
    const float JC02 = J00 * Cc[2] + J02 * Cc[8];
    const float JC10 = J11 * Cc[3] + J12 * Cc[6];
    const float JC11 = J11 * Cc[4] + J12 * Cc[7];
    const float JC12 = J11 * Cc[5] + J12 * Cc[8];
    float c00 = JC00 * J00 + JC02 * J02;
    const float c01 = JC01 * J11 + JC02 * J12;
    const float c10 = JC10 * J00 + JC12 * J02;
    float c11 = JC11 * J11 + JC12 * J12;
    (void)JC01;
    const float m2x = cam.fx * mx * rz + cam.cx;
    const float m2y = cam.fy * my * rz + cam.cy;

    const float det_orig = c00 * c11 - c01 * c10;
    c00 += cfg.eps2d;
    c11 += cfg.eps2d;
    const float det = c00 * c11 - c01 * c10;
    const float comp =
        __builtin_sqrtf(smax(sx::kMinCompensation * sx::kMinCompensation, det_orig / det));
    if (det <= 0.0f) return o;

    const float rdet = 1.0f / det;
    const float conic_a = c11 * rdet;
    const float conic_b = -c10 * rdet;
    const float conic_c = c00 * rdet;

    float extend = sx::kGaussianExtend;
    if (cfg.has_opac) {
        float op = opacity;
        if (cfg.calc_comp) op *= comp;
        if (op < sx::kAlphaThreshold) return o;
        extend = smin(sx::kGaussianExtend,
                      __builtin_sqrtf(2.0f * sxm::logf_(op / sx::kAlphaThreshold)));
    }
    const float radius_x = __builtin_ceilf(extend * __builtin_sqrtf(c00));
    const float radius_y = __builtin_ceilf(extend * __builtin_sqrtf(c11));
    if (radius_x <= cfg.radius_clip && radius_y <= cfg.radius_clip) return o;
    if (m2x + radius_x <= 0.0f || m2x - radius_x >= cam.width || m2y + radius_y <= 0.0f ||
        m2y - radius_y >= cam.height)
        return o;

    o.alive = true;
    o.rx = sxm::f2i_trunc(radius_x);
    o.ry = sxm::f2i_trunc(radius_y);
    o.m2x = m2x;
    o.m2y = m2y;
    o.depth = mz;
    o.ca = conic_a;
    o.cb = conic_b;
    o.cc = conic_c;
    o.comp = comp;
    return o;
}

// ---------------------------------------------------------------------------------------------
// SH color for one channel — CpuKernels.cpp:284-353 expression forms (no fma), degrees 0..4.
// `co(k)` returns coefficient k of this channel.
// ---------------------------------------------------------------------------------------------
template <class CoeffFn>
SX_DEV float sh_color(uint32_t degree, float dx, float dy, float dz, CoeffFn co) {
    float result = 0.2820947917738781f * co(0);
    if (degree >= 1) {
        const float inorm = 1.0f / __builtin_sqrtf(dx * dx + dy * dy + dz * dz);
        const float x = dx * inorm;
        const float y = dy * inorm;
        const float z = dz * inorm;
        result += 0.48860251190292f * (-y * co(1) + z * co(2) - x * co(3));
        if (degree >= 2) {
            const float z2 = z * z;
            const float fTmp0B = -1.092548430592079f * z;
            const float fC1 = x * x - y * y;
            const float fS1 = 2.f * x * y;
            const float pSH6 = 0.9461746957575601f * z2 - 0.3153915652525201f;
            const float pSH7 = fTmp0B * x;
            const float pSH5 = fTmp0B * y;
            const float pSH8 = 0.5462742152960395f * fC1;
            const float pSH4 = 0.5462742152960395f * fS1;
            result += pSH4 * co(4) + pSH5 * co(5) + pSH6 * co(6) + pSH7 * co(7) + pSH8 * co(8);
            if (degree >= 3) {
                const float fTmp0C = -2.285228997322329f * z2 + 0.4570457994644658f;
                const float fTmp1B = 1.445305721320277f * z;
                const float fC2 = x * fC1 - y * fS1;
                const float fS2 = x * fS1 + y * fC1;
                const float pSH12 = z * (1.865881662950577f * z2 - 1.119528997770346f);
                const float pSH13 = fTmp0C * x;
                const float pSH11 = fTmp0C * y;
                const float pSH14 = fTmp1B * fC1;
                const float pSH10 = fTmp1B * fS1;
                const float pSH15 = -0.5900435899266435f * fC2;
                const float pSH9 = -0.5900435899266435f * fS2;
                result += pSH9 * co(9) + pSH10 * co(10) + pSH11 * co(11) + pSH12 * co(12) +
                          pSH13 * co(13) + pSH14 * co(14) + pSH15 * co(15);
                if (degree >= 4) {
                    const float fTmp0D = z * (-4.683325804901025f * z2 + 2.007139630671868f);
                    const float fTmp1C = 3.31161143515146f * z2 - 0.47308734787878f;
                    const float fTmp2B = -1.770130769779931f * z;
                    const float fC3 = x * fC2 - y * fS2;
                    const float fS3 = x * fS2 + y * fC2;
                    const float pSH20 = 1.984313483298443f * z * pSH12 - 1.006230589874905f * pSH6;
                    const float pSH21 = fTmp0D * x;
                    const float pSH19 = fTmp0D * y;
                    const float pSH22 = fTmp1C * fC1;
                    const float pSH18 = fTmp1C * fS1;
                    const float pSH23 = fTmp2B * fC2;
                    const float pSH17 = fTmp2B * fS2;
                    const float pSH24 = 0.6258357354491763f * fC3;
                    const float pSH16 = 0.6258357354491763f * fS3;
                    result += pSH16 * co(16) + pSH17 * co(17) + pSH18 * co(18) + pSH19 * co(19) +
                              pSH20 * co(20) + pSH21 * co(21) + pSH22 * co(22) + pSH23 * co(23) +
                              pSH24 * co(24);
                }
            }
        }
    }
    return result;
}

// SH basis values Y_k (k < 25) at the normalized direction, for the backward pass. Returns the
// number of bases for `degree` and fills the Cartesian partials needed for v_dir.
// The vector-Jacobian product follows SphericalHarmonics.metal:145-389 (gsplat
// sh_coeffs_to_color_fast_vjp): per channel, v_coeff[k] += Y_k * v_color and
// v_dir += v_color * sum_k dY_k/d(xyz) * coeff[k], then the normalization Jacobian.
struct ShBasis {
    float Y[25];
    float dX[25], dY[25], dZ[25];  // partials w.r.t. the normalized x, y, z
    float x, y, z, inorm;
};

SX_DEV void sh_basis(uint32_t degree, float dx, float dy, float dz, ShBasis& b) {
#pragma unroll
    for (int k = 0; k < 25; k++) {
        b.Y[k] = 0.f;
        b.dX[k] = 0.f;
        b.dY[k] = 0.f;
        b.dZ[k] = 0.f;
    }
    b.Y[0] = 0.2820947917738781f;
    b.x = b.y = b.z = 0.f;
    b.inorm = 0.f;
    if (degree < 1) return;
    const float inorm = 1.0f / __builtin_sqrtf(dx * dx + dy * dy + dz * dz);
    const float x = dx * inorm, y = dy * inorm, z = dz * inorm;
    b.x = x; b.y = y; b.z = z; b.inorm = inorm;
    const float c1 = 0.48860251190292f;
    b.Y[1] = -c1 * y; b.Y[2] = c1 * z; b.Y[3] = -c1 * x;
    b.dY[1] = -c1; b.dZ[2] = c1; b.dX[3] = -c1;
    if (degree < 2) return;
    const float z2 = z * z;
    const float fTmp0B = -1.092548430592079f * z;
    const float fC1 = x * x - y * y, fS1 = 2.f * x * y;
    const float pSH6 = 0.9461746957575601f * z2 - 0.3153915652525201f;
    b.Y[4] = 0.5462742152960395f * fS1;
    b.Y[5] = fTmp0B * y;
    b.Y[6] = pSH6;
    b.Y[7] = fTmp0B * x;
    b.Y[8] = 0.5462742152960395f * fC1;
    const float fC1_x = 2.f * x, fC1_y = -2.f * y, fS1_x = 2.f * y, fS1_y = 2.f * x;
    const float pSH6_z = 2.f * 0.9461746957575601f * z;
    const float fTmp0B_z = -1.092548430592079f;
    b.dX[4] = 0.5462742152960395f * fS1_x; b.dY[4] = 0.5462742152960395f * fS1_y;
    b.dY[5] = fTmp0B; b.dZ[5] = fTmp0B_z * y;
    b.dZ[6] = pSH6_z;
    b.dX[7] = fTmp0B; b.dZ[7] = fTmp0B_z * x;
    b.dX[8] = 0.5462742152960395f * fC1_x; b.dY[8] = 0.5462742152960395f * fC1_y;
    if (degree < 3) return;
    const float fTmp0C = -2.285228997322329f * z2 + 0.4570457994644658f;
    const float fTmp1B = 1.445305721320277f * z;
    const float fC2 = x * fC1 - y * fS1, fS2 = x * fS1 + y * fC1;
    const float pSH12 = z * (1.865881662950577f * z2 - 1.119528997770346f);
    b.Y[9] = -0.5900435899266435f * fS2;
    b.Y[10] = fTmp1B * fS1;
    b.Y[11] = fTmp0C * y;
    b.Y[12] = pSH12;
    b.Y[13] = fTmp0C * x;
    b.Y[14] = fTmp1B * fC1;
    b.Y[15] = -0.5900435899266435f * fC2;
    const float fTmp0C_z = -2.285228997322329f * 2.f * z, fTmp1B_z = 1.445305721320277f;
    const float fC2_x = fC1 + x * fC1_x - y * fS1_x, fC2_y = x * fC1_y - fS1 - y * fS1_y;
    const float fS2_x = fS1 + x * fS1_x + y * fC1_x, fS2_y = x * fS1_y + fC1 + y * fC1_y;
    const float pSH12_z = 3.f * 1.865881662950577f * z2 - 1.119528997770346f;
    b.dX[9] = -0.5900435899266435f * fS2_x; b.dY[9] = -0.5900435899266435f * fS2_y;
    b.dX[10] = fTmp1B * fS1_x; b.dY[10] = fTmp1B * fS1_y; b.dZ[10] = fTmp1B_z * fS1;
    b.dY[11] = fTmp0C; b.dZ[11] = fTmp0C_z * y;
    b.dZ[12] = pSH12_z;
    b.dX[13] = fTmp0C; b.dZ[13] = fTmp0C_z * x;
    b.dX[14] = fTmp1B * fC1_x; b.dY[14] = fTmp1B * fC1_y; b.dZ[14] = fTmp1B_z * fC1;
    b.dX[15] = -0.5900435899266435f * fC2_x; b.dY[15] = -0.5900435899266435f * fC2_y;
    if (degree < 4) return;
    const float fTmp0D = z * (-4.683325804901025f * z2 + 2.007139630671868f);
    const float fTmp1C = 3.31161143515146f * z2 - 0.47308734787878f;
    const float fTmp2B = -1.770130769779931f * z;
    const float fC3 = x * fC2 - y * fS2, fS3 = x * fS2 + y * fC2;
    b.Y[16] = 0.6258357354491763f * fS3;
    b.Y[17] = fTmp2B * fS2;
    b.Y[18] = fTmp1C * fS1;
    b.Y[19] = fTmp0D * y;
    b.Y[20] = 1.984313483298443f * z * pSH12 - 1.006230589874905f * pSH6;
    b.Y[21] = fTmp0D * x;
    b.Y[22] = fTmp1C * fC1;
    b.Y[23] = fTmp2B * fC2;
    b.Y[24] = 0.6258357354491763f * fC3;
    const float fTmp0D_z = 3.f * -4.683325804901025f * z2 + 2.007139630671868f;
    const float fTmp1C_z = 2.f * 3.31161143515146f * z;
    const float fTmp2B_z = -1.770130769779931f;
    const float fC3_x = fC2 + x * fC2_x - y * fS2_x, fC3_y = x * fC2_y - fS2 - y * fS2_y;
    const float fS3_x = fS2 + y * fC2_x + x * fS2_x, fS3_y = x * fS2_y + fC2 + y * fC2_y;
    b.dX[16] = 0.6258357354491763f * fS3_x; b.dY[16] = 0.6258357354491763f * fS3_y;
    b.dX[17] = fTmp2B * fS2_x; b.dY[17] = fTmp2B * fS2_y; b.dZ[17] = fTmp2B_z * fS2;
    b.dX[18] = fTmp1C * fS1_x; b.dY[18] = fTmp1C * fS1_y; b.dZ[18] = fTmp1C_z * fS1;
    b.dY[19] = fTmp0D; b.dZ[19] = fTmp0D_z * y;
    b.dZ[20] = 1.984313483298443f * (pSH12 + z * pSH12_z) - 1.006230589874905f * pSH6_z;
    b.dX[21] = fTmp0D; b.dZ[21] = fTmp0D_z * x;
    b.dX[22] = fTmp1C * fC1_x; b.dY[22] = fTmp1C * fC1_y; b.dZ[22] = fTmp1C_z * fC1;
    b.dX[23] = fTmp2B * fC2_x; b.dY[23] = fTmp2B * fC2_y; b.dZ[23] = fTmp2B_z * fC2;
    b.dX[24] = 0.6258357354491763f * fC3_x; b.dY[24] = 0.6258357354491763f * fC3_y;
}

// Normalization Jacobian of the direction: v_raw = (v_n - (v_n . n) n) / |raw|.
SX_DEV void sh_dir_vjp(const ShBasis& b, float vx, float vy, float vz, float* out) {
    const float dot = vx * b.x + vy * b.y + vz * b.z;
    out[0] = (vx - dot * b.x) * b.inorm;
    out[1] = (vy - dot * b.y) * b.inorm;
    out[2] = (vz - dot * b.z) * b.inorm;
}

// ---------------------------------------------------------------------------------------------
// Tile sets — CpuKernels.cpp:390-564 (AABB rectangle; AccuTile SNUGBOX + strip sweep).
// The sweep calls `emit(tile_id)` for every tile in the reference emit order.
// ---------------------------------------------------------------------------------------------
struct TileRect {
    int32_t min_x, min_y, max_x, max_y;
};

SX_DEV TileRect aabb_rect(float mean_x, float mean_y, float radius_x, float radius_y, float ts,
                          int32_t tw, int32_t th) {
    const float trx = radius_x / ts, try_ = radius_y / ts;
    const float tx = mean_x / ts, ty = mean_y / ts;
    TileRect r;
    r.min_x = imin(imax(0, sxm::f2i_trunc(__builtin_floorf(tx - trx))), tw);
    r.min_y = imin(imax(0, sxm::f2i_trunc(__builtin_floorf(ty - try_))), th);
    r.max_x = imin(imax(0, sxm::f2i_trunc(__builtin_ceilf(tx + trx))), tw);
    r.max_y = imin(imax(0, sxm::f2i_trunc(__builtin_ceilf(ty + try_))), th);
    return r;
}

struct F2 {
    float x, y;
};

SX_DEV F2 ellipse_intersection(float A, float B, float C, float disc, float t, F2 p, bool isY,
                               float coord) {
    const float p_u = isY ? p.y : p.x;
    const float p_v = isY ? p.x : p.y;
    const float coeff = isY ? A : C;
    const float h = coord - p_u;
    const float sqrt_term = __builtin_sqrtf(disc * h * h + t * coeff);
    F2 r;
    r.x = (-B * h - sqrt_term) / coeff + p_v;
    r.y = (-B * h + sqrt_term) / coeff + p_v;
    return r;
}

// AccuTile sweep state of one Gaussian after SNUGBOX and the line/column swap: lines u in
// [rect_min_x, rect_max_x), each a run of tiles v in [vmin, vmax) of the other axis.
struct AccuSweep {
    float A, B, C, disc, t;
    F2 p, bbox_min, bbox_max, bbox_argmin, bbox_argmax;
    int32_t rect_min_x, rect_min_y, rect_max_x, rect_max_y;
    bool isY;
};

// false when the Gaussian covers no tile
SX_DEV bool accutile_setup(float A, float B, float C, float opacity, float mean_x, float mean_y, float ts,
                           int32_t tw, int32_t th, AccuSweep& s) {
    s.A = A;
    s.B = B;
    s.C = C;
    s.disc = B * B - A * C;
    s.t = __builtin_fminf(sx::kGaussianExtend * sx::kGaussianExtend,
                          2.0f * sxm::logf_(opacity / sx::kAlphaThreshold));
    if (s.t <= 0.f) return false;
    const float neg_t_over_disc = -s.t / s.disc;
    const float x_extent = __builtin_sqrtf(neg_t_over_disc * C);
    const float y_extent = __builtin_sqrtf(neg_t_over_disc * A);
    F2 bbox_min = {mean_x - x_extent, mean_y - y_extent};
    F2 bbox_max = {mean_x + x_extent, mean_y + y_extent};
    const float Bx_over_C = B * x_extent / C;
    const float By_over_A = B * y_extent / A;
    F2 bbox_argmin = {mean_y + Bx_over_C, mean_x + By_over_A};
    F2 bbox_argmax = {mean_y - Bx_over_C, mean_x - By_over_A};
    int32_t rect_min_x = imax(0, imin(tw, sxm::f2i_trunc(bbox_min.x / ts)));
    int32_t rect_min_y = imax(0, imin(th, sxm::f2i_trunc(bbox_min.y / ts)));
    int32_t rect_max_x = imax(0, imin(tw, sxm::f2i_trunc(bbox_max.x / ts + 1.f)));
    int32_t rect_max_y = imax(0, imin(th, sxm::f2i_trunc(bbox_max.y / ts + 1.f)));
    const int32_t y_span = rect_max_y - rect_min_y;
    const int32_t x_span = rect_max_x - rect_min_x;
    if (y_span * x_span == 0) return false;
    s.isY = y_span < x_span;
    s.p = {mean_x, mean_y};
    if (s.isY) {
        int32_t tmp = rect_min_x; rect_min_x = rect_min_y; rect_min_y = tmp;
        tmp = rect_max_x; rect_max_x = rect_max_y; rect_max_y = tmp;
        bbox_min = {bbox_min.y, bbox_min.x};
        bbox_max = {bbox_max.y, bbox_max.x};
        bbox_argmin = {bbox_argmin.y, bbox_argmin.x};
        bbox_argmax = {bbox_argmax.y, bbox_argmax.x};
    }
    s.bbox_min = bbox_min;
    s.bbox_max = bbox_max;
    s.bbox_argmin = bbox_argmin;
    s.bbox_argmax = bbox_argmax;
    s.rect_min_x = rect_min_x;
    s.rect_min_y = rect_min_y;
    s.rect_max_x = rect_max_x;
    s.rect_max_y = rect_max_y;
    return true;
}

SX_DEV F2 accutile_cut(const AccuSweep& s, float coord) {
    return ellipse_intersection(s.A, s.B, s.C, s.disc, s.t, s.p, s.isY, coord);
}

// The tile run of the line [min_line, max_line) given the ellipse cuts at its two edges.
SX_DEV void accutile_span(const AccuSweep& s, float min_line, float max_line, F2 imin_line, F2 imax_line, float ts,
                          int32_t& vmin, int32_t& vmax) {
    float emin, emax;
    if (min_line <= s.bbox_argmin.y && s.bbox_argmin.y < max_line) emin = s.bbox_min.y;
    else emin = __builtin_fminf(imin_line.x, imax_line.x);
    if (min_line <= s.bbox_argmax.y && s.bbox_argmax.y < max_line) emax = s.bbox_max.y;
    else emax = __builtin_fmaxf(imin_line.y, imax_line.y);
    vmin = imax(s.rect_min_y, imin(s.rect_max_y, sxm::f2i_trunc(emin / ts)));
    vmax = imin(s.rect_max_y, imax(s.rect_min_y, sxm::f2i_trunc(emax / ts + 1.f)));
}

// The sweep's cut state, stated per line (lines can then be evaluated independently): line u spans
// [u ts, (u + 1) ts) (exact in float), its upper cut is the ellipse cut at (u + 1) ts while that edge
// is <= bbox_max.x and otherwise the last such cut (the start value {bbox_max.y, bbox_min.y} if there
// was none), and its lower cut is the previous line's upper cut — for the first line the cut at its
// own edge when bbox_min.x <= that edge, else the start value.
SX_DEV F2 accutile_start(const AccuSweep& s) { return F2{s.bbox_max.y, s.bbox_min.y}; }

// AccuTile for one Gaussian as a sweep over lines: calls line(u, vmin, vmax, isY) for every line u
// of the sweep in order, the line's tiles being v in [vmin, vmax) with tile id u * tw + v when isY,
// else v * tw + u (the reference's emit order). line returns false to end the sweep early.
template <class Line>
SX_DEV void accutile_lines(float A, float B, float C, float opacity, float mean_x, float mean_y, float ts,
                           int32_t tw, int32_t th, Line line) {
    AccuSweep s;
    if (!accutile_setup(A, B, C, opacity, mean_x, mean_y, ts, tw, th, s)) return;
    const float BLOCK = ts;
    F2 imin_line, imax_line;
    imax_line = accutile_start(s);
    float min_line = s.rect_min_x * BLOCK;
    if (s.bbox_min.x <= min_line) imin_line = accutile_cut(s, min_line);
    else imin_line = imax_line;
    for (int32_t u = s.rect_min_x; u < s.rect_max_x; ++u) {
        const float max_line = min_line + BLOCK;
        if (max_line <= s.bbox_max.x) imax_line = accutile_cut(s, max_line);
        int32_t vmin, vmax;
        accutile_span(s, min_line, max_line, imin_line, imax_line, BLOCK, vmin, vmax);
        if (!line(u, vmin, vmax, s.isY)) return;
        imin_line = imax_line;
        min_line = max_line;
    }
}

// AccuTile for one Gaussian. Returns the tile count; calls emit(tile_id) in emit order when
// EMIT is true.
template <bool EMIT, class Emit>
SX_DEV uint32_t accutile(float A, float B, float C, float opacity, float mean_x, float mean_y, float ts,
                         int32_t tw, int32_t th, Emit emit) {
    uint32_t count = 0;
    accutile_lines(A, B, C, opacity, mean_x, mean_y, ts, tw, th, [&](int32_t u, int32_t vmin, int32_t vmax, bool isY) {
        if (EMIT) {
            for (int32_t v = vmin; v < vmax; ++v) emit(isY ? u * tw + v : v * tw + u);
        }
        if (vmax > vmin) count += static_cast<uint32_t>(vmax - vmin);
        return true;
    });
    return count;
}

} // namespace sxd
