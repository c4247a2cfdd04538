// sx_dev_bwd.h — gfx950 device functions of the backward pass shared by the per-op kernels and
// the fused resident-step kernels: the projection VJP (ProjectionEWA.metal:186-560 mathematics),
// the quaternion/scale covariance VJP, and the MCMC position perturbation of one Gaussian
// (CpuKernels.cpp:969-1008 expression forms).
#pragma once

#include "sx_dev.h"

namespace sxd {

__device__ __forceinline__ void mm3(const float* a, const float* b, float* c) {  // c = a b
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) c[i * 3 + j] = a[i * 3] * b[j] + a[i * 3 + 1] * b[3 + j] + a[i * 3 + 2] * b[6 + j];
}
__device__ __forceinline__ void mm3_tn(const float* a, const float* b, float* c) {  // c = a^T b
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) c[i * 3 + j] = a[i] * b[j] + a[3 + i] * b[3 + j] + a[6 + i] * b[6 + j];
}
__device__ __forceinline__ void mm3_nt(const float* a, const float* b, float* c) {  // c = a b^T
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++)
            c[i * 3 + j] = a[i * 3] * b[j * 3] + a[i * 3 + 1] * b[j * 3 + 1] + a[i * 3 + 2] * b[j * 3 + 2];
}

struct ProjGrad {
    float vmean[3];
    float vcov[9];   // world covariance gradient (row-major)
    float vR[9];
    float vt[3];
};

// Gradient of one (camera, Gaussian) pair with respect to the world mean, world covariance and
// the view rotation/translation.
__device__ __forceinline__ void proj_vjp_one(const sxd::Cam& cam, const float* mw, const float* Cw, float ca,
                                    float cb, float cc, float v_m2x, float v_m2y, float v_depth,
                                    float va, float vb, float vc, bool has_comp, float comp,
                                    float v_comp, float eps2d, ProjGrad& out) {
    // B1: v_cov2d = -P vP P
    const float P00 = ca, P01 = cb, P11 = cc;
    const float q00 = va, q01 = vb * 0.5f, q11 = vc;
    const float t00 = P00 * q00 + P01 * q01, t01 = P00 * q01 + P01 * q11;
    const float t10 = P01 * q00 + P11 * q01, t11 = P01 * q01 + P11 * q11;
    float g00 = -(t00 * P00 + t01 * P01), g01 = -(t00 * P01 + t01 * P11);
    float g10 = -(t10 * P00 + t11 * P01), g11 = -(t10 * P01 + t11 * P11);
    // B2: compensation
    if (has_comp) {
        const float det_cb = P00 * P11 - P01 * P01;
        const float v_sqr = v_comp * 0.5f / (comp + 1e-6f);
        const float om = 1.f - comp * comp;
        g00 += v_sqr * (om * P00 - eps2d * det_cb);
        g01 += v_sqr * (om * P01);
        g10 += v_sqr * (om * P01);
        g11 += v_sqr * (om * P11 - eps2d * det_cb);
    }
    // B3: rematerialize
    const float* R = cam.R;
    float pc[3];
#pragma unroll
    for (int i = 0; i < 3; i++) pc[i] = R[i * 3] * mw[0] + R[i * 3 + 1] * mw[1] + R[i * 3 + 2] * mw[2] + cam.t[i];
    float RC[9], Cc[9];
    mm3(R, Cw, RC);
    mm3_nt(RC, R, Cc);
    const float x = pc[0], y = pc[1], z = pc[2];
    const float rz = 1.f / z, rz2 = rz * rz, rz3 = rz2 * rz;
    const float xr = x * rz, yr = y * rz;
    const float tx = z * sxd::smin(cam.lim_x_pos, sxd::smax(-cam.lim_x_neg, xr));
    const float ty = z * sxd::smin(cam.lim_y_pos, sxd::smax(-cam.lim_y_neg, yr));
    const float J[6] = {cam.fx * rz, 0.f, -cam.fx * tx * rz2, 0.f, cam.fy * rz, -cam.fy * ty * rz2};
    const float G[4] = {g00, g01, g10, g11};
    // v_cov_c = J^T G J
    float vCc[9];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) {
            float s = 0.f;
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int q = 0; q < 2; q++) s += J[p * 3 + i] * G[p * 2 + q] * J[q * 3 + j];
            vCc[i * 3 + j] = s;
        }
    float vpc[3] = {cam.fx * rz * v_m2x, cam.fy * rz * v_m2y, -(cam.fx * x * v_m2x + cam.fy * y * v_m2y) * rz2};
    // v_J = G J Cc^T + G^T J Cc
    float vJ[6];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int j = 0; j < 3; j++) {
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int k = 0; k < 3; k++)
                    s += G[p * 2 + q] * J[q * 3 + k] * Cc[j * 3 + k] + G[q * 2 + p] * J[q * 3 + k] * Cc[k * 3 + j];
            vJ[p * 3 + j] = s;
        }
    if (xr <= cam.lim_x_pos && xr >= -cam.lim_x_neg) vpc[0] += -cam.fx * rz2 * vJ[2];
    else vpc[2] += -cam.fx * rz3 * vJ[2] * tx;
    if (yr <= cam.lim_y_pos && yr >= -cam.lim_y_neg) vpc[1] += -cam.fy * rz2 * vJ[5];
    else vpc[2] += -cam.fy * rz3 * vJ[5] * ty;
    vpc[2] += -cam.fx * rz2 * vJ[0] - cam.fy * rz2 * vJ[4] + 2.f * cam.fx * tx * rz3 * vJ[2] +
              2.f * cam.fy * ty * rz3 * vJ[5];
    vpc[2] += v_depth;
    // B6: world
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) out.vR[i * 3 + j] = vpc[i] * mw[j];
#pragma unroll
    for (int i = 0; i < 3; i++) out.vt[i] = vpc[i];
#pragma unroll
    for (int j = 0; j < 3; j++) out.vmean[j] = R[j] * vpc[0] + R[3 + j] * vpc[1] + R[6 + j] * vpc[2];
    float t1[9], a1[9], t2[9], a2[9];
    mm3(vCc, R, t1);
    mm3_nt(t1, Cw, a1);       // vCc R Cw^T
    mm3_tn(vCc, R, t2);       // vCc^T R
    mm3(t2, Cw, a2);          // vCc^T R Cw
#pragma unroll
    for (int i = 0; i < 9; i++) out.vR[i] += a1[i] + a2[i];
    float t3[9];
    mm3_tn(R, vCc, t3);       // R^T vCc
    mm3(t3, R, out.vcov);     // R^T vCc R
}

// quat_scale_to_covar VJP (ProjectionEWA.metal:295-337): normalized rotation, M = R diag(s),
// v_M = (G + G^T) M, v_R = v_M diag(s), v_s_j = col_j(R) . col_j(v_M); quaternion VJP projected
// onto the tangent plane of the unit sphere.
__device__ __forceinline__ void quat_scale_vjp(const float* q, const float* s, const float* vcov, float* vq,
                                      float* vs) {
    float w = q[0], x = q[1], y = q[2], z = q[3];
    const float inv_norm = 1.f / __builtin_sqrtf(x * x + y * y + z * z + w * w);
    w *= inv_norm; x *= inv_norm; y *= inv_norm; z *= inv_norm;
    float R[9];
    R[0] = 1.f - 2.f * (y * y + z * z); R[1] = 2.f * (x * y - w * z); R[2] = 2.f * (x * z + w * y);
    R[3] = 2.f * (x * y + w * z); R[4] = 1.f - 2.f * (x * x + z * z); R[5] = 2.f * (y * z - w * x);
    R[6] = 2.f * (x * z - w * y); R[7] = 2.f * (y * z + w * x); R[8] = 1.f - 2.f * (x * x + y * y);
    float M[9], S2[9], vM[9], VR[9];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) {
            M[i * 3 + j] = R[i * 3 + j] * s[j];
            S2[i * 3 + j] = vcov[i * 3 + j] + vcov[j * 3 + i];
        }
    mm3(S2, M, vM);
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) VR[i * 3 + j] = vM[i * 3 + j] * s[j];
#define V(r, c) VR[(r) * 3 + (c)]
    const float vqn0 = 2.f * (x * (V(2, 1) - V(1, 2)) + y * (V(0, 2) - V(2, 0)) + z * (V(1, 0) - V(0, 1)));
    const float vqn1 = 2.f * (-2.f * x * (V(1, 1) + V(2, 2)) + y * (V(1, 0) + V(0, 1)) +
                              z * (V(2, 0) + V(0, 2)) + w * (V(2, 1) - V(1, 2)));
    const float vqn2 = 2.f * (x * (V(1, 0) + V(0, 1)) - 2.f * y * (V(0, 0) + V(2, 2)) +
                              z * (V(2, 1) + V(1, 2)) + w * (V(0, 2) - V(2, 0)));
    const float vqn3 = 2.f * (x * (V(2, 0) + V(0, 2)) + y * (V(2, 1) + V(1, 2)) -
                              2.f * z * (V(0, 0) + V(1, 1)) + w * (V(1, 0) - V(0, 1)));
#undef V
    const float dot = vqn0 * w + vqn1 * x + vqn2 * y + vqn3 * z;
    vq[0] = (vqn0 - dot * w) * inv_norm;
    vq[1] = (vqn1 - dot * x) * inv_norm;
    vq[2] = (vqn2 - dot * y) * inv_norm;
    vq[3] = (vqn3 - dot * z) * inv_norm;
#pragma unroll
    for (int j = 0; j < 3; j++) vs[j] = R[j] * vM[j] + R[3 + j] * vM[3 + j] + R[6 + j] * vM[6 + j];
}


// Eq.9 relocation of one source (CpuKernels.cpp:924-960 forms: clamp first, then the (i,k)
// ascending sum) — shared by the per-op kernel and the device refine. Returns the new opacity and
// the factor that scales the linear scales.
__device__ __forceinline__ float relocation_one(float old_op, int n_idx, const float* __restrict__ binoms, int n_max,
                                                float min_opacity, float* coeff) {
    float nop = 1.0f - sxm::powf_(1.0f - old_op, 1.0f / static_cast<float>(n_idx));
    nop = smin(smax(nop, min_opacity), 1.0f - 1.1920928955078125e-07f);
    float denom = 0.0f;
    for (int i = 1; i <= n_idx; i++)
        for (int k = 0; k <= i - 1; k++) {
            const float bin = binoms[(i - 1) * n_max + k];
            const float sign = (k & 1) ? -1.0f : 1.0f;
            const float term = (sign / __builtin_sqrtf(static_cast<float>(k + 1))) *
                               sxm::powf_(nop, static_cast<float>(k + 1));
            denom += bin * term;
        }
    *coeff = old_op / denom;
    return nop;
}

// Perturbation of one Gaussian (CpuKernels.cpp:969-1008 forms) — shared with the fused step.
__device__ __forceinline__ void perturb_one(float* pos, const float* q, const float* slog, float logit, const float* nz,
                            float noise_scale, float tt, float kk) {
    float w = q[0], x = q[1], y = q[2], z = q[3];
    const float inv_norm = 1.0f / __builtin_sqrtf(x * x + y * y + z * z + w * w);
    x *= inv_norm; y *= inv_norm; z *= inv_norm; w *= inv_norm;
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    const float wx = w * x, wy = w * y, wz = w * z;
    const float R[9] = {1.f - 2.f * (y2 + z2), 2.f * (xy - wz), 2.f * (xz + wy),
                        2.f * (xy + wz), 1.f - 2.f * (x2 + z2), 2.f * (yz - wx),
                        2.f * (xz - wy), 2.f * (yz + wx), 1.f - 2.f * (x2 + y2)};
    const float s[3] = {sxm::expf_(slog[0]), sxm::expf_(slog[1]), sxm::expf_(slog[2])};
    float M[9], Cm[9];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) M[i * 3 + j] = R[i * 3 + j] * s[j];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++)
            Cm[i * 3 + j] = M[i * 3] * M[j * 3] + M[i * 3 + 1] * M[j * 3 + 1] + M[i * 3 + 2] * M[j * 3 + 2];
    const float density = 1.0f / (1.0f + sxm::expf_(-logit));
    const float gate = 1.0f / (1.0f + sxm::expf_(kk * (density - tt)));
    const float wgt = gate * noise_scale;
    const float n0 = nz[0] * wgt, n1 = nz[1] * wgt, n2 = nz[2] * wgt;
    pos[0] += Cm[0] * n0 + Cm[1] * n1 + Cm[2] * n2;
    pos[1] += Cm[3] * n0 + Cm[4] * n1 + Cm[5] * n2;
    pos[2] += Cm[6] * n0 + Cm[7] * n1 + Cm[8] * n2;
}


} // namespace sxd
