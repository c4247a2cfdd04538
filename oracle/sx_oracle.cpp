// sx_oracle.cpp — CPU oracle of the splatx 3DGS training step. TEST INFRASTRUCTURE ONLY: it is
// the checker for the gfx950 backend and the timed CPU baseline, never part of the product path.
//
// Forward ops restate /root/reference Sources/SplatXCore/CpuKernels.cpp (+ Math.cpp) statement
// by statement, keeping the reference's expression forms and evaluation order so that results
// stay bit-comparable; each function cites the lines it follows. Backward ops restate the
// mathematics of the reference kernels (the reference has no CPU backward). Transcendentals go
// through o_exp/o_log/... which are glibc (SX_ORACLE_LIBM, identical to the reference) or the
// deterministic sx_fmath.h functions shared with the device code.
#include "sx_oracle.h"

#include <algorithm>
#include <cfloat>
#include <chrono>
#include <cmath>
#include <cstring>
#include <numeric>
#include <random>
#include <sstream>
#include <unordered_map>
#include <stdexcept>
#include <string>
#include <vector>

#include "sx_common.h"
#include "sx_fmath.h"

namespace {

thread_local std::string g_err;

#ifdef SX_ORACLE_LIBM
inline float o_exp(float x) { return std::exp(x); }
inline float o_exp_raster(float x) { return std::exp(x); }
inline float o_log(float x) { return std::log(x); }
inline float o_pow(float x, float y) { return std::pow(x, y); }
inline void o_sincos(float x, float* s, float* c) {
    *s = std::sin(x);
    *c = std::cos(x);
}
#else
inline float o_exp(float x) { return sxm::expf_(x); }
inline float o_exp_raster(float x) { return sxm::expf_fast(x); }
inline float o_log(float x) { return sxm::logf_(x); }
inline float o_pow(float x, float y) { return sxm::powf_(x, y); }
inline void o_sincos(float x, float* s, float* c) { sxm::sincosf_(x, s, c); }
#endif

[[noreturn]] void invalid(const char* what, const std::string& msg) {
    throw std::invalid_argument(std::string(what) + ": " + msg);
}

struct CapacityError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

template <class F>
int32_t guarded(F&& f) {
    try {
        f();
        g_err.clear();
        return SXH_OK;
    } catch (const std::invalid_argument& e) {
        g_err = e.what();
        return SXH_ERR_INVALID_ARGUMENT;
    } catch (const CapacityError& e) {
        g_err = e.what();
        return SXH_ERR_CAPACITY;
    } catch (const std::exception& e) {
        g_err = e.what();
        return SXH_ERR_RUNTIME;
    }
}

// ------------------------------------------------------------------------------------------
// Math.cpp:9-45 (row-major 3x3, mat3_mul accumulates s = 0; s += a*b in k order)
// ------------------------------------------------------------------------------------------
struct M3 {
    float m[9];
};

M3 mat3_mul(const M3& a, const M3& b) {
    M3 c;
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) {
            float s = 0;
            for (int k = 0; k < 3; k++) s += a.m[i * 3 + k] * b.m[k * 3 + j];
            c.m[i * 3 + j] = s;
        }
    return c;
}

M3 mat3_transpose(const M3& a) {
    M3 t;
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) t.m[i * 3 + j] = a.m[j * 3 + i];
    return t;
}

M3 quat_to_rotmat(const float q[4]) { // Math.cpp:9-18
    float w = q[0], x = q[1], y = q[2], z = q[3];
    float n = std::sqrt(w * w + x * x + y * y + z * z);
    if (n > 0.0f) {
        w /= n;
        x /= n;
        y /= n;
        z /= n;
    }
    M3 R;
    R.m[0] = 1 - 2 * (y * y + z * z);
    R.m[1] = 2 * (x * y - w * z);
    R.m[2] = 2 * (x * z + w * y);
    R.m[3] = 2 * (x * y + w * z);
    R.m[4] = 1 - 2 * (x * x + z * z);
    R.m[5] = 2 * (y * z - w * x);
    R.m[6] = 2 * (x * z - w * y);
    R.m[7] = 2 * (y * z + w * x);
    R.m[8] = 1 - 2 * (x * x + y * y);
    return R;
}

M3 quat_scale_to_covar(const float q[4], const float s[3]) { // Math.cpp:37-43
    M3 R = quat_to_rotmat(q);
    M3 M = R;
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) M.m[i * 3 + j] *= s[j];
    return mat3_mul(M, mat3_transpose(M));
}

} // namespace

extern "C" {

const char* sxo_last_error(void) { return g_err.c_str(); }

int32_t sxo_uses_libm(void) {
#ifdef SX_ORACLE_LIBM
    return 1;
#else
    return 0;
#endif
}

int32_t sxo_quat_scale_to_covar(const float* quats, const float* scales, int64_t n, float* out) {
    return guarded([&] {
        for (int64_t i = 0; i < n; i++) {
            const M3 c = quat_scale_to_covar(quats + i * 4, scales + i * 3);
            std::memcpy(out + i * 9, c.m, sizeof(c.m));
        }
    });
}

// ------------------------------------------------------------------------------------------
// fused_adam — CpuKernels.cpp:127-144 (Validate.h:40-45)
// ------------------------------------------------------------------------------------------
int32_t sxo_fused_adam(const sxh_adam_inputs* in) {
    return guarded([&] {
        if (in->n_elems == 0) return;
        if (!in->param || !in->grad || !in->exp_avg || !in->exp_avg_sq)
            invalid("fused_adam_cpu", "null tensor");
        if (in->n_elems < 0 || in->n_gauss <= 0 || in->n_elems % in->n_gauss != 0)
            invalid("fused_adam_cpu", "n_elems must be a positive multiple of n_gauss");
        const int64_t D = in->n_elems / in->n_gauss;
        for (int64_t p = 0; p < in->n_elems; p++) {
            if (in->valid && in->valid[p / D] == 0) continue;
            const float g = in->grad[p];
            float m = in->exp_avg[p];
            float v = in->exp_avg_sq[p];
            m = in->b1 * m + (1.0f - in->b1) * g;
            v = in->b2 * v + (1.0f - in->b2) * g * g;
            const float step = -in->lr * m / (std::sqrt(v) + in->eps);
            in->param[p] += step;
            in->exp_avg[p] = m;
            in->exp_avg_sq[p] = v;
        }
    });
}

// ------------------------------------------------------------------------------------------
// projection_fused_fwd — CpuKernels.cpp:155-272 (Validate.h:50-62)
// ------------------------------------------------------------------------------------------
static void validate_projection(const sxh_projection_inputs* in, const char* what) {
    if (in->camera_model != 0)
        throw std::runtime_error(std::string(what) + ": only PINHOLE (camera_model=0) supported");
    if (!in->means || !in->viewmats || !in->Ks) invalid(what, "null means/viewmats/Ks");
    if (!in->covars && (!in->quats || !in->scales))
        invalid(what, "need covars (6-triu) or quats+scales");
    if (in->N < 0 || in->C < 0) invalid(what, "negative N or C");
}

int32_t sxo_projection_fused_fwd(const sxh_projection_inputs* in, sxh_projection_outputs* out) {
    return guarded([&] {
        validate_projection(in, "projection_fused_fwd");
        const int64_t N = in->N, C = in->C;
        const size_t CN = static_cast<size_t>(C * N);
        if (!out->radii || !out->means2d || !out->depths || !out->conics ||
            (in->calc_compensations && !out->compensations))
            invalid("projection_fused_fwd", "null output buffer");
        std::fill(out->radii, out->radii + CN * 2, 0);
        std::fill(out->means2d, out->means2d + CN * 2, 0.0f);
        std::fill(out->depths, out->depths + CN, 0.0f);
        std::fill(out->conics, out->conics + CN * 3, 0.0f);
        if (in->calc_compensations) std::fill(out->compensations, out->compensations + CN, 0.0f);

        for (int64_t c = 0; c < C; c++) {
            const float* V = in->viewmats + c * 16;
            const M3 R = {{V[0], V[1], V[2], V[4], V[5], V[6], V[8], V[9], V[10]}};
            const float tx_ = V[3], ty_ = V[7], tz_ = V[11];
            const float* K = in->Ks + c * 9;
            const float fx = K[0], fy = K[4], cx = K[2], cy = K[5];
            const float tan_fovx = 0.5f * static_cast<float>(in->width) / fx;
            const float tan_fovy = 0.5f * static_cast<float>(in->height) / fy;
            const float lim_x_pos = (static_cast<float>(in->width) - cx) / fx + 0.3f * tan_fovx;
            const float lim_x_neg = cx / fx + 0.3f * tan_fovx;
            const float lim_y_pos = (static_cast<float>(in->height) - cy) / fy + 0.3f * tan_fovy;
            const float lim_y_neg = cy / fy + 0.3f * tan_fovy;

            for (int64_t n = 0; n < N; n++) {
                const size_t gi = static_cast<size_t>(c * N + n);
                const float* mw = in->means + n * 3;
                const float mx = R.m[0] * mw[0] + R.m[1] * mw[1] + R.m[2] * mw[2] + tx_;
                const float my = R.m[3] * mw[0] + R.m[4] * mw[1] + R.m[5] * mw[2] + ty_;
                const float mz = R.m[6] * mw[0] + R.m[7] * mw[1] + R.m[8] * mw[2] + tz_;
                if (mz < in->near_plane || mz > in->far_plane) continue;

                M3 Cw;
                if (in->covars) {
                    const float* cv = in->covars + n * 6;
                    Cw = {{cv[0], cv[1], cv[2], cv[1], cv[3], cv[4], cv[2], cv[4], cv[5]}};
                } else {
                    Cw = quat_scale_to_covar(in->quats + n * 4, in->scales + n * 3);
                }
                const M3 Cc = mat3_mul(mat3_mul(R, Cw), mat3_transpose(R));

                const float rz = 1.0f / mz, rz2 = rz * rz;
                const float txc = mz * std::min(lim_x_pos, std::max(-lim_x_neg, mx * rz));
                const float tyc = mz * std::min(lim_y_pos, std::max(-lim_y_neg, my * rz));
                const float J00 = fx * rz, J02 = -fx * txc * rz2;
                const float J11 = fy * rz, J12 = -fy * tyc * rz2;
                const float JC0[3] = {J00 * Cc.m[0] + J02 * Cc.m[6], J00 * Cc.m[1] + J02 * Cc.m[7],
                                      J00 * Cc.m[2] + J02 * Cc.m[8]};
                const float JC1[3] = {J11 * Cc.m[3] + J12 * Cc.m[6], J11 * Cc.m[4] + J12 * Cc.m[7],
                                      J11 * Cc.m[5] + J12 * Cc.m[8]};
                float c00 = JC0[0] * J00 + JC0[2] * J02;
                const float c01 = JC0[1] * J11 + JC0[2] * J12;
                const float c10 = JC1[0] * J00 + JC1[2] * J02;
                float c11 = JC1[1] * J11 + JC1[2] * J12;
                const float m2x = fx * mx * rz + cx;
                const float m2y = fy * my * rz + cy;

                const float det_orig = c00 * c11 - c01 * c10;
                c00 += in->eps2d;
                c11 += in->eps2d;
                const float det = c00 * c11 - c01 * c10;
                const float compensation =
                    std::sqrt(std::max(sx::kMinCompensation * sx::kMinCompensation, det_orig / det));
                if (det <= 0.0f) continue;

                const float rdet = 1.0f / det;
                const float conic_a = c11 * rdet;
                const float conic_b = -c10 * rdet;
                const float conic_c = c00 * rdet;

                float extend = sx::kGaussianExtend;
                if (in->opacities) {
                    float opacity = in->opacities[n];
                    if (in->calc_compensations) opacity *= compensation;
                    if (opacity < sx::kAlphaThreshold) continue;
                    extend = std::min(sx::kGaussianExtend,
                                      std::sqrt(2.0f * o_log(opacity / sx::kAlphaThreshold)));
                }
                const float radius_x = std::ceil(extend * std::sqrt(c00));
                const float radius_y = std::ceil(extend * std::sqrt(c11));
                if (radius_x <= in->radius_clip && radius_y <= in->radius_clip) continue;
                if (m2x + radius_x <= 0.0f || m2x - radius_x >= static_cast<float>(in->width) ||
                    m2y + radius_y <= 0.0f || m2y - radius_y >= static_cast<float>(in->height))
                    continue;

                out->radii[gi * 2] = static_cast<int32_t>(radius_x);
                out->radii[gi * 2 + 1] = static_cast<int32_t>(radius_y);
                out->means2d[gi * 2] = m2x;
                out->means2d[gi * 2 + 1] = m2y;
                out->depths[gi] = mz;
                out->conics[gi * 3] = conic_a;
                out->conics[gi * 3 + 1] = conic_b;
                out->conics[gi * 3 + 2] = conic_c;
                if (in->calc_compensations) out->compensations[gi] = compensation;
            }
        }
    });
}

// ------------------------------------------------------------------------------------------
// projection_fused_bwd — own CPU restatement of the VJP in ProjectionEWA.metal:186-560
// (inverse_vjp, add_blur_vjp, persp_proj_vjp, posW2C/covarW2C VJPs, quat_scale_to_covar_vjp).
// Rematerializes the forward with the same covariance expression as the forward above.
// Scalar row-major matrices; sums accumulate in double (reference-quality gradients).
// ------------------------------------------------------------------------------------------
namespace {
struct D3 {
    double m[9];
};
inline double& at(D3& a, int r, int c) { return a.m[r * 3 + c]; }
D3 dmul(const D3& a, const D3& b) {
    D3 c{};
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) {
            double s = 0;
            for (int k = 0; k < 3; k++) s += a.m[i * 3 + k] * b.m[k * 3 + j];
            c.m[i * 3 + j] = s;
        }
    return c;
}
D3 dtr(const D3& a) {
    D3 t;
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) t.m[i * 3 + j] = a.m[j * 3 + i];
    return t;
}
D3 dfrom(const M3& a) {
    D3 d;
    for (int i = 0; i < 9; i++) d.m[i] = a.m[i];
    return d;
}
} // namespace

int32_t sxo_projection_fused_bwd(const sxh_projection_inputs* in, const sxh_projection_grads_in* g,
                                 sxh_projection_grads* out) {
    return guarded([&] {
        validate_projection(in, "projection_fused_bwd");
        if (!g->radii || !g->conics || !g->v_means2d || !g->v_depths || !g->v_conics)
            invalid("projection_fused_bwd", "null radii/conics/v_means2d/v_depths/v_conics");
        if (g->v_compensations && !g->compensations)
            invalid("projection_fused_bwd", "v_compensations requires compensations (fwd output)");
        const int64_t N = in->N, C = in->C;
        const bool use_covars = in->covars != nullptr;
        std::vector<double> v_means(N * 3, 0.0), v_covars(use_covars ? N * 6 : 0, 0.0),
            v_quats(use_covars ? 0 : N * 4, 0.0), v_scales(use_covars ? 0 : N * 3, 0.0),
            v_view(C * 16, 0.0);
        for (int64_t c = 0; c < C; c++) {
            const float* vm = in->viewmats + c * 16;
            D3 R;
            for (int i = 0; i < 3; i++)
                for (int j = 0; j < 3; j++) at(R, i, j) = vm[i * 4 + j];
            const double t[3] = {vm[3], vm[7], vm[11]};
            const float* K = in->Ks + c * 9;
            const double fx = K[0], fy = K[4], cx = K[2], cy = K[5];
            const double W = in->width, H = in->height;
            const double tan_fovx = 0.5 * W / fx, tan_fovy = 0.5 * H / fy;
            const double lim_x_pos = (W - cx) / fx + 0.3 * tan_fovx;
            const double lim_x_neg = cx / fx + 0.3 * tan_fovx;
            const double lim_y_pos = (H - cy) / fy + 0.3 * tan_fovy;
            const double lim_y_neg = cy / fy + 0.3 * tan_fovy;
            for (int64_t n = 0; n < N; n++) {
                const int64_t gi = c * N + n;
                if (!(g->radii[gi * 2] > 0 && g->radii[gi * 2 + 1] > 0)) continue;
                // B1: conic -> covar2d VJP: v_cov2d = -P v_P P (P symmetric conic)
                const double a = g->conics[gi * 3], b = g->conics[gi * 3 + 1],
                             cc = g->conics[gi * 3 + 2];
                const double P[2][2] = {{a, b}, {b, cc}};
                const double vP[2][2] = {{g->v_conics[gi * 3], g->v_conics[gi * 3 + 1] * 0.5},
                                         {g->v_conics[gi * 3 + 1] * 0.5, g->v_conics[gi * 3 + 2]}};
                double tmp[2][2], vC2[2][2];
                for (int i = 0; i < 2; i++)
                    for (int j = 0; j < 2; j++)
                        tmp[i][j] = P[i][0] * vP[0][j] + P[i][1] * vP[1][j];
                for (int i = 0; i < 2; i++)
                    for (int j = 0; j < 2; j++)
                        vC2[i][j] = -(tmp[i][0] * P[0][j] + tmp[i][1] * P[1][j]);
                // B2: compensation VJP
                if (g->v_compensations) {
                    const double comp = g->compensations[gi];
                    const double det_cb = a * cc - b * b;
                    const double v_sqr = g->v_compensations[gi] * 0.5 / (comp + 1e-6);
                    const double om = 1.0 - comp * comp;
                    const double e2 = in->eps2d;
                    vC2[0][0] += v_sqr * (om * a - e2 * det_cb);
                    vC2[0][1] += v_sqr * (om * b);
                    vC2[1][0] += v_sqr * (om * b);
                    vC2[1][1] += v_sqr * (om * cc - e2 * det_cb);
                }
                // B3: rematerialize the forward chain
                D3 Cw;
                float qf[4] = {0, 0, 0, 0}, sf[3] = {0, 0, 0};
                if (use_covars) {
                    const float* cv = in->covars + n * 6;
                    const double v6[9] = {cv[0], cv[1], cv[2], cv[1], cv[3], cv[4], cv[2], cv[4], cv[5]};
                    for (int i = 0; i < 9; i++) Cw.m[i] = v6[i];
                } else {
                    std::memcpy(qf, in->quats + n * 4, sizeof(qf));
                    std::memcpy(sf, in->scales + n * 3, sizeof(sf));
                    Cw = dfrom(quat_scale_to_covar(qf, sf));
                }
                const double pw[3] = {in->means[n * 3], in->means[n * 3 + 1], in->means[n * 3 + 2]};
                double pc[3];
                for (int i = 0; i < 3; i++)
                    pc[i] = at(R, i, 0) * pw[0] + at(R, i, 1) * pw[1] + at(R, i, 2) * pw[2] + t[i];
                D3 Cc = dmul(dmul(R, Cw), dtr(R));
                // B4: persp_proj VJP (PINHOLE)
                const double x = pc[0], y = pc[1], z = pc[2];
                const double rz = 1.0 / z, rz2 = rz * rz, rz3 = rz2 * rz;
                const double tx = z * std::min(lim_x_pos, std::max(-lim_x_neg, x * rz));
                const double ty = z * std::min(lim_y_pos, std::max(-lim_y_neg, y * rz));
                const double J[2][3] = {{fx * rz, 0.0, -fx * tx * rz2}, {0.0, fy * rz, -fy * ty * rz2}};
                D3 vCc{};
                for (int i = 0; i < 3; i++)
                    for (int j = 0; j < 3; j++) {
                        double s = 0;
                        for (int p = 0; p < 2; p++)
                            for (int q = 0; q < 2; q++) s += J[p][i] * vC2[p][q] * J[q][j];
                        at(vCc, i, j) = s;
                    }
                const double vm2x = g->v_means2d[gi * 2], vm2y = g->v_means2d[gi * 2 + 1];
                double vpc[3] = {fx * rz * vm2x, fy * rz * vm2y, -(fx * x * vm2x + fy * y * vm2y) * rz2};
                // v_J = vC2 J Cc^T + vC2^T J Cc (2x3)
                double vJ[2][3];
                for (int p = 0; p < 2; p++)
                    for (int j = 0; j < 3; j++) {
                        double s = 0;
                        for (int q = 0; q < 2; q++)
                            for (int k = 0; k < 3; k++)
                                s += vC2[p][q] * J[q][k] * at(Cc, j, k) + vC2[q][p] * J[q][k] * at(Cc, k, j);
                        vJ[p][j] = s;
                    }
                if (x * rz <= lim_x_pos && x * rz >= -lim_x_neg) vpc[0] += -fx * rz2 * vJ[0][2];
                else vpc[2] += -fx * rz3 * vJ[0][2] * tx;
                if (y * rz <= lim_y_pos && y * rz >= -lim_y_neg) vpc[1] += -fy * rz2 * vJ[1][2];
                else vpc[2] += -fy * rz3 * vJ[1][2] * ty;
                vpc[2] += -fx * rz2 * vJ[0][0] - fy * rz2 * vJ[1][1] + 2.0 * fx * tx * rz3 * vJ[0][2] +
                          2.0 * fy * ty * rz3 * vJ[1][2];
                // B5
                vpc[2] += g->v_depths[gi];
                // B6: camera -> world
                D3 vR{};
                for (int i = 0; i < 3; i++)
                    for (int j = 0; j < 3; j++) at(vR, i, j) += vpc[i] * pw[j];
                double vt[3] = {vpc[0], vpc[1], vpc[2]};
                double vpw[3];
                for (int j = 0; j < 3; j++)
                    vpw[j] = at(R, 0, j) * vpc[0] + at(R, 1, j) * vpc[1] + at(R, 2, j) * vpc[2];
                {
                    D3 a1 = dmul(dmul(vCc, R), dtr(Cw));
                    D3 a2 = dmul(dmul(dtr(vCc), R), Cw);
                    for (int i = 0; i < 9; i++) vR.m[i] += a1.m[i] + a2.m[i];
                }
                D3 vCw = dmul(dmul(dtr(R), vCc), R);
                for (int j = 0; j < 3; j++) v_means[n * 3 + j] += vpw[j];
                if (use_covars) {
                    v_covars[n * 6 + 0] += at(vCw, 0, 0);
                    v_covars[n * 6 + 1] += at(vCw, 0, 1) + at(vCw, 1, 0);
                    v_covars[n * 6 + 2] += at(vCw, 0, 2) + at(vCw, 2, 0);
                    v_covars[n * 6 + 3] += at(vCw, 1, 1);
                    v_covars[n * 6 + 4] += at(vCw, 1, 2) + at(vCw, 2, 1);
                    v_covars[n * 6 + 5] += at(vCw, 2, 2);
                } else {
                    // B7: quat_scale_to_covar VJP (normalized rotation, M = R diag(s), covar = M M^T)
                    double w = qf[0], qx = qf[1], qy = qf[2], qz = qf[3];
                    const double inv_norm = 1.0 / std::sqrt(qx * qx + qy * qy + qz * qz + w * w);
                    w *= inv_norm; qx *= inv_norm; qy *= inv_norm; qz *= inv_norm;
                    D3 Rg;
                    at(Rg, 0, 0) = 1 - 2 * (qy * qy + qz * qz); at(Rg, 0, 1) = 2 * (qx * qy - w * qz);
                    at(Rg, 0, 2) = 2 * (qx * qz + w * qy);     at(Rg, 1, 0) = 2 * (qx * qy + w * qz);
                    at(Rg, 1, 1) = 1 - 2 * (qx * qx + qz * qz); at(Rg, 1, 2) = 2 * (qy * qz - w * qx);
                    at(Rg, 2, 0) = 2 * (qx * qz - w * qy);     at(Rg, 2, 1) = 2 * (qy * qz + w * qx);
                    at(Rg, 2, 2) = 1 - 2 * (qx * qx + qy * qy);
                    const double s3[3] = {sf[0], sf[1], sf[2]};
                    D3 M;
                    for (int i = 0; i < 3; i++)
                        for (int j = 0; j < 3; j++) at(M, i, j) = at(Rg, i, j) * s3[j];
                    D3 S2;
                    for (int i = 0; i < 9; i++) S2.m[i] = vCw.m[i];
                    D3 S2t = dtr(S2);
                    for (int i = 0; i < 9; i++) S2.m[i] += S2t.m[i];
                    D3 vM = dmul(S2, M);
                    D3 VR;
                    for (int i = 0; i < 3; i++)
                        for (int j = 0; j < 3; j++) at(VR, i, j) = at(vM, i, j) * s3[j];
                    const double vqn[4] = {
                        2 * (qx * (at(VR, 2, 1) - at(VR, 1, 2)) + qy * (at(VR, 0, 2) - at(VR, 2, 0)) +
                             qz * (at(VR, 1, 0) - at(VR, 0, 1))),
                        2 * (-2 * qx * (at(VR, 1, 1) + at(VR, 2, 2)) + qy * (at(VR, 1, 0) + at(VR, 0, 1)) +
                             qz * (at(VR, 2, 0) + at(VR, 0, 2)) + w * (at(VR, 2, 1) - at(VR, 1, 2))),
                        2 * (qx * (at(VR, 1, 0) + at(VR, 0, 1)) - 2 * qy * (at(VR, 0, 0) + at(VR, 2, 2)) +
                             qz * (at(VR, 2, 1) + at(VR, 1, 2)) + w * (at(VR, 0, 2) - at(VR, 2, 0))),
                        2 * (qx * (at(VR, 2, 0) + at(VR, 0, 2)) + qy * (at(VR, 2, 1) + at(VR, 1, 2)) -
                             2 * qz * (at(VR, 0, 0) + at(VR, 1, 1)) + w * (at(VR, 1, 0) - at(VR, 0, 1)))};
                    const double qn[4] = {w, qx, qy, qz};
                    const double dot = vqn[0] * qn[0] + vqn[1] * qn[1] + vqn[2] * qn[2] + vqn[3] * qn[3];
                    for (int k = 0; k < 4; k++) v_quats[n * 4 + k] += (vqn[k] - dot * qn[k]) * inv_norm;
                    for (int j = 0; j < 3; j++)
                        v_scales[n * 3 + j] += at(Rg, 0, j) * at(vM, 0, j) + at(Rg, 1, j) * at(vM, 1, j) +
                                               at(Rg, 2, j) * at(vM, 2, j);
                }
                if (g->viewmats_grad) {
                    for (int i = 0; i < 3; i++) {
                        for (int j = 0; j < 3; j++) v_view[c * 16 + i * 4 + j] += at(vR, i, j);
                        v_view[c * 16 + i * 4 + 3] += vt[i];
                    }
                }
            }
        }
        auto put = [](float* dst, const std::vector<double>& src) {
            if (dst)
                for (size_t i = 0; i < src.size(); i++) dst[i] = static_cast<float>(src[i]);
        };
        if (!out->v_means) invalid("projection_fused_bwd", "null v_means");
        put(out->v_means, v_means);
        if (use_covars) put(out->v_covars, v_covars);
        else {
            put(out->v_quats, v_quats);
            put(out->v_scales, v_scales);
        }
        if (g->viewmats_grad) put(out->v_viewmats, v_view);
    });
}

// ------------------------------------------------------------------------------------------
// sh_fwd — CpuKernels.cpp:284-377 (sh_coeffs_to_color_fast_cpu + sh_fwd_cpu), Validate.h:79-90
// ------------------------------------------------------------------------------------------
static void validate_sh(const sxh_sh_inputs* in, const char* what) {
    if (!in->dirs || !in->coeffs) invalid(what, "null dirs/coeffs");
    if (in->B < 0 || in->N < 0) invalid(what, "negative B or N");
    if (in->K < 1 || in->D == 0) invalid(what, "K and D must be positive");
    if (in->degrees_to_use > 4) invalid(what, "degrees_to_use must be 0..4");
    const int64_t bands = static_cast<int64_t>(in->degrees_to_use) + 1;
    if (bands * bands > in->K) invalid(what, "(degrees_to_use+1)^2 must be <= K");
}

static void sh_color_cpu(uint32_t degree, uint32_t D, uint32_t c, const float* dir,
                         const float* coeffs, float* colors) {
    float result = 0.2820947917738781f * coeffs[c];
    if (degree >= 1) {
        const float inorm = 1.0f / std::sqrt(dir[0] * dir[0] + dir[1] * dir[1] + dir[2] * dir[2]);
        const float x = dir[0] * inorm;
        const float y = dir[1] * inorm;
        const float z = dir[2] * inorm;
        result += 0.48860251190292f *
                  (-y * coeffs[1 * D + c] + z * coeffs[2 * D + c] - x * coeffs[3 * D + c]);
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
            result += pSH4 * coeffs[4 * D + c] + pSH5 * coeffs[5 * D + c] + pSH6 * coeffs[6 * D + c] +
                      pSH7 * coeffs[7 * D + c] + pSH8 * coeffs[8 * D + c];
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
                result += pSH9 * coeffs[9 * D + c] + pSH10 * coeffs[10 * D + c] +
                          pSH11 * coeffs[11 * D + c] + pSH12 * coeffs[12 * D + c] +
                          pSH13 * coeffs[13 * D + c] + pSH14 * coeffs[14 * D + c] +
                          pSH15 * coeffs[15 * D + c];
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
                    result += pSH16 * coeffs[16 * D + c] + pSH17 * coeffs[17 * D + c] +
                              pSH18 * coeffs[18 * D + c] + pSH19 * coeffs[19 * D + c] +
                              pSH20 * coeffs[20 * D + c] + pSH21 * coeffs[21 * D + c] +
                              pSH22 * coeffs[22 * D + c] + pSH23 * coeffs[23 * D + c] +
                              pSH24 * coeffs[24 * D + c];
                }
            }
        }
    }
    colors[c] = result;
}

int32_t sxo_sh_fwd(const sxh_sh_inputs* in, float* colors) {
    return guarded([&] {
        validate_sh(in, "sh_fwd_cpu");
        const size_t BN = static_cast<size_t>(in->B) * static_cast<size_t>(in->N);
        const size_t N = static_cast<size_t>(in->N);
        const size_t KD = static_cast<size_t>(in->K) * in->D;
        if (BN > 0 && !colors) invalid("sh_fwd_cpu", "null colors");
        for (size_t elem = 0; elem < BN; elem++) {
            if (in->masks && in->masks[elem] == 0) continue; // unwritten (CpuKernels.cpp:369)
            const size_t gid = elem % N;
            for (uint32_t c = 0; c < in->D; c++)
                sh_color_cpu(in->degrees_to_use, in->D, c, in->dirs + elem * 3, in->coeffs + gid * KD,
                             colors + elem * in->D);
        }
    });
}

// ------------------------------------------------------------------------------------------
// sh_bwd — own CPU restatement of sh_coeffs_to_color_fast_vjp (SphericalHarmonics.metal:124-389)
// and the kernel's accumulation (:422-446). Double accumulators.
// ------------------------------------------------------------------------------------------
static void sh_vjp_cpu(uint32_t degree, uint32_t D, uint32_t c, const float* dirf, const float* coeffs,
                       double vc, double* v_coeffs, double v_dir[3], bool want_dir) {
    auto C = [&](int k) { return static_cast<double>(coeffs[k * D + c]); };
    v_coeffs[0 * D + c] += 0.2820947917738781 * vc;
    if (degree < 1) return;
    const double dx = dirf[0], dy = dirf[1], dz = dirf[2];
    const double inorm = 1.0 / std::sqrt(dx * dx + dy * dy + dz * dz);
    const double x = dx * inorm, y = dy * inorm, z = dz * inorm;
    double v_x = 0, v_y = 0, v_z = 0;
    v_coeffs[1 * D + c] += -0.48860251190292 * y * vc;
    v_coeffs[2 * D + c] += 0.48860251190292 * z * vc;
    v_coeffs[3 * D + c] += -0.48860251190292 * x * vc;
    v_x += -0.48860251190292 * C(3) * vc;
    v_y += -0.48860251190292 * C(1) * vc;
    v_z += 0.48860251190292 * C(2) * vc;
    auto finish = [&] {
        if (!want_dir) return;
        const double dot = v_x * x + v_y * y + v_z * z;
        v_dir[0] += (v_x - dot * x) * inorm;
        v_dir[1] += (v_y - dot * y) * inorm;
        v_dir[2] += (v_z - dot * z) * inorm;
    };
    if (degree < 2) { finish(); return; }
    const double z2 = z * z;
    const double fTmp0B = -1.092548430592079 * z;
    const double fC1 = x * x - y * y, fS1 = 2 * x * y;
    const double pSH6 = 0.9461746957575601 * z2 - 0.3153915652525201;
    const double pSH7 = fTmp0B * x, pSH5 = fTmp0B * y;
    const double pSH8 = 0.5462742152960395 * fC1, pSH4 = 0.5462742152960395 * fS1;
    v_coeffs[4 * D + c] += pSH4 * vc;
    v_coeffs[5 * D + c] += pSH5 * vc;
    v_coeffs[6 * D + c] += pSH6 * vc;
    v_coeffs[7 * D + c] += pSH7 * vc;
    v_coeffs[8 * D + c] += pSH8 * vc;
    const double fTmp0B_z = -1.092548430592079;
    const double fC1_x = 2 * x, fC1_y = -2 * y, fS1_x = 2 * y, fS1_y = 2 * x;
    const double pSH6_z = 2 * 0.9461746957575601 * z;
    const double pSH7_x = fTmp0B, pSH7_z = fTmp0B_z * x;
    const double pSH5_y = fTmp0B, pSH5_z = fTmp0B_z * y;
    const double pSH8_x = 0.5462742152960395 * fC1_x, pSH8_y = 0.5462742152960395 * fC1_y;
    const double pSH4_x = 0.5462742152960395 * fS1_x, pSH4_y = 0.5462742152960395 * fS1_y;
    v_x += vc * (pSH4_x * C(4) + pSH8_x * C(8) + pSH7_x * C(7));
    v_y += vc * (pSH4_y * C(4) + pSH8_y * C(8) + pSH5_y * C(5));
    v_z += vc * (pSH6_z * C(6) + pSH7_z * C(7) + pSH5_z * C(5));
    if (degree < 3) { finish(); return; }
    const double fTmp0C = -2.285228997322329 * z2 + 0.4570457994644658;
    const double fTmp1B = 1.445305721320277 * z;
    const double fC2 = x * fC1 - y * fS1, fS2 = x * fS1 + y * fC1;
    const double pSH12 = z * (1.865881662950577 * z2 - 1.119528997770346);
    const double pSH13 = fTmp0C * x, pSH11 = fTmp0C * y;
    const double pSH14 = fTmp1B * fC1, pSH10 = fTmp1B * fS1;
    const double pSH15 = -0.5900435899266435 * fC2, pSH9 = -0.5900435899266435 * fS2;
    v_coeffs[9 * D + c] += pSH9 * vc;
    v_coeffs[10 * D + c] += pSH10 * vc;
    v_coeffs[11 * D + c] += pSH11 * vc;
    v_coeffs[12 * D + c] += pSH12 * vc;
    v_coeffs[13 * D + c] += pSH13 * vc;
    v_coeffs[14 * D + c] += pSH14 * vc;
    v_coeffs[15 * D + c] += pSH15 * vc;
    const double fTmp0C_z = -2.285228997322329 * 2 * z, fTmp1B_z = 1.445305721320277;
    const double fC2_x = fC1 + x * fC1_x - y * fS1_x, fC2_y = x * fC1_y - fS1 - y * fS1_y;
    const double fS2_x = fS1 + x * fS1_x + y * fC1_x, fS2_y = x * fS1_y + fC1 + y * fC1_y;
    const double pSH12_z = 3 * 1.865881662950577 * z2 - 1.119528997770346;
    const double pSH13_x = fTmp0C, pSH13_z = fTmp0C_z * x;
    const double pSH11_y = fTmp0C, pSH11_z = fTmp0C_z * y;
    const double pSH14_x = fTmp1B * fC1_x, pSH14_y = fTmp1B * fC1_y, pSH14_z = fTmp1B_z * fC1;
    const double pSH10_x = fTmp1B * fS1_x, pSH10_y = fTmp1B * fS1_y, pSH10_z = fTmp1B_z * fS1;
    const double pSH15_x = -0.5900435899266435 * fC2_x, pSH15_y = -0.5900435899266435 * fC2_y;
    const double pSH9_x = -0.5900435899266435 * fS2_x, pSH9_y = -0.5900435899266435 * fS2_y;
    v_x += vc * (pSH9_x * C(9) + pSH15_x * C(15) + pSH10_x * C(10) + pSH14_x * C(14) + pSH13_x * C(13));
    v_y += vc * (pSH9_y * C(9) + pSH15_y * C(15) + pSH10_y * C(10) + pSH14_y * C(14) + pSH11_y * C(11));
    v_z += vc * (pSH12_z * C(12) + pSH13_z * C(13) + pSH11_z * C(11) + pSH14_z * C(14) + pSH10_z * C(10));
    if (degree < 4) { finish(); return; }
    const double fTmp0D = z * (-4.683325804901025 * z2 + 2.007139630671868);
    const double fTmp1C = 3.31161143515146 * z2 - 0.47308734787878;
    const double fTmp2B = -1.770130769779931 * z;
    const double fC3 = x * fC2 - y * fS2, fS3 = x * fS2 + y * fC2;
    const double pSH20 = 1.984313483298443 * z * pSH12 - 1.006230589874905 * pSH6;
    const double pSH21 = fTmp0D * x, pSH19 = fTmp0D * y;
    const double pSH22 = fTmp1C * fC1, pSH18 = fTmp1C * fS1;
    const double pSH23 = fTmp2B * fC2, pSH17 = fTmp2B * fS2;
    const double pSH24 = 0.6258357354491763 * fC3, pSH16 = 0.6258357354491763 * fS3;
    v_coeffs[16 * D + c] += pSH16 * vc;
    v_coeffs[17 * D + c] += pSH17 * vc;
    v_coeffs[18 * D + c] += pSH18 * vc;
    v_coeffs[19 * D + c] += pSH19 * vc;
    v_coeffs[20 * D + c] += pSH20 * vc;
    v_coeffs[21 * D + c] += pSH21 * vc;
    v_coeffs[22 * D + c] += pSH22 * vc;
    v_coeffs[23 * D + c] += pSH23 * vc;
    v_coeffs[24 * D + c] += pSH24 * vc;
    const double fTmp0D_z = 3 * -4.683325804901025 * z2 + 2.007139630671868;
    const double fTmp1C_z = 2 * 3.31161143515146 * z;
    const double fTmp2B_z = -1.770130769779931;
    const double fC3_x = fC2 + x * fC2_x - y * fS2_x, fC3_y = x * fC2_y - fS2 - y * fS2_y;
    const double fS3_x = fS2 + y * fC2_x + x * fS2_x, fS3_y = x * fS2_y + fC2 + y * fC2_y;
    const double pSH20_z = 1.984313483298443 * (pSH12 + z * pSH12_z) - 1.006230589874905 * pSH6_z;
    const double pSH21_x = fTmp0D, pSH21_z = fTmp0D_z * x;
    const double pSH19_y = fTmp0D, pSH19_z = fTmp0D_z * y;
    const double pSH22_x = fTmp1C * fC1_x, pSH22_y = fTmp1C * fC1_y, pSH22_z = fTmp1C_z * fC1;
    const double pSH18_x = fTmp1C * fS1_x, pSH18_y = fTmp1C * fS1_y, pSH18_z = fTmp1C_z * fS1;
    const double pSH23_x = fTmp2B * fC2_x, pSH23_y = fTmp2B * fC2_y, pSH23_z = fTmp2B_z * fC2;
    const double pSH17_x = fTmp2B * fS2_x, pSH17_y = fTmp2B * fS2_y, pSH17_z = fTmp2B_z * fS2;
    const double pSH24_x = 0.6258357354491763 * fC3_x, pSH24_y = 0.6258357354491763 * fC3_y;
    const double pSH16_x = 0.6258357354491763 * fS3_x, pSH16_y = 0.6258357354491763 * fS3_y;
    v_x += vc * (pSH16_x * C(16) + pSH24_x * C(24) + pSH17_x * C(17) + pSH23_x * C(23) +
                 pSH18_x * C(18) + pSH22_x * C(22) + pSH21_x * C(21));
    v_y += vc * (pSH16_y * C(16) + pSH24_y * C(24) + pSH17_y * C(17) + pSH23_y * C(23) +
                 pSH18_y * C(18) + pSH22_y * C(22) + pSH19_y * C(19));
    v_z += vc * (pSH20_z * C(20) + pSH21_z * C(21) + pSH19_z * C(19) + pSH22_z * C(22) +
                 pSH18_z * C(18) + pSH23_z * C(23) + pSH17_z * C(17));
    finish();
}

int32_t sxo_sh_bwd(const sxh_sh_inputs* in, const float* v_colors, float* v_coeffs, float* v_dirs) {
    return guarded([&] {
        validate_sh(in, "sh_bwd_cpu");
        const size_t BN = static_cast<size_t>(in->B) * static_cast<size_t>(in->N);
        const size_t N = static_cast<size_t>(in->N);
        const size_t KD = static_cast<size_t>(in->K) * in->D;
        if (BN > 0 && (!v_colors || !v_coeffs)) invalid("sh_bwd_cpu", "null v_colors/v_coeffs");
        if (in->compute_v_dirs && BN > 0 && !v_dirs) invalid("sh_bwd_cpu", "null v_dirs");
        std::vector<double> acc(N * KD, 0.0), vd(in->compute_v_dirs ? BN * 3 : 0, 0.0);
        for (size_t elem = 0; elem < BN; elem++) {
            if (in->masks && in->masks[elem] == 0) continue;
            const size_t gid = elem % N;
            double vdir[3] = {0, 0, 0};
            for (uint32_t c = 0; c < in->D; c++)
                sh_vjp_cpu(in->degrees_to_use, in->D, c, in->dirs + elem * 3, in->coeffs + gid * KD,
                           v_colors[elem * in->D + c], acc.data() + gid * KD, vdir,
                           in->compute_v_dirs != 0);
            if (in->compute_v_dirs)
                for (int k = 0; k < 3; k++) vd[elem * 3 + k] += vdir[k];
        }
        for (size_t i = 0; i < acc.size(); i++) v_coeffs[i] = static_cast<float>(acc[i]);
        if (in->compute_v_dirs)
            for (size_t i = 0; i < vd.size(); i++) v_dirs[i] = static_cast<float>(vd[i]);
    });
}

// ------------------------------------------------------------------------------------------
// isect_tiles — CpuKernels.cpp:381-664 (AABB rect, AccuTile SNUGBOX + sweep, 2-pass emit)
// ------------------------------------------------------------------------------------------
namespace {
struct TileRect {
    int32_t min_x, min_y, max_x, max_y;
};
TileRect aabb_tile_rect(float mean_x, float mean_y, float radius_x, float radius_y, float ts,
                        int32_t tw, int32_t th) { // CpuKernels.cpp:390-406
    const float trx = radius_x / ts, try_ = radius_y / ts;
    const float tx = mean_x / ts, ty = mean_y / ts;
    TileRect r;
    r.min_x = std::min(std::max(0, sxm::f2i_trunc(std::floor(tx - trx))), tw);
    r.min_y = std::min(std::max(0, sxm::f2i_trunc(std::floor(ty - try_))), th);
    r.max_x = std::min(std::max(0, sxm::f2i_trunc(std::ceil(tx + trx))), tw);
    r.max_y = std::min(std::max(0, sxm::f2i_trunc(std::ceil(ty + try_))), th);
    return r;
}
struct F2 {
    float x, y;
};
F2 accutile_ellipse_intersection(float A, float B, float C, float disc, float t, F2 p, bool isY,
                                 float coord) { // CpuKernels.cpp:423-432
    const float p_u = isY ? p.y : p.x;
    const float p_v = isY ? p.x : p.y;
    const float coeff = isY ? A : C;
    const float h = coord - p_u;
    const float sqrt_term = std::sqrt(disc * h * h + t * coeff);
    return {(-B * h - sqrt_term) / coeff + p_v, (-B * h + sqrt_term) / coeff + p_v};
}
uint32_t accutile_process_tiles(float A, float B, float C, float disc, float t, F2 p, F2 bbox_min,
                                F2 bbox_max, F2 bbox_argmin, F2 bbox_argmax, int32_t rect_min_x,
                                int32_t rect_min_y, int32_t rect_max_x, int32_t rect_max_y,
                                float BLOCK, int32_t tile_width, bool isY, uint64_t iid_enc,
                                uint64_t depth_id_enc, int32_t flatten_idx, uint64_t* isect_ids,
                                int32_t* flatten_ids, int64_t* cur_idx) { // CpuKernels.cpp:439-505
    if (isY) {
        std::swap(rect_min_x, rect_min_y);
        std::swap(rect_max_x, rect_max_y);
        bbox_min = {bbox_min.y, bbox_min.x};
        bbox_max = {bbox_max.y, bbox_max.x};
        bbox_argmin = {bbox_argmin.y, bbox_argmin.x};
        bbox_argmax = {bbox_argmax.y, bbox_argmax.x};
    }
    uint32_t tiles_count = 0;
    F2 intersect_min_line, intersect_max_line;
    float ellipse_min, ellipse_max, min_line, max_line;
    intersect_max_line = {bbox_max.y, bbox_min.y};
    min_line = rect_min_x * BLOCK;
    if (bbox_min.x <= min_line)
        intersect_min_line = accutile_ellipse_intersection(A, B, C, disc, t, p, isY, min_line);
    else
        intersect_min_line = intersect_max_line;
    for (int32_t u = rect_min_x; u < rect_max_x; ++u) {
        max_line = min_line + BLOCK;
        if (max_line <= bbox_max.x)
            intersect_max_line = accutile_ellipse_intersection(A, B, C, disc, t, p, isY, max_line);
        if (min_line <= bbox_argmin.y && bbox_argmin.y < max_line) ellipse_min = bbox_min.y;
        else ellipse_min = std::fmin(intersect_min_line.x, intersect_max_line.x);
        if (min_line <= bbox_argmax.y && bbox_argmax.y < max_line) ellipse_max = bbox_max.y;
        else ellipse_max = std::fmax(intersect_min_line.y, intersect_max_line.y);
        const int32_t min_tile_v =
            std::max(rect_min_y, std::min(rect_max_y, sxm::f2i_trunc(ellipse_min / BLOCK)));
        const int32_t max_tile_v =
            std::min(rect_max_y, std::max(rect_min_y, sxm::f2i_trunc(ellipse_max / BLOCK + 1.f)));
        for (int32_t v = min_tile_v; v < max_tile_v; ++v) {
            ++tiles_count;
            if (isect_ids != nullptr) {
                const uint64_t tile_id =
                    static_cast<uint64_t>(isY ? u * tile_width + v : v * tile_width + u);
                isect_ids[*cur_idx] = iid_enc | (tile_id << 32) | depth_id_enc;
                flatten_ids[*cur_idx] = flatten_idx;
                ++(*cur_idx);
            }
        }
        intersect_min_line = intersect_max_line;
        min_line = max_line;
    }
    return tiles_count;
}
uint32_t accutile_element(const float* conic, float opacity, float mean_x, float mean_y, float ts,
                          int32_t tw, int32_t th, uint64_t iid_enc, uint64_t depth_id_enc,
                          int32_t flatten_idx, uint64_t* isect_ids, int32_t* flatten_ids,
                          int64_t* cur_idx) { // CpuKernels.cpp:510-564
    const float A = conic[0], B = conic[1], C = conic[2];
    const float disc = B * B - A * C;
    const float t = std::fmin(sx::kGaussianExtend * sx::kGaussianExtend,
                              2.0f * o_log(opacity / sx::kAlphaThreshold));
    if (t <= 0.f) return 0;
    const float neg_t_over_disc = -t / disc;
    const float x_extent = std::sqrt(neg_t_over_disc * C);
    const float y_extent = std::sqrt(neg_t_over_disc * A);
    const F2 bbox_min = {mean_x - x_extent, mean_y - y_extent};
    const F2 bbox_max = {mean_x + x_extent, mean_y + y_extent};
    const float Bx_over_C = B * x_extent / C;
    const float By_over_A = B * y_extent / A;
    const F2 bbox_argmin = {mean_y + Bx_over_C, mean_x + By_over_A};
    const F2 bbox_argmax = {mean_y - Bx_over_C, mean_x - By_over_A};
    const int32_t rect_min_x = std::max(0, std::min(tw, sxm::f2i_trunc(bbox_min.x / ts)));
    const int32_t rect_min_y = std::max(0, std::min(th, sxm::f2i_trunc(bbox_min.y / ts)));
    const int32_t rect_max_x = std::max(0, std::min(tw, sxm::f2i_trunc(bbox_max.x / ts + 1.f)));
    const int32_t rect_max_y = std::max(0, std::min(th, sxm::f2i_trunc(bbox_max.y / ts + 1.f)));
    const int32_t y_span = rect_max_y - rect_min_y;
    const int32_t x_span = rect_max_x - rect_min_x;
    if (y_span * x_span == 0) return 0;
    const bool isY = y_span < x_span;
    return accutile_process_tiles(A, B, C, disc, t, {mean_x, mean_y}, bbox_min, bbox_max,
                                  bbox_argmin, bbox_argmax, rect_min_x, rect_min_y, rect_max_x,
                                  rect_max_y, ts, tw, isY, iid_enc, depth_id_enc, flatten_idx,
                                  isect_ids, flatten_ids, cur_idx);
}
} // namespace

// The two-pass host orchestration of isect_tiles_cpu (CpuKernels.cpp:576-664): count, int64
// cumsum, emit into [cum[i-1], cum[i]).
static void isect_core(const sxh_isect_inputs* in, int32_t* tiles_per_gauss,
                       std::vector<uint64_t>& ids, std::vector<int32_t>& flat, int64_t* n_isects,
                       uint32_t* tnb, uint32_t* inb) {
    const char* what = "isect_tiles_cpu";
    if (!in->means2d || !in->radii || !in->depths) invalid(what, "null means2d/radii/depths");
    if ((in->conics != nullptr) != (in->opacities != nullptr))
        invalid(what, "conics and opacities must be given together (AccuTile) or both null (AABB)");
    if (in->I < 0 || in->N < 0) invalid(what, "negative I or N");
    if (in->tile_size == 0 || in->tile_width == 0 || in->tile_height == 0)
        invalid(what, "tile_size/tile_width/tile_height must be positive");
    const uint32_t tile_n_bits =
        sx::bits_for_count(static_cast<int64_t>(in->tile_width) * in->tile_height);
    const uint32_t image_n_bits = sx::bits_for_count(in->I);
    if (image_n_bits + tile_n_bits > 32) invalid(what, "image_n_bits + tile_n_bits must be <= 32");
    if (in->N > 0 && in->I > INT32_MAX / in->N) invalid(what, "I*N must fit in int32 (flatten_ids)");
    const int64_t n_el = in->I * in->N;
    *tnb = tile_n_bits;
    *inb = image_n_bits;
    *n_isects = 0;
    ids.clear();
    flat.clear();
    if (n_el > 0 && !tiles_per_gauss) invalid(what, "null tiles_per_gauss");
    std::fill(tiles_per_gauss, tiles_per_gauss + n_el, 0);
    if (n_el == 0) return;
    const bool accu = in->conics != nullptr;
    const float ts = static_cast<float>(in->tile_size);
    const int32_t TW = static_cast<int32_t>(in->tile_width), TH = static_cast<int32_t>(in->tile_height);
    for (int64_t idx = 0; idx < n_el; idx++) {
        const float rx = static_cast<float>(in->radii[idx * 2]);
        const float ry = static_cast<float>(in->radii[idx * 2 + 1]);
        if (rx <= 0.f || ry <= 0.f) continue;
        if (accu) {
            tiles_per_gauss[idx] = static_cast<int32_t>(
                accutile_element(in->conics + idx * 3, in->opacities[idx], in->means2d[idx * 2],
                                 in->means2d[idx * 2 + 1], ts, TW, TH, 0, 0,
                                 static_cast<int32_t>(idx), nullptr, nullptr, nullptr));
            continue;
        }
        const TileRect r = aabb_tile_rect(in->means2d[idx * 2], in->means2d[idx * 2 + 1], rx, ry,
                                          ts, TW, TH);
        tiles_per_gauss[idx] = (r.max_y - r.min_y) * (r.max_x - r.min_x);
    }
    std::vector<int64_t> cum(static_cast<size_t>(n_el));
    int64_t running = 0;
    for (int64_t i = 0; i < n_el; i++) cum[i] = (running += tiles_per_gauss[i]);
    *n_isects = cum.back();
    if (*n_isects == 0) return;
    ids.resize(static_cast<size_t>(*n_isects));
    flat.resize(static_cast<size_t>(*n_isects));
    for (int64_t idx = 0; idx < n_el; idx++) {
        const float rx = static_cast<float>(in->radii[idx * 2]);
        const float ry = static_cast<float>(in->radii[idx * 2 + 1]);
        if (rx <= 0.f || ry <= 0.f) continue;
        const int64_t iid = idx / in->N;
        const uint64_t iid_enc = static_cast<uint64_t>(iid) << (32 + tile_n_bits);
        const float depth_f = in->depths[idx];
        if (!(depth_f >= 0.f)) invalid(what, "depth must be >= 0 at idx " + std::to_string(idx));
        uint32_t depth_bits;
        std::memcpy(&depth_bits, &depth_f, 4);
        const uint64_t depth_id_enc = depth_bits;
        int64_t cur = (idx == 0) ? 0 : cum[idx - 1];
        if (accu) {
            accutile_element(in->conics + idx * 3, in->opacities[idx], in->means2d[idx * 2],
                             in->means2d[idx * 2 + 1], ts, TW, TH, iid_enc, depth_id_enc,
                             static_cast<int32_t>(idx), ids.data(), flat.data(), &cur);
            continue;
        }
        const TileRect r = aabb_tile_rect(in->means2d[idx * 2], in->means2d[idx * 2 + 1], rx, ry,
                                          ts, TW, TH);
        for (int32_t i = r.min_y; i < r.max_y; i++)
            for (int32_t j = r.min_x; j < r.max_x; j++) {
                const uint64_t tile_id = static_cast<uint64_t>(i * TW + j);
                ids[cur] = iid_enc | (tile_id << 32) | depth_id_enc;
                flat[cur] = static_cast<int32_t>(idx);
                ++cur;
            }
    }
}

int32_t sxo_isect_tiles(const sxh_isect_inputs* in, sxh_isect_outputs* out) {
    return guarded([&] {
        std::vector<uint64_t> ids;
        std::vector<int32_t> flat;
        isect_core(in, out->tiles_per_gauss, ids, flat, &out->n_isects, &out->tile_n_bits,
                   &out->image_n_bits);
        if (out->n_isects == 0) return;
        if (out->capacity < out->n_isects)
            throw CapacityError("isect_tiles_cpu: capacity " + std::to_string(out->capacity) +
                                " < n_isects " + std::to_string(out->n_isects));
        if (!out->isect_ids || !out->flatten_ids) invalid("isect_tiles_cpu", "null isect_ids/flatten_ids");
        std::memcpy(out->isect_ids, ids.data(), ids.size() * 8);
        std::memcpy(out->flatten_ids, flat.data(), flat.size() * 4);
    });
}

int32_t sxo_prefix_scan_i64(const int32_t* in, int64_t n, int64_t* out) { // CpuKernels.h:81-89
    return guarded([&] {
        if (n < 0) invalid("prefix_scan_i64", "negative n");
        int64_t running = 0;
        for (int64_t i = 0; i < n; i++) out[i] = (running += in[i]);
    });
}

// sort_isect — CpuKernels.cpp:674-700 (a stable ascending sort of the pairs on the u64 key). The stable
// order is unique (equal keys keep their input order), so any stable sort yields the reference's
// std::stable_sort result. It is computed here in linear time (166 M keys in seconds, where the
// comparison sort over an index array takes over a minute): a stable counting pass on the key's top
// (at most 16) significant bits, then, within each run of equal top bits, stable LSD counting passes of
// 8 bits over the remaining bits (runs are small and stay in cache). The values travel with the keys.
namespace {
void lsd_runs(uint64_t* k, int32_t* v, uint64_t* tk, int32_t* tv, size_t n, uint32_t bits) {
    for (uint32_t shift = 0; shift < bits; shift += 8) {
        size_t start[256] = {};
        for (size_t i = 0; i < n; i++) start[(k[i] >> shift) & 255u]++;
        if (start[(k[0] >> shift) & 255u] == n) continue;  // one digit value: the pass keeps the order
        size_t run = 0;
        for (int d = 0; d < 256; d++) {
            const size_t c = start[d];
            start[d] = run;
            run += c;
        }
        for (size_t i = 0; i < n; i++) {  // in input order: equal digits keep their order (stable)
            const size_t pos = start[(k[i] >> shift) & 255u]++;
            tk[pos] = k[i];
            tv[pos] = v[i];
        }
        std::copy(tk, tk + n, k);
        std::copy(tv, tv + n, v);
    }
}
}  // namespace

int32_t sxo_sort_isect(const sxh_sort_inputs* in, uint64_t* keys_sorted, int32_t* values_sorted) {
    return guarded([&] {
        const char* what = "sort_isect_cpu";
        if (in->n < 0) invalid(what, "negative n");
        if (in->n > 0 && (!in->keys || !in->values)) invalid(what, "null keys/values");
        if (in->n > INT32_MAX) invalid(what, "n must fit in int32 (flatten_ids/GPU params)");
        if (in->key_n_bits < 1 || in->key_n_bits > 64) invalid(what, "key_n_bits must be 1..64");
        const size_t n = static_cast<size_t>(in->n);
        if (n == 0) return;
        if (in->key_n_bits < 64)
            for (size_t i = 0; i < n; i++)
                if (in->keys[i] >> in->key_n_bits)
                    invalid(what, "key has bits above key_n_bits at idx " + std::to_string(i));
        const uint32_t top = std::min<uint32_t>(16, in->key_n_bits), low = in->key_n_bits - top;
        const size_t buckets = size_t{1} << top;
        // stable counting pass on the top bits, straight into the outputs
        std::vector<size_t> start(buckets + 1, 0);
        for (size_t i = 0; i < n; i++) start[(in->keys[i] >> low) + 1]++;
        for (size_t b = 0; b < buckets; b++) start[b + 1] += start[b];
        std::vector<size_t> next(start.begin(), start.end() - 1);
        for (size_t i = 0; i < n; i++) {
            const size_t pos = next[in->keys[i] >> low]++;
            keys_sorted[pos] = in->keys[i];
            values_sorted[pos] = in->values[i];
        }
        // each run of equal top bits sorted stably on the low bits
        if (low == 0) return;
        size_t longest = 0;
        for (size_t b = 0; b < buckets; b++) longest = std::max(longest, start[b + 1] - start[b]);
        std::vector<uint64_t> tk(longest);
        std::vector<int32_t> tv(longest);
        for (size_t b = 0; b < buckets; b++) {
            const size_t r = start[b + 1] - start[b];
            if (r > 1) lsd_runs(keys_sorted + start[b], values_sorted + start[b], tk.data(), tv.data(), r, low);
        }
    });
}

// isect_offset_encode — CpuKernels.cpp:708-740
int32_t sxo_isect_offset_encode(const sxh_offset_inputs* in, int32_t* offsets) {
    return guarded([&] {
        const char* what = "isect_offset_encode_cpu";
        if (in->n_isects < 0) invalid(what, "negative n_isects");
        if (in->n_isects > 0 && !in->isect_ids) invalid(what, "null isect_ids");
        if (in->I < 0) invalid(what, "negative I");
        if (in->n_isects > 0 && in->I == 0) invalid(what, "n_isects > 0 requires I > 0 (keys encode image ids)");
        if (in->tile_width == 0 || in->tile_height == 0) invalid(what, "tile_width/tile_height must be positive");
        const int64_t n_tiles = static_cast<int64_t>(in->tile_width) * in->tile_height;
        if (sx::bits_for_count(in->I) + sx::bits_for_count(n_tiles) > 32)
            invalid(what, "image_n_bits + tile_n_bits must be <= 32");
        if (in->n_isects > INT32_MAX) invalid(what, "n_isects must fit in int32 (offsets values)");
        if (in->I > 0 && n_tiles > INT32_MAX / in->I) invalid(what, "I*n_tiles must fit in int32 (offsets table)");
        const int64_t total = in->I * n_tiles;
        std::fill(offsets, offsets + total, 0);
        if (in->n_isects == 0) return;
        const uint32_t tile_n_bits = sx::bits_for_count(n_tiles);
        const uint64_t tile_mask = (static_cast<uint64_t>(1) << tile_n_bits) - 1;
        auto flat_tile_id = [&](uint64_t key) {
            const uint64_t isect_id = key >> 32;
            return static_cast<int64_t>(isect_id >> tile_n_bits) * n_tiles +
                   static_cast<int64_t>(isect_id & tile_mask);
        };
        for (int64_t idx = 0; idx < in->n_isects; idx++) {
            const int64_t id_curr = flat_tile_id(in->isect_ids[idx]);
            if (idx == 0)
                for (int64_t i = 0; i <= id_curr; i++) offsets[i] = 0;
            if (idx == in->n_isects - 1)
                for (int64_t i = id_curr + 1; i < total; i++) offsets[i] = static_cast<int32_t>(in->n_isects);
            if (idx > 0) {
                if ((in->isect_ids[idx - 1] >> 32) == (in->isect_ids[idx] >> 32)) continue;
                const int64_t id_prev = flat_tile_id(in->isect_ids[idx - 1]);
                for (int64_t i = id_prev + 1; i <= id_curr; i++) offsets[i] = static_cast<int32_t>(idx);
            }
        }
    });
}

// ------------------------------------------------------------------------------------------
// rasterize_fwd — CpuKernels.cpp:747-855 (Validate.h:165-195)
// ------------------------------------------------------------------------------------------
static void validate_raster(const sxh_raster_inputs* in, const char* what) {
    if (!in->means2d || !in->conics || !in->colors || !in->opacities || !in->isect_offsets)
        invalid(what, "null means2d/conics/colors/opacities/isect_offsets");
    if (in->n_isects > 0 && !in->flatten_ids) invalid(what, "null flatten_ids");
    if (in->I < 0 || in->N < 0 || in->n_isects < 0) invalid(what, "negative I/N/n_isects");
    if (in->n_isects > 0 && in->N == 0) invalid(what, "n_isects > 0 requires N > 0 (flatten_ids reference gaussians)");
    if (in->tile_size != 16) invalid(what, "tile_size must be 16 (Phase 1 rasterize instantiation)");
    if (in->image_width == 0 || in->image_height == 0) invalid(what, "image_width/image_height must be positive");
    if (in->tile_width == 0 || in->tile_height == 0) invalid(what, "tile_width/tile_height must be positive");
    if (static_cast<uint64_t>(in->tile_width) * in->tile_size < in->image_width ||
        static_cast<uint64_t>(in->tile_height) * in->tile_size < in->image_height)
        invalid(what, "tile grid must cover the image");
    if (in->n_isects > INT32_MAX) invalid(what, "n_isects must fit in int32 (last_ids)");
    const int64_t n_tiles = static_cast<int64_t>(in->tile_width) * in->tile_height;
    if (in->I > 0 && n_tiles > INT32_MAX / in->I) invalid(what, "I*n_tiles must fit in int32 (offsets table)");
}

int32_t sxo_rasterize_fwd(const sxh_raster_inputs* in, sxh_raster_outputs* out) {
    return guarded([&] {
        validate_raster(in, "rasterize_fwd_cpu");
        const size_t I = static_cast<size_t>(in->I);
        const size_t H = in->image_height, W = in->image_width;
        const size_t n_tiles = static_cast<size_t>(in->tile_width) * in->tile_height;
        for (size_t img = 0; img < I; img++) {
            const int32_t* offsets = in->isect_offsets + img * n_tiles;
            const float* bg = in->backgrounds ? in->backgrounds + img * 3 : nullptr;
            const uint8_t* masks = in->masks ? in->masks + img * n_tiles : nullptr;
            float* rc = out->render_colors + img * H * W * 3;
            float* ra = out->render_alphas + img * H * W;
            int32_t* li = out->last_ids + img * H * W;
            for (size_t tile = 0; tile < n_tiles; tile++) {
                const size_t tile_x = tile % in->tile_width, tile_y = tile / in->tile_width;
                const bool masked = masks && masks[tile] == 0;
                const int32_t range_start = offsets[tile];
                const int32_t range_end = (img == I - 1 && tile == n_tiles - 1)
                                              ? static_cast<int32_t>(in->n_isects)
                                              : offsets[tile + 1];
                for (size_t yy = 0; yy < in->tile_size; yy++) {
                    const size_t out_y = tile_y * in->tile_size + yy;
                    if (out_y >= H) continue;
                    for (size_t xx = 0; xx < in->tile_size; xx++) {
                        const size_t out_x = tile_x * in->tile_size + xx;
                        if (out_x >= W) continue;
                        const size_t pix = out_y * W + out_x;
                        if (masked) {
                            for (size_t k = 0; k < 3; k++) rc[pix * 3 + k] = bg ? bg[k] : 0.f;
                            ra[pix] = 0.f;
                            li[pix] = 0;
                            continue;
                        }
                        const float px = static_cast<float>(out_x) + 0.5f;
                        const float py = static_cast<float>(out_y) + 0.5f;
                        float T = 1.0f;
                        uint32_t cur_idx = 0u;
                        float pix_out[3] = {0.f, 0.f, 0.f};
                        for (int32_t idx = range_start; idx < range_end; idx++) {
                            const int32_t g = in->flatten_ids[idx];
                            const float dx = in->means2d[2 * g] - px;
                            const float dy = in->means2d[2 * g + 1] - py;
                            const float* cn = in->conics + 3 * g;
                            const float sigma = 0.5f * (cn[0] * dx * dx + cn[2] * dy * dy) + cn[1] * dx * dy;
                            const float vis = o_exp_raster(-sigma);
                            const float alpha = std::min(sx::kMaxAlpha, in->opacities[g] * vis);
                            if (sigma < 0.f || alpha < sx::kAlphaThreshold) continue;
                            const float next_T = T * (1.0f - alpha);
                            if (next_T <= sx::kTransmittanceThreshold) break;
                            const float w = alpha * T;
                            for (size_t k = 0; k < 3; k++)
                                pix_out[k] = std::fma(in->colors[g * 3 + k], w, pix_out[k]);
                            cur_idx = static_cast<uint32_t>(idx);
                            T = next_T;
                        }
                        ra[pix] = 1.0f - T;
                        for (size_t k = 0; k < 3; k++)
                            rc[pix * 3 + k] = bg ? std::fma(T, bg[k], pix_out[k]) : pix_out[k];
                        li[pix] = static_cast<int32_t>(cur_idx);
                    }
                }
            }
        }
    });
}

// ------------------------------------------------------------------------------------------
// rasterize_bwd — own CPU restatement of Rasterize3DGSBwd.metal:142-297 (back-to-front walk,
// T recovered by division, v_alpha terms, clamp gate), pixel by pixel; double accumulators.
// ------------------------------------------------------------------------------------------
int32_t sxo_rasterize_bwd(const sxh_raster_inputs* in, const sxh_raster_grads_in* gin,
                          sxh_raster_grads* out) {
    return guarded([&] {
        validate_raster(in, "rasterize_bwd_cpu");
        if (!gin->render_alphas || !gin->last_ids) invalid("rasterize_bwd_cpu", "null render_alphas/last_ids (fwd outputs)");
        if (!gin->v_render_colors || !gin->v_render_alphas) invalid("rasterize_bwd_cpu", "null v_render_colors/v_render_alphas");
        const size_t I = static_cast<size_t>(in->I), Ng = static_cast<size_t>(in->I * in->N);
        const size_t H = in->image_height, W = in->image_width;
        const size_t n_tiles = static_cast<size_t>(in->tile_width) * in->tile_height;
        std::vector<double> vm2(Ng * 2, 0.0), vcn(Ng * 3, 0.0), vcol(Ng * 3, 0.0), vop(Ng, 0.0),
            vabs(gin->absgrad ? Ng * 2 : 0, 0.0);
        if (in->n_isects > 0) {
            for (size_t img = 0; img < I; img++) {
                const int32_t* offsets = in->isect_offsets + img * n_tiles;
                const float* bg = in->backgrounds ? in->backgrounds + img * 3 : nullptr;
                const uint8_t* masks = in->masks ? in->masks + img * n_tiles : nullptr;
                const float* ralpha = gin->render_alphas + img * H * W;
                const int32_t* lids = gin->last_ids + img * H * W;
                const float* vrc = gin->v_render_colors + img * H * W * 3;
                const float* vra = gin->v_render_alphas + img * H * W;
                for (size_t tile = 0; tile < n_tiles; tile++) {
                    if (masks && masks[tile] == 0) continue;
                    const size_t tile_x = tile % in->tile_width, tile_y = tile / in->tile_width;
                    const int32_t range_start = offsets[tile];
                    const int32_t range_end = (img == I - 1 && tile == n_tiles - 1)
                                                  ? static_cast<int32_t>(in->n_isects)
                                                  : offsets[tile + 1];
                    for (size_t yy = 0; yy < 16; yy++) {
                        const size_t py_i = tile_y * 16 + yy;
                        if (py_i >= H) continue;
                        for (size_t xx = 0; xx < 16; xx++) {
                            const size_t px_i = tile_x * 16 + xx;
                            if (px_i >= W) continue;
                            const size_t pix = py_i * W + px_i;
                            const float px = static_cast<float>(px_i) + 0.5f;
                            const float py = static_cast<float>(py_i) + 0.5f;
                            const float T_final = 1.0f - ralpha[pix];
                            float T = T_final;
                            float buf[3] = {0.f, 0.f, 0.f};
                            const int32_t bin_final = lids[pix];
                            const float vc[3] = {vrc[pix * 3], vrc[pix * 3 + 1], vrc[pix * 3 + 2]};
                            const float va = vra[pix];
                            // entries past the pixel's last contributor are skipped (the reference's
                            // `if (idx > bin_final) continue`): the walk starts at that entry
                            for (int32_t idx = std::min(range_end - 1, bin_final); idx >= range_start; idx--) {
                                const int32_t g = in->flatten_ids[idx];
                                const float* cn = in->conics + 3 * g;
                                const float opac = in->opacities[g];
                                const float dx = in->means2d[2 * g] - px;
                                const float dy = in->means2d[2 * g + 1] - py;
                                const float sigma = 0.5f * (cn[0] * dx * dx + cn[2] * dy * dy) + cn[1] * dx * dy;
                                const float vis = o_exp_raster(-sigma);
                                const float alpha = std::min(sx::kMaxAlpha, opac * vis);
                                if (sigma < 0.f || alpha < sx::kAlphaThreshold) continue;
                                const float ra = 1.0f / std::max(sx::kMinOneMinusAlpha, 1.0f - alpha);
                                T *= ra;
                                const float fac = alpha * T;
                                const float* col = in->colors + 3 * g;
                                float v_alpha = 0.f;
                                for (int k = 0; k < 3; k++) v_alpha += (col[k] * T - buf[k] * ra) * vc[k];
                                v_alpha += T_final * ra * va;
                                if (bg) {
                                    float accum = 0.f;
                                    for (int k = 0; k < 3; k++) accum += bg[k] * vc[k];
                                    v_alpha += -T_final * ra * accum;
                                }
                                for (int k = 0; k < 3; k++) vcol[g * 3 + k] += static_cast<double>(fac) * vc[k];
                                if (opac * vis <= sx::kMaxAlpha) {
                                    const double v_sigma = -static_cast<double>(opac) * vis * v_alpha;
                                    vcn[g * 3 + 0] += 0.5 * v_sigma * dx * dx;
                                    vcn[g * 3 + 1] += v_sigma * dx * dy;
                                    vcn[g * 3 + 2] += 0.5 * v_sigma * dy * dy;
                                    const double vx = v_sigma * (static_cast<double>(cn[0]) * dx + static_cast<double>(cn[1]) * dy);
                                    const double vy = v_sigma * (static_cast<double>(cn[1]) * dx + static_cast<double>(cn[2]) * dy);
                                    vm2[g * 2] += vx;
                                    vm2[g * 2 + 1] += vy;
                                    if (gin->absgrad) {
                                        vabs[g * 2] += std::fabs(vx);
                                        vabs[g * 2 + 1] += std::fabs(vy);
                                    }
                                    vop[g] += static_cast<double>(vis) * v_alpha;
                                }
                                for (int k = 0; k < 3; k++) buf[k] += col[k] * fac;
                            }
                        }
                    }
                }
            }
        }
        for (size_t i = 0; i < Ng * 2; i++) out->v_means2d[i] = static_cast<float>(vm2[i]);
        for (size_t i = 0; i < Ng * 3; i++) out->v_conics[i] = static_cast<float>(vcn[i]);
        for (size_t i = 0; i < Ng * 3; i++) out->v_colors[i] = static_cast<float>(vcol[i]);
        for (size_t i = 0; i < Ng; i++) out->v_opacities[i] = static_cast<float>(vop[i]);
        if (gin->absgrad && out->v_means2d_abs)
            for (size_t i = 0; i < Ng * 2; i++) out->v_means2d_abs[i] = static_cast<float>(vabs[i]);
    });
}

// ------------------------------------------------------------------------------------------
// RNG — CpuKernels.cpp:863-900 with the Philox core restated from RngPhilox.h:50-98
// ------------------------------------------------------------------------------------------
namespace {
void philox_block(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1,
                  uint32_t out[4]) {
    for (int r = 0; r < 10; ++r) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
        const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
        const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
        c1 = static_cast<uint32_t>(p1);
        c3 = static_cast<uint32_t>(p0);
        c0 = n0;
        c2 = n2;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}
float u32_uniform(uint32_t x) { return (static_cast<float>(x) + 1.0f) * (1.0f / 4294967296.0f); }
void box_muller(uint32_t x0, uint32_t x1, float* z0, float* z1) {
    const float u1 = u32_uniform(x0), u2 = u32_uniform(x1);
    const float r = std::sqrt(-2.0f * o_log(u1));
    const float theta = 6.28318530717958647692f * u2;
    float s, c;
    o_sincos(theta, &s, &c);
    *z0 = r * c;
    *z1 = r * s;
}
void validate_rng(const sxh_rng_inputs* in, const char* what) {
    if (in->count < 0) invalid(what, "negative count");
    if (in->count > static_cast<int64_t>(UINT32_MAX)) invalid(what, "count must fit in uint32 (RngParams.count)");
}
} // namespace

int32_t sxo_rng_philox_u32(const sxh_rng_inputs* in, uint32_t* out) {
    return guarded([&] {
        validate_rng(in, "rng_philox_u32_cpu");
        const size_t n = static_cast<size_t>(in->count);
        for (size_t t = 0; t < (n + 3) / 4; t++) {
            uint32_t r[4];
            philox_block(static_cast<uint32_t>(t), static_cast<uint32_t>(in->offset),
                         static_cast<uint32_t>(in->offset >> 32), 0u, static_cast<uint32_t>(in->seed),
                         static_cast<uint32_t>(in->seed >> 32), r);
            for (size_t j = 0; j < 4 && t * 4 + j < n; j++) out[t * 4 + j] = r[j];
        }
    });
}

int32_t sxo_rng_normal_f32(const sxh_rng_inputs* in, float* out) {
    return guarded([&] {
        validate_rng(in, "rng_normal_f32_cpu");
        const size_t n = static_cast<size_t>(in->count);
        for (size_t t = 0; t < (n + 3) / 4; t++) {
            uint32_t r[4];
            philox_block(static_cast<uint32_t>(t), static_cast<uint32_t>(in->offset),
                         static_cast<uint32_t>(in->offset >> 32), 0u, static_cast<uint32_t>(in->seed),
                         static_cast<uint32_t>(in->seed >> 32), r);
            float z[4];
            box_muller(r[0], r[1], &z[0], &z[1]);
            box_muller(r[2], r[3], &z[2], &z[3]);
            for (size_t j = 0; j < 4 && t * 4 + j < n; j++) out[t * 4 + j] = z[j];
        }
    });
}

// make_binoms_lut — CpuKernels.cpp:906-917 (Pascal's triangle in u64, cast to float)
int32_t sxo_make_binoms_lut(int32_t n_max, float* out) {
    return guarded([&] {
        if (n_max < 1) invalid("make_binoms_lut", "n_max must be >= 1");
        std::fill(out, out + static_cast<size_t>(n_max) * n_max, 0.0f);
        std::vector<uint64_t> row(static_cast<size_t>(n_max), 0);
        for (int n = 0; n < n_max; n++) {
            for (int k = n; k >= 1; k--) row[k] += row[k - 1];
            row[0] = 1;
            for (int k = 0; k <= n; k++) out[static_cast<size_t>(n) * n_max + k] = static_cast<float>(row[k]);
        }
    });
}

// mcmc_relocation — CpuKernels.cpp:924-960 (Validate.h:221-229)
int32_t sxo_mcmc_relocation(const sxh_relocation_inputs* in, float* new_op, float* new_sc) {
    return guarded([&] {
        const char* what = "mcmc_relocation_cpu";
        if (!in->opacities || !in->scales || !in->ratios || !in->binoms)
            invalid(what, "null opacities/scales/ratios/binoms");
        if (in->N < 0) invalid(what, "negative N");
        if (in->n_max < 1) invalid(what, "n_max must be >= 1");
        for (int64_t idx = 0; idx < in->N; idx++) {
            const int n_idx = in->ratios[idx];
            if (n_idx < 1 || n_idx > in->n_max)
                invalid(what, "ratios[" + std::to_string(idx) + "] out of [1, n_max] (host clamp contract)");
            const float old_op = in->opacities[idx];
            float new_opacity = 1.0f - o_pow(1.0f - old_op, 1.0f / static_cast<float>(n_idx));
            new_opacity = std::min(std::max(new_opacity, in->min_opacity), 1.0f - FLT_EPSILON);
            new_op[idx] = new_opacity;
            float denom_sum = 0.0f;
            for (int i = 1; i <= n_idx; i++)
                for (int k = 0; k <= i - 1; k++) {
                    const float bin_coeff = in->binoms[static_cast<size_t>(i - 1) * in->n_max + k];
                    const float sign = (k & 1) ? -1.0f : 1.0f;
                    const float term = (sign / std::sqrt(static_cast<float>(k + 1))) *
                                       o_pow(new_opacity, static_cast<float>(k + 1));
                    denom_sum += bin_coeff * term;
                }
            const float coeff = old_op / denom_sum;
            for (int i = 0; i < 3; i++) new_sc[idx * 3 + i] = coeff * in->scales[idx * 3 + i];
        }
    });
}

// mcmc_perturb_positions — CpuKernels.cpp:969-1008 (Validate.h:257-263)
int32_t sxo_mcmc_perturb_positions(const sxh_perturb_inputs* in) {
    return guarded([&] {
        if (in->N == 0) return;
        const char* what = "mcmc_perturb_positions_cpu";
        if (!in->positions || !in->quats || !in->scales_log || !in->opacities_logit || !in->noise)
            invalid(what, "null positions/quats/scales_log/opacities_logit/noise");
        if (in->N < 0) invalid(what, "negative N");
        for (int64_t idx = 0; idx < in->N; idx++) {
            const float* q = in->quats + idx * 4;
            float w = q[0], x = q[1], y = q[2], z = q[3];
            const float inv_norm = 1.0f / std::sqrt(x * x + y * y + z * z + w * w);
            x *= inv_norm; y *= inv_norm; z *= inv_norm; w *= inv_norm;
            const float x2 = x * x, y2 = y * y, z2 = z * z;
            const float xy = x * y, xz = x * z, yz = y * z;
            const float wx = w * x, wy = w * y, wz = w * z;
            const float R[3][3] = {
                {1.f - 2.f * (y2 + z2), 2.f * (xy - wz), 2.f * (xz + wy)},
                {2.f * (xy + wz), 1.f - 2.f * (x2 + z2), 2.f * (yz - wx)},
                {2.f * (xz - wy), 2.f * (yz + wx), 1.f - 2.f * (x2 + y2)},
            };
            const float s[3] = {o_exp(in->scales_log[idx * 3 + 0]), o_exp(in->scales_log[idx * 3 + 1]),
                                o_exp(in->scales_log[idx * 3 + 2])};
            float M[3][3];
            for (int i = 0; i < 3; i++)
                for (int j = 0; j < 3; j++) M[i][j] = R[i][j] * s[j];
            float C[3][3];
            for (int i = 0; i < 3; i++)
                for (int j = 0; j < 3; j++)
                    C[i][j] = M[i][0] * M[j][0] + M[i][1] * M[j][1] + M[i][2] * M[j][2];
            const float density = 1.0f / (1.0f + o_exp(-in->opacities_logit[idx]));
            const float gate = 1.0f / (1.0f + o_exp(in->k * (density - in->t)));
            const float wgt = gate * in->noise_scale;
            const float n0 = in->noise[idx * 3 + 0] * wgt;
            const float n1 = in->noise[idx * 3 + 1] * wgt;
            const float n2 = in->noise[idx * 3 + 2] * wgt;
            in->positions[idx * 3 + 0] += C[0][0] * n0 + C[0][1] * n1 + C[0][2] * n2;
            in->positions[idx * 3 + 1] += C[1][0] * n0 + C[1][1] * n1 + C[1][2] * n2;
            in->positions[idx * 3 + 2] += C[2][0] * n0 + C[2][1] * n1 + C[2][2] * n2;
        }
    });
}

// ------------------------------------------------------------------------------------------
// SSIM — fwd restates CpuKernels.cpp:1019-1106; bwd restates Ssim.metal:175-268 (the adjoint of
// the valid correlation as a zero-padded separable pass, fma chains in tap order, then
// G·(c1 + 2x·c2 + y·c3) with G = -v_loss/M computed in f64).
// ------------------------------------------------------------------------------------------
static const float kTaps[11] = SX_SSIM_TAPS;

static void validate_ssim(const sxh_ssim_inputs* in, const char* what) {
    if (!in->img1 || !in->img2) invalid(what, "null img1/img2");
    if (in->I <= 0 || in->C <= 0) invalid(what, "I and C must be positive (ssim mean undefined on empty batch)");
    if (in->H < 11 || in->W < 11) invalid(what, "H and W must be >= 11 (valid map would be empty)");
    if (in->H > UINT32_MAX || in->W > UINT32_MAX) invalid(what, "H/W exceed uint32 (SsimParams)");
    if (in->I > static_cast<int64_t>(UINT32_MAX) / in->C) invalid(what, "I*C exceeds uint32 (dispatch grid z)");
}

int32_t sxo_ssim_fwd(const sxh_ssim_inputs* in, sxh_ssim_outputs* out) {
    return guarded([&] {
        validate_ssim(in, "ssim_fwd_cpu");
        const size_t H = in->H, W = in->W, C = in->C;
        const size_t map_h = H - 10, map_w = W - 10;
        const size_t map_count = static_cast<size_t>(in->I) * map_h * map_w * C;
        if (!out->ssim_map || (in->need_coeffs && (!out->coeff_mu || !out->coeff_sigma || !out->coeff_cross)))
            invalid("ssim_fwd_cpu", "null output buffer");
        std::vector<float> h_m1(H * map_w), h_m2(H * map_w), h_e11(H * map_w), h_e22(H * map_w), h_e12(H * map_w);
        for (int64_t i = 0; i < in->I; i++) {
            for (size_t c = 0; c < C; c++) {
                for (size_t y = 0; y < H; y++)
                    for (size_t xw = 0; xw < map_w; xw++) {
                        float m1 = 0.f, m2 = 0.f, e11 = 0.f, e22 = 0.f, e12 = 0.f;
                        for (uint32_t u = 0; u < 11; u++) {
                            const float w = kTaps[u];
                            const size_t off = (((static_cast<size_t>(i) * H + y) * W) + xw + u) * C + c;
                            const float x = in->img1[off], g = in->img2[off];
                            m1 = std::fma(w, x, m1);
                            m2 = std::fma(w, g, m2);
                            e11 = std::fma(w * x, x, e11);
                            e22 = std::fma(w * g, g, e22);
                            e12 = std::fma(w * x, g, e12);
                        }
                        const size_t ho = y * map_w + xw;
                        h_m1[ho] = m1; h_m2[ho] = m2; h_e11[ho] = e11; h_e22[ho] = e22; h_e12[ho] = e12;
                    }
                for (size_t my = 0; my < map_h; my++)
                    for (size_t mx = 0; mx < map_w; mx++) {
                        float mu1 = 0.f, mu2 = 0.f, e11 = 0.f, e22 = 0.f, e12 = 0.f;
                        for (uint32_t v = 0; v < 11; v++) {
                            const float w = kTaps[v];
                            const size_t ho = (my + v) * map_w + mx;
                            mu1 = std::fma(w, h_m1[ho], mu1);
                            mu2 = std::fma(w, h_m2[ho], mu2);
                            e11 = std::fma(w, h_e11[ho], e11);
                            e22 = std::fma(w, h_e22[ho], e22);
                            e12 = std::fma(w, h_e12[ho], e12);
                        }
                        const float sigma1 = std::fma(-mu1, mu1, e11);
                        const float sigma2 = std::fma(-mu2, mu2, e22);
                        const float sigma12 = std::fma(-mu1, mu2, e12);
                        const float A1 = 2.f * mu1 * mu2 + sx::kSsimC1;
                        const float B1 = mu1 * mu1 + mu2 * mu2 + sx::kSsimC1;
                        const float A2 = 2.f * sigma12 + sx::kSsimC2;
                        const float B2 = sigma1 + sigma2 + sx::kSsimC2;
                        const float denom = B1 * B2;
                        const float S = (A1 * A2) / denom;
                        const size_t mo = (((static_cast<size_t>(i) * map_h + my) * map_w) + mx) * C + c;
                        out->ssim_map[mo] = S;
                        if (in->need_coeffs) {
                            const float dS_dmu1 = 2.f * (mu2 * A2 / denom - mu1 * S / B1);
                            const float dS_dsigma1 = -S / B2;
                            const float dS_dsigma12 = 2.f * A1 / denom;
                            out->coeff_mu[mo] = dS_dmu1 - 2.f * mu1 * dS_dsigma1 - mu2 * dS_dsigma12;
                            out->coeff_sigma[mo] = dS_dsigma1;
                            out->coeff_cross[mo] = dS_dsigma12;
                        }
                    }
            }
        }
        double sum = 0.0; // ssim_reduce_mean_f64 (CpuKernels.h:198-202)
        for (size_t k = 0; k < map_count; k++) sum += static_cast<double>(out->ssim_map[k]);
        out->ssim = sum / static_cast<double>(map_count);
    });
}

int32_t sxo_ssim_bwd(const sxh_ssim_inputs* in, const sxh_ssim_grads_in* gin, float* v_img1) {
    return guarded([&] {
        validate_ssim(in, "ssim_bwd_cpu");
        if (!gin->coeff_mu || !gin->coeff_sigma || !gin->coeff_cross)
            invalid("ssim_bwd_cpu", "null coeff maps (run ssim_fwd with need_coeffs=true)");
        const int64_t H = in->H, W = in->W, C = in->C, mh = H - 10, mw = W - 10;
        const size_t M = static_cast<size_t>(in->I) * mh * mw * C;
        const float G = static_cast<float>(-static_cast<double>(gin->v_loss) / static_cast<double>(M));
        std::vector<float> h1(static_cast<size_t>((mh + 20) * W)), h2(h1.size()), h3(h1.size());
        for (int64_t i = 0; i < in->I; i++)
            for (int64_t c = 0; c < C; c++) {
                auto D = [&](const float* map, int64_t y, int64_t x) -> float {
                    if (y < 0 || y >= mh || x < 0 || x >= mw) return 0.f;
                    return map[(((i * mh + y) * mw) + x) * C + c];
                };
                // horizontal pass for map rows y in [-10, mh+10): h[y][qx] = sum_u w[u] D(y, qx+u-10)
                for (int64_t yy = 0; yy < mh + 20; yy++) {
                    const int64_t y = yy - 10;
                    for (int64_t qx = 0; qx < W; qx++) {
                        float s1 = 0.f, s2 = 0.f, s3 = 0.f;
                        for (int u = 0; u < 11; u++) {
                            const float w = kTaps[u];
                            s1 = std::fma(w, D(gin->coeff_mu, y, qx + u - 10), s1);
                            s2 = std::fma(w, D(gin->coeff_sigma, y, qx + u - 10), s2);
                            s3 = std::fma(w, D(gin->coeff_cross, y, qx + u - 10), s3);
                        }
                        h1[yy * W + qx] = s1; h2[yy * W + qx] = s2; h3[yy * W + qx] = s3;
                    }
                }
                for (int64_t qy = 0; qy < H; qy++)
                    for (int64_t qx = 0; qx < W; qx++) {
                        float c1 = 0.f, c2 = 0.f, c3 = 0.f;
                        for (int v = 0; v < 11; v++) {
                            const float w = kTaps[v];
                            const int64_t yy = qy + v - 10 + 10; // row qy+v-10 of the map, offset by 10
                            c1 = std::fma(w, h1[yy * W + qx], c1);
                            c2 = std::fma(w, h2[yy * W + qx], c2);
                            c3 = std::fma(w, h3[yy * W + qx], c3);
                        }
                        const size_t q = (((static_cast<size_t>(i) * H + qy) * W) + qx) * C + c;
                        const float x = in->img1[q], y = in->img2[q];
                        v_img1[q] = G * (c1 + 2.f * x * c2 + y * c3);
                    }
            }
    });
}

// ------------------------------------------------------------------------------------------
// transcendental primitives (pinning surface)
// ------------------------------------------------------------------------------------------
void sxo_logf_array(const float* x, float* y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = sxm::logf_(x[i]); }
void sxo_expf_array(const float* x, float* y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = sxm::expf_(x[i]); }
void sxo_expf_fast_array(const float* x, float* y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = sxm::expf_fast(x[i]); }
void sxo_powf_array(const float* x, const float* p, float* y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = sxm::powf_(x[i], p[i]); }
void sxo_sincosf_array(const float* x, float* s, float* c, int64_t n) { for (int64_t i = 0; i < n; i++) sxm::sincosf_(x[i], &s[i], &c[i]); }

} // extern "C"

// ------------------------------------------------------------------------------------------
// One full training step on the host — Trainer.cpp:716-832 (forward_pass) and :971-1131 (step),
// with the MCMC noise tail of the resident step (MetalBackend.cpp:2198-2229): rng_normal_f32 with
// (seed, offset, N*3) then mcmc_perturb_positions on the post-Adam parameters.
// ------------------------------------------------------------------------------------------
namespace {
const char* kStageNames[16] = {"activation", "projection_fwd", "sh_fwd", "isect", "sort",
                               "offsets", "raster_fwd", "l1_loss", "ssim_fwd", "ssim_bwd",
                               "raster_bwd", "sh_bwd", "projection_bwd", "grad_chains", "adam",
                               "noise"};
using clk = std::chrono::steady_clock;
inline double ms_since(clk::time_point t0) {
    return std::chrono::duration<double, std::milli>(clk::now() - t0).count();
}
void check(int32_t rc) {
    if (rc == SXH_ERR_INVALID_ARGUMENT) throw std::invalid_argument(g_err);
    if (rc != SXH_OK) throw std::runtime_error(g_err);
}
} // namespace

extern "C" const char* sxo_stage_name(int32_t i) {
    return (i >= 0 && i < 16) ? kStageNames[i] : "";
}

extern "C" int32_t sxo_train_step(sxo_step_args* a) {
    return guarded([&] {
        for (double& t : a->stage_ms) t = 0.0;
        const int64_t N = a->count;
        if (N < 1) invalid("train_step", "count must be >= 1");
        if (a->width < 1 || a->height < 1) invalid("train_step", "width/height must be positive");
        if (a->sh_degree < 0 || a->sh_degree > 3) invalid("train_step", "sh_degree must be in [0,3]");
        if (!a->viewmat || !a->K) invalid("train_step", "null viewmat/K");
        if (!a->forward_only && !a->gt_rgb) invalid("train_step", "null gt_rgb");
        const int64_t K = static_cast<int64_t>(a->sh_degree + 1) * (a->sh_degree + 1);
        const bool aa = a->antialiased != 0;
        const int W = a->width, H = a->height;
        const size_t HW = static_cast<size_t>(W) * H, n_px = HW * 3;
        float* means = a->params[0];
        float* quats = a->params[1];
        float* log_scales = a->params[2];
        float* logits = a->params[3];
        float* sh0 = a->params[4];
        float* shN = a->params[5];

        // (host) activation — Trainer.cpp:438-460
        auto t0 = clk::now();
        std::vector<float> scales_lin(N * 3), opacs_act(N);
        for (int64_t i = 0; i < N * 3; i++) scales_lin[i] = o_exp(log_scales[i]);
        for (int64_t i = 0; i < N; i++) opacs_act[i] = 1.0f / (1.0f + o_exp(-logits[i]));
        a->stage_ms[0] += ms_since(t0);

        // [01] projection fwd — Trainer.cpp:603-628, :731-733
        t0 = clk::now();
        sxh_projection_inputs pin{};
        pin.means = means; pin.quats = quats; pin.scales = scales_lin.data();
        pin.opacities = opacs_act.data(); pin.viewmats = a->viewmat; pin.Ks = a->K;
        pin.N = N; pin.C = 1; pin.width = W; pin.height = H;
        pin.eps2d = a->eps2d; pin.near_plane = a->near_plane; pin.far_plane = a->far_plane;
        pin.radius_clip = a->radius_clip; pin.camera_model = 0; pin.calc_compensations = aa;
        std::vector<int32_t> radii(N * 2);
        std::vector<float> means2d(N * 2), depths(N), conics(N * 3), comps(aa ? N : 0);
        sxh_projection_outputs pout{radii.data(), means2d.data(), depths.data(), conics.data(),
                                    aa ? comps.data() : nullptr};
        check(sxo_projection_fused_fwd(&pin, &pout));
        std::vector<float> opacs_aa;
        if (aa) { // Trainer.cpp:741-745
            opacs_aa.resize(N);
            for (int64_t i = 0; i < N; i++) opacs_aa[i] = opacs_act[i] * comps[i];
        }
        const std::vector<float>& raster_opacs = aa ? opacs_aa : opacs_act;
        std::vector<uint8_t> valid(N);
        int64_t n_vis = 0;
        for (int64_t i = 0; i < N; i++) {
            valid[i] = (radii[i * 2] > 0 && radii[i * 2 + 1] > 0) ? 1 : 0;
            n_vis += valid[i];
        }
        a->n_visible = n_vis;
        a->stage_ms[1] += ms_since(t0);

        // [02] SH fwd + post-op — Trainer.cpp:752-788
        t0 = clk::now();
        const float* vm = a->viewmat;
        float campos[3];
        for (int i = 0; i < 3; i++)
            campos[i] = -(vm[0 * 4 + i] * vm[0 * 4 + 3] + vm[1 * 4 + i] * vm[1 * 4 + 3] +
                          vm[2 * 4 + i] * vm[2 * 4 + 3]);
        std::vector<float> dirs(N * 3);
        for (int64_t i = 0; i < N; i++)
            for (int k = 0; k < 3; k++) dirs[i * 3 + k] = means[i * 3 + k] - campos[k];
        std::vector<float> coeffs(N * K * 3);
        for (int64_t i = 0; i < N; i++) {
            for (int c = 0; c < 3; c++) coeffs[(i * K) * 3 + c] = sh0[i * 3 + c];
            for (int64_t k = 1; k < K; k++)
                for (int c = 0; c < 3; c++)
                    coeffs[(i * K + k) * 3 + c] = shN[(i * (K - 1) + (k - 1)) * 3 + c];
        }
        sxh_sh_inputs sin{};
        sin.dirs = dirs.data(); sin.coeffs = coeffs.data(); sin.masks = valid.data();
        sin.degrees_to_use = a->degrees_to_use; sin.B = 1; sin.N = N; sin.K = K; sin.D = 3;
        std::vector<float> colors(N * 3, 0.0f);
        check(sxo_sh_fwd(&sin, colors.data()));
        std::vector<uint8_t> relu_mask(N * 3);
        for (size_t i = 0; i < colors.size(); i++) {
            const float pre = colors[i] + 0.5f;
            relu_mask[i] = pre > 0.0f ? 1 : 0;
            colors[i] = std::max(pre, 0.0f);
        }
        a->stage_ms[2] += ms_since(t0);

        // [03] isect — Trainer.cpp:790-806 (AccuTile; AABB when isect_mode says so)
        t0 = clk::now();
        const uint32_t tw = static_cast<uint32_t>((W + 15) / 16), th = static_cast<uint32_t>((H + 15) / 16);
        sxh_isect_inputs iin{};
        iin.means2d = means2d.data(); iin.radii = radii.data(); iin.depths = depths.data();
        if (a->isect_mode == SXH_ISECT_ACCUTILE) {
            iin.conics = conics.data();
            iin.opacities = raster_opacs.data();
        }
        iin.I = 1; iin.N = N; iin.tile_size = 16; iin.tile_width = tw; iin.tile_height = th;
        std::vector<int32_t> tiles(N);
        std::vector<uint64_t> ids;
        std::vector<int32_t> flat;
        int64_t n_isects = 0;
        uint32_t tnb = 0, inb = 0;
        isect_core(&iin, tiles.data(), ids, flat, &n_isects, &tnb, &inb);
        a->n_isects = n_isects;
        a->stage_ms[3] += ms_since(t0);

        // [04] sort + [03] offsets — Trainer.cpp:808-827
        t0 = clk::now();
        std::vector<uint64_t> keys_sorted(n_isects);
        std::vector<int32_t> vals_sorted(n_isects);
        sxh_sort_inputs srt{ids.data(), flat.data(), n_isects, 32 + tnb + inb};
        check(sxo_sort_isect(&srt, keys_sorted.data(), vals_sorted.data()));
        a->stage_ms[4] += ms_since(t0);
        t0 = clk::now();
        std::vector<int32_t> offsets(static_cast<size_t>(tw) * th);
        sxh_offset_inputs oin{keys_sorted.data(), n_isects, 1, tw, th};
        check(sxo_isect_offset_encode(&oin, offsets.data()));
        a->stage_ms[5] += ms_since(t0);

        // [05] raster fwd
        t0 = clk::now();
        sxh_raster_inputs rin{};
        rin.means2d = means2d.data(); rin.conics = conics.data(); rin.colors = colors.data();
        rin.opacities = raster_opacs.data(); rin.isect_offsets = offsets.data();
        rin.flatten_ids = vals_sorted.data(); rin.I = 1; rin.N = N; rin.n_isects = n_isects;
        rin.image_width = W; rin.image_height = H; rin.tile_size = 16; rin.tile_width = tw;
        rin.tile_height = th;
        std::vector<float> render(n_px), ralpha(HW);
        std::vector<int32_t> last_ids(HW);
        sxh_raster_outputs rout{render.data(), ralpha.data(), last_ids.data()};
        check(sxo_rasterize_fwd(&rin, &rout));
        a->stage_ms[6] += ms_since(t0);
        if (a->render_colors) std::memcpy(a->render_colors, render.data(), n_px * 4);
        a->loss = 0.0f;
        if (a->forward_only) return;

        // (host) L1 loss and grad — Trainer.cpp:330-345
        t0 = clk::now();
        std::vector<float> v_render(n_px);
        const float gsc = 1.0f / static_cast<float>(n_px);
        double acc = 0.0;
        for (size_t i = 0; i < n_px; i++) {
            const float d = render[i] - a->gt_rgb[i];
            acc += std::fabs(static_cast<double>(d));
            v_render[i] = d > 0.0f ? gsc : (d < 0.0f ? -gsc : 0.0f);
        }
        const float l1 = static_cast<float>(acc / static_cast<double>(n_px));
        float loss = l1;
        a->stage_ms[7] += ms_since(t0);

        // SSIM combination — Trainer.cpp:995-1017
        if (a->ssim_weight > 0.0f) {
            t0 = clk::now();
            const float lam = a->ssim_weight;
            sxh_ssim_inputs si{render.data(), a->gt_rgb, 1, H, W, 3, 1};
            const size_t mc = static_cast<size_t>(H - 10) * (W - 10) * 3;
            std::vector<float> smap(mc), cmu(mc), csg(mc), ccr(mc);
            sxh_ssim_outputs so{0.0, smap.data(), cmu.data(), csg.data(), ccr.data()};
            check(sxo_ssim_fwd(&si, &so));
            a->stage_ms[8] += ms_since(t0);
            t0 = clk::now();
            sxh_ssim_grads_in sg{cmu.data(), csg.data(), ccr.data(), lam};
            std::vector<float> v_dssim(n_px);
            check(sxo_ssim_bwd(&si, &sg, v_dssim.data()));
            const float w_l1 = 1.0f - lam;
            for (size_t i = 0; i < n_px; i++) v_render[i] = w_l1 * v_render[i] + v_dssim[i];
            loss = w_l1 * l1 + lam * (1.0f - static_cast<float>(so.ssim));
            a->stage_ms[9] += ms_since(t0);
        }
        a->loss = loss;

        // [05] raster bwd (v_render_alphas = 0)
        t0 = clk::now();
        std::vector<float> v_ra(HW, 0.0f), v_m2(N * 2), v_cn(N * 3), v_col(N * 3), v_op(N);
        sxh_raster_grads_in rgi{ralpha.data(), last_ids.data(), v_render.data(), v_ra.data(), 0};
        sxh_raster_grads rg{v_m2.data(), v_cn.data(), v_col.data(), v_op.data(), nullptr};
        check(sxo_rasterize_bwd(&rin, &rgi, &rg));
        a->stage_ms[10] += ms_since(t0);

        // relu mask + [02] SH bwd — Trainer.cpp:1029-1038
        t0 = clk::now();
        for (size_t i = 0; i < v_col.size(); i++)
            if (!relu_mask[i]) v_col[i] = 0.0f;
        sin.compute_v_dirs = 1;
        std::vector<float> v_coeffs(N * K * 3), v_dirs(N * 3);
        check(sxo_sh_bwd(&sin, v_col.data(), v_coeffs.data(), v_dirs.data()));
        a->stage_ms[11] += ms_since(t0);

        // AA chain + [01] proj bwd — Trainer.cpp:1040-1067
        t0 = clk::now();
        std::vector<float> v_comp;
        if (aa) { // chain_aa_opacity_grads_inplace (Trainer.cpp:526-536)
            v_comp.resize(N);
            for (int64_t i = 0; i < N; i++) {
                const float v_op_aa = v_op[i];
                v_comp[i] = v_op_aa * opacs_act[i];
                v_op[i] = v_op_aa * comps[i];
            }
        }
        std::vector<float> v_depths(N, 0.0f), v_means(N * 3), v_quats(N * 4), v_scales(N * 3);
        sxh_projection_grads_in pg{radii.data(), conics.data(), aa ? comps.data() : nullptr,
                                   v_m2.data(), v_depths.data(), v_cn.data(),
                                   aa ? v_comp.data() : nullptr, 0};
        sxh_projection_grads pgo{v_means.data(), nullptr, v_quats.data(), v_scales.data(), nullptr};
        check(sxo_projection_fused_bwd(&pin, &pg, &pgo));
        a->stage_ms[12] += ms_since(t0);

        // chains + reg + split — Trainer.cpp:1069-1097 (resident forms, TrainStep.metal:187-213)
        t0 = clk::now();
        for (int64_t i = 0; i < N * 3; i++) v_means[i] += v_dirs[i];
        for (int64_t i = 0; i < N * 3; i++) {
            float v = v_scales[i] * scales_lin[i];
            if (a->scale_reg_w > 0.0f) v += a->scale_reg_w * scales_lin[i];
            v_scales[i] = v;
        }
        for (int64_t i = 0; i < N; i++) {
            const float s = opacs_act[i];
            float v = v_op[i] * (s * (1.0f - s));
            if (a->opacity_reg_w > 0.0f) v += a->opacity_reg_w * s * (1.0f - s);
            v_op[i] = v;
        }
        std::vector<float> v_sh0(N * 3), v_shN(N * (K - 1) * 3);
        for (int64_t i = 0; i < N; i++) {
            for (int c = 0; c < 3; c++) v_sh0[i * 3 + c] = v_coeffs[(i * K) * 3 + c];
            for (int64_t k = 1; k < K; k++)
                for (int c = 0; c < 3; c++)
                    v_shN[(i * (K - 1) + (k - 1)) * 3 + c] = v_coeffs[(i * K + k) * 3 + c];
        }
        a->stage_ms[13] += ms_since(t0);

        // [06] fused_adam x6 — Trainer.cpp:1099-1108
        t0 = clk::now();
        const float* grads[6] = {v_means.data(), v_quats.data(), v_scales.data(), v_op.data(),
                                 v_sh0.data(), v_shN.data()};
        const int64_t dims[6] = {3, 4, 3, 1, 3, (K - 1) * 3};
        for (int g = 0; g < 6; g++) {
            if (dims[g] == 0) continue;
            sxh_adam_inputs ai{a->params[g], grads[g], a->exp_avg[g], a->exp_avg_sq[g], valid.data(),
                               N * dims[g], N, a->lr[g], a->b1, a->b2, a->eps};
            check(sxo_fused_adam(&ai));
        }
        a->stage_ms[14] += ms_since(t0);

        // MCMC noise (non-refine step)
        if (a->inject_noise) {
            t0 = clk::now();
            std::vector<float> noise(N * 3);
            sxh_rng_inputs ri{a->noise_seed, a->noise_offset, N * 3};
            check(sxo_rng_normal_f32(&ri, noise.data()));
            sxh_perturb_inputs pi{means, quats, log_scales, logits, noise.data(), N, a->noise_scale,
                                  0.005f, 100.0f};
            check(sxo_mcmc_perturb_positions(&pi));
            a->stage_ms[15] += ms_since(t0);
        }
    });
}

// ------------------------------------------------------------------------------------------
// MCMC refine — Trainer::mcmc_refine (Trainer.cpp:1273-1280): mcmc_relocate (:1284-1338) then
// mcmc_add (:1342-1395), with multinomial_with_replacement (:1199-1218), run_relocation_for
// (:1231-1258) and mcmc_zero_adam_rows (:1422-1435), on host AoS arrays of arena rows (the
// reference's cap_max arena, :686-709). The engine is std::mt19937_64 itself; its state crosses
// the C boundary in libstdc++'s text layout (312 words, then the position).
// ------------------------------------------------------------------------------------------
namespace {

std::mt19937_64 mt_from(const sxh_mt64_state& st) {
    std::ostringstream os;
    for (int i = 0; i < 312; i++) os << st.x[i] << ' ';
    os << st.p;
    std::istringstream is(os.str());
    std::mt19937_64 g;
    is >> g;
    if (!is) throw std::invalid_argument("mcmc_refine: malformed rng state");
    return g;
}

void mt_to(const std::mt19937_64& g, sxh_mt64_state* st) {
    std::ostringstream os;
    os << g;
    std::istringstream is(os.str());
    for (int i = 0; i < 312; i++) is >> st->x[i];
    is >> st->p;
}

float sigmoid_o(float x) { return 1.0f / (1.0f + o_exp(-x)); }  // Trainer.cpp:430

float logit_o(float p) {  // Trainer.cpp:432-436
    if (!(p > 0.0f && p < 1.0f)) throw std::invalid_argument("logit_f32: p must be in (0,1)");
    return o_log(p / (1.0f - p));
}

// Trainer.cpp:1199-1218
std::vector<int64_t> multinomial_o(const float* w, int64_t n_w, int64_t n_samples, std::mt19937_64& rng) {
    std::vector<double> cdf(static_cast<size_t>(n_w));
    double acc = 0.0;
    for (int64_t i = 0; i < n_w; i++) {
        if (!(w[i] >= 0.0f)) throw std::invalid_argument("multinomial: weights must be >= 0 and finite");
        acc += static_cast<double>(w[i]);
        cdf[static_cast<size_t>(i)] = acc;
    }
    if (!(acc > 0.0)) throw std::invalid_argument("multinomial: weight sum must be > 0");
    std::vector<int64_t> out(static_cast<size_t>(n_samples));
    for (int64_t j = 0; j < n_samples; j++) {
        const double u = static_cast<double>(rng() >> 11) * 0x1.0p-53 * acc;
        const int64_t idx = std::upper_bound(cdf.begin(), cdf.end(), u) - cdf.begin();
        out[static_cast<size_t>(j)] = std::min(idx, n_w - 1);
    }
    return out;
}

struct RefineArrays {
    float* p[6];
    float* m[6];
    float* v[6];
    int64_t dim[6];
};

// Trainer.cpp:1231-1258 (gather + bincount ratios + the relocation op), then the source
// opacity / scale writes of :1310-1321 (or :1367-1377)
void relocate_sources(RefineArrays& a, const std::vector<float>& op_act, const std::vector<int64_t>& sampled,
                      const float* binoms, int32_t n_max, float min_opacity, const char* what) {
    const int64_t n = static_cast<int64_t>(sampled.size());
    std::unordered_map<int64_t, int32_t> counts;
    for (int64_t s : sampled) counts[s]++;
    std::vector<float> g_op(static_cast<size_t>(n)), g_sc(static_cast<size_t>(n) * 3);
    std::vector<int32_t> ratios(static_cast<size_t>(n));
    for (int64_t j = 0; j < n; j++) {
        const int64_t s = sampled[static_cast<size_t>(j)];
        g_op[static_cast<size_t>(j)] = op_act[static_cast<size_t>(s)];
        for (int k = 0; k < 3; k++) g_sc[static_cast<size_t>(j) * 3 + k] = o_exp(a.p[2][s * 3 + k]);
        ratios[static_cast<size_t>(j)] = std::min(counts[s] + 1, n_max);
    }
    std::vector<float> new_op(static_cast<size_t>(n)), new_sc(static_cast<size_t>(n) * 3);
    sxh_relocation_inputs rin{g_op.data(), g_sc.data(), ratios.data(), binoms, n, n_max, min_opacity};
    if (sxo_mcmc_relocation(&rin, new_op.data(), new_sc.data()) != SXH_OK) throw std::runtime_error(g_err);
    for (int64_t j = 0; j < n; j++) {
        const int64_t s = sampled[static_cast<size_t>(j)];
        a.p[3][s] = logit_o(new_op[static_cast<size_t>(j)]);
        for (int k = 0; k < 3; k++) {
            const float ns = new_sc[static_cast<size_t>(j) * 3 + k];
            if (!(ns > 0.0f)) throw std::logic_error(std::string(what) + ": non-positive new_scale");
            a.p[2][s * 3 + k] = o_log(ns);
        }
    }
}

void copy_row(RefineArrays& a, int64_t dst, int64_t src) {  // Trainer.cpp:1223-1225 over all groups
    for (int g = 0; g < 6; g++)
        for (int64_t k = 0; k < a.dim[g]; k++) a.p[g][dst * a.dim[g] + k] = a.p[g][src * a.dim[g] + k];
}

void zero_moments(RefineArrays& a, int64_t row) {  // Trainer.cpp:1422-1435
    for (int g = 0; g < 6; g++)
        for (int64_t k = 0; k < a.dim[g]; k++) {
            a.m[g][row * a.dim[g] + k] = 0.0f;
            a.v[g][row * a.dim[g] + k] = 0.0f;
        }
}

}  // namespace

// std::mt19937_64(seed) itself, in the C layout
extern "C" int32_t sxo_mt64_seed(uint64_t seed, sxh_mt64_state* out) {
    return guarded([&] {
        std::mt19937_64 g(seed);
        mt_to(g, out);
    });
}

// n raw draws of std::mt19937_64 from a state (advances the state)
extern "C" int32_t sxo_mt64_draw(sxh_mt64_state* st, int64_t n, uint64_t* out) {
    return guarded([&] {
        std::mt19937_64 g = mt_from(*st);
        for (int64_t i = 0; i < n; i++) out[i] = g();
        mt_to(g, st);
    });
}

// the multinomial's running f64 sum (Trainer.cpp:1202-1208), left to right
extern "C" int32_t sxo_running_sum_f64(const float* w, int64_t n, double* out) {
    return guarded([&] {
        double acc = 0.0;
        for (int64_t i = 0; i < n; i++) {
            acc += static_cast<double>(w[i]);
            out[i] = acc;
        }
    });
}

extern "C" int32_t sxo_mcmc_refine(sxo_refine_args* r) {
    return guarded([&] {
        const char* what = "mcmc_refine";
        if (!r || !r->rng || !r->binoms) invalid(what, "null argument");
        if (r->count < 1 || r->cap_max < r->count) invalid(what, "bad count / cap_max");
        const int64_t K3 = static_cast<int64_t>((r->sh_degree + 1) * (r->sh_degree + 1) - 1) * 3;
        RefineArrays a{};
        const int64_t dims[6] = {3, 4, 3, 1, 3, K3};
        for (int g = 0; g < 6; g++) {
            a.p[g] = r->params[g];
            a.m[g] = r->exp_avg[g];
            a.v[g] = r->exp_avg_sq[g];
            a.dim[g] = dims[g];
        }
        std::mt19937_64 rng = mt_from(*r->rng);
        r->new_count = r->count;
        r->n_relocated = 0;
        r->n_added = 0;
        struct SaveRng {  // the engine state is handed back even when a phase throws
            std::mt19937_64& g;
            sxh_mt64_state* st;
            ~SaveRng() { mt_to(g, st); }
        } save{rng, r->rng};

        // relocate (Trainer.cpp:1284-1338)
        {
            const int64_t N = r->count;
            std::vector<float> op_act(static_cast<size_t>(N));
            for (int64_t i = 0; i < N; i++) op_act[static_cast<size_t>(i)] = sigmoid_o(a.p[3][i]);
            std::vector<int64_t> dead, alive;
            for (int64_t i = 0; i < N; i++) (op_act[static_cast<size_t>(i)] <= r->min_opacity ? dead : alive).push_back(i);
            if (!dead.empty() && !alive.empty()) {
                std::vector<float> probs(alive.size());
                for (size_t j = 0; j < alive.size(); j++) probs[j] = op_act[static_cast<size_t>(alive[j])];
                const std::vector<int64_t> local = multinomial_o(probs.data(), static_cast<int64_t>(alive.size()),
                                                                 static_cast<int64_t>(dead.size()), rng);
                std::vector<int64_t> sampled(dead.size());
                for (size_t j = 0; j < dead.size(); j++) sampled[j] = alive[static_cast<size_t>(local[j])];
                relocate_sources(a, op_act, sampled, r->binoms, r->n_max, r->min_opacity, "Trainer::mcmc_relocate");
                for (size_t j = 0; j < dead.size(); j++) copy_row(a, dead[j], sampled[j]);
                for (int64_t s : sampled) zero_moments(a, s);
                r->n_relocated = static_cast<int64_t>(dead.size());
                if (r->relocated_dead && r->capacity >= r->n_relocated)
                    std::copy(dead.begin(), dead.end(), r->relocated_dead);
                if (r->relocation_src && r->capacity >= r->n_relocated)
                    std::copy(sampled.begin(), sampled.end(), r->relocation_src);
            }
        }
        // add (Trainer.cpp:1342-1395)
        {
            const int64_t N = r->count;
            const int64_t target = std::min(r->cap_max, (N * 21 + 19) / 20);
            const int64_t n_add = target - N;
            if (n_add > 0) {
                std::vector<float> op_act(static_cast<size_t>(N));
                for (int64_t i = 0; i < N; i++) op_act[static_cast<size_t>(i)] = sigmoid_o(a.p[3][i]);
                const std::vector<int64_t> sampled = multinomial_o(op_act.data(), N, n_add, rng);
                relocate_sources(a, op_act, sampled, r->binoms, r->n_max, r->min_opacity, "Trainer::mcmc_add");
                for (int64_t j = 0; j < n_add; j++) copy_row(a, N + j, sampled[static_cast<size_t>(j)]);
                for (int64_t j = 0; j < n_add; j++) zero_moments(a, N + j);
                r->n_added = n_add;
                r->new_count = N + n_add;
                if (r->added_src && r->capacity >= n_add) std::copy(sampled.begin(), sampled.end(), r->added_src);
            }
        }
    });
}
