// Shared device math for the bundle-adjustment kernels (gfx950).
//
// One observation o sees image i (node n, cam c), track t.  The per-observation
// model follows the reference kernels in
// src/blast3r/extensions/cujac/sfm_jacobian_rigs.cu (".cu" below):
//   residual, Huber error and IRLS weight in fp32      (.cu:129-259)
//   Jacobian blocks in fp64 from fp32 inputs           (.cu:323-509)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ba_hip.h"

#define BA_MAX_C 24          // z-coefficient columns supported by the fused path

namespace ba {

// ---------------------------------------------------------------- observation -> image
// Upper bound of idx over cum[0..n_imgs-2] (.cu:72-88): image of observation idx.
__device__ __forceinline__ int obs_image(const int* __restrict__ cum, int n_imgs, int idx) {
    int a = 0, b = n_imgs;
    while (b - a > 1) {
        int m = (a + b) >> 1;
        if (idx < cum[m - 1]) b = m; else a = m;
    }
    return a;
}

// ---------------------------------------------------------------- camera parameters
struct CamF {           // fp32 view of the parameters an observation needs
    float fx, fy, cx, cy;
    float Rrw[9], trw[3];
    float Rcr[9], tcr[3];
};

__device__ __forceinline__ void load_cam(CamF& cp, const float* __restrict__ K, const float* __restrict__ Prc,
                                         int64_t prc_stride, const float* __restrict__ Pwr, int cam, int node) {
    const float* k = K + (int64_t)cam * 9;
    cp.fx = k[0]; cp.cx = k[2]; cp.fy = k[4]; cp.cy = k[5];
    const float* p = Pwr + (int64_t)node * 16;
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        cp.Rrw[3 * r + 0] = p[4 * r + 0]; cp.Rrw[3 * r + 1] = p[4 * r + 1]; cp.Rrw[3 * r + 2] = p[4 * r + 2];
        cp.trw[r] = p[4 * r + 3];
    }
    const float* q = Prc + (int64_t)cam * prc_stride;
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        cp.Rcr[3 * r + 0] = q[4 * r + 0]; cp.Rcr[3 * r + 1] = q[4 * r + 1]; cp.Rcr[3 * r + 2] = q[4 * r + 2];
        cp.tcr[r] = q[4 * r + 3];
    }
}

// ---------------------------------------------------------------- residual (fp32)
struct ResOut {
    float r[3], err[3], w[3];
    bool valid;
};

typedef ba_huber HuberParams;

// Same operation order as .cu:201-258 (matmul with bias, then projection, then Huber).
__device__ __forceinline__ void eval_residual(const CamF& cp, const float X[3], float u, float v, float su, float sv,
                                              float guidance, const HuberParams& hp, ResOut& o) {
    float Xr[3], Xc[3];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 3; ++k) s += cp.Rrw[3 * r + k] * X[k];
        Xr[r] = s + cp.trw[r];
    }
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 3; ++k) s += cp.Rcr[3 * r + k] * Xr[k];
        Xc[r] = s + cp.tcr[r];
    }
    float z = Xc[2];
    o.valid = z > 1e-3f;
#pragma unroll
    for (int i = 0; i < 3; ++i) { o.r[i] = 0.f; o.err[i] = 0.f; o.w[i] = 0.f; }
    if (!o.valid) return;
    float p0 = (cp.fx * Xc[0] + cp.cx * Xc[2]) / z;
    float p1 = (cp.fy * Xc[1] + cp.cy * Xc[2]) / z;
    o.r[0] = (p0 - u) / su;
    o.r[1] = (p1 - v) / sv;
    float avg_focal = 0.5f * (cp.fx + cp.fy);
    if (hp.is_depth_log) o.r[2] = avg_focal * (guidance - logf(z));
    else                 o.r[2] = avg_focal * logf(guidance / z);
    if (hp.pnorm > 0.f) {
        float a = 0.5f * hp.pnorm * powf(hp.huber_delta, hp.pnorm - 2.f);
        float b = powf(hp.huber_delta, hp.pnorm) - a * hp.huber_delta * hp.huber_delta;
        float wz[3] = {1.f, 1.f, hp.weight_z};
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            float r = fabsf(o.r[i]);
            r = (r > hp.max_pix_err) ? hp.max_pix_err : r;
            o.err[i] = wz[i] * ((r <= hp.huber_delta) ? a * r * r : powf(r, hp.pnorm) - b);
            r = (r < hp.huber_delta) ? hp.huber_delta : r;
            o.w[i] = (r == hp.max_pix_err) ? hp.w_pts_null : wz[i] * powf(r, hp.pnorm - 2.f);
        }
    }
}

// ---------------------------------------------------------------- Jacobian (fp64)
// Jcam: 3x8 row-major [fx, fy, wx, wy, wz, vx, vy, vz]; Jz: C entries of row 2; Jp: 3x3.
struct JacOut {
    double Jcam[24];
    double Jp[9];
    double fbar;         // d r2 / d zcf_c = fbar * dep_c (log mode)
    double zscale;       // lin mode: fbar / g (or 0); log mode: fbar
    bool valid;
};

__device__ __forceinline__ void eval_jacobian(const CamF& cp, const float Xf[3], float su, float sv, double guidance,
                                              int is_depth_log, JacOut& J) {
    double X[3] = {Xf[0], Xf[1], Xf[2]};
    double Rrw[9], trw[3], Rcr[9], tcr[3];
#pragma unroll
    for (int k = 0; k < 9; ++k) { Rrw[k] = cp.Rrw[k]; Rcr[k] = cp.Rcr[k]; }
#pragma unroll
    for (int k = 0; k < 3; ++k) { trw[k] = cp.trw[k]; tcr[k] = cp.tcr[k]; }
    double fx = cp.fx, fy = cp.fy, cx = cp.cx, cy = cp.cy;
    double Xr[3], Xc[3];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < 3; ++k) s += Rrw[3 * r + k] * X[k];
        Xr[r] = s + trw[r];
    }
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < 3; ++k) s += Rcr[3 * r + k] * Xr[k];
        Xc[r] = s + tcr[r];
    }
    double p0 = fx * Xc[0] + cx * Xc[2];
    double p1 = fy * Xc[1] + cy * Xc[2];
    double z = Xc[2];
    J.valid = z > 1e-3;
    if (!J.valid) {
#pragma unroll
        for (int k = 0; k < 24; ++k) J.Jcam[k] = 0.0;
#pragma unroll
        for (int k = 0; k < 9; ++k) J.Jp[k] = 0.0;
        J.fbar = 0.0; J.zscale = 0.0;
        return;
    }
    double inv_z = 1.0 / z;
    double inv_z2 = inv_z * inv_z;
    double avg_focal = 0.5 * (fx + fy);
    double s0 = su, s1 = sv;
    // d(proj)/d X_cam, rows scaled by 1/std (.cu:415-435)
    double Jpc[9];
    Jpc[0] = fx * inv_z / s0;  Jpc[1] = 0.0;             Jpc[2] = (cx * inv_z - p0 * inv_z2) / s0;
    Jpc[3] = 0.0;              Jpc[4] = fy * inv_z / s1; Jpc[5] = (cy * inv_z - p1 * inv_z2) / s1;
    Jpc[6] = 0.0;              Jpc[7] = 0.0;             Jpc[8] = -avg_focal * inv_z;
    double Jpr[9];   // (.cu:441)
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            double s = 0.0;
#pragma unroll
            for (int k = 0; k < 3; ++k) s += Jpc[3 * r + k] * Rcr[3 * k + c];
            Jpr[3 * r + c] = s;
        }
    // tau block = Jpr @ [-skew(Xr) | I] (.cu:444-458)
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        double a0 = Jpr[3 * r + 0], a1 = Jpr[3 * r + 1], a2 = Jpr[3 * r + 2];
        J.Jcam[8 * r + 2] = -a1 * Xr[2] + a2 * Xr[1];
        J.Jcam[8 * r + 3] = a0 * Xr[2] - a2 * Xr[0];
        J.Jcam[8 * r + 4] = -a0 * Xr[1] + a1 * Xr[0];
        J.Jcam[8 * r + 5] = a0;
        J.Jcam[8 * r + 6] = a1;
        J.Jcam[8 * r + 7] = a2;
    }
    // points (.cu:463)
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            double s = 0.0;
#pragma unroll
            for (int k = 0; k < 3; ++k) s += Jpr[3 * r + k] * Rrw[3 * k + c];
            J.Jp[3 * r + c] = s;
        }
    // focal columns (.cu:473-489): J_k_f gated on g > 0 and rounded to fp32
    J.Jcam[0] = Xc[0] * inv_z / s0;  J.Jcam[1] = 0.0;
    J.Jcam[8] = 0.0;                 J.Jcam[9] = Xc[1] * inv_z / s1;
    float jkf = 0.0f;
    if (guidance > 0) {
        if (is_depth_log) jkf = (float)(0.5 * (guidance + log(inv_z)));
        else              jkf = (float)(0.5 * log(guidance * inv_z));
    }
    J.Jcam[16] = (double)jkf;
    J.Jcam[17] = (double)jkf;
    J.fbar = avg_focal;
    if (is_depth_log) J.zscale = avg_focal;
    else              J.zscale = (guidance != 0) ? avg_focal / guidance : 0.0;
}

}  // namespace ba
