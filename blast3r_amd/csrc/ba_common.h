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

// ---------------------------------------------------------------- XCD-aware block order
// The dispatcher hands workgroup b to XCD b mod 8 (MI355X: 8 XCDs, one L2 each).  xcd_block maps
// the hardware id onto a logical id so that each XCD takes one contiguous range of logical blocks,
// in order: neighbouring blocks that read the same data (one image's map, one image's tiles) then
// share an L2 instead of fetching it into all eight.  A bijection on [0, nb) for any nb.
#define BA_N_XCD 8
__device__ __forceinline__ unsigned xcd_block(unsigned b, unsigned nb) {
    const unsigned x = b % BA_N_XCD, k = b / BA_N_XCD, q = nb / BA_N_XCD, r = nb % BA_N_XCD;
    return x * q + (x < r ? x : r) + k;
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

// x^p and x^(p-2) for the Huber exponent p: in closed form when PC = 1 (x, 1/x) or PC = 2 (x*x, 1), else
// powf (a general powf costs some 150 instructions per wave, uniform input or not).
template <int PC>
__device__ __forceinline__ float hub_pow_p(float x, float p) { return PC == 1 ? x : (PC == 2 ? x * x : powf(x, p)); }
template <int PC>
__device__ __forceinline__ float hub_pow_pm2(float x, float p) {
    return PC == 1 ? 1.f / x : (PC == 2 ? 1.f : powf(x, p - 2.f));
}

// Huber errors and IRLS weights of the three residuals (.cu:240-258), with the constants
// a = p delta^(p-2) / 2 and b = delta^p - a delta^2 of the reference's formula.
template <int PC>
__device__ __forceinline__ void huber_rows(const HuberParams& hp, ResOut& o) {
    const float p = hp.pnorm, dl = hp.huber_delta;
    const float a = 0.5f * p * hub_pow_pm2<PC>(dl, p);
    const float b = hub_pow_p<PC>(dl, p) - a * dl * dl;
    const float wz[3] = {1.f, 1.f, hp.weight_z};
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        float r = fabsf(o.r[i]);
        r = (r > hp.max_pix_err) ? hp.max_pix_err : r;
        o.err[i] = wz[i] * ((r <= dl) ? a * r * r : hub_pow_p<PC>(r, p) - b);
        r = (r < dl) ? dl : r;
        o.w[i] = (r == hp.max_pix_err) ? hp.w_pts_null : wz[i] * hub_pow_pm2<PC>(r, p);
    }
}

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
    // .cu:212 compares the fp32 depth with the double literal 1e-3: z = 1e-3f (just above 1e-3) is kept
    o.valid = (double)z > 1e-3;
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
        // exponent 1 is the reference's default (args.py:61); the exponent is uniform, so each case is its
        // own branch (no speculated powf)
        if (hp.pnorm == 1.f)      huber_rows<1>(hp, o);
        else if (hp.pnorm == 2.f) huber_rows<2>(hp, o);
        else                      huber_rows<0>(hp, o);
    }
}

// ---------------------------------------------------------------- Jacobian (fp64)
// Every Jacobian entry of one observation is formed from a small core (.cu:323-509):
//   Jpr = d(proj)/d X_cam * R_cr, rows scaled by 1/std           (.cu:415-441)
//   tau block of row r = Jpr_r @ [-skew(Xr) | I]                 (.cu:444-458)
//   points block       = Jpr @ R_rw                              (.cu:463)
//   focal columns: Xc0/z/s0, Xc1/z/s1, and for row 2 J_k_f, gated on g > 0 and rounded to fp32
//   (.cu:473-489).
struct JacCore {
    double Xr[3];
    double Jpr[9];
    double fx_col, fy_col;   // row 0 column fx, row 1 column fy
    double jkf;              // row 2, both focal columns
    double fbar;             // d r2 / d zcf_c = fbar * dep_c (log mode)
    double zscale;           // lin mode: fbar / g (or 0); log mode: fbar
    bool valid;
};

__device__ __forceinline__ void eval_jac_core(const CamF& cp, const float Xf[3], float su, float sv, double guidance,
                                              int is_depth_log, JacCore& J) {
    double X[3] = {Xf[0], Xf[1], Xf[2]};
    double Xc[3];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < 3; ++k) s += (double)cp.Rrw[3 * r + k] * X[k];
        J.Xr[r] = s + (double)cp.trw[r];
    }
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < 3; ++k) s += (double)cp.Rcr[3 * r + k] * J.Xr[k];
        Xc[r] = s + (double)cp.tcr[r];
    }
    const double fx = cp.fx, fy = cp.fy, cx = cp.cx, cy = cp.cy;
    const double p0 = fx * Xc[0] + cx * Xc[2];
    const double p1 = fy * Xc[1] + cy * Xc[2];
    const double z = Xc[2];
    J.valid = z > 1e-3;
    if (!J.valid) {
#pragma unroll
        for (int k = 0; k < 9; ++k) J.Jpr[k] = 0.0;
        J.fx_col = J.fy_col = J.jkf = J.fbar = J.zscale = 0.0;
        return;
    }
    const double inv_z = 1.0 / z;
    const double inv_z2 = inv_z * inv_z;
    const double avg_focal = 0.5 * (fx + fy);
    const double s0 = su, s1 = sv;
    double Jpc[9];
    Jpc[0] = fx * inv_z / s0;  Jpc[1] = 0.0;             Jpc[2] = (cx * inv_z - p0 * inv_z2) / s0;
    Jpc[3] = 0.0;              Jpc[4] = fy * inv_z / s1; Jpc[5] = (cy * inv_z - p1 * inv_z2) / s1;
    Jpc[6] = 0.0;              Jpc[7] = 0.0;             Jpc[8] = -avg_focal * inv_z;
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            double s = 0.0;
#pragma unroll
            for (int k = 0; k < 3; ++k) s += Jpc[3 * r + k] * (double)cp.Rcr[3 * k + c];
            J.Jpr[3 * r + c] = s;
        }
    J.fx_col = Xc[0] * inv_z / s0;
    J.fy_col = Xc[1] * inv_z / s1;
    float jkf = 0.0f;
    if (guidance > 0) {
        if (is_depth_log) jkf = (float)(0.5 * (guidance + log(inv_z)));
        else              jkf = (float)(0.5 * log(guidance * inv_z));
    }
    J.jkf = (double)jkf;
    J.fbar = avg_focal;
    if (is_depth_log) J.zscale = avg_focal;
    else              J.zscale = (guidance != 0) ? avg_focal / guidance : 0.0;
}

// tau column k (0..5: w_x, w_y, w_z, v_x, v_y, v_z) of residual row r
__device__ __forceinline__ double jac_tau(const JacCore& J, int r, int k) {
    const double a0 = J.Jpr[3 * r], a1 = J.Jpr[3 * r + 1], a2 = J.Jpr[3 * r + 2];
    switch (k) {
        case 0: return -a1 * J.Xr[2] + a2 * J.Xr[1];
        case 1: return a0 * J.Xr[2] - a2 * J.Xr[0];
        case 2: return -a0 * J.Xr[1] + a1 * J.Xr[0];
        case 3: return a0;
        case 4: return a1;
        default: return a2;
    }
}

// focal column k (0 = fx, 1 = fy) of residual row r
__device__ __forceinline__ double jac_foc(const JacCore& J, int r, int k) {
    if (r == 0) return k == 0 ? J.fx_col : 0.0;
    if (r == 1) return k == 1 ? J.fy_col : 0.0;
    return J.jkf;
}

// point column c of residual row r
__device__ __forceinline__ double jac_pts(const JacCore& J, const CamF& cp, int r, int c) {
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < 3; ++k) s += J.Jpr[3 * r + k] * (double)cp.Rrw[3 * k + c];
    return s;
}

// Full blocks, for the operator-level jacobians_with_rigs.
// Jcam: 3x8 row-major [fx, fy, wx, wy, wz, vx, vy, vz]; Jp: 3x3.
struct JacOut {
    double Jcam[24];
    double Jp[9];
    double fbar, zscale;
    bool valid;
};

__device__ __forceinline__ void eval_jacobian(const CamF& cp, const float Xf[3], float su, float sv, double guidance,
                                              int is_depth_log, JacOut& O) {
    JacCore J;
    eval_jac_core(cp, Xf, su, sv, guidance, is_depth_log, J);
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        O.Jcam[8 * r + 0] = jac_foc(J, r, 0);
        O.Jcam[8 * r + 1] = jac_foc(J, r, 1);
#pragma unroll
        for (int k = 0; k < 6; ++k) O.Jcam[8 * r + 2 + k] = jac_tau(J, r, k);
#pragma unroll
        for (int c = 0; c < 3; ++c) O.Jp[3 * r + c] = jac_pts(J, cp, r, c);
    }
    O.fbar = J.fbar;
    O.zscale = J.zscale;
    O.valid = J.valid;
}

// Running maximum of non-negative floating-point values: their bit patterns order as the values, so
// an integer atomic max combines them in any order with the same result.
__device__ __forceinline__ void atomic_max_nonneg(double* p, double v) {
    atomicMax(reinterpret_cast<unsigned long long*>(p), (unsigned long long)__double_as_longlong(v));
}
__device__ __forceinline__ void atomic_max_nonneg(float* p, float v) {
    atomicMax(reinterpret_cast<unsigned int*>(p), __float_as_uint(v));
}

}  // namespace ba
