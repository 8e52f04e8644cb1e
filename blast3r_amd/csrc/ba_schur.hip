// Fused linearisation + Schur reduction for MI355X (gfx950).
//
// Replaces, for one LM step, the reference sequence
//   compute_jacobians (src/blast3r/inference/ba_solver.py:34-40)
//   -> solve_delta: W, J^T W r, J *= sqrt(W), gram_matrix, dampen_ (ba_solver.py:110-177)
//   -> _solve_CG rhs and the Schur operator (ba_solver.py:184-206)
// with four kernels over a precomputed structure plan (ba_plan.cpp):
//   k_track_pp     per chunk: point blocks H_pp, g_p per track (+ max diag for the damping)
//   k_schur        per batch: camera-pair blocks of S = H_cc - H_cp H_pp^-1 H_pc, accumulated
//                  in fp64 MFMA tiles held in registers, plus rhs and diag(H_cc) per image
//   k_pair_reduce  per image pair: deterministic sum of the batch partials
//   k_backsub      per chunk: delta_p = H_pp^-1 (g_p - H_pc delta_c)
// Every per-observation quantity is recomputed from the inputs (no J is stored).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ba_common.h"
#include "ba_error.h"
#include "ba_plan.h"

namespace ba {

typedef double dbl4 __attribute__((ext_vector_type(4)));

typedef ba_layout LinLayout;
typedef ba_lin_args LinArgs;

// ----------------------------------------------------------------------------- per observation
struct ObsLin {
    double Jc[3][16];     // sqrt(W)-weighted camera rows in the image-level layout [foc|tau|zcf]
    double Jp[3][3];      // sqrt(W)-weighted point rows
    double gJ[16];        // J_c^T (W r)
    double gP[3];         // J_p^T (W r)
};

__device__ __forceinline__ float clampw(float w, float lo, float hi) {
    // torch.clamp semantics: NaN propagates
    return w < lo ? lo : (w > hi ? hi : w);
}

template <int HK, int HP>
__device__ __forceinline__ void linearize_obs(const CamF& cp, const float* __restrict__ zc_img, const float X[3],
                                              float2 uv, float2 sv, const float* __restrict__ dep,
                                              const HuberParams& hp, const LinLayout& lay, bool enK, bool enP,
                                              bool enZ, bool enX, bool first_obs, const float* given_r,
                                              const float* given_w, ObsLin& L) {
    constexpr int OT = 2 * HK, OZ = OT + 6 * HP;     // image-level columns [foc | tau | zcf]
    const int C = lay.C;
    ResOut ro;
    if (given_r) {
        // residuals and weights handed to solve_delta by the caller
#pragma unroll
        for (int k = 0; k < 3; ++k) { ro.r[k] = given_r[k]; ro.w[k] = given_w[k]; }
    } else {
        // residual and weights in fp32 (residuals_with_rigs, .cu:129-259)
        float gf = 0.f;
        for (int c = 0; c < C; ++c) gf += zc_img[c] * dep[c];
        eval_residual(cp, X, uv.x, uv.y, sv.x, sv.y, gf, hp, ro);
    }
    // Jacobian in fp64 (.cu:323-509); guidance = float products summed in double
    double gd = 0.0;
    for (int c = 0; c < C; ++c) { float pr = zc_img[c] * dep[c]; gd += (double)pr; }
    JacOut J;
    eval_jacobian(cp, X, sv.x, sv.y, gd, hp.is_depth_log, J);
    // W = clamp(w), g uses (W*r) in fp32 cast to fp64, J *= sqrt(W) with sqrt in fp32 (ba_solver.py:123-132)
    double Wr[3], sW[3];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        float W = clampw(ro.w[r], lay.wmin, lay.wmax);
        Wr[r] = (double)(W * ro.r[r]);
        sW[r] = (double)sqrtf(W);
    }
    const double mK = enK ? 1.0 : 0.0, mP = enP ? 1.0 : 0.0;
    const bool zon = lay.hasZ && enZ && J.valid;
    const bool z0off = !lay.optim_Z0 || (first_obs && !lay.optim_Z_1st_cam);      // ba_solver.py:38-39
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        double u0 = 0.0, u1 = 0.0, u2 = 0.0;
        if (j < OT) {
            u0 = J.Jcam[j] * mK;
            u1 = J.Jcam[8 + j] * mK;
            u2 = lay.no_grad_f_from_rz ? 0.0 : J.Jcam[16 + j] * mK;             // ba_solver.py:59-60
        } else if (j < OZ) {
            u0 = J.Jcam[2 + (j - OT)] * mP;
            u1 = J.Jcam[10 + (j - OT)] * mP;
            u2 = J.Jcam[18 + (j - OT)] * mP;
        } else {
            const int c = j - OZ;
            if (zon && c < C && !(c == 0 && z0off)) u2 = J.zscale * (double)dep[c];
        }
        L.gJ[j] = u0 * Wr[0] + u1 * Wr[1] + u2 * Wr[2];
        L.Jc[0][j] = u0 * sW[0];
        L.Jc[1][j] = u1 * sW[1];
        L.Jc[2][j] = u2 * sW[2];
    }
    bool xon = enX && !lay.x_off;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        double jp0 = xon ? J.Jp[k] : 0.0, jp1 = xon ? J.Jp[3 + k] : 0.0, jp2 = xon ? J.Jp[6 + k] : 0.0;
        L.gP[k] = jp0 * Wr[0] + jp1 * Wr[1] + jp2 * Wr[2];
        L.Jp[0][k] = jp0 * sW[0];
        L.Jp[1][k] = jp1 * sW[1];
        L.Jp[2][k] = jp2 * sW[2];
    }
}

// Damped point block -> Cholesky factor with the chol3x3_solve rules (.cu:560-634):
// + jitter on the diagonal, averaged off-diagonals, non-positive pivots + jitter.
__device__ __forceinline__ void chol3_factor(const double H[6], double lam, double L[6]) {
    const double jit = 1e-12;
    double a00 = (H[0] + lam) + jit, a11 = (H[3] + lam) + jit, a22 = (H[5] + lam) + jit;
    double a01 = H[1], a02 = H[2], a12 = H[4];
    a00 = a00 > 0.0 ? a00 : a00 + jit;
    double l00 = sqrt(a00);
    double l10 = a01 / l00, l20 = a02 / l00;
    double t11 = a11 - l10 * l10;
    t11 = t11 > 0.0 ? t11 : t11 + jit;
    double l11 = sqrt(t11);
    double l21 = (a12 - l10 * l20) / l11;
    double t22 = a22 - l20 * l20 - l21 * l21;
    t22 = t22 > 0.0 ? t22 : t22 + jit;
    double l22 = sqrt(t22);
    L[0] = l00; L[1] = l10; L[2] = l20; L[3] = l11; L[4] = l21; L[5] = l22;
}

__device__ __forceinline__ void chol3_fwd(const double L[6], const double b[3], double y[3]) {
    y[0] = b[0] / L[0];
    y[1] = (b[1] - L[1] * y[0]) / L[3];
    y[2] = (b[2] - L[2] * y[0] - L[4] * y[1]) / L[5];
}

__device__ __forceinline__ void chol3_bwd(const double L[6], const double z[3], double x[3]) {
    x[2] = z[2] / L[5];
    x[1] = (z[1] - L[4] * x[2]) / L[3];
    x[0] = (z[0] - L[1] * x[1] - L[2] * x[2]) / L[0];
}

struct ObsCtx {   // everything one lane needs to linearise its observation
    CamF cp;
    const float* zc;
    bool enK, enP, enZ;
};

__device__ __forceinline__ void load_obs_ctx(const LinArgs& a, int img, ObsCtx& c) {
    int node = a.infos[a.n_imgs + img];
    int cam = a.infos[2 * a.n_imgs + img];
    load_cam(c.cp, a.K, a.P_rig2cam, a.P_rig2cam_stride, a.P_w2rig, cam, node);
    c.zc = a.z_coefs + (int64_t)img * a.lay.C;
    c.enK = a.enK ? a.enK[cam] != 0 : true;
    c.enP = a.enP ? a.enP[node] != 0 : true;
    c.enZ = a.enZ ? a.enZ[img] != 0 : true;
}

template <int HK, int HP>
__device__ __forceinline__ void linearize_slot(const LinArgs& a, int64_t slot, int obs, const ObsCtx& c, ObsLin& L,
                                               int& pid) {
    pid = a.s_pid[slot];
    float X[3] = {a.pts3d[3 * (int64_t)pid], a.pts3d[3 * (int64_t)pid + 1], a.pts3d[3 * (int64_t)pid + 2]};
    float2 uv = reinterpret_cast<const float2*>(a.s_pix)[slot];
    float2 sv = reinterpret_cast<const float2*>(a.s_std)[slot];
    bool enX = a.enX ? a.enX[pid] != 0 : true;
    float gr[3], gw[3];
    if (a.r_in) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            gr[k] = a.r_in[(int64_t)obs * a.r_s0 + k * a.r_s1];
            gw[k] = a.w_in[(int64_t)obs * a.w_s0 + k * a.w_s1];
        }
    }
    linearize_obs<HK, HP>(c.cp, c.zc, X, uv, sv, a.s_dep + slot * a.lay.C, a.hp, a.lay, c.enK, c.enP, c.enZ, enX,
                          obs == 0, a.r_in ? gr : nullptr, a.r_in ? gw : nullptr, L);
}

// ----------------------------------------------------------------------------- point blocks
template <int HK, int HP>
__global__ void __launch_bounds__(BA_CHUNK) k_track_pp(LinArgs a) {
    __shared__ double sh[BA_CHUNK][9];
    __shared__ double smax[BA_CHUNK];
    const int chunk = blockIdx.x, tid = threadIdx.x;
    const int64_t slot = (int64_t)chunk * BA_CHUNK + tid;
    const int obs = a.chunk_obs[slot];
    double c[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) c[k] = 0.0;
    if (obs >= 0) {
        ObsCtx ctx;
        load_obs_ctx(a, a.s_img[slot], ctx);
        ObsLin L;
        int pid;
        linearize_slot<HK, HP>(a, slot, obs, ctx, L, pid);
        // J_pts gram (ba_solver.py:911-924) and J_pts^T W r
        const int pr[6][2] = {{0, 0}, {0, 1}, {0, 2}, {1, 1}, {1, 2}, {2, 2}};
#pragma unroll
        for (int q = 0; q < 6; ++q) {
            int i = pr[q][0], j = pr[q][1];
            c[q] = L.Jp[0][i] * L.Jp[0][j] + L.Jp[1][i] * L.Jp[1][j] + L.Jp[2][i] * L.Jp[2][j];
        }
        c[6] = L.gP[0]; c[7] = L.gP[1]; c[8] = L.gP[2];
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) sh[tid][k] = c[k];
    __syncthreads();
    const int first_ct = a.chunk_meta[4 * chunk + 1], n_ct = a.chunk_meta[4 * chunk + 2];
    double mx = 0.0;
    if (tid < n_ct) {
        int f = a.ct_first[first_ct + tid], m = a.ct_m[first_ct + tid], pid = a.ct_pid[first_ct + tid];
        double s[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) s[k] = 0.0;
        for (int q = 0; q < m; ++q)
#pragma unroll
            for (int k = 0; k < 9; ++k) s[k] += sh[f + q][k];
#pragma unroll
        for (int k = 0; k < 6; ++k) a.Hpp[6 * (int64_t)pid + k] = s[k];
#pragma unroll
        for (int k = 0; k < 3; ++k) a.gp[3 * (int64_t)pid + k] = s[6 + k];
        mx = fmax(fmax(fabs(s[0]), fabs(s[3])), fabs(s[5]));
    }
    smax[tid] = mx;
    __syncthreads();
    for (int w = BA_CHUNK / 2; w > 0; w >>= 1) {
        if (tid < w) smax[tid] = fmax(smax[tid], smax[tid + w]);
        __syncthreads();
    }
    if (tid == 0) a.chunk_max[chunk] = smax[0];
}

// lam_p = dampen * max diag over all tracks (BlockDiagMat.dampen_, ba_solver.py:575-582)
__global__ void __launch_bounds__(256) k_lam_reduce(const double* __restrict__ cmax, int64_t n, double dampen,
                                                    int adaptive, int x_off, double* __restrict__ out) {
    __shared__ double s[256];
    double m = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) m = fmax(m, cmax[i]);
    s[threadIdx.x] = m;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) s[threadIdx.x] = fmax(s[threadIdx.x], s[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = (adaptive && !x_off) ? dampen * s[0] : dampen;
}

// ----------------------------------------------------------------------------- camera-pair blocks
__device__ __forceinline__ int pop_lowest(uint64_t& m0, uint64_t& m1) {
    if (m0) { int b = __builtin_ctzll(m0); m0 &= m0 - 1; return b; }
    int b = __builtin_ctzll(m1); m1 &= m1 - 1; return 64 + b;
}

__device__ __forceinline__ int sel4(int q, int v0, int v1, int v2, int v3) {
    return q == 0 ? v0 : (q == 1 ? v1 : (q == 2 ? v2 : v3));
}

// One 16x16 fp64 tile: acc += sign * X_a^T X_b over K-elements (group item, component).
// Items come 4 at a time from a uniform bit mask; item q maps to LDS rows (ra, rb).
template <bool DIAG_J>
__device__ __forceinline__ void mfma_items(dbl4& acc, uint64_t m0, uint64_t m1, const double* __restrict__ X,
                                           const unsigned char* __restrict__ rowsA, const unsigned char* __restrict__ rowsB,
                                           int rstride, int la, int lb, int d, double sign, int lane) {
    int cnt = __builtin_popcountll(m0) + __builtin_popcountll(m1);
    const int i = lane & 15;
    const int kk = lane >> 4;
    for (int g = 0; g < cnt; g += 4) {
        int nt = cnt - g < 4 ? cnt - g : 4;
        int it[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) it[q] = (q < nt) ? pop_lowest(m0, m1) : 0;
        int ra[4], rb[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (DIAG_J) { ra[q] = it[q]; rb[q] = it[q]; }
            else { ra[q] = rowsA[it[q] * rstride + la]; rb[q] = rowsB[it[q] * rstride + lb]; }
        }
        int nk = 3 * nt;
#pragma unroll
        for (int mm = 0; mm < 3; ++mm) {
            if (4 * mm >= nk) break;
            int k = 4 * mm + kk;
            int q = k / 3, comp = k - 3 * (k / 3);
            bool ok = (k < nk) && (i < d);
            int rowa = sel4(q, ra[0], ra[1], ra[2], ra[3]);
            int rowb = sel4(q, rb[0], rb[1], rb[2], rb[3]);
            double A = ok ? sign * X[(rowa * 3 + comp) * d + i] : 0.0;
            double B = ok ? X[(rowb * 3 + comp) * d + i] : 0.0;
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(A, B, acc, 0, 0, 0);
        }
    }
}

template <int HK, int HP>
__global__ void __launch_bounds__(BA_WAVES * 64) k_schur(LinArgs a) {
    extern __shared__ double dyn[];
    const int d = a.lay.d, C = a.lay.C;
    double* sV = dyn;                                 // [CHUNK][3][d]  V = H_cp L^-T per observation
    double* sJ = sV + BA_CHUNK * 3 * d;               // [CHUNK][3][d]  weighted J_c rows
    double* sE = sJ + BA_CHUNK * 3 * d;               // [CHUNK][d]     rhs contribution
    double* sD = sE + BA_CHUNK * d;                   // [CHUNK][d]     diag(J_c^T J_c) contribution
    __shared__ int sInfo[BA_CHUNK];
    __shared__ unsigned sMask[BA_CHUNK];
    __shared__ unsigned char sRow[BA_CHUNK * BA_MAX_LOCAL];
    __shared__ CamF sCam[BA_MAX_LOCAL];
    __shared__ float sZc[BA_MAX_LOCAL * BA_MAX_C];
    __shared__ unsigned char sEn[BA_MAX_LOCAL * 3];
    __shared__ unsigned char sLa[BA_MAX_SLOTS], sLb[BA_MAX_SLOTS];
    __shared__ double sVec[BA_MAX_LOCAL * 2 * 16];       // per local image: rhs (d) | diag(H_cc) (d)

    const int batch = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nimg = a.b_nimgs[batch];
    const int s0 = a.b_slot_ptr[batch], ns = a.b_slot_ptr[batch + 1] - s0;
    const double lam = a.lam_p[0];

    // local image parameters
    if (tid < nimg) {
        int img = a.b_imgs[(int64_t)batch * a.L + tid];
        int node = a.infos[a.n_imgs + img], cam = a.infos[2 * a.n_imgs + img];
        load_cam(sCam[tid], a.K, a.P_rig2cam, a.P_rig2cam_stride, a.P_w2rig, cam, node);
        for (int c = 0; c < C; ++c) sZc[tid * BA_MAX_C + c] = a.z_coefs[(int64_t)img * C + c];
        sEn[3 * tid + 0] = a.enK ? a.enK[cam] : 1;
        sEn[3 * tid + 1] = a.enP ? a.enP[node] : 1;
        sEn[3 * tid + 2] = a.enZ ? a.enZ[img] : 1;
    }

    for (int q = tid; q < ns; q += BA_WAVES * 64) {
        const int pr = a.slot_pair[s0 + q];
        sLa[q] = (unsigned char)(pr & 0xff);
        sLb[q] = (unsigned char)((pr >> 8) & 0xff);
    }
    for (int q = tid; q < BA_MAX_LOCAL * 2 * 16; q += BA_WAVES * 64) sVec[q] = 0.0;

    dbl4 acc[BA_SLOTS_PER_WAVE];
#pragma unroll
    for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) acc[q] = dbl4{0.0, 0.0, 0.0, 0.0};
    // K-element of this lane in the three MFMAs of a 4-track group: k = 4*mm + lane/16
    const int mi = lane & 15, kk = lane >> 4;

    const int c_begin = a.b_chunk_ptr[batch], c_end = a.b_chunk_ptr[batch + 1];
    for (int ck = c_begin; ck < c_end; ++ck) {
        __syncthreads();    // previous chunk fully consumed; local params visible
        const int first_ct = a.chunk_meta[4 * ck + 1], n_ct = a.chunk_meta[4 * ck + 2];
        if (tid < BA_CHUNK) {
            const int64_t slot = (int64_t)ck * BA_CHUNK + tid;
            const int info = a.slot_info[slot];
            sInfo[tid] = info;
            if (info >= 0) {
                const int li = info & 0xff, ctr = (info >> 8) & 0xff, leader = info >> 16;
                const int obs = a.chunk_obs[slot];
                ObsCtx ctx;
                ctx.cp = sCam[li];
                ctx.zc = sZc + li * BA_MAX_C;
                ctx.enK = sEn[3 * li] != 0; ctx.enP = sEn[3 * li + 1] != 0; ctx.enZ = sEn[3 * li + 2] != 0;
                ObsLin L;
                int pid;
                linearize_slot<HK, HP>(a, slot, obs, ctx, L, pid);
                double H[6], g[3], Lf[6];
#pragma unroll
                for (int k = 0; k < 6; ++k) H[k] = a.Hpp[6 * (int64_t)pid + k];
#pragma unroll
                for (int k = 0; k < 3; ++k) g[k] = a.gp[3 * (int64_t)pid + k];
                chol3_factor(H, lam, Lf);
                double P[3][3], w[3];
#pragma unroll
                for (int r = 0; r < 3; ++r) chol3_fwd(Lf, L.Jp[r], P[r]);    // P = Jp L^-T (row-wise)
                chol3_fwd(Lf, g, w);                                          // w = L^-1 g_p
                double* v = sV + tid * 3 * d;
                double* jj = sJ + tid * 3 * d;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    if (j < d) {
                        double v0 = L.Jc[0][j] * P[0][0] + L.Jc[1][j] * P[1][0] + L.Jc[2][j] * P[2][0];
                        double v1 = L.Jc[0][j] * P[0][1] + L.Jc[1][j] * P[1][1] + L.Jc[2][j] * P[2][1];
                        double v2 = L.Jc[0][j] * P[0][2] + L.Jc[1][j] * P[1][2] + L.Jc[2][j] * P[2][2];
                        v[0 * d + j] = v0; v[1 * d + j] = v1; v[2 * d + j] = v2;
                        jj[0 * d + j] = L.Jc[0][j]; jj[1 * d + j] = L.Jc[1][j]; jj[2 * d + j] = L.Jc[2][j];
                        sE[tid * d + j] = L.gJ[j] - (v0 * w[0] + v1 * w[1] + v2 * w[2]);
                        sD[tid * d + j] = L.Jc[0][j] * L.Jc[0][j] + L.Jc[1][j] * L.Jc[1][j] + L.Jc[2][j] * L.Jc[2][j];
                    }
                }
                if (leader == tid) sRow[ctr * BA_MAX_LOCAL + li] = (unsigned char)tid;
            }
        }
        if (tid < n_ct) sMask[tid] = (unsigned)a.ct_mask[first_ct + tid];
        __syncthreads();
        // several observations of one track in one image: sum their V into the leader row
        if (tid < BA_CHUNK) {
            int info = sInfo[tid];
            if (info >= 0 && (info >> 16) == tid) {
                for (int f = tid + 1; f < BA_CHUNK; ++f) {
                    int fi = sInfo[f];
                    if (fi < 0 || (fi >> 16) != tid) break;
                    for (int e = 0; e < 3 * d; ++e) sV[tid * 3 * d + e] += sV[f * 3 * d + e];
                }
            }
        }
        __syncthreads();

        // camera-pair tiles: groups of 4 chunk tracks outermost, so that every owned slot the group
        // covers gets its 3 MFMAs back to back on independent accumulators
        for (int t0 = 0; t0 < n_ct; t0 += 4) {
            const unsigned gm0 = sMask[t0];
            const unsigned gm1 = t0 + 1 < n_ct ? sMask[t0 + 1] : 0u;
            const unsigned gm2 = t0 + 2 < n_ct ? sMask[t0 + 2] : 0u;
            const unsigned gm3 = t0 + 3 < n_ct ? sMask[t0 + 3] : 0u;
#pragma unroll
            for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
                const int sl = wave + BA_WAVES * q;
                if (sl < ns) {
                    const int la = sLa[sl], lb = sLb[sl];
                    const unsigned cov = ((gm0 >> la) & (gm0 >> lb) & 1u) | (((gm1 >> la) & (gm1 >> lb) & 1u) << 1) |
                                         (((gm2 >> la) & (gm2 >> lb) & 1u) << 2) |
                                         (((gm3 >> la) & (gm3 >> lb) & 1u) << 3);
                    if (cov) {
#pragma unroll
                        for (int mm = 0; mm < 3; ++mm) {
                            const int kq = 4 * mm + kk, tq = kq / 3, gcomp = kq - 3 * tq;
                            const bool on = ((cov >> tq) & 1u) && mi < d;
                            const int t = t0 + tq < BA_CHUNK ? t0 + tq : BA_CHUNK - 1;
                            const int ra = sRow[t * BA_MAX_LOCAL + la], rb = sRow[t * BA_MAX_LOCAL + lb];
                            const double A = on ? -sV[(ra * 3 + gcomp) * d + mi] : 0.0;
                            const double B = on ? sV[(rb * 3 + gcomp) * d + mi] : 0.0;
                            acc[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(A, B, acc[q], 0, 0, 0);
                        }
                    }
                }
            }
        }
        // diagonal slots: + J_c^T J_c of every observation in the image, and the image's rhs and
        // diag(H_cc) contributions (each image has exactly one diagonal slot, owned by one wave)
#pragma unroll
        for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
            const int sl = wave + BA_WAVES * q;
            if (sl < ns && sLa[sl] == sLb[sl]) {
                const int la = sLa[sl];
                int i0 = sInfo[lane], i1 = sInfo[lane + 64];
                bool o0 = i0 >= 0 && (i0 & 0xff) == la;
                bool o1 = i1 >= 0 && (i1 & 0xff) == la;
                uint64_t n0 = __ballot(o0), n1 = __ballot(o1);
                if (lane < d) {
                    double e = sVec[la * 32 + lane], g = sVec[la * 32 + 16 + lane];
                    uint64_t c0 = n0, c1 = n1;
                    while (c0 | c1) {
                        int s = pop_lowest(c0, c1);
                        e += sE[s * d + lane];
                        g += sD[s * d + lane];
                    }
                    sVec[la * 32 + lane] = e;
                    sVec[la * 32 + 16 + lane] = g;
                }
                mfma_items<true>(acc[q], n0, n1, sJ, nullptr, nullptr, 0, la, la, d, 1.0, lane);
            }
        }
    }

    // flush this batch's partial blocks (row-major d x d, local orientation)
#pragma unroll
    for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
        const int sl = wave + BA_WAVES * q;
        if (sl < ns) {
            double* P = a.partials + (int64_t)(s0 + sl) * d * d;
            // v_mfma_f64_16x16x4f64 accumulator layout: lane l, element v holds D[4v + l/16][l%16]
            const int j = lane & 15;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                int i = 4 * v + (lane >> 4);
                if (i < d && j < d) P[i * d + j] = acc[q][v];
            }
        }
    }
    __syncthreads();
    {
        const int va = tid >> 4, vj = tid & 15;
        if (va < nimg && vj < d) {
            double* o = a.img_partials + ((int64_t)batch * a.L + va) * 2 * d;
            o[vj] = sVec[va * 32 + vj];
            o[d + vj] = sVec[va * 32 + 16 + vj];
        }
    }
}

// ----------------------------------------------------------------------------- reductions
__global__ void __launch_bounds__(256) k_pair_reduce(const int* __restrict__ pair_ptr, const int* __restrict__ pair_src,
                                                     const double* __restrict__ partials, int64_t n_pairs, int d,
                                                     double* __restrict__ out) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int dd = d * d;
    if (tid >= n_pairs * dd) return;
    int64_t p = tid / dd;
    int e = (int)(tid - p * dd);
    int i = e / d, j = e - (e / d) * d;
    double acc = 0.0;
    for (int q = pair_ptr[p]; q < pair_ptr[p + 1]; ++q) {
        int src = pair_src[q];
        int64_t s = src >> 1;
        acc += partials[s * dd + ((src & 1) ? j * d + i : i * d + j)];
    }
    out[tid] = acc;
}

__global__ void __launch_bounds__(256) k_img_reduce(const int* __restrict__ img_ptr, const int* __restrict__ img_src,
                                                    const double* __restrict__ ip, int n_imgs, int d,
                                                    double* __restrict__ e_out, double* __restrict__ dg_out) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= (int64_t)n_imgs * d) return;
    int i = (int)(tid / d), j = (int)(tid - (tid / d) * d);
    double e = 0.0, g = 0.0;
    for (int q = img_ptr[i]; q < img_ptr[i + 1]; ++q) {
        const double* s = ip + (int64_t)img_src[q] * 2 * d;
        e += s[j];
        g += s[d + j];
    }
    e_out[tid] = e;
    dg_out[tid] = g;
}

// ----------------------------------------------------------------------------- back-substitution
template <int HK, int HP>
__global__ void __launch_bounds__(BA_CHUNK) k_backsub(LinArgs a) {
    __shared__ double sh[BA_CHUNK][3];
    const int chunk = blockIdx.x, tid = threadIdx.x;
    const int64_t slot = (int64_t)chunk * BA_CHUNK + tid;
    const int obs = a.chunk_obs[slot];
    const int d = a.lay.d;
    double y[3] = {0.0, 0.0, 0.0};
    if (obs >= 0) {
        const int img = a.s_img[slot];
        ObsCtx ctx;
        load_obs_ctx(a, img, ctx);
        ObsLin L;
        int pid;
        linearize_slot<HK, HP>(a, slot, obs, ctx, L, pid);
        double t[3] = {0.0, 0.0, 0.0};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (j < d) {
                int u = a.umap[(int64_t)img * d + j];
                double x = u >= 0 ? a.dc[u] : 0.0;
                t[0] += L.Jc[0][j] * x; t[1] += L.Jc[1][j] * x; t[2] += L.Jc[2][j] * x;
            }
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) y[k] = L.Jp[0][k] * t[0] + L.Jp[1][k] * t[1] + L.Jp[2][k] * t[2];
    }
    sh[tid][0] = y[0]; sh[tid][1] = y[1]; sh[tid][2] = y[2];
    __syncthreads();
    const int first_ct = a.chunk_meta[4 * chunk + 1], n_ct = a.chunk_meta[4 * chunk + 2];
    if (tid < n_ct) {
        int f = a.ct_first[first_ct + tid], m = a.ct_m[first_ct + tid], pid = a.ct_pid[first_ct + tid];
        double s[3] = {0.0, 0.0, 0.0};
        for (int q = 0; q < m; ++q) { s[0] += sh[f + q][0]; s[1] += sh[f + q][1]; s[2] += sh[f + q][2]; }
        double H[6], Lf[6], b[3], z[3], x[3];
#pragma unroll
        for (int k = 0; k < 6; ++k) H[k] = a.Hpp[6 * (int64_t)pid + k];
#pragma unroll
        for (int k = 0; k < 3; ++k) b[k] = a.gp[3 * (int64_t)pid + k] - s[k];
        chol3_factor(H, a.lam_p[0], Lf);
        chol3_fwd(Lf, b, z);
        chol3_bwd(Lf, z, x);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            a.dX[3 * (int64_t)pid + k] = (float)x[k];
            if (a.dX64) a.dX64[3 * (int64_t)pid + k] = x[k];
        }
    }
}

}  // namespace ba

using namespace ba;

// ============================================================================= C ABI

static inline unsigned nblk(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

// instantiate the kernels for the four (focal on/off, pose on/off) column layouts
#define BA_DISPATCH_KP(lay, ...)                                                   \
    do {                                                                           \
        if ((lay).hasK && (lay).hasP) { constexpr int HK_ = 1, HP_ = 1; __VA_ARGS__; } \
        else if ((lay).hasK)          { constexpr int HK_ = 1, HP_ = 0; __VA_ARGS__; } \
        else if ((lay).hasP)          { constexpr int HK_ = 0, HP_ = 1; __VA_ARGS__; } \
        else                          { constexpr int HK_ = 0, HP_ = 0; __VA_ARGS__; } \
    } while (0)

extern "C" int ba_linearize_stage(const ba_lin_args* args, int32_t stage, void* stream);

extern "C" int ba_linearize_schur(const ba_lin_args* args, void* stream) {
    for (int s = 0; s < 3; ++s) {
        int rc = ba_linearize_stage(args, s, stream);
        if (rc) return rc;
    }
    return BA_OK;
}

// stage 0: point blocks + damping value; 1: camera-pair batches; 2: deterministic reductions
extern "C" int ba_linearize_stage(const ba_lin_args* args, int32_t stage, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_lin_args& a = *args;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.lay.d >= 1 && a.lay.d <= 16, "fused path supports 1 <= d <= 16 image-level parameters");
    BA_REQUIRE(a.lay.off_tau == 2 * a.lay.hasK && a.lay.off_zcf == a.lay.off_tau + 6 * a.lay.hasP &&
                   a.lay.d == a.lay.off_zcf + (a.lay.hasZ ? a.lay.C : 0),
               "inconsistent image-level layout");
    BA_REQUIRE(a.lay.C >= 0 && a.lay.C <= BA_MAX_C, "fused path supports at most 24 z-coefficient columns");
    BA_REQUIRE(a.L >= 1 && a.L <= BA_MAX_LOCAL, "bad plan L");
    if (stage == 0 && a.n_chunks == 0) {
        BA_HIP(hipMemsetAsync(a.lam_p, 0, sizeof(double), st));
    } else if (stage == 0) {
        BA_DISPATCH_KP(a.lay, hipLaunchKernelGGL((k_track_pp<HK_, HP_>), dim3((unsigned)a.n_chunks), dim3(BA_CHUNK), 0, st, a));
        BA_LAUNCHED();
    }
    if (stage == 0) {
        hipLaunchKernelGGL(k_lam_reduce, dim3(1), dim3(256), 0, st, a.chunk_max, a.n_chunks, a.lay.dampen,
                           a.lay.adaptive, a.lay.x_off, a.lam_p);
        BA_LAUNCHED();
        return BA_OK;
    }
    if (stage == 1 && a.n_batches > 0) {
        size_t lds = (size_t)BA_CHUNK * 8 * a.lay.d * sizeof(double);
        BA_DISPATCH_KP(a.lay, {
            BA_HIP(hipFuncSetAttribute((const void*)k_schur<HK_, HP_>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds));
            hipLaunchKernelGGL((k_schur<HK_, HP_>), dim3((unsigned)a.n_batches), dim3(BA_WAVES * 64), lds, st, a);
        });
        BA_LAUNCHED();
    }
    if (stage == 1) return BA_OK;
    int d = a.lay.d;
    if (a.n_pairs > 0) {
        hipLaunchKernelGGL(k_pair_reduce, dim3(nblk(a.n_pairs * d * d, 256)), dim3(256), 0, st, a.pair_ptr, a.pair_src,
                           a.partials, a.n_pairs, d, a.S_pairs);
        BA_LAUNCHED();
    }
    hipLaunchKernelGGL(k_img_reduce, dim3(nblk((int64_t)a.n_imgs * d, 256)), dim3(256), 0, st, a.img_ptr, a.img_src,
                       a.img_partials, a.n_imgs, d, a.e_img, a.dg_img);
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int ba_backsubstitute(const ba_lin_args* args, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_lin_args& a = *args;
    BA_REQUIRE(a.lay.d >= 1 && a.lay.d <= 16, "fused path supports 1 <= d <= 16 image-level parameters");
    if (a.n_chunks == 0) return BA_OK;
    hipStream_t st = (hipStream_t)stream;
    BA_DISPATCH_KP(a.lay, hipLaunchKernelGGL((k_backsub<HK_, HP_>), dim3((unsigned)a.n_chunks), dim3(BA_CHUNK), 0, st, a));
    BA_LAUNCHED();
    return BA_OK;
}
