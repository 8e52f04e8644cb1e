// Fused linearisation + Schur reduction for MI355X (gfx950).
//
// Replaces, for one LM step, the reference sequence
//   compute_jacobians (src/blast3r/inference/ba_solver.py:34-40)
//   -> solve_delta: W, J^T W r, J *= sqrt(W), gram_matrix, dampen_ (ba_solver.py:110-177)
//   -> _solve_CG rhs and the Schur operator (ba_solver.py:184-206)
// with four kernels over a precomputed structure plan (ba_plan.cpp):
//   k_track_pp     per chunk: point blocks H_pp, g_p per track (+ max diag for the damping)
//   k_schur        per batch: camera-pair blocks of S = H_cc - H_cp H_pp^-1 H_pc, accumulated
//                  in MFMA tiles of the working precision (fp64, or fp32 for the fp32 solver) held in
//                  registers, plus rhs and diag(H_cc) per image
//   k_pair_reduce  per image pair: deterministic sum of the batch partials
//   k_backsub      per chunk: delta_p = H_pp^-1 (g_p - H_pc delta_c)
// The expensive per-observation work (residual, IRLS weight, Jacobian core) is done once, in
// k_track_pp, and kept as a 160-byte record per observation; the weighted rows are re-formed from it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ba_common.h"
#include "ba_error.h"
#include "ba_plan.h"

namespace ba {

typedef double dbl4 __attribute__((ext_vector_type(4)));
typedef float flt4 __attribute__((ext_vector_type(4)));

typedef ba_layout LinLayout;
typedef ba_lin_args LinArgs;

// ----------------------------------------------------------------------------- per observation
#define BA_PRE_C 8          // depth-guidance channels held in registers (further channels are read from memory)
// The MFMA entry lists come from the plan (32-bit entries holding the LDS offsets of the A and B
// rows, see ba_plan.h): one entry per (track, image pair) of an off-diagonal slot, per observation
// and per (track, image) run of a diagonal slot.  The planner rejects a chunk that would need more
// than BA_LIST_CAP entries; the kernel copies whole lists of that capacity.
static_assert(BA_LIST_CAP * 4 % 1024 == 0 && BA_MAX_SLOTS % 4 == 0, "list copies are whole 16-byte lanes");
static_assert(BA_ZERO + 48 < 65536 && BA_LIST_CAP < 4096, "entry offsets fit their fields");
#define BA_CORE 20          // doubles per observation in the linearisation record
#define BA_CORE32 24        // floats per observation in the fp32 solver's record (22 used)
static_assert(BA_CORE * BA_CHUNK % 256 == 0, "a chunk's record block is copied 256 doubles at a time");

// Depth-guidance channels of one observation: the first BA_PRE_C in registers, the rest in memory.
// Every access uses a compile-time channel index, so the register part never spills.
struct DepSrc {
    float r[BA_PRE_C];
    const float* g;
    __device__ __forceinline__ float operator()(int c) const { return c < BA_PRE_C ? r[c] : g[c]; }
};

__device__ __forceinline__ void load_dep(DepSrc& s, const float* g, int C) {
    s.g = g;
#pragma unroll
    for (int c = 0; c < BA_PRE_C; ++c) s.r[c] = c < C ? g[c] : 0.f;
}

// The sqrt(W)-weighted camera rows (image-level layout [foc|tau|zcf], columns 0..15, zero beyond d)
// are handed element by element to a sink (r, j, value) as they are formed, so no caller holds all
// of them in registers at once.
struct NoSink {
    __device__ __forceinline__ void operator()(int, int, double) const {}
};

__device__ __forceinline__ float clampw(float w, float lo, float hi) {
    // torch.clamp semantics: NaN propagates
    return w < lo ? lo : (w > hi ? hi : w);
}

// Residuals and IRLS weights handed over by the caller (the `residuals`, `w_pts` of solve_delta)
struct GivenRW {
    float r[3], w[3];
};

// Everything the weighted rows of one observation are formed from.
struct ObsCore {
    JacCore J;
    double sW[3];         // sqrt(W), W = clamp(w), sqrt in fp32 (ba_solver.py:123-132)
    double Wr[3];         // W*r formed in fp32, widened (ba_solver.py:128)
    double Rs[3];         // W*r / sqrt(W): the residual that pairs with the weighted rows in J^T W r
};

__device__ __forceinline__ void obs_core(const CamF& cp, const float* __restrict__ zc_img, const float X[3], float2 uv,
                                         float2 sv, const DepSrc& dep, const HuberParams& hp, const LinLayout& lay,
                                         bool given, const GivenRW& grw, ObsCore& o) {
    const int C = lay.C;
    ResOut ro;
    if (given) {
#pragma unroll
        for (int k = 0; k < 3; ++k) { ro.r[k] = grw.r[k]; ro.w[k] = grw.w[k]; }
    } else {
        // residual and weights in fp32 (residuals_with_rigs, .cu:129-259)
        float gf = 0.f;
#pragma unroll
        for (int c = 0; c < BA_MAX_C; ++c)
            if (c < C) gf += zc_img[c] * dep(c);
        eval_residual(cp, X, uv.x, uv.y, sv.x, sv.y, gf, hp, ro);
    }
    // Jacobian in fp64 (.cu:323-509); guidance = float products summed in double
    double gd = 0.0;
#pragma unroll
    for (int c = 0; c < BA_MAX_C; ++c)
        if (c < C) { float pr = zc_img[c] * dep(c); gd += (double)pr; }
    eval_jac_core(cp, X, sv.x, sv.y, gd, hp.is_depth_log, o.J);
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        float W = clampw(ro.w[r], lay.wmin, lay.wmax);
        o.Wr[r] = (double)(W * ro.r[r]);
        o.sW[r] = (double)sqrtf(W);
        o.Rs[r] = o.Wr[r] * (1.0 / o.sW[r]);
    }
}

// The linearisation record of one observation slot, written by the point-block pass and read by
// the camera-pair and back-substitution passes: chunk-blocked structure of arrays, field f of slot
// (chunk, t) at rec[(chunk * BA_CORE + f) * BA_CHUNK + t] (coalesced per field).
//   0-2 X_rig | 3-11 Jpr | 12 d r0/d fx | 13 d r1/d fy | 14 zscale | 15-17 W r / sqrt(W)
//   18 (J_k_f, sqrt(W_0)) | 19 (sqrt(W_1), sqrt(W_2))  as fp32 pairs (both are fp32 values)
__device__ __forceinline__ void core_store(double* __restrict__ rec, int t, const ObsCore& o) {
    // streamed out (the records of a pass exceed every cache; k_schur reads them back after the point pass)
    auto put = [&](int f, double v) { __builtin_nontemporal_store(v, rec + f * BA_CHUNK + t); };
#pragma unroll
    for (int k = 0; k < 3; ++k) put(k, o.J.Xr[k]);
#pragma unroll
    for (int k = 0; k < 9; ++k) put(3 + k, o.J.Jpr[k]);
    put(12, o.J.fx_col);
    put(13, o.J.fy_col);
    put(14, o.J.zscale);
#pragma unroll
    for (int k = 0; k < 3; ++k) put(15 + k, o.Rs[k]);
    float2* p = reinterpret_cast<float2*>(rec);
    const float2 a = make_float2((float)o.J.jkf, (float)o.sW[0]), b = make_float2((float)o.sW[1], (float)o.sW[2]);
    __builtin_nontemporal_store(__builtin_bit_cast(double, a), reinterpret_cast<double*>(p + 18 * BA_CHUNK + t));
    __builtin_nontemporal_store(__builtin_bit_cast(double, b), reinterpret_cast<double*>(p + 19 * BA_CHUNK + t));
}

// NT: non-temporal loads (a record read once from memory, by the back-substitution)
template <bool NT = false>
__device__ __forceinline__ void core_load(const double* __restrict__ rec, int t, ObsCore& o) {
    auto get = [&](int f) { return NT ? __builtin_nontemporal_load(rec + f * BA_CHUNK + t) : rec[f * BA_CHUNK + t]; };
#pragma unroll
    for (int k = 0; k < 3; ++k) o.J.Xr[k] = get(k);
#pragma unroll
    for (int k = 0; k < 9; ++k) o.J.Jpr[k] = get(3 + k);
    o.J.fx_col = get(12);
    o.J.fy_col = get(13);
    o.J.zscale = get(14);
#pragma unroll
    for (int k = 0; k < 3; ++k) o.Rs[k] = get(15 + k);
    const double* p2 = reinterpret_cast<const double*>(reinterpret_cast<const float2*>(rec));
    const float2 a = __builtin_bit_cast(float2, NT ? __builtin_nontemporal_load(p2 + 18 * BA_CHUNK + t) : p2[18 * BA_CHUNK + t]);
    const float2 b = __builtin_bit_cast(float2, NT ? __builtin_nontemporal_load(p2 + 19 * BA_CHUNK + t) : p2[19 * BA_CHUNK + t]);
    o.J.jkf = a.x;
    o.sW[0] = a.y; o.sW[1] = b.x; o.sW[2] = b.y;
}

// The fp32 solver's record (real32): the same fields rounded to fp32, one float each,
//   0-2 X_rig | 3-11 Jpr | 12, 13 focal columns | 14 zscale | 15-17 W r / sqrt(W) | 18 J_k_f | 19-21 sqrt(W)
// (22, 23 unused: a chunk's block stays a whole number of 2 KB copies), 96 bytes per slot against 160.
__device__ __forceinline__ void core_store(float* __restrict__ rec, int t, const ObsCore& o) {
    auto put = [&](int f, double v) { __builtin_nontemporal_store((float)v, rec + f * BA_CHUNK + t); };
#pragma unroll
    for (int k = 0; k < 3; ++k) put(k, o.J.Xr[k]);
#pragma unroll
    for (int k = 0; k < 9; ++k) put(3 + k, o.J.Jpr[k]);
    put(12, o.J.fx_col);
    put(13, o.J.fy_col);
    put(14, o.J.zscale);
#pragma unroll
    for (int k = 0; k < 3; ++k) put(15 + k, o.Rs[k]);
    put(18, o.J.jkf);
#pragma unroll
    for (int k = 0; k < 3; ++k) put(19 + k, o.sW[k]);
}

template <bool NT = false>
__device__ __forceinline__ void core_load(const float* __restrict__ rec, int t, ObsCore& o) {
    auto get = [&](int f) { return (double)(NT ? __builtin_nontemporal_load(rec + f * BA_CHUNK + t) : rec[f * BA_CHUNK + t]); };
#pragma unroll
    for (int k = 0; k < 3; ++k) o.J.Xr[k] = get(k);
#pragma unroll
    for (int k = 0; k < 9; ++k) o.J.Jpr[k] = get(3 + k);
    o.J.fx_col = get(12);
    o.J.fy_col = get(13);
    o.J.zscale = get(14);
#pragma unroll
    for (int k = 0; k < 3; ++k) o.Rs[k] = get(15 + k);
    o.J.jkf = get(18);
#pragma unroll
    for (int k = 0; k < 3; ++k) o.sW[k] = get(19 + k);
}

// the record type and its fields per slot, by working precision
template <typename Real> struct CoreRec;
template <> struct CoreRec<double> { typedef double T; static constexpr int NF = BA_CORE; };
template <> struct CoreRec<float> { typedef float T; static constexpr int NF = BA_CORE32; };

// Weighted camera row R, element by element, from the core (.cu:444-501, ba_solver.py:38-39, :59-60);
// only the columns j in [JLO, JHI) are formed.
template <int HK, int HP, int R, int JLO = 0, int JHI = 16, class RowSink>
__device__ __forceinline__ void emit_jc_row(const ObsCore& o, const LinLayout& lay, bool enK, bool enP, bool enZ,
                                            bool first_obs, const DepSrc& dep, RowSink&& sink) {
    constexpr int OT = 2 * HK, OZ = OT + 6 * HP;     // image-level columns [foc | tau | zcf]
    const int C = lay.C;
    const double mK = enK ? 1.0 : 0.0, mP = enP ? 1.0 : 0.0;
    const bool zon = lay.hasZ && enZ;                 // an invalid observation has zscale = 0
    const bool z0off = !lay.optim_Z0 || (first_obs && !lay.optim_Z_1st_cam);
#pragma unroll
    for (int j = JLO; j < JHI; ++j) {
        double u = 0.0;
        if (j < OT) {
            u = (R == 2 && lay.no_grad_f_from_rz) ? 0.0 : jac_foc(o.J, R, j) * mK;
        } else if (j < OZ) {
            u = jac_tau(o.J, R, j - OT) * mP;
        } else if (R == 2) {
            const int c = j - OZ;
            if (zon && c < C && !(c == 0 && z0off)) u = o.J.zscale * (double)dep(c);
        }
        sink(j, u * o.sW[R]);
    }
}

// All three weighted camera rows; sink(r, j, value).
template <int HK, int HP, class JcSink>
__device__ __forceinline__ void emit_jc(const ObsCore& o, const LinLayout& lay, bool enK, bool enP, bool enZ,
                                        bool first_obs, const DepSrc& dep, JcSink&& sink) {
    emit_jc_row<HK, HP, 0>(o, lay, enK, enP, enZ, first_obs, dep, [&](int j, double v) { sink(0, j, v); });
    emit_jc_row<HK, HP, 1>(o, lay, enK, enP, enZ, first_obs, dep, [&](int j, double v) { sink(1, j, v); });
    emit_jc_row<HK, HP, 2>(o, lay, enK, enP, enZ, first_obs, dep, [&](int j, double v) { sink(2, j, v); });
}

// Weighted point row R of Jp.
template <int R>
__device__ __forceinline__ void point_row(const ObsCore& o, const CamF& cp, bool xon, double Jp[3]) {
#pragma unroll
    for (int k = 0; k < 3; ++k) Jp[k] = (xon ? jac_pts(o.J, cp, R, k) : 0.0) * o.sW[R];
}

// Weighted point rows Jp (3x3) and, when asked, the point gradient J_p^T (W r) (unweighted rows).
template <bool GRAD_P>
__device__ __forceinline__ void point_rows(const ObsCore& o, const CamF& cp, bool xon, double Jp[3][3],
                                           double gP[3]) {
    double jp[3][3];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) jp[r][k] = xon ? jac_pts(o.J, cp, r, k) : 0.0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (GRAD_P) gP[k] = jp[0][k] * o.Wr[0] + jp[1][k] * o.Wr[1] + jp[2][k] * o.Wr[2];
        Jp[0][k] = jp[0][k] * o.sW[0];
        Jp[1][k] = jp[1][k] * o.sW[1];
        Jp[2][k] = jp[2][k] * o.sW[2];
    }
}

// Damped point block -> Cholesky factor with the chol3x3_solve rules (.cu:560-634):
// + jitter on the diagonal, averaged off-diagonals, non-positive pivots + jitter; in the working
// precision R (the reference's fp32 solver factors its fp32 blocks in fp32).
template <typename R>
__device__ __forceinline__ void chol3_factor(const R H[6], R lam, R L[6]) {
    const R jit = R(1e-12);
    R a00 = (H[0] + lam) + jit, a11 = (H[3] + lam) + jit, a22 = (H[5] + lam) + jit;
    R a01 = H[1], a02 = H[2], a12 = H[4];
    a00 = a00 > R(0) ? a00 : a00 + jit;
    R l00 = sqrt(a00);
    R l10 = a01 / l00, l20 = a02 / l00;
    R t11 = a11 - l10 * l10;
    t11 = t11 > R(0) ? t11 : t11 + jit;
    R l11 = sqrt(t11);
    R l21 = (a12 - l10 * l20) / l11;
    R t22 = a22 - l20 * l20 - l21 * l21;
    t22 = t22 > R(0) ? t22 : t22 + jit;
    R l22 = sqrt(t22);
    L[0] = l00; L[1] = l10; L[2] = l20; L[3] = l11; L[4] = l21; L[5] = l22;
}

template <typename R>
__device__ __forceinline__ void chol3_fwd(const R L[6], const R b[3], R y[3]) {
    y[0] = b[0] / L[0];
    y[1] = (b[1] - L[1] * y[0]) / L[3];
    y[2] = (b[2] - L[2] * y[0] - L[4] * y[1]) / L[5];
}

template <typename R>
__device__ __forceinline__ void chol3_bwd(const R L[6], const R z[3], R x[3]) {
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

// Core of the observation in plan slot `slot`, every input gathered from memory.
__device__ __forceinline__ void obs_core_slot(const LinArgs& a, int64_t slot, int obs, const ObsCtx& c, int pid,
                                              const DepSrc& dep, ObsCore& o) {
    float X[3] = {a.pts3d[3 * (int64_t)pid], a.pts3d[3 * (int64_t)pid + 1], a.pts3d[3 * (int64_t)pid + 2]};
    float2 uv = reinterpret_cast<const float2*>(a.s_pix)[slot];
    float2 sv = reinterpret_cast<const float2*>(a.s_std)[slot];
    GivenRW grw = {{0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}};
    if (a.r_in) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            grw.r[k] = a.r_in[(int64_t)obs * a.r_s0 + k * a.r_s1];
            grw.w[k] = a.w_in[(int64_t)obs * a.w_s0 + k * a.w_s1];
        }
    }
    obs_core(c.cp, c.zc, X, uv, sv, dep, a.hp, a.lay, a.r_in != nullptr, grw, o);
}

// ----------------------------------------------------------------------------- point blocks
// One chunk per block.  Linearises every observation (residual, weights, Jacobian) once per LM
// iteration and writes its linearisation record; writes, per chunk track (index first_ct + t),
// H_pp upper, g_p, the point with its enable flag, and the chunk's largest point-block diagonal
// (for the damping value).
template <int HK, int HP, typename Real>
__global__ void __launch_bounds__(BA_CHUNK, 5) k_track_pp(LinArgs a) {   // 5 waves per SIMD: 96 VGPRs, no spills
    __shared__ Real sh[BA_CHUNK][9];
    __shared__ Real smax[BA_CHUNK];
    const int chunk = blockIdx.x, tid = threadIdx.x;
    const int64_t slot = (int64_t)chunk * BA_CHUNK + tid;
    // Everything that depends only on the slot or the chunk is requested at once (an empty slot
    // holds gather index 0 in the slot arrays, so every lane's reads are valid), then what those
    // give: the image's camera and pose, the point; then the chunk track of this lane.
    const int obs = a.chunk_obs[slot];
    const int img = a.s_img[slot], pid = a.s_pid[slot];
    const float2 uv = reinterpret_cast<const float2*>(a.s_pix)[slot];
    const float2 sv = reinterpret_cast<const float2*>(a.s_std)[slot];
    DepSrc dep;
    load_dep(dep, a.s_dep + slot * a.lay.C, a.lay.C);
    const int first_ct = a.chunk_meta[4 * chunk + 1], n_ct = a.chunk_meta[4 * chunk + 2];
    int64_t ct = first_ct + (tid < n_ct ? tid : 0);
    ct = ct < a.n_ctracks ? ct : a.n_ctracks - 1;
    const int ct_f = a.ct_first[ct], ct_m = a.ct_m[ct], ct_pid = a.ct_pid[ct];
    const float X[3] = {a.pts3d[3 * (int64_t)pid], a.pts3d[3 * (int64_t)pid + 1], a.pts3d[3 * (int64_t)pid + 2]};
    Real c[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) c[k] = Real(0);
    if (obs >= 0) {
        ObsCtx ctx;
        load_obs_ctx(a, img, ctx);
        GivenRW grw = {{0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}};
        if (a.r_in) {
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                grw.r[k] = a.r_in[(int64_t)obs * a.r_s0 + k * a.r_s1];
                grw.w[k] = a.w_in[(int64_t)obs * a.w_s0 + k * a.w_s1];
            }
        }
        ObsCore o;
        float Xo[3] = {X[0], X[1], X[2]};
        obs_core(ctx.cp, ctx.zc, Xo, uv, sv, dep, a.hp, a.lay, a.r_in != nullptr, grw, o);
        typedef CoreRec<Real> CR;
        core_store(reinterpret_cast<typename CR::T*>(a.core) + (int64_t)chunk * CR::NF * BA_CHUNK, tid, o);
        const bool xon = (a.enX ? a.enX[pid] != 0 : true) && !a.lay.x_off;
        double Jp[3][3], gP[3];
        point_rows<true>(o, ctx.cp, xon, Jp, gP);
        // J_pts gram (ba_solver.py:911-924) and J_pts^T W r
        const int pr[6][2] = {{0, 0}, {0, 1}, {0, 2}, {1, 1}, {1, 2}, {2, 2}};
#pragma unroll
        for (int q = 0; q < 6; ++q) {
            int i = pr[q][0], j = pr[q][1];
            c[q] = (Real)(Jp[0][i] * Jp[0][j] + Jp[1][i] * Jp[1][j] + Jp[2][i] * Jp[2][j]);
        }
        c[6] = (Real)gP[0]; c[7] = (Real)gP[1]; c[8] = (Real)gP[2];
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) sh[tid][k] = c[k];
    const float* Xc = a.pts3d + 3 * (int64_t)ct_pid;
    const float4 cpt = make_float4(Xc[0], Xc[1], Xc[2], (a.enX ? a.enX[ct_pid] != 0 : true) ? 1.f : 0.f);
    __syncthreads();
    Real mx = Real(0);
    if (tid < n_ct) {
        const int f = ct_f, m = ct_m;
        Real s[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) s[k] = Real(0);
        for (int q = 0; q < m; ++q)
#pragma unroll
            for (int k = 0; k < 9; ++k) s[k] += sh[f + q][k];
#pragma unroll
        for (int k = 0; k < 6; ++k) ((Real*)a.Hpp)[6 * ct + k] = s[k];
#pragma unroll
        for (int k = 0; k < 3; ++k) ((Real*)a.gp)[3 * ct + k] = s[6 + k];
        reinterpret_cast<float4*>(a.ct_pt)[ct] = cpt;
        mx = fmax(fmax(fabs(s[0]), fabs(s[3])), fabs(s[5]));
    }
    smax[tid] = mx;
    __syncthreads();
    for (int w = BA_CHUNK / 2; w > 0; w >>= 1) {
        if (tid < w) smax[tid] = fmax(smax[tid], smax[tid + w]);
        __syncthreads();
    }
    if (tid == 0) ((Real*)a.chunk_max)[chunk] = smax[0];
}

// lam_p = dampen * max diag over all tracks (BlockDiagMat.dampen_, ba_solver.py:575-582).
// The maximum of non-negative floating-point values is the maximum of their bit patterns, so blocks
// combine with an integer atomic max into word n of cmax (cleared by k_lam_clear); the result is
// order-free.
template <typename R>
__global__ void k_lam_clear(R* __restrict__ cmax, int64_t n) { cmax[n] = R(0); }

template <typename R>
__global__ void __launch_bounds__(256) k_lam_reduce(R* __restrict__ cmax, int64_t n) {
    __shared__ R s[256];
    R m = R(0);
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) m = fmax(m, cmax[i]);
    s[threadIdx.x] = m;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) s[threadIdx.x] = fmax(s[threadIdx.x], s[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) atomic_max_nonneg(cmax + n, s[0]);
}

template <typename R>
__global__ void k_lam_final(const R* __restrict__ cmax, int64_t n, double dampen, int adaptive, int x_off,
                            R* __restrict__ out) {
    out[0] = (adaptive && !x_off) ? R(dampen) * cmax[n] : R(dampen);
}

// Point factors of every chunk track once the damping value is known: L = chol(H_pp + lam_p I) with
// the chol3x3_solve rules, w = L^-1 g_p and the reciprocal pivots, 12 values per chunk track
// (L0..L5 | w0 w1 w2 | 1/L0 1/L3 1/L5), read by the camera-pair kernel two values per copy; in the
// working precision R.
template <typename R>
__global__ void __launch_bounds__(256) k_point_factor(const R* __restrict__ Hpp, const R* __restrict__ gp,
                                                      const R* __restrict__ lam_p, int64_t n_ct, R* __restrict__ pf) {
    typedef R R2 __attribute__((ext_vector_type(2)));
    __shared__ R2 rec[256 * 7];                        // the block's records, 6 vectors each (+1: row stride)
    const int64_t ct0 = (int64_t)blockIdx.x * 256, ct = ct0 + threadIdx.x;
    const int nt = (int)min((int64_t)256, n_ct - ct0);
    if (ct < n_ct) {
        R H[6], Lf[6];
        const R2* h2 = reinterpret_cast<const R2*>(Hpp + 6 * ct);            // 16-byte aligned rows (fp64)
#pragma unroll
        for (int k = 0; k < 3; ++k) { const R2 v = h2[k]; H[2 * k] = v.x; H[2 * k + 1] = v.y; }
        chol3_factor(H, lam_p[0], Lf);
        const R r0 = R(1) / Lf[0], r1 = R(1) / Lf[3], r2 = R(1) / Lf[5];
        const R g0 = gp[3 * ct], g1 = gp[3 * ct + 1], g2 = gp[3 * ct + 2];
        const R w0 = g0 * r0;
        const R w1 = (g1 - Lf[1] * w0) * r1;
        const R w2 = (g2 - Lf[2] * w0 - Lf[4] * w1) * r2;
        R2* o = rec + threadIdx.x * 7;
        o[0] = (R2){Lf[0], Lf[1]}; o[1] = (R2){Lf[2], Lf[3]}; o[2] = (R2){Lf[4], Lf[5]};
        o[3] = (R2){w0, w1}; o[4] = (R2){w2, r0}; o[5] = (R2){r1, r2};
    }
    __syncthreads();
    // the block's records leave as one contiguous range, 16 bytes per lane and store
    R2* dst = reinterpret_cast<R2*>(pf + 12 * ct0);
    for (int e = threadIdx.x; e < nt * 6; e += 256) dst[e] = rec[(e / 6) * 7 + e % 6];
}

// ----------------------------------------------------------------------------- camera-pair blocks
//
// k_schur: one workgroup (16 waves, four per SIMD) per CU, taking batches from a work queue.  Per
// chunk of 128 observation slots:
//   A1  waves 0-5, lane per (slot, row r): row r of the weighted camera rows J_c from the slot's
//       linearisation record (rows 3-5 of the slot's LDS block, column 15 = W r / sqrt(W)) and row
//       r of the point rows J_p, except the z-coefficient columns of row 2 (the depth row), which
//       waves 6-7 form, lane per slot (waves w and w + 4 share a SIMD: this spreads phase A evenly
//       over the four).  The point blocks' Cholesky factors come precomputed (k_point_factor).
//   A2  waves 0-11, lane per (slot, column c, half h): column c of V = J_c^T J_p L^-T at the image-level
//       columns [8h, 8h + 8) (row c of the block, column 15 = w for the first observation of the track
//       in the image, else 0); several
//       observations of one track in one image are then summed into the first one.
//   B   every wave, for each camera-pair slot it owns (accumulator in registers), over the slot's
//       entry list (built by the planner once per structure):
//         off-diagonal (a,b):  acc += V_ta^T V_tb        per covering track t
//         diagonal (a,a):      acc += V_ta^T V_ta        per covering track
//                              acc -= J_o^T J_o          per observation o in image a
//       The entries of a slot are taken four at a time along the MFMA's K dimension: lane group k
//       of a 16x16x4 MFMA reads row c of entry k's blocks, and one MFMA per row c = 0..2
//       sums c over four entries.  The partial block is -acc; column 15 of a diagonal tile then
//       holds sum J_c^T W r - V w = the image's rhs term, and diag(J_c^T J_c) is summed from the
//       squared B operands of the J entries.
// The next chunk's inputs (its linearisation records, slot streams, the chunk-track state written by
// k_track_pp, its entry list) are copied into LDS while the current chunk's MFMAs run.  Four waves
// per SIMD keep four independent accumulation chains in flight on each MFMA pipe.

__device__ __forceinline__ uint64_t uni64(uint64_t x) {
    uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// The next chunk's inputs are copied straight into LDS staging arrays while the current chunk's
// MFMAs run (global_load_lds: lane l of the issuing wave writes dst + 4 l or dst + 16 l; dst is
// uniform),
// so no registers hold them across the MFMA phase.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glob_void;
__device__ __forceinline__ void dma4_to_lds(const void* src, void* wave_dst) {
    __builtin_amdgcn_global_load_lds((glob_void*)src, (lds_void*)wave_dst, 4, 0, 0);
}
__device__ __forceinline__ void dma16_to_lds(const void* src, void* wave_dst) {
    __builtin_amdgcn_global_load_lds((glob_void*)src, (lds_void*)wave_dst, 16, 0, 0);
}

// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// LDS reads of the MFMA phase, issued from inline asm.  The next chunk's inputs are being copied
// into LDS (global_load_lds) while the MFMA phase runs, and the compiler cannot tell that these
// reads touch other arrays, so a read it issued itself would first wait for the whole copy
// (vmcnt 0).  lds_rd* issue reads the compiler does not wait for; lds_wait waits for every
// outstanding LDS read (lgkmcnt 0, so the count never depends on what else is in flight) and
// passes the values through, so nothing can read (or copy) a destination register before its data
// has arrived.  The "; ba_pf" / "; ba_pw" tags let the code-generation test check exactly that in
// the compiled kernel.
__device__ __forceinline__ uint32_t lds_rd_u32(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1 ; ba_pf" : "=v"(v) : "v"(addr));
    return v;
}
__device__ __forceinline__ void lds_rd3(uint32_t addr, double (&v)[3]) {
    asm volatile("ds_read_b64 %0, %1 ; ba_pf" : "=v"(v[0]) : "v"(addr));
    asm volatile("ds_read_b64 %0, %1 offset:128 ; ba_pf" : "=v"(v[1]) : "v"(addr));
    asm volatile("ds_read_b64 %0, %1 offset:256 ; ba_pf" : "=v"(v[2]) : "v"(addr));
}
// fp32 blocks: rows 16 floats (64 bytes) apart
__device__ __forceinline__ void lds_rd3(uint32_t addr, float (&v)[3]) {
    asm volatile("ds_read_b32 %0, %1 ; ba_pf" : "=v"(v[0]) : "v"(addr));
    asm volatile("ds_read_b32 %0, %1 offset:64 ; ba_pf" : "=v"(v[1]) : "v"(addr));
    asm volatile("ds_read_b32 %0, %1 offset:128 ; ba_pf" : "=v"(v[2]) : "v"(addr));
}
__device__ __forceinline__ void lds_wait(uint32_t& a) {
    asm volatile("s_waitcnt lgkmcnt(0) ; ba_pw" : "+v"(a));
}
template <typename Real>
__device__ __forceinline__ void lds_wait(Real (&A)[3], uint32_t& d) {
    asm volatile("s_waitcnt lgkmcnt(0) ; ba_pw" : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(d));
}
template <typename Real>
__device__ __forceinline__ void lds_wait(Real (&A)[3], Real (&B)[3], uint32_t& d) {
    asm volatile("s_waitcnt lgkmcnt(0) ; ba_pw"
                 : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(B[0]), "+v"(B[1]), "+v"(B[2]), "+v"(d));
}
// LDS atomic add (no return) at a byte address, also outside the compiler's view of LDS.
__device__ __forceinline__ void lds_add(uint32_t addr, double v) {
    asm volatile("ds_add_f64 %0, %1 ; ba_pa" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_add(uint32_t addr, float v) {
    asm volatile("ds_add_f32 %0, %1 ; ba_pa" : : "v"(addr), "v"(v) : "memory");
}

// The camera-pair tiles in the working precision: a 16 x 16 x 4 MFMA, the J groups with A negated
// (fp64: the MFMA's neg modifier; fp32: the operand's sign, an exact flip), and the accumulator
// layout (lane l, element v holds D[row(l, v)][l % 16]).
template <typename Real> struct SchurMfma;
template <>
struct SchurMfma<double> {
    typedef dbl4 V4;
    static __device__ __forceinline__ V4 mac(double a, double b, V4 c) {
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ V4 mac_neg(double a, V4 c) {
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, a, c, 0, 0, 1);      // neg:[1,0,0]
    }
    static __device__ __forceinline__ int row(int lane, int v) { return 4 * v + (lane >> 4); }
};
template <>
struct SchurMfma<float> {
    typedef flt4 V4;
    static __device__ __forceinline__ V4 mac(float a, float b, V4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ V4 mac_neg(float a, V4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(-a, a, c, 0, 0, 0);
    }
    static __device__ __forceinline__ int row(int lane, int v) { return 4 * (lane >> 4) + v; }
};

// One chunk's inputs, laid out as the copies write them.  The point factors of a chunk track (12 values
// in the working precision) arrive in 16-byte copies: element i of track ct at pf[i / PF][ct][i % PF].
template <typename Real>
struct Staging {
    static constexpr int PF = 16 / sizeof(Real);            // values per 16-byte copy
    typename CoreRec<Real>::T rec[CoreRec<Real>::NF * BA_CHUNK];   // the chunk's linearisation records (field-major,
                                                                    // as in memory)
    int info[BA_CHUNK];                     // slot_info per slot
    int obs[BA_CHUNK];                      // chunk_obs per slot
    float dep[BA_PRE_C][BA_CHUNK];          // depth guidance channels c < min(C, BA_PRE_C)
    Real pf[12 / PF][BA_MAX_CT][PF];        // point factors of each chunk track (L | w | 1/pivots)
    float4 X[BA_MAX_CT];                    // point, enable flag
    __device__ __forceinline__ Real f(int i, int ct) const { return pf[i / PF][ct][i % PF]; }
};

// waves 0-1: the slots of chunk ck; wave 2: its chunk tracks (first_ct ..), n_ct; wave 3: its entry list
template <typename Real>
__device__ __forceinline__ void stage_chunk(const LinArgs& a, Staging<Real>& S, int* sNct,
                                            uint32_t (*lists)[BA_LIST_CAP], int (*tabs)[BA_MAX_SLOTS], int ck,
                                            int first_ct, int C, int wave, int lane) {
    constexpr int PF = Staging<Real>::PF;
    if (wave < 2) {
        const int w = __builtin_amdgcn_readfirstlane(wave);
        const int64_t slot = (int64_t)ck * BA_CHUNK + 64 * w + lane;
        // the record block, 16 bytes per lane per copy (2 KB per copy of the two waves)
        if constexpr (sizeof(Real) == 8) {
            const double* rec = a.core + (int64_t)ck * BA_CORE * BA_CHUNK;
#pragma unroll
            for (int i = 0; i < BA_CORE * BA_CHUNK / 256; ++i)
                dma16_to_lds(rec + 256 * i + 128 * w + 2 * lane, S.rec + 256 * i + 128 * w);
        } else {
            constexpr int RB = (int)sizeof(S.rec);
            static_assert(RB % 2048 == 0, "a chunk's record block is a whole number of 2 KB copies");
            const char* rec = reinterpret_cast<const char*>(a.core) + (int64_t)ck * RB;
            char* dst = reinterpret_cast<char*>(S.rec);
#pragma unroll
            for (int i = 0; i < RB / 2048; ++i)
                dma16_to_lds(rec + 2048 * i + 1024 * w + 16 * lane, dst + 2048 * i + 1024 * w);
        }
        dma4_to_lds(a.slot_info + slot, S.info + 64 * w);
        dma4_to_lds(a.chunk_obs + slot, S.obs + 64 * w);
#pragma unroll
        for (int c = 0; c < BA_PRE_C; ++c)
            if (c < C) dma4_to_lds(a.s_dep + slot * C + c, &S.dep[c][64 * w]);
    } else if (wave == 2) {
        int64_t ct = (int64_t)first_ct + lane;
        ct = ct < a.n_ctracks ? ct : a.n_ctracks - 1;
        const Real* pfac = (const Real*)a.pfac;
#pragma unroll
        for (int k = 0; k < 12 / PF; ++k) dma16_to_lds(pfac + 12 * ct + PF * k, &S.pf[k][0][0]);
        dma16_to_lds(a.ct_pt + 4 * ct, S.X);
        if (lane == 0) *sNct = a.chunk_meta[4 * ck + 2];
    } else if (wave == 3) {
        // the chunk's MFMA entry list, in whole 1 KB pieces (the plan pads its array for a copy of
        // full capacity), and its slot table, into buffer ck & 1
        const int ep0 = a.chunk_eptr[ck], ep1 = a.chunk_eptr[ck + 1];
        const char* src = reinterpret_cast<const char*>(a.chunk_ent) + (int64_t)ep0 * 16;
        char* dst = reinterpret_cast<char*>(lists[ck & 1]);
        const int nbytes = __builtin_amdgcn_readfirstlane((ep1 - ep0) * 16);
#pragma unroll
        for (int i = 0; i < BA_LIST_CAP * 4 / 1024; ++i)
            if (1024 * i < nbytes) dma16_to_lds(src + 1024 * i + 16 * lane, dst + 1024 * i);
        if (lane < BA_MAX_SLOTS / 4)
            dma16_to_lds(a.chunk_slots + (int64_t)ck * BA_MAX_SLOTS + 4 * lane, tabs[ck & 1]);
    }
}

template <int HK, int HP, typename Real>
__global__ void __launch_bounds__(BA_WAVES * 64) k_schur(LinArgs a) {
    typedef SchurMfma<Real> M;
    typedef typename M::V4 V4;
    extern __shared__ __align__(16) char sBlkRaw[];     // [BA_CHUNK][BA_BLK] observation blocks + zero block
    Real* const sBlk = reinterpret_cast<Real*>(sBlkRaw);
    __shared__ Staging<Real> sSt;                        // this chunk's inputs (the next chunk's, in phase B)
    __shared__ Real sJp[BA_CHUNK][9];                    // weighted point rows J_p of each slot
    __shared__ Real sDv[BA_MAX_LOCAL][16];               // per local image: diag(J_c^T J_c)
    __shared__ int sInfo[BA_CHUNK];
    __shared__ CamF sCam[BA_MAX_LOCAL];
    __shared__ unsigned char sEn[BA_MAX_LOCAL * 3];
    __shared__ int sPair[BA_MAX_SLOTS];                  // per kernel place: the slot's pair, -1 if none
    __shared__ int sQ[BA_MAX_SLOTS];                     // per kernel place: the batch slot
    __shared__ uint32_t sList[2][BA_LIST_CAP];           // MFMA entry lists (chunk ck in buffer ck & 1)
    __shared__ int sSlotTab[2][BA_MAX_SLOTS];            // per slot: entry offset | padded count << 16
    __shared__ int sDup[2];
    __shared__ int sNct;
    __shared__ int sNext;

    const int d = a.lay.d, C = a.lay.C;
    static_assert(BA_WAVES >= 8, "phase A needs eight waves");

    // Work queue: with a counter, each workgroup (one per CU) takes the next batch of the dispatch
    // order until none is left, so a CU that finishes early starts the next batch at once (the
    // hardware dispatcher hands each XCD its workgroups in launch order, and one long batch
    // then holds back every later workgroup of its XCD).  Without one, workgroup b takes batch b.
    for (int bq = blockIdx.x;;) {
    // the lane indices are re-derived for every batch (through an opaque copy of the thread id), so
    // that nothing computed from them is hoisted out of this loop and kept live across the inner ones
    int tid_ = threadIdx.x;
    asm volatile("" : "+v"(tid_));
    const int tid = tid_, wave = tid >> 6, lane = tid & 63;
    // phase A roles: waves 0-5 take one (slot, row) each (slot tid % 128, row tid / 128), waves 6-7
    // the z-coefficient columns of row 2 (rr = 3)
    const bool row_lane = tid < 4 * BA_CHUNK;
    const int t = tid & (BA_CHUNK - 1), rr = tid >> 7;
    if (a.work_ctr != nullptr) {
        if (tid == 0) sNext = atomicAdd(a.work_ctr, 1);
        __syncthreads();
        bq = sNext;
    }
    if (bq >= a.n_batches) break;
    const int batch = a.b_order != nullptr ? a.b_order[bq] : bq;             // most expensive first
    const int nimg = a.b_nimgs[batch];
    const int s0 = a.b_slot_ptr[batch], ns = a.b_slot_ptr[batch + 1] - s0;
    const int c_begin = a.b_chunk_ptr[batch], c_end = a.b_chunk_ptr[batch + 1];
    int first_ct = a.chunk_meta[4 * c_begin + 1];

    {
        stage_chunk(a, sSt, &sNct, sList, sSlotTab, c_begin, first_ct, C, wave, lane);
        // local image parameters
        if (tid < nimg) {
            int img = a.b_imgs[(int64_t)batch * a.L + tid];
            int node = a.infos[a.n_imgs + img], cam = a.infos[2 * a.n_imgs + img];
            load_cam(sCam[tid], a.K, a.P_rig2cam, a.P_rig2cam_stride, a.P_w2rig, cam, node);
            sEn[3 * tid + 0] = a.enK ? a.enK[cam] : 1;
            sEn[3 * tid + 1] = a.enP ? a.enP[node] : 1;
            sEn[3 * tid + 2] = a.enZ ? a.enZ[img] : 1;
        }
        // kernel place p = wave + BA_WAVES * k holds batch slot sQ[p] with pair (a | b << 8), or -1
        for (int p = tid; p < BA_MAX_SLOTS; p += BA_WAVES * 64) {
            const int q = a.b_pos_slot[(int64_t)batch * BA_MAX_SLOTS + p];
            sQ[p] = q;
            sPair[p] = q >= 0 && q < ns ? a.slot_pair[s0 + q] : -1;
        }
        for (int q = tid; q < BA_MAX_LOCAL * 16; q += BA_WAVES * 64) sDv[q >> 4][q & 15] = Real(0);
        for (int q = tid; q < 48; q += BA_WAVES * 64) sBlk[BA_ZERO + q] = Real(0);
    }
    __syncthreads();

    V4 acc[BA_SLOTS_PER_WAVE];
    int my_pq[BA_SLOTS_PER_WAVE], my_q[BA_SLOTS_PER_WAVE];       // this wave's slots: pair, batch slot
#pragma unroll
    for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
        acc[q] = V4{Real(0), Real(0), Real(0), Real(0)};
        my_pq[q] = __builtin_amdgcn_readfirstlane(sPair[wave + BA_WAVES * q]);
        my_q[q] = __builtin_amdgcn_readfirstlane(sQ[wave + BA_WAVES * q]);
    }
    // MFMA operand element of this lane: K index lane/16 (the entry), column lane%16
    const int kq = lane >> 4, l15 = lane & 15;

    for (int ck = c_begin; ck < c_end; ++ck) {
        if (ck != c_begin) __syncthreads();    // previous chunk consumed; this chunk's inputs staged
        const int n_ct = sNct;

        // ---------------- A1
        const int info = row_lane ? sSt.info[t] : -1;
        const bool valid = info >= 0;
        const int li = info & 0xff, ct = (info >> 8) & 0xff, leader = info >> 16;
        if (row_lane) {
            if (rr == 0) sInfo[t] = info;
            if (valid && rr == 3) {                        // row 2's z-coefficient columns: zscale, sqrt(W_2)
                ObsCore o;
                o.J.zscale = sSt.rec[14 * BA_CHUNK + t];
                if constexpr (sizeof(Real) == 8)
                    o.sW[2] = reinterpret_cast<const float2*>(sSt.rec)[19 * BA_CHUNK + t].y;
                else
                    o.sW[2] = sSt.rec[21 * BA_CHUNK + t];
                const bool eZ = sEn[3 * li + 2] != 0, first = sSt.obs[t] == 0;
                Real* blk2 = sBlk + t * BA_BLK + BA_JROW + 32;
                auto sink2 = [&](int j, double v) { if (j < 15) blk2[j] = j < d ? (Real)v : Real(0); };
                DepSrc dep;
#pragma unroll
                for (int c = 0; c < BA_PRE_C; ++c) dep.r[c] = c < C ? sSt.dep[c][t] : 0.f;
                dep.g = a.s_dep + ((int64_t)ck * BA_CHUNK + t) * C;
                emit_jc_row<HK, HP, 2, 2 * HK + 6 * HP, 15>(o, a.lay, true, true, eZ, first, dep, sink2);
            } else if (valid) {
                ObsCore o;
                core_load(sSt.rec, t, o);
                const bool eK = sEn[3 * li] != 0, eP = sEn[3 * li + 1] != 0, eZ = sEn[3 * li + 2] != 0;
                const bool first = sSt.obs[t] == 0, xon = sSt.X[ct].w != 0.f && !a.lay.x_off;
                Real* blk = sBlk + t * BA_BLK + BA_JROW + 16 * rr;
                auto sink = [&](int j, double v) { if (j < 15) blk[j] = j < d ? (Real)v : Real(0); };
                double jp[3];
                DepSrc dep;
                if (rr == 0) {
                    emit_jc_row<HK, HP, 0>(o, a.lay, eK, eP, eZ, first, dep, sink);
                    blk[15] = (Real)o.Rs[0];
                    point_row<0>(o, sCam[li], xon, jp);
                } else if (rr == 1) {
                    emit_jc_row<HK, HP, 1>(o, a.lay, eK, eP, eZ, first, dep, sink);
                    blk[15] = (Real)o.Rs[1];
                    point_row<1>(o, sCam[li], xon, jp);
                } else {
                    emit_jc_row<HK, HP, 2, 0, 2 * HK + 6 * HP>(o, a.lay, eK, eP, eZ, first, dep, sink);
                    blk[15] = (Real)o.Rs[2];
                    point_row<2>(o, sCam[li], xon, jp);
                }
#pragma unroll
                for (int k = 0; k < 3; ++k) sJp[t][3 * rr + k] = (Real)jp[k];
            }
            if (rr == 0) {
                const uint64_t dup = __ballot(valid && leader != t);
                if (lane == 0) sDup[wave] = dup != 0;
            }
        }
        __syncthreads();

        // ---------------- A2: V = J_c^T P with P = J_p L^-T; waves 0-11, lane (slot t, task q = tid / 128)
        // forms column c = q % 3 of V at the image-level columns [8h, 8h + 8), h = q / 3 (h = 1 also
        // writes column 15, the rhs term); the slot's status comes from sInfo (written in A1)
        if (tid < 6 * BA_CHUNK) {
            const int info2 = sInfo[t];
            if (info2 >= 0) {
                const int q = tid >> 7, c = q % 3, h = q / 3;
                const int ct2 = (info2 >> 8) & 0xff, leader2 = info2 >> 16;
                // the chunk track's factor: L (0-5), w = L^-1 g_p (6-8), reciprocal pivots (9-11)
                const Real l10 = sSt.f(1, ct2), l20 = sSt.f(2, ct2), l21 = sSt.f(4, ct2);
                const Real r0 = sSt.f(9, ct2), r1 = sSt.f(10, ct2), r2 = sSt.f(11, ct2);
                Real Pc[3];
#pragma unroll
                for (int r = 0; r < 3; ++r) {
                    const Real p0 = sJp[t][3 * r] * r0;
                    const Real p1 = (sJp[t][3 * r + 1] - l10 * p0) * r1;
                    const Real p2 = (sJp[t][3 * r + 2] - l20 * p0 - l21 * p1) * r2;
                    Pc[r] = c == 0 ? p0 : (c == 1 ? p1 : p2);
                }
                Real* blk = sBlk + t * BA_BLK;
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int j = 8 * h + jj;
                    if (j < 15) {
                        const Real j0 = blk[BA_JROW + j], j1 = blk[BA_JROW + 16 + j], j2 = blk[BA_JROW + 32 + j];
                        blk[16 * c + j] = j < d ? j0 * Pc[0] + j1 * Pc[1] + j2 * Pc[2] : Real(0);
                    }
                }
                if (h == 1) {
                    const Real wc = c == 0 ? sSt.f(6, ct2) : (c == 1 ? sSt.f(7, ct2) : sSt.f(8, ct2));
                    blk[16 * c + 15] = leader2 == t ? wc : Real(0);
                }
            }
        }
        __syncthreads();
        if (sDup[0] | sDup[1]) {
            // several observations of one track in one image: V of the run is summed into its first slot
            if (row_lane && rr < 3 && valid && leader == t) {   // lane (slot, rr): V row rr
                Real* dst = sBlk + t * BA_BLK + 16 * rr;
                for (int f = t + 1; f < BA_CHUNK; ++f) {
                    const int fi = sInfo[f];
                    if (fi < 0 || (fi >> 16) != t) break;
                    const Real* src = sBlk + f * BA_BLK + 16 * rr;
#pragma unroll
                    for (int j = 0; j < 15; ++j) dst[j] += src[j];
                }
            }
            __syncthreads();
        }

        // next chunk's inputs: copied into the staging arrays while the MFMAs run (this chunk's A1,
        // the only reader of the staging arrays, is past)
        if (ck + 1 < c_end) {
            first_ct += n_ct;
            stage_chunk(a, sSt, &sNct, sList, sSlotTab, ck + 1, first_ct, C, wave, lane);
        }

        // ---------------- B: camera-pair tiles
        // one group of four entries: lane group kq reads row c of its entry's A and B rows (the
        // entry holds their LDS offsets), then one MFMA per row c; the next group's entry is read
        // with this group's operands.  A diagonal slot starts with its J groups (A = B = the J rows
        // of one observation each, A negated by the MFMA's modifier, and their squares summed into
        // diag(J_c^T J_c)), then its V groups.  Every LDS read here goes through lds_rd* (above).
        constexpr uint32_t RB = sizeof(Real);            // bytes per value
        const uint32_t lane_base = lds_addr(sBlk) + RB * (uint32_t)l15;
        auto run_v = [&](uint32_t Lb, int g0, int g1, V4 acc_l) -> V4 {
            if (g0 >= g1) return acc_l;
            uint32_t e = lds_rd_u32(Lb + 16u * (uint32_t)g0);
            lds_wait(e);
            for (int g = g0; g < g1; ++g) {
                Real A[3], B[3];
                lds_rd3(lane_base + RB * (e & 0xffffu), A);
                lds_rd3(lane_base + RB * (e >> 16), B);
                uint32_t en = lds_rd_u32(Lb + 16u * (uint32_t)min(g + 1, g1 - 1));
                lds_wait(A, B, en);
#pragma unroll
                for (int c = 0; c < 3; ++c) acc_l = M::mac(A[c], B[c], acc_l);
                e = en;
            }
            return acc_l;
        };
        // the V groups of a diagonal slot: each entry's A and B rows are the same rows (one run with
        // itself), read once
        auto run_vd = [&](uint32_t Lb, int g0, int g1, V4 acc_l) -> V4 {
            if (g0 >= g1) return acc_l;
            uint32_t e = lds_rd_u32(Lb + 16u * (uint32_t)g0);
            lds_wait(e);
            for (int g = g0; g < g1; ++g) {
                Real A[3];
                lds_rd3(lane_base + RB * (e & 0xffffu), A);
                uint32_t en = lds_rd_u32(Lb + 16u * (uint32_t)min(g + 1, g1 - 1));
                lds_wait(A, en);
#pragma unroll
                for (int c = 0; c < 3; ++c) acc_l = M::mac(A[c], A[c], acc_l);
                e = en;
            }
            return acc_l;
        };
        auto run_j = [&](uint32_t Lb, int ng, V4 acc_l, Real& dsq) -> V4 {
            if (ng <= 0) return acc_l;
            uint32_t e = lds_rd_u32(Lb);
            lds_wait(e);
            for (int g = 0; g < ng; ++g) {
                Real A[3];
                lds_rd3(lane_base + RB * (e & 0xffffu), A);
                uint32_t en = lds_rd_u32(Lb + 16u * (uint32_t)min(g + 1, ng - 1));
                lds_wait(A, en);
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    dsq += A[c] * A[c];
                    acc_l = M::mac_neg(A[c], acc_l);
                }
                e = en;
            }
            return acc_l;
        };
        const uint32_t tab_base = lds_addr(sSlotTab[ck & 1]), list_base = lds_addr(sList[ck & 1]) + 4u * (uint32_t)kq;
#pragma unroll
        for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
            const int pq = my_pq[q];
            if (pq < 0) continue;
            const int la = pq & 0xff, lb = (pq >> 8) & 0xff;
            uint32_t tv = lds_rd_u32(tab_base + 4u * (uint32_t)my_q[q]);
            lds_wait(tv);
            const int tab = __builtin_amdgcn_readfirstlane((int)tv);
            const uint32_t Lb = list_base + 4u * (uint32_t)BA_TAB_OFF(tab);
            const int ng = BA_TAB_NG(tab);
            if (la != lb) {
                acc[q] = run_v(Lb, 0, ng, acc[q]);
            } else {
                const int njg = BA_TAB_NJG(tab);
                Real dsq = Real(0);
                acc[q] = run_j(Lb, njg, acc[q], dsq);
                acc[q] = run_vd(Lb, njg, ng, acc[q]);
                dsq += __shfl_xor(dsq, 16);
                dsq += __shfl_xor(dsq, 32);
                if (lane < 16) lds_add(lds_addr(&sDv[la][lane]), dsq);
            }
        }
    }

    // flush this batch's partial blocks (-acc, row-major d x d, local orientation); accumulator
    // layout: lane l, element v holds D[M::row(l, v)][l % 16]
    const int jc = lane & 15;
#pragma unroll
    for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
        const int pq = my_pq[q];
        if (pq >= 0) {
            const int sl = my_q[q];
            Real* P = (Real*)a.partials + (int64_t)(s0 + sl) * d * d;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = M::row(lane, v);
                if (i < d && jc < d) P[i * d + jc] = -acc[q][v];
            }
            const int la = pq & 0xff, lb = (pq >> 8) & 0xff;
            if (la == lb && jc == 15) {
                Real* o = (Real*)a.img_partials + ((int64_t)batch * a.L + la) * 2 * d;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int i = M::row(lane, v);
                    if (i < d) o[i] = -acc[q][v];
                }
            }
        }
    }
    __syncthreads();
    {
        const int va = tid >> 4, vj = tid & 15;
        if (va < nimg && vj < d) ((Real*)a.img_partials)[((int64_t)batch * a.L + va) * 2 * d + d + vj] = sDv[va][vj];
    }
    if (a.work_ctr == nullptr) break;
    __syncthreads();                     // this batch's LDS fully read before the next one is staged
    }
}

__global__ void k_ctr_clear(int* ctr) { *ctr = 0; }

// ----------------------------------------------------------------------------- reductions
template <typename Real>
__global__ void __launch_bounds__(256) k_pair_reduce(const int* __restrict__ pair_ptr, const int* __restrict__ pair_src,
                                                     const Real* __restrict__ partials, int64_t n_pairs, int d,
                                                     Real* __restrict__ out) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int dd = d * d;
    if (tid >= n_pairs * dd) return;
    int64_t p = tid / dd;
    int e = (int)(tid - p * dd);
    int i = e / d, j = e - (e / d) * d;
    Real acc = Real(0);
    for (int q = pair_ptr[p]; q < pair_ptr[p + 1]; ++q) {
        int src = pair_src[q];
        int64_t s = src >> 1;
        acc += partials[s * dd + ((src & 1) ? j * d + i : i * d + j)];
    }
    out[tid] = acc;
}

template <typename Real>
__global__ void __launch_bounds__(256) k_img_reduce(const int* __restrict__ img_ptr, const int* __restrict__ img_src,
                                                    const Real* __restrict__ ip, int n_imgs, int d,
                                                    Real* __restrict__ e_out, Real* __restrict__ dg_out) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= (int64_t)n_imgs * d) return;
    int i = (int)(tid / d), j = (int)(tid - (tid / d) * d);
    Real e = Real(0), g = Real(0);
    for (int q = img_ptr[i]; q < img_ptr[i + 1]; ++q) {
        const Real* s = ip + (int64_t)img_src[q] * 2 * d;
        e += s[j];
        g += s[d + j];
    }
    e_out[tid] = e;
    dg_out[tid] = g;
}

// ----------------------------------------------------------------------------- back-substitution
// In fp32 (Real = float) the weighted rows and point rows are rounded from the fp64 core and every
// product and sum after them is fp32, as on the pair-major path.
template <int HK, int HP, typename Real>
__global__ void __launch_bounds__(BA_CHUNK) k_backsub(LinArgs a) {
    __shared__ Real sh[BA_CHUNK][3];
    const int chunk = blockIdx.x, tid = threadIdx.x;
    const int64_t slot = (int64_t)chunk * BA_CHUNK + tid;
    // slot- and chunk-only inputs first (as in k_track_pp): the observation's slot data, and this
    // lane's chunk track with its point block and gradient
    const int obs = a.chunk_obs[slot];
    const int img = a.s_img[slot], pid = a.s_pid[slot];
    const int d = a.lay.d;
    DepSrc dep;
    load_dep(dep, a.s_dep + slot * a.lay.C, a.lay.C);
    const int first_ct = a.chunk_meta[4 * chunk + 1], n_ct = a.chunk_meta[4 * chunk + 2];
    int64_t ctk = first_ct + (tid < n_ct ? tid : 0);
    ctk = ctk < a.n_ctracks ? ctk : a.n_ctracks - 1;
    const int ct_f = a.ct_first[ctk], ct_m = a.ct_m[ctk], ct_pid = a.ct_pid[ctk];
    Real H[6], gpt[3];
#pragma unroll
    for (int k = 0; k < 6; ++k) H[k] = ((const Real*)a.Hpp)[6 * ctk + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) gpt[k] = ((const Real*)a.gp)[3 * ctk + k];
    Real y[3] = {Real(0), Real(0), Real(0)};
    if (obs >= 0) {
        ObsCtx ctx;
        load_obs_ctx(a, img, ctx);
        ObsCore o;
        typedef CoreRec<Real> CR;
        core_load<true>(reinterpret_cast<const typename CR::T*>(a.core) + (int64_t)chunk * CR::NF * BA_CHUNK, tid, o);
        // t = J_c delta_c, with delta_c of this image gathered through the unknown map
        Real xs[16];
        if (a.dc_img != nullptr) {                     // image-level copy: one load fewer
#pragma unroll
            for (int j = 0; j < 16; ++j) xs[j] = j < d ? ((const Real*)a.dc_img)[(int64_t)img * d + j] : Real(0);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int u = j < d ? a.umap[(int64_t)img * d + j] : -1;
                xs[j] = u >= 0 ? ((const Real*)a.dc)[u] : Real(0);
            }
        }
        Real t[3] = {Real(0), Real(0), Real(0)};
        emit_jc<HK, HP>(o, a.lay, ctx.enK, ctx.enP, ctx.enZ, obs == 0, dep,
                        [&](int r, int j, double v) { t[r] += (Real)v * xs[j]; });
        const bool xon = (a.enX ? a.enX[pid] != 0 : true) && !a.lay.x_off;
        double Jp[3][3], gP[3];
        point_rows<false>(o, ctx.cp, xon, Jp, gP);
#pragma unroll
        for (int k = 0; k < 3; ++k)
            y[k] = (Real)Jp[0][k] * t[0] + (Real)Jp[1][k] * t[1] + (Real)Jp[2][k] * t[2];
    }
    sh[tid][0] = y[0]; sh[tid][1] = y[1]; sh[tid][2] = y[2];
    __syncthreads();
    if (tid < n_ct) {
        const int f = ct_f, m = ct_m, pid = ct_pid;
        Real s[3] = {Real(0), Real(0), Real(0)};
        for (int q = 0; q < m; ++q) { s[0] += sh[f + q][0]; s[1] += sh[f + q][1]; s[2] += sh[f + q][2]; }
        Real Lf[6], b[3], z[3], x[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) b[k] = gpt[k] - s[k];
        chol3_factor(H, ((const Real*)a.lam_p)[0], Lf);
        chol3_fwd(Lf, b, z);
        chol3_bwd(Lf, z, x);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            a.dX[3 * (int64_t)pid + k] = (float)x[k];
            if (a.dX64) ((Real*)a.dX64)[3 * (int64_t)pid + k] = x[k];
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

// The first pointer a stage (0, 1, 2) or the back-substitution (3) dereferences that the caller left
// NULL, or nullptr when all are set (the optional ones: enable masks, r_in / w_in, dX64, b_order,
// work_ctr).
static const char* missing_pointer(const ba_lin_args& a, int stage) {
    const bool C = a.lay.C > 0;
#define BA_NEED(cond, p) do { if ((cond) && (p) == nullptr) return "null pointer " #p; } while (0)
    BA_NEED(stage != 2, a.infos);
    BA_NEED(stage != 2, a.chunk_obs); BA_NEED(stage != 2, a.chunk_meta);
    BA_NEED(stage != 2, a.ct_pid); BA_NEED(stage != 2, a.ct_first); BA_NEED(stage != 2, a.ct_m);
    BA_NEED(stage != 2 && C, a.s_dep);
    BA_NEED(stage != 2, a.s_pid); BA_NEED(stage != 2, a.s_img);
    BA_NEED(stage != 2, a.K); BA_NEED(stage != 2, a.P_rig2cam); BA_NEED(stage != 2, a.P_w2rig);
    BA_NEED(stage != 2 && C, a.z_coefs);
    BA_NEED(stage != 2, a.Hpp); BA_NEED(stage != 2, a.gp); BA_NEED(stage != 2, a.lam_p);
    BA_NEED(stage != 2, a.core);
    BA_NEED(stage == 0, a.s_pix); BA_NEED(stage == 0, a.s_std); BA_NEED(stage == 0, a.pts3d);
    BA_NEED(stage == 0, a.chunk_max); BA_NEED(stage == 0, a.ct_pt); BA_NEED(stage == 0, a.pfac);
    BA_NEED(stage == 0 && a.r_in != nullptr, a.w_in);
    BA_NEED(stage == 1, a.slot_info); BA_NEED(stage == 1, a.b_chunk_ptr); BA_NEED(stage == 1, a.b_imgs);
    BA_NEED(stage == 1, a.b_nimgs); BA_NEED(stage == 1, a.b_slot_ptr); BA_NEED(stage == 1, a.slot_pair);
    BA_NEED(stage == 1, a.chunk_slots); BA_NEED(stage == 1, a.chunk_ent); BA_NEED(stage == 1, a.chunk_eptr);
    BA_NEED(stage == 1, a.b_pos_slot); BA_NEED(stage == 1, a.ct_pt); BA_NEED(stage == 1, a.pfac);
    BA_NEED(stage == 1, a.partials); BA_NEED(stage == 1, a.img_partials);
    BA_NEED(stage == 2, a.pair_ptr); BA_NEED(stage == 2, a.pair_src); BA_NEED(stage == 2, a.img_ptr);
    BA_NEED(stage == 2, a.img_src); BA_NEED(stage == 2, a.partials); BA_NEED(stage == 2, a.img_partials);
    BA_NEED(stage == 2, a.S_pairs); BA_NEED(stage == 2, a.e_img); BA_NEED(stage == 2, a.dg_img);
    BA_NEED(stage == 3 && a.dc_img == nullptr, a.dc); BA_NEED(stage == 3 && a.dc_img == nullptr, a.umap);
    BA_NEED(stage == 3, a.dX);
#undef BA_NEED
    return nullptr;
}

// stage 0: point blocks + damping value; 1: camera-pair batches; 2: deterministic reductions
// stages of the batched pass in the working precision Real (the checks are made by the caller)
template <typename Real>
static int lin_stage(const ba_lin_args& a, int32_t stage, hipStream_t st) {
    Real* const chunk_max = (Real*)a.chunk_max;
    Real* const lam_p = (Real*)a.lam_p;
    if (stage == 0) {
        hipLaunchKernelGGL(k_lam_clear<Real>, dim3(1), dim3(1), 0, st, chunk_max, a.n_chunks);
        if (a.n_chunks > 0) {
            BA_REQUIRE(a.n_ctracks >= 1 && a.ct_pt != nullptr, "chunk-track state missing");
            BA_DISPATCH_KP(a.lay, hipLaunchKernelGGL((k_track_pp<HK_, HP_, Real>), dim3((unsigned)a.n_chunks),
                                                     dim3(BA_CHUNK), 0, st, a));
            const int64_t nb = a.n_chunks < 256 * 256 ? (a.n_chunks + 255) / 256 : 256;
            hipLaunchKernelGGL(k_lam_reduce<Real>, dim3((unsigned)nb), dim3(256), 0, st, chunk_max, a.n_chunks);
        }
        hipLaunchKernelGGL(k_lam_final<Real>, dim3(1), dim3(1), 0, st, chunk_max, a.n_chunks, a.lay.dampen,
                           a.lay.adaptive, a.lay.x_off, lam_p);
        if (a.n_chunks > 0) {
            BA_REQUIRE(a.pfac != nullptr, "point-factor scratch missing");
            BA_REQUIRE((((uintptr_t)a.pfac | (uintptr_t)a.Hpp) & 15) == 0, "Hpp and pfac must be 16-byte aligned");
            hipLaunchKernelGGL(k_point_factor<Real>, dim3(nblk(a.n_ctracks, 256)), dim3(256), 0, st, (const Real*)a.Hpp,
                               (const Real*)a.gp, (const Real*)lam_p, a.n_ctracks, (Real*)a.pfac);
        }
        BA_LAUNCHED();
        return BA_OK;
    }
    if (stage == 1 && a.n_batches > 0) {
        size_t lds = ((size_t)BA_CHUNK * BA_BLK + 48) * sizeof(Real);
        // one workgroup per CU (the kernel's LDS allows one) pulling batches from the work queue
        unsigned grid = (unsigned)a.n_batches;
        if (a.work_ctr != nullptr) {
            int dev = 0, n_cu = 0;
            BA_HIP(hipGetDevice(&dev));
            BA_HIP(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
            if (n_cu > 0 && (int64_t)n_cu < a.n_batches) grid = (unsigned)n_cu;
            hipLaunchKernelGGL(k_ctr_clear, dim3(1), dim3(1), 0, st, a.work_ctr);
        }
        BA_DISPATCH_KP(a.lay, {
            BA_HIP(hipFuncSetAttribute((const void*)k_schur<HK_, HP_, Real>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds));
            hipLaunchKernelGGL((k_schur<HK_, HP_, Real>), dim3(grid), dim3(BA_WAVES * 64), lds, st, a);
        });
        BA_LAUNCHED();
    }
    if (stage == 1) return BA_OK;
    int d = a.lay.d;
    if (a.n_pairs > 0) {
        hipLaunchKernelGGL(k_pair_reduce<Real>, dim3(nblk(a.n_pairs * d * d, 256)), dim3(256), 0, st, a.pair_ptr,
                           a.pair_src, (const Real*)a.partials, a.n_pairs, d, (Real*)a.S_pairs);
        BA_LAUNCHED();
    }
    hipLaunchKernelGGL(k_img_reduce<Real>, dim3(nblk((int64_t)a.n_imgs * d, 256)), dim3(256), 0, st, a.img_ptr,
                       a.img_src, (const Real*)a.img_partials, a.n_imgs, d, (Real*)a.e_img, (Real*)a.dg_img);
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int ba_linearize_stage(const ba_lin_args* args, int32_t stage, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_lin_args& a = *args;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.lay.d >= 1 && a.lay.d <= 15, "fused path supports 1 <= d <= 15 image-level parameters");
    BA_REQUIRE(a.lay.off_tau == 2 * a.lay.hasK && a.lay.off_zcf == a.lay.off_tau + 6 * a.lay.hasP &&
                   a.lay.d == a.lay.off_zcf + (a.lay.hasZ ? a.lay.C : 0),
               "inconsistent image-level layout");
    BA_REQUIRE(a.lay.C >= 0 && a.lay.C <= BA_MAX_C, "fused path supports at most 24 z-coefficient columns");
    BA_REQUIRE(a.L >= 1 && a.L <= BA_MAX_LOCAL, "bad plan L");
    BA_REQUIRE(stage >= 0 && stage <= 2, "stage must be 0, 1 or 2");
    BA_REQUIRE(a.real32 == 0 || a.real32 == 1, "real32 must be 0 or 1");
    if (a.n_chunks > 0) {
        const char* miss = missing_pointer(a, stage);
        BA_REQUIRE(miss == nullptr, miss);
    }
    return a.real32 ? lin_stage<float>(a, stage, st) : lin_stage<double>(a, stage, st);
}

extern "C" int ba_backsubstitute(const ba_lin_args* args, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_lin_args& a = *args;
    BA_REQUIRE(a.lay.d >= 1 && a.lay.d <= 15, "fused path supports 1 <= d <= 15 image-level parameters");
    BA_REQUIRE(a.real32 == 0 || a.real32 == 1, "real32 must be 0 or 1");
    if (a.n_chunks == 0) return BA_OK;
    BA_REQUIRE(a.n_ctracks >= 1, "chunk-track state missing");
    const char* miss = missing_pointer(a, 3);
    BA_REQUIRE(miss == nullptr, miss);
    hipStream_t st = (hipStream_t)stream;
    if (a.real32)
        BA_DISPATCH_KP(a.lay, hipLaunchKernelGGL((k_backsub<HK_, HP_, float>), dim3((unsigned)a.n_chunks), dim3(BA_CHUNK), 0,
                                                 st, a));
    else
        BA_DISPATCH_KP(a.lay, hipLaunchKernelGGL((k_backsub<HK_, HP_, double>), dim3((unsigned)a.n_chunks), dim3(BA_CHUNK),
                                                 0, st, a));
    BA_LAUNCHED();
    return BA_OK;
}

// ============================================================================= pair-major path
// The reduced system built per run, per image and per image pair instead of per chunk batch (no
// limit on track length, up to 32 image-level parameters, any co-visibility), over the plan of
// ba_pm_plan_create.  Every sum runs in a fixed order, so the result does not depend on scheduling.
namespace ba {

#define PM_T 256
#define PM_SPAN BA_PM_SPAN  // observations (runs) per wave of k_pm_obs (k_pm_runs)
// waves of k_pm_obs sharing one staging buffer: two in fp64 (the buffer, not the registers, limited
// the CU to 1.5 waves per SIMD; measured at config 3: 17.33 -> 17.05 ms per pass), one in fp32 (the
// registers already allow no more waves than buffers; two waves there cost 3.5% in their turns)
template <typename Real> struct PmObsWaves { static constexpr int N = sizeof(Real) == 8 ? 2 : 1; };
static_assert(PM_SPAN % 64 == 0, "a span is whole rounds of 64 observations");

typedef ba_pm_args PmArgs;

__device__ __forceinline__ void pm_ctx(const PmArgs& a, int img, ObsCtx& c) {
    const int node = a.infos[a.n_imgs + img];
    const int cam = a.infos[2 * a.n_imgs + img];
    load_cam(c.cp, a.K, a.P_rig2cam, a.P_rig2cam_stride, a.P_w2rig, cam, node);
    c.zc = a.z_coefs + (int64_t)img * a.lay.C;
    c.enK = a.enK ? a.enK[cam] != 0 : true;
    c.enP = a.enP ? a.enP[node] != 0 : true;
    c.enZ = a.enZ ? a.enZ[img] != 0 : true;
}

// linearisation of observation o (residual or the caller's, weights, Jacobian core)
__device__ __forceinline__ void pm_core(const PmArgs& a, int o, const ObsCtx& c, ObsCore& oc, DepSrc& dep,
                                        bool& xon) {
    const int pid = a.pids[o];
    float X[3] = {a.pts3d[3 * (int64_t)pid], a.pts3d[3 * (int64_t)pid + 1], a.pts3d[3 * (int64_t)pid + 2]};
    const float2 uv = reinterpret_cast<const float2*>(a.pix2d)[o];
    const float2 sv = reinterpret_cast<const float2*>(a.pix2d_std)[o];
    load_dep(dep, a.pix2d_dep + (int64_t)o * a.lay.C, a.lay.C);
    GivenRW grw = {{0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}};
    if (a.r_in) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            grw.r[k] = a.r_in[(int64_t)o * a.r_s0 + k * a.r_s1];
            grw.w[k] = a.w_in[(int64_t)o * a.w_s0 + k * a.w_s1];
        }
    }
    obs_core(c.cp, c.zc, X, uv, sv, dep, a.hp, a.lay, a.r_in != nullptr, grw, oc);
    xon = (a.enX ? a.enX[pid] != 0 : true) && !a.lay.x_off;
}

// The Jacobian core of observation o of track t (point X, from the track's factor record) with the
// sqrt(W) k_pm_obs stored for it (no residual, no IRLS weights: the run pass needs neither).
__device__ __forceinline__ void pm_jcore(const PmArgs& a, int o, int t, const float X[3], const ObsCtx& c, ObsCore& oc,
                                         DepSrc& dep, bool& xon) {
    const float2 sv = reinterpret_cast<const float2*>(a.pix2d_std)[o];
    load_dep(dep, a.pix2d_dep + (int64_t)o * a.lay.C, a.lay.C);
    double gd = 0.0;
#pragma unroll
    for (int k = 0; k < BA_MAX_C; ++k)
        if (k < a.lay.C) { float pr = c.zc[k] * dep(k); gd += (double)pr; }
    eval_jac_core(c.cp, X, sv.x, sv.y, gd, a.hp.is_depth_log, oc.J);
    const float4 w = reinterpret_cast<const float4*>(a.wobs)[o];
    oc.sW[0] = w.x; oc.sW[1] = w.y; oc.sW[2] = w.z;
    xon = (a.enX ? a.enX[t] != 0 : true) && !a.lay.x_off;
}

// Weighted camera-row element (R, j) of an observation (the element emit_jc_row hands its sink).
template <int HK, int HP, int R>
__device__ __forceinline__ double jc_elem(const ObsCore& o, const LinLayout& lay, double mK, double mP, bool zon,
                                          bool z0off, const DepSrc& dep, int j) {
    constexpr int OT = 2 * HK, OZ = OT + 6 * HP;
    double u = 0.0;
    if (j < OT) {
        u = (R == 2 && lay.no_grad_f_from_rz) ? 0.0 : jac_foc(o.J, R, j) * mK;
    } else if (j < OZ) {
        u = jac_tau(o.J, R, j - OT) * mP;
    } else if (R == 2) {
        const int c = j - OZ;
        if (zon && c < lay.C && !(c == 0 && z0off)) u = o.J.zscale * (double)dep(c);
    }
    return u * o.sW[R];
}

// The 16 x 16 x 4 MFMA of the working precision: A[i][k] from lane i + 16 k, B[k][j] from lane
// j + 16 k (both kinds); the four accumulator values of a lane are column lane & 15 of rows
// row(lane, v), which the two kinds lay out differently.
template <typename Real>
struct PmMfma;
template <>
struct PmMfma<double> {
    typedef dbl4 V4;
    static __device__ __forceinline__ V4 mac(double a, double b, V4 c) {
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ int row(int lane, int v) { return 4 * v + (lane >> 4); }
};
template <>
struct PmMfma<float> {
    typedef flt4 V4;
    static __device__ __forceinline__ V4 mac(float a, float b, V4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ int row(int lane, int v) { return 4 * (lane >> 4) + v; }
};

// One wave's running sum of X^T X (or -X^T X) over the rows it staged for one image: the lower
// DP/16 x DP/16 tiles of the working precision's 16 x 16 x 4 MFMA, flushed to the slot (wave +
// image) when the image changes.  Column d of every staged row holds its right-hand-side value, so
// row d of the sum is the image's rhs part.  A slot (w, i) is unique: obs (runs) are image-sorted,
// so waves w and w + 1 cannot hold images i + 1 and i respectively.
template <int DP, typename Real>
struct PmTileAcc {
    typedef PmMfma<Real> M;
    static constexpr int NT = DP / 16, NTL = NT * (NT + 1) / 2;
    typename M::V4 acc[NTL];
    int img;
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int q = 0; q < NTL; ++q) acc[q] = (typename M::V4){Real(0), Real(0), Real(0), Real(0)};
    }
    __device__ __forceinline__ void flush(Real* __restrict__ slots, int64_t wave, int lane) const {
        Real* dst = slots + (wave + img) * (int64_t)(NTL * 256);
#pragma unroll
        for (int q = 0; q < NTL; ++q)
#pragma unroll
            for (int v = 0; v < 4; ++v) dst[q * 256 + M::row(lane, v) * 16 + (lane & 15)] = acc[q][v];
    }
    // rows [row_lo, row_hi) of X (LDS, row stride DP + 1) into the sum, A operand scaled by sg
    __device__ __forceinline__ void add_rows(const Real (*X)[DP + 1], int row_lo, int row_hi, Real sg, int lane) {
        const int c = lane & 15, k = lane >> 4;
        for (int g = row_lo >> 2; 4 * g < row_hi; ++g) {
            const int row = 4 * g + k;
            const bool ok = row >= row_lo && row < row_hi;
            Real av[NT], bw[NT];
#pragma unroll
            for (int h = 0; h < NT; ++h) {
                const Real x = ok ? X[row][16 * h + c] : Real(0);
                av[h] = sg * x;
                bw[h] = x;
            }
            int q = 0;
#pragma unroll
            for (int hi = 0; hi < NT; ++hi)
#pragma unroll
                for (int hj = 0; hj <= hi; ++hj) {
                    acc[q] = M::mac(av[hi], bw[hj], acc[q]);
                    ++q;
                }
        }
    }
    // the 64 staged entities of one round (3 rows each), image ids simg[0..64) (-1 = none, only at
    // the end; the others non-decreasing): every image segment into the sum
    __device__ __forceinline__ void add_round(const Real (*X)[DP + 1], const int* simg, Real sg, Real* slots,
                                              int64_t wave, int lane) {
        const int my = simg[lane];
        int lo = 0;
        while (lo < 64) {
            const int i = __shfl(my, lo);
            if (i < 0) break;
            const int hi = lo + __popcll(__ballot(my == i));
            if (i != img) {
                if (img >= 0) flush(slots, wave, lane);
                zero();
                img = i;
            }
            add_rows(X, 3 * lo, 3 * hi, sg, lane);
            lo = hi;
        }
    }
};

// Per observation (one wave per PM_SPAN observations, 64 at a time): J_p^T J_p (upper 6) and
// J_p^T W r (3) to pobs, sqrt(W) to wobs; the weighted camera rows, with sqrt(W) r in column d,
// staged in LDS and summed per image (X^T X) into the J slots.  PmObsWaves waves share one staging
// buffer and take turns with it: each wave linearises its observations of a round in registers (the
// loads that bound this kernel), then stages and sums them in its turn, so the buffer (26 KB in fp64)
// limits the CU to half as many buffers as waves.  Every wave sums its own rows in the same order as
// alone.
template <int HK, int HP, int DP, typename Real>
__global__ void __launch_bounds__(64 * PmObsWaves<Real>::N, 3) k_pm_obs(PmArgs a) {
    constexpr int NW = PmObsWaves<Real>::N;
    __shared__ Real X[192][DP + 1];
    __shared__ int simg[64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t w = (int64_t)blockIdx.x * NW + wv;
    const int64_t o_begin = w * PM_SPAN, o_end = min(o_begin + PM_SPAN, a.n_obs);   // empty past the end
    const int d = a.lay.d;
    PmTileAcc<DP, Real> T;
    T.img = -1;
    T.zero();
#pragma unroll 1
    for (int rnd = 0; rnd < PM_SPAN / 64; ++rnd) {     // the same rounds in every wave (barriers below)
        const int64_t o = o_begin + 64 * rnd + lane;
        int img = -1;
        ObsCtx c;
        ObsCore oc;
        DepSrc dep;
        if (o < o_end) {
            img = a.obs_img[o];
            bool xon;
            pm_ctx(a, img, c);
            pm_core(a, (int)o, c, oc, dep, xon);
            double Jp[3][3], gP[3];
            point_rows<true>(oc, c.cp, xon, Jp, gP);
            const int pr[6][2] = {{0, 0}, {0, 1}, {0, 2}, {1, 1}, {1, 2}, {2, 2}};
            // plain stores: a store instruction covers only part of each line of these 9-value rows,
            // which the L2 then completes (non-temporal, the kernel took 5% longer at config 3 in fp64)
            Real* q = (Real*)a.pobs + 9 * o;
#pragma unroll
            for (int k = 0; k < 6; ++k) {
                const int i = pr[k][0], j = pr[k][1];
                q[k] = (Real)(Jp[0][i] * Jp[0][j] + Jp[1][i] * Jp[1][j] + Jp[2][i] * Jp[2][j]);
            }
            q[6] = (Real)gP[0];
            q[7] = (Real)gP[1];
            q[8] = (Real)gP[2];
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 wv4 = {(float)oc.sW[0], (float)oc.sW[1], (float)oc.sW[2], 0.f};
            __builtin_nontemporal_store(wv4, reinterpret_cast<f4*>(a.wobs) + o);
        }
#pragma unroll 1
        for (int turn = 0; turn < NW; ++turn) {
            if (wv == turn) {
                if (img >= 0) {
                    const bool first = o == 0;
                    emit_jc_row<HK, HP, 0, 0, DP>(oc, a.lay, c.enK, c.enP, c.enZ, first, dep,
                                                  [&](int j, double v) { X[3 * lane][j] = (Real)v; });
                    emit_jc_row<HK, HP, 1, 0, DP>(oc, a.lay, c.enK, c.enP, c.enZ, first, dep,
                                                  [&](int j, double v) { X[3 * lane + 1][j] = (Real)v; });
                    emit_jc_row<HK, HP, 2, 0, DP>(oc, a.lay, c.enK, c.enP, c.enZ, first, dep,
                                                  [&](int j, double v) { X[3 * lane + 2][j] = (Real)v; });
#pragma unroll
                    for (int k = 0; k < 3; ++k) X[3 * lane + k][d] = (Real)oc.Rs[k];
                }
                simg[lane] = img;
            }
            __syncthreads();
            if (wv == turn) T.add_round(X, simg, Real(1), (Real*)a.jslots, w, lane);
            __syncthreads();
        }
    }
    if (T.img >= 0) T.flush((Real*)a.jslots, w, lane);
}

// per track: H_pp and g_p summed over its observations in image order; the block's largest diagonal
template <typename Real>
__global__ void __launch_bounds__(PM_T) k_pm_track(PmArgs a) {
    __shared__ Real sm[PM_T];
    const int64_t t = (int64_t)blockIdx.x * PM_T + threadIdx.x;
    Real m = Real(0);
    if (t < a.n_tracks) {
        Real h[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) h[k] = Real(0);
        for (int q = a.trk_obs_ptr[t]; q < a.trk_obs_ptr[t + 1]; ++q) {
            const Real* s = (const Real*)a.pobs + 9 * (int64_t)a.trk_obs[q];
#pragma unroll
            for (int k = 0; k < 9; ++k) h[k] += s[k];
        }
#pragma unroll
        for (int k = 0; k < 6; ++k) ((Real*)a.Hpp)[6 * t + k] = h[k];
#pragma unroll
        for (int k = 0; k < 3; ++k) ((Real*)a.gp)[3 * t + k] = h[6 + k];
        m = fmax(fabs(h[0]), fmax(fabs(h[3]), fabs(h[5])));
    }
    sm[threadIdx.x] = m;
    __syncthreads();
    for (int w = PM_T / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) sm[threadIdx.x] = fmax(sm[threadIdx.x], sm[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) ((Real*)a.tmax)[blockIdx.x] = sm[0];
}

// Per track: the point block's factor record of the pair-major passes, PM_PF values per track in the
// working precision, so that one aligned line (fp64) or half line (fp32) holds all a run reads:
//   0-2 L1 L2 L4 | 3-5 1/L0 1/L3 1/L5 | 6-8 w = L^-1 g_p | 9-11 the point X | 12-14 L0 L3 L5 | 15 zero
// (L the chol3x3_solve factor of H_pp + lam_p I).  The runs gather it by track, once each; with the
// point inside, they do not gather pts3d as well.
#define PM_PF 16
template <typename Real>
__global__ void __launch_bounds__(256) k_pm_factor(PmArgs a, const Real* __restrict__ lam_p) {
    typedef Real R2 __attribute__((ext_vector_type(2)));
    constexpr int NV = PM_PF / 2, STR = NV + 1;         // 16-byte vectors per record; LDS row stride
    __shared__ R2 rec[256 * STR];
    const int64_t t0 = (int64_t)blockIdx.x * 256, t = t0 + threadIdx.x;
    const int nt = (int)min((int64_t)256, a.n_tracks - t0);
    if (t < a.n_tracks) {
        const R2* h2 = reinterpret_cast<const R2*>((const Real*)a.Hpp + 6 * t);     // 16-byte aligned rows (fp64)
        Real H[6], Lf[6];
#pragma unroll
        for (int k = 0; k < 3; ++k) { const R2 v = h2[k]; H[2 * k] = v.x; H[2 * k + 1] = v.y; }
        chol3_factor(H, lam_p[0], Lf);
        const Real* gp = (const Real*)a.gp + 3 * t;
        const Real r0 = Real(1) / Lf[0], r1 = Real(1) / Lf[3], r2 = Real(1) / Lf[5];
        const Real w0 = gp[0] * r0;
        const Real w1 = (gp[1] - Lf[1] * w0) * r1;
        const Real w2 = (gp[2] - Lf[2] * w0 - Lf[4] * w1) * r2;
        const float* X = a.pts3d + 3 * t;
        R2* o = rec + threadIdx.x * STR;
        o[0] = (R2){Lf[1], Lf[2]}; o[1] = (R2){Lf[4], r0}; o[2] = (R2){r1, r2}; o[3] = (R2){w0, w1};
        o[4] = (R2){w2, (Real)X[0]}; o[5] = (R2){(Real)X[1], (Real)X[2]};
        o[6] = (R2){Lf[0], Lf[3]}; o[7] = (R2){Lf[5], Real(0)};
    }
    __syncthreads();
    // the block's records leave as one contiguous range, 16 bytes per lane and store
    R2* dst = reinterpret_cast<R2*>((Real*)a.pfac + PM_PF * t0);
    for (int e = threadIdx.x; e < nt * NV; e += 256) dst[e] = rec[(e / NV) * STR + e % NV];
}

// Per run (one wave per PM_SPAN runs, 64 at a time): V = sum over the run's observations of
// sum_R jc_R (L^-1 jp_R)^T (= (sum J_c^T J_p) L^-T), staged in LDS with L^-1 g_p in column d,
// summed per image (-X^T X) into the V slots and copied to V (run-major, 3 x DP per run).
template <int HK, int HP, int DP, typename Real>
__global__ void __launch_bounds__(64, 2) k_pm_runs(PmArgs a) {
    __shared__ Real X[192][DP + 1];
    __shared__ int simg[64];
    const int lane = threadIdx.x;
    const int64_t w = blockIdx.x;
    const int64_t r_begin = w * PM_SPAN, r_end = min(r_begin + PM_SPAN, a.n_runs);
    const int d = a.lay.d;
    PmTileAcc<DP, Real> T;
    T.img = -1;
    T.zero();
    // a round's run indices are requested one round ahead (its first observation's index at the end of
    // the round before), so a round starts with its factor and observation loads
    int n_img = -1, n_t = 0, n_q0 = 0, n_q1 = 0, n_o0 = 0;
    auto fetch_idx = [&](int64_t r) {
        n_img = -1;
        if (r < r_end) { n_img = a.run_img[r]; n_t = a.run_trk[r]; n_q0 = a.run_ptr[r]; n_q1 = a.run_ptr[r + 1]; }
    };
    fetch_idx(r_begin + lane);
    if (n_img >= 0) n_o0 = a.run_obs[n_q0];
    for (int64_t base = r_begin; base < r_end; base += 64) {
        const int img = n_img, t = n_t, q0 = n_q0, q1 = n_q1, o0 = n_o0;
        fetch_idx(base + 64 + lane);
        if (img >= 0) {
            ObsCtx c;
            pm_ctx(a, img, c);
            const double mK = c.enK ? 1.0 : 0.0, mP = c.enP ? 1.0 : 0.0;
            const bool zon = a.lay.hasZ && c.enZ;
            typedef Real R4 __attribute__((ext_vector_type(4)));
            const R4* pf = reinterpret_cast<const R4*>((const Real*)a.pfac + PM_PF * (int64_t)t);
            const R4 f0 = pf[0], f1 = pf[1], f2 = pf[2];
            const Real L1 = f0.x, L2 = f0.y, L4 = f0.z, i0 = f0.w, i1 = f1.x, i2 = f1.y;
            const float Xp[3] = {(float)f2.y, (float)f2.z, (float)f2.w};
            // column d: L^-1 g_p, stored first (the column loops skip it), so that its registers are free
            // during the loops (the fp64 kernel stays within 256 VGPRs without spills)
            X[3 * lane][d] = f1.z;
            X[3 * lane + 1][d] = f1.w;
            X[3 * lane + 2][d] = f2.x;
            for (int q = q0; q < q1; ++q) {
                const int o = q == q0 ? o0 : a.run_obs[q];
                ObsCore oc;
                DepSrc dep;
                bool xon;
                pm_jcore(a, o, t, Xp, c, oc, dep, xon);
                double Jp[3][3], gP[3];
                point_rows<false>(oc, c.cp, xon, Jp, gP);
                Real wv[3][3];                       // L^-1 jp_R, R = 0..2
#pragma unroll
                for (int R = 0; R < 3; ++R) {
                    wv[R][0] = (Real)Jp[R][0] * i0;
                    wv[R][1] = ((Real)Jp[R][1] - L1 * wv[R][0]) * i1;
                    wv[R][2] = ((Real)Jp[R][2] - L2 * wv[R][0] - L4 * wv[R][1]) * i2;
                }
                const bool z0off = !a.lay.optim_Z0 || (o == 0 && !a.lay.optim_Z_1st_cam);
                auto col = [&](int j, Real v[3]) {
                    const Real e0 = (Real)jc_elem<HK, HP, 0>(oc, a.lay, mK, mP, zon, z0off, dep, j);
                    const Real e1 = (Real)jc_elem<HK, HP, 1>(oc, a.lay, mK, mP, zon, z0off, dep, j);
                    const Real e2 = (Real)jc_elem<HK, HP, 2>(oc, a.lay, mK, mP, zon, z0off, dep, j);
#pragma unroll
                    for (int k = 0; k < 3; ++k) v[k] = e0 * wv[0][k] + e1 * wv[1][k] + e2 * wv[2][k];
                };
                if (q == q0) {
#pragma unroll
                    for (int j = 0; j < DP; ++j) {
                        if (j == d) continue;
                        Real v[3];
                        col(j, v);
#pragma unroll
                        for (int k = 0; k < 3; ++k) X[3 * lane + k][j] = v[k];
                    }
                } else {                             // several observations of the track in this image
#pragma unroll
                    for (int j = 0; j < DP; ++j) {
                        if (j == d) continue;
                        Real v[3];
                        col(j, v);
#pragma unroll
                        for (int k = 0; k < 3; ++k) X[3 * lane + k][j] += v[k];
                    }
                }
            }
        }
        if (n_img >= 0) n_o0 = a.run_obs[n_q0];
        simg[lane] = img;
        __syncthreads();
        T.add_round(X, simg, Real(-1), (Real*)a.vslots, w, lane);
        const int nr = (int)min((int64_t)64, r_end - base);
        Real* dst = (Real*)a.V + base * 3 * DP;
        // streamed out (V of a pass exceeds every cache)
        for (int e = lane; e < nr * 3 * DP; e += 64) __builtin_nontemporal_store(X[e / DP][e % DP], dst + e);
        __syncthreads();
    }
    if (T.img >= 0) T.flush((Real*)a.vslots, w, lane);
}

// Per image i: the J and V slots of the waves that held its observations and runs, summed in wave
// order: S_ii (lower tiles, mirrored), rhs_i (row d) and diag(H_cc)_i (the J part's diagonal).
template <int DP, typename Real>
__global__ void __launch_bounds__(256) k_pm_diag(PmArgs a) {
    constexpr int NT = DP / 16, NTL = NT * (NT + 1) / 2;
    const int i = blockIdx.x, t = threadIdx.x, d = a.lay.d;
    const int pd = a.diag_pair[i];
    Real* const e_img = (Real*)a.e_img;
    Real* const dg_img = (Real*)a.dg_img;
    if (pd < 0) {
        if (t < d) { e_img[(int64_t)i * d + t] = Real(0); dg_img[(int64_t)i * d + t] = Real(0); }
        return;
    }
    const int64_t o0 = i ? a.infos[i - 1] : 0, o1 = a.infos[i];
    const int64_t r0 = a.img_run_ptr[i], r1 = a.img_run_ptr[i + 1];
    const int64_t wj0 = o0 / PM_SPAN, wj1 = (o1 - 1) / PM_SPAN, wv0 = r0 / PM_SPAN, wv1 = (r1 - 1) / PM_SPAN;
    Real* S = (Real*)a.S_pairs + (int64_t)pd * d * d;
    const Real* jslots = (const Real*)a.jslots;
    const Real* vslots = (const Real*)a.vslots;
    for (int e = t; e < NTL * 256; e += 256) {
        Real sj = Real(0), sv = Real(0);
        for (int64_t w = wj0; w <= wj1; ++w) sj += jslots[(w + i) * (NTL * 256) + e];
        for (int64_t w = wv0; w <= wv1; ++w) sv += vslots[(w + i) * (NTL * 256) + e];
        const int q = e >> 8, ri = (e >> 4) & 15, cj = e & 15;
        int hi = 0, hj = 0, qq = 0;
#pragma unroll
        for (int x = 0; x < NT; ++x)
#pragma unroll
            for (int y = 0; y <= x; ++y) { if (qq == q) { hi = x; hj = y; } ++qq; }
        const int rr = 16 * hi + ri, cc = 16 * hj + cj;
        if (rr < d && cc < d && (hi != hj || cc <= rr)) {
            const Real s = sj + sv;
            S[rr * d + cc] = s;
            S[cc * d + rr] = s;
            if (rr == cc) dg_img[(int64_t)i * d + rr] = sj;
        } else if (rr == d && cc < d) {
            e_img[(int64_t)i * d + cc] = sj + sv;
        }
    }
}

// Block -> work index with consecutive indices on one XCD (blocks are dispatched round-robin over
// the 8 XCDs, each with its own L2): neighbouring pairs share image runs.
__device__ __forceinline__ int64_t xcd_block(int64_t b, int64_t nb) {
    const int64_t x = b & 7, q = nb >> 3, r = nb & 7;
    return x * q + (x < r ? x : r) + (b >> 3);
}

// per off-diagonal image pair (one wave): S_ij = - sum over the pair's terms of V_ti V_tj^T, four
// terms (twelve rows) per three 16 x 16 x 4 MFMAs per tile; the term indices of 64 terms are read at
// once and handed to the row lanes by shuffles, the rows of the next 8 terms are requested before
// the MFMAs of the current 8.  The pairs are taken in the plan's schedule (pairs whose
// terms come from the same neighbourhood of images run together and find each other's V rows in the L2)
template <int DP, typename Real>
__global__ void __launch_bounds__(PM_T) k_pm_pairs(PmArgs a) {
    typedef PmMfma<Real> M;
    constexpr int NT = DP / 16;
    const Real* const Vg = (const Real*)a.V;
    const int lane = threadIdx.x & 63;
    const int64_t q = xcd_block(blockIdx.x, gridDim.x) * (PM_T / 64) + (threadIdx.x >> 6);
    if (q >= a.n_pairs) return;
    const int64_t p = a.pair_sched != nullptr ? a.pair_sched[q] : q;     // the plan's processing order
    const int i1 = a.pair_i1[p], i2 = a.pair_i2[p];
    if (i1 == i2) return;
    const int d = a.lay.d;
    const int k = lane >> 4, c = lane & 15;
    typename M::V4 acc[NT][NT];
#pragma unroll
    for (int x = 0; x < NT; ++x)
#pragma unroll
        for (int y = 0; y < NT; ++y) acc[x][y] = (typename M::V4){Real(0), Real(0), Real(0), Real(0)};
    const int q0 = a.term_ptr[p], q1 = a.term_ptr[p + 1];
    const int n = q1 - q0, nbat = (n + 7) >> 3;
    // The loop body has no branches (indices clamped, out-of-range rows zeroed by a factor), so the
    // accumulators stay in the MFMA registers across iterations.
    // term indices of window w (64 terms) in lane order, -1 past the end
    auto window = [&](int w, int& ra, int& rb) {
        const int q = q0 + 64 * w + lane;
        const int qc = min(q, q1 - 1);
        ra = a.term[2 * (int64_t)qc];
        rb = a.term[2 * (int64_t)qc + 1];
        if (q >= q1) { ra = -1; rb = -1; }
    };
    // rows of batch b (8 terms, 24 rows = 6 groups of 4): group g, lane (c, k) holds row 4 g + k
    auto fetch = [&](int b, int ra_w, int rb_w, Real (&A)[6][NT], Real (&B)[6][NT]) {
#pragma unroll
        for (int g = 0; g < 6; ++g) {
            const int row = 4 * g + k, tj = 8 * (b & 7) + row / 3, kk = row % 3;
            const int ra = __shfl(ra_w, tj), rb = __shfl(rb_w, tj);
            const Real ma = ra >= 0 ? Real(1) : Real(0), mb = rb >= 0 ? Real(1) : Real(0);
            const int64_t oa = (int64_t)max(ra, 0) * 3 * DP + kk * DP + c, ob = (int64_t)max(rb, 0) * 3 * DP + kk * DP + c;
#pragma unroll
            for (int h = 0; h < NT; ++h) {
                A[g][h] = ma * Vg[oa + 16 * h];
                B[g][h] = mb * __builtin_nontemporal_load(Vg + ob + 16 * h);
            }
        }
    };
    int ra_c, rb_c, ra_n, rb_n;
    window(0, ra_c, rb_c);
    window(1, ra_n, rb_n);
    Real A[6][NT], B[6][NT], An[6][NT], Bn[6][NT];
    fetch(0, ra_c, rb_c, A, B);
    for (int b = 0; b < nbat; ++b) {
        const int nb = b + 1;
        const bool wrap = (nb & 7) == 0;
        const int raw = wrap ? ra_n : ra_c, rbw = wrap ? rb_n : rb_c;
        fetch(nb, nb < nbat ? raw : -1, nb < nbat ? rbw : -1, An, Bn);
#pragma unroll
        for (int g = 0; g < 6; ++g)
#pragma unroll
            for (int x = 0; x < NT; ++x)
#pragma unroll
                for (int y = 0; y < NT; ++y) acc[x][y] = M::mac(A[g][x], B[g][y], acc[x][y]);
#pragma unroll
        for (int g = 0; g < 6; ++g)
#pragma unroll
            for (int h = 0; h < NT; ++h) { A[g][h] = An[g][h]; B[g][h] = Bn[g][h]; }
        // after the last batch of a window: the next window becomes current, the one after is read
        int ra_f, rb_f;
        window((nb >> 3) + 1, ra_f, rb_f);
        ra_c = wrap ? ra_n : ra_c; rb_c = wrap ? rb_n : rb_c;
        ra_n = wrap ? ra_f : ra_n; rb_n = wrap ? rb_f : rb_n;
    }
    Real* S = (Real*)a.S_pairs + p * d * d;
#pragma unroll
    for (int x = 0; x < NT; ++x)
#pragma unroll
        for (int y = 0; y < NT; ++y)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int rr = 16 * x + M::row(lane, v), cc = 16 * y + (lane & 15);
                if (rr < d && cc < d) S[rr * d + cc] = -acc[x][y][v];
            }
}

// per track: delta_p = L^-T (L^-1 g_p - sum over its runs of V_ti^T delta_c(i)), DP lanes per track
// (lane c holds column c of the run's three V rows, so every V load is coalesced over the group): per
// run, the three products summed over the DP lanes by an xor tree, then added over the track's runs in
// trk_run order; lane 0 then solves with the k_pm_factor record.  Two runs per step: the run ids two
// steps ahead and their images one step ahead are requested early, so that a step's V rows and delta_c
// are requested together.
template <int DP, typename Real>
__global__ void __launch_bounds__(256) k_pm_backsub(PmArgs a) {
    const int d = a.lay.d;
    const int c = threadIdx.x % DP;
    const int64_t t = (int64_t)blockIdx.x * (256 / DP) + threadIdx.x / DP;
    const bool live = t < a.n_tracks;
    const int q0 = live ? a.trk_run_ptr[t] : 0, q1 = live ? a.trk_run_ptr[t + 1] : 0;
    Real s[3] = {Real(0), Real(0), Real(0)};
    auto run_at = [&](int q) { return q < q1 ? a.trk_run[q] : -1; };
    auto img_of = [&](int r) { return r >= 0 ? a.run_img[r] : 0; };
    int ra = run_at(q0), rb = run_at(q0 + 1);
    int ia = img_of(ra), ib = img_of(rb);
    int rc = run_at(q0 + 2), rd = run_at(q0 + 3);
    auto prod = [&](int r, int img, Real (&v)[3]) {
        v[0] = v[1] = v[2] = Real(0);
        if (r >= 0 && c < d) {
            const Real dc = ((const Real*)a.dc_img)[(int64_t)img * d + c];
            const Real* V = (const Real*)a.V + (int64_t)r * 3 * DP + c;
#pragma unroll
            for (int k = 0; k < 3; ++k) v[k] = V[k * DP] * dc;
        }
    };
    for (int q = q0; q < q1; q += 2) {
        Real va[3], vb[3];
        prod(ra, ia, va);
        prod(rb, ib, vb);
        ra = rc; rb = rd;
        ia = img_of(ra); ib = img_of(rb);
        rc = run_at(q + 4); rd = run_at(q + 5);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
#pragma unroll
            for (int m = DP / 2; m >= 1; m >>= 1) {
                va[k] += __shfl_xor(va[k], m);
                vb[k] += __shfl_xor(vb[k], m);
            }
            s[k] += va[k];
            if (q + 1 < q1) s[k] += vb[k];
        }
    }
    if (!live || c != 0) return;
    const Real* pf = (const Real*)a.pfac + PM_PF * t;       // the k_pm_factor record
    const Real z0 = pf[6] - s[0], z1 = pf[7] - s[1], z2 = pf[8] - s[2];
    const Real x2 = z2 * pf[5];
    const Real x1 = (z1 - pf[2] * x2) * pf[4];
    const Real x0 = (z0 - pf[0] * x1 - pf[1] * x2) * pf[3];
    a.dX[3 * t] = (float)x0; a.dX[3 * t + 1] = (float)x1; a.dX[3 * t + 2] = (float)x2;
    if (a.dX64) {
        Real* o = (Real*)a.dX64;
        o[3 * t] = x0; o[3 * t + 1] = x1; o[3 * t + 2] = x2;
    }
}

static const char* pm_missing(const ba_pm_args& a, bool backsub) {
#define BA_NEED(cond, p) do { if ((cond) && (p) == nullptr) return "null pointer " #p; } while (0)
    const bool C = a.lay.C > 0;
    BA_NEED(true, a.trk_run_ptr); BA_NEED(true, a.trk_run); BA_NEED(true, a.run_img); BA_NEED(true, a.V);
    BA_NEED(true, a.pfac);
    BA_NEED(backsub, a.dc_img); BA_NEED(backsub, a.dX);
    if (backsub) return nullptr;
    BA_NEED(true, a.jslots); BA_NEED(true, a.vslots); BA_NEED(true, a.wobs);
    BA_NEED(true, a.infos); BA_NEED(true, a.run_ptr); BA_NEED(true, a.run_obs); BA_NEED(true, a.run_trk);
    BA_NEED(true, a.img_run_ptr); BA_NEED(true, a.trk_obs_ptr); BA_NEED(true, a.trk_obs); BA_NEED(true, a.obs_img);
    BA_NEED(true, a.pair_i1); BA_NEED(true, a.pair_i2); BA_NEED(true, a.diag_pair); BA_NEED(true, a.term_ptr);
    BA_NEED(true, a.term); BA_NEED(true, a.pids); BA_NEED(true, a.pix2d); BA_NEED(true, a.pix2d_std);
    BA_NEED(C, a.pix2d_dep); BA_NEED(true, a.K); BA_NEED(true, a.P_rig2cam); BA_NEED(true, a.P_w2rig);
    BA_NEED(C, a.z_coefs); BA_NEED(true, a.pts3d); BA_NEED(a.r_in != nullptr, a.w_in);
    BA_NEED(true, a.pobs); BA_NEED(true, a.Hpp); BA_NEED(true, a.gp); BA_NEED(true, a.tmax); BA_NEED(true, a.lam_p);
    BA_NEED(true, a.S_pairs); BA_NEED(true, a.e_img); BA_NEED(true, a.dg_img);
#undef BA_NEED
    return nullptr;
}

}  // namespace ba

// the launches of one stage of ba_pm_linearize_stage in the working precision Real
template <typename Real>
static void pm_stage(const ba_pm_args& a, int stage, hipStream_t st) {
    const int64_t nbt = (a.n_tracks + PM_T - 1) / PM_T;
    const bool wide = a.lay.d > 15;
    if (stage == 1) {
        if (a.n_pairs > 0) {
            const unsigned g = (unsigned)((a.n_pairs + PM_T / 64 - 1) / (PM_T / 64));
            if (wide) hipLaunchKernelGGL((k_pm_pairs<32, Real>), dim3(g), dim3(PM_T), 0, st, a);
            else      hipLaunchKernelGGL((k_pm_pairs<16, Real>), dim3(g), dim3(PM_T), 0, st, a);
        }
        return;
    }
    Real* const tmax = (Real*)a.tmax;
    Real* const lam_p = (Real*)a.lam_p;
    hipLaunchKernelGGL(k_lam_clear<Real>, dim3(1), dim3(1), 0, st, tmax, nbt);
    if (a.n_obs > 0) {
        const int64_t nw = (a.n_obs + PM_SPAN - 1) / PM_SPAN;          // waves (spans of PM_SPAN observations)
        constexpr int NW = PmObsWaves<Real>::N;
        const unsigned g = (unsigned)((nw + NW - 1) / NW);
        BA_DISPATCH_KP(a.lay, {
            if (wide) hipLaunchKernelGGL((k_pm_obs<HK_, HP_, 32, Real>), dim3(g), dim3(64 * NW), 0, st, a);
            else      hipLaunchKernelGGL((k_pm_obs<HK_, HP_, 16, Real>), dim3(g), dim3(64 * NW), 0, st, a);
        });
    }
    if (a.n_tracks > 0) {
        hipLaunchKernelGGL(k_pm_track<Real>, dim3((unsigned)nbt), dim3(PM_T), 0, st, a);
        const int64_t nb = nbt < 256 * 256 ? (nbt + 255) / 256 : 256;
        hipLaunchKernelGGL(k_lam_reduce<Real>, dim3((unsigned)nb), dim3(256), 0, st, tmax, nbt);
    }
    hipLaunchKernelGGL(k_lam_final<Real>, dim3(1), dim3(1), 0, st, tmax, nbt, a.lay.dampen, a.lay.adaptive,
                       a.lay.x_off, lam_p);
    if (a.n_tracks > 0)
        hipLaunchKernelGGL(k_pm_factor<Real>, dim3(nblk(a.n_tracks, 256)), dim3(256), 0, st, a, (const Real*)lam_p);
    if (a.n_runs > 0) {
        const unsigned g = (unsigned)((a.n_runs + PM_SPAN - 1) / PM_SPAN);
        BA_DISPATCH_KP(a.lay, {
            if (wide) hipLaunchKernelGGL((k_pm_runs<HK_, HP_, 32, Real>), dim3(g), dim3(64), 0, st, a);
            else      hipLaunchKernelGGL((k_pm_runs<HK_, HP_, 16, Real>), dim3(g), dim3(64), 0, st, a);
        });
    }
    if (wide) hipLaunchKernelGGL((k_pm_diag<32, Real>), dim3((unsigned)a.n_imgs), dim3(256), 0, st, a);
    else      hipLaunchKernelGGL((k_pm_diag<16, Real>), dim3((unsigned)a.n_imgs), dim3(256), 0, st, a);
}

template <typename Real>
static void pm_backsub(const ba_pm_args& a, hipStream_t st) {
    if (a.lay.d > 15)
        hipLaunchKernelGGL((k_pm_backsub<32, Real>), dim3(nblk(a.n_tracks, 256 / 32)), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((k_pm_backsub<16, Real>), dim3(nblk(a.n_tracks, 256 / 16)), dim3(256), 0, st, a);
}

// elements (of the working precision) of one slot array
extern "C" int64_t ba_pm_slot_doubles(int64_t n_items, int32_t n_imgs, int32_t d) {
    if (n_items < 0 || n_imgs < 0 || d < 1 || d > 31) return -1;
    const int64_t ntl = d < 16 ? 1 : 3;
    return ((n_items + PM_SPAN - 1) / PM_SPAN + n_imgs) * ntl * 256;
}

extern "C" int ba_pm_linearize_stage(const ba_pm_args* args, int stage, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    BA_REQUIRE(stage == 0 || stage == 1, "stage must be 0 (observations, tracks, runs, images) or 1 (pairs)");
    const ba_pm_args& a = *args;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.lay.d >= 1 && a.lay.d <= 31, "pair-major path supports 1 <= d <= 31 image-level parameters");
    BA_REQUIRE(a.lay.off_tau == 2 * a.lay.hasK && a.lay.off_zcf == a.lay.off_tau + 6 * a.lay.hasP &&
                   a.lay.d == a.lay.off_zcf + (a.lay.hasZ ? a.lay.C : 0),
               "inconsistent image-level layout");
    BA_REQUIRE(a.lay.C >= 0 && a.lay.C <= BA_MAX_C, "at most 24 z-coefficient columns");
    BA_REQUIRE(a.n_imgs >= 1 && a.n_tracks >= 0 && a.n_obs >= 0 && a.n_runs >= 0 && a.n_pairs >= 0, "bad sizes");
    BA_REQUIRE(a.n_obs < ((int64_t)1 << 31) && a.n_runs <= a.n_obs, "bad observation / run counts");
    const char* miss = pm_missing(a, false);
    BA_REQUIRE(miss == nullptr, miss);
    BA_REQUIRE((((uintptr_t)a.Hpp | (uintptr_t)a.wobs) & 15) == 0, "Hpp and wobs must be 16-byte aligned");
    BA_REQUIRE(((uintptr_t)a.pfac & (a.real32 ? 15 : 31)) == 0, "pfac must be 32-byte aligned (16 in fp32)");
    if (a.real32) pm_stage<float>(a, stage, st);
    else          pm_stage<double>(a, stage, st);
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int ba_pm_linearize_schur(const ba_pm_args* args, void* stream) {
    const int rc = ba_pm_linearize_stage(args, 0, stream);
    return rc != BA_OK ? rc : ba_pm_linearize_stage(args, 1, stream);
}

extern "C" int ba_pm_backsubstitute(const ba_pm_args* args, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_pm_args& a = *args;
    BA_REQUIRE(a.lay.d >= 1 && a.lay.d <= 31, "pair-major path supports 1 <= d <= 31 image-level parameters");
    if (a.n_tracks == 0) return BA_OK;
    const char* miss = pm_missing(a, true);
    BA_REQUIRE(miss == nullptr, miss);
    hipStream_t st = (hipStream_t)stream;
    if (a.real32) pm_backsub<float>(a, st);
    else          pm_backsub<double>(a, st);
    BA_LAUNCHED();
    return BA_OK;
}
