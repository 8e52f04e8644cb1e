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
// The expensive per-observation work (residual, IRLS weight, Jacobian core) is done once, in
// k_track_pp, and kept as a 160-byte record per observation; the weighted rows are re-formed from it.
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
#define BA_PRE_C 8          // depth-guidance channels held in registers (further channels are read from memory)
#define BA_BLK 129          // doubles per observation block in LDS: 8 rows x 16 columns + 1 pad (spreads banks)
#define BA_CORE 20          // doubles per observation in the linearisation record

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
    auto put = [&](int f, double v) { rec[f * BA_CHUNK + t] = v; };
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
    p[18 * BA_CHUNK + t] = make_float2((float)o.J.jkf, (float)o.sW[0]);
    p[19 * BA_CHUNK + t] = make_float2((float)o.sW[1], (float)o.sW[2]);
}

__device__ __forceinline__ void core_load(const double* __restrict__ rec, int t, ObsCore& o) {
    auto get = [&](int f) { return rec[f * BA_CHUNK + t]; };
#pragma unroll
    for (int k = 0; k < 3; ++k) o.J.Xr[k] = get(k);
#pragma unroll
    for (int k = 0; k < 9; ++k) o.J.Jpr[k] = get(3 + k);
    o.J.fx_col = get(12);
    o.J.fy_col = get(13);
    o.J.zscale = get(14);
#pragma unroll
    for (int k = 0; k < 3; ++k) o.Rs[k] = get(15 + k);
    const float2* p = reinterpret_cast<const float2*>(rec);
    const float2 a = p[18 * BA_CHUNK + t], b = p[19 * BA_CHUNK + t];
    o.J.jkf = a.x;
    o.sW[0] = a.y; o.sW[1] = b.x; o.sW[2] = b.y;
}

// Weighted camera rows, element by element, from the core (.cu:444-501, ba_solver.py:38-39, :59-60).
template <int HK, int HP, class JcSink>
__device__ __forceinline__ void emit_jc(const ObsCore& o, const LinLayout& lay, bool enK, bool enP, bool enZ,
                                        bool first_obs, const DepSrc& dep, JcSink&& sink) {
    constexpr int OT = 2 * HK, OZ = OT + 6 * HP;     // image-level columns [foc | tau | zcf]
    const int C = lay.C;
    const double mK = enK ? 1.0 : 0.0, mP = enP ? 1.0 : 0.0;
    const bool zon = lay.hasZ && enZ;                 // an invalid observation has zscale = 0
    const bool z0off = !lay.optim_Z0 || (first_obs && !lay.optim_Z_1st_cam);
#pragma unroll
    for (int r = 0; r < 3; ++r) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            double u = 0.0;
            if (j < OT) {
                u = (r == 2 && lay.no_grad_f_from_rz) ? 0.0 : jac_foc(o.J, r, j) * mK;
            } else if (j < OZ) {
                u = jac_tau(o.J, r, j - OT) * mP;
            } else if (r == 2) {
                const int c = j - OZ;
                if (zon && c < C && !(c == 0 && z0off)) u = o.J.zscale * (double)dep(c);
            }
            sink(r, j, u * o.sW[r]);
        }
    }
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
        const int pid = a.s_pid[slot];
        DepSrc dep;
        load_dep(dep, a.s_dep + slot * a.lay.C, a.lay.C);
        ObsCore o;
        obs_core_slot(a, slot, obs, ctx, pid, dep, o);
        core_store(a.core + (int64_t)chunk * BA_CORE * BA_CHUNK, tid, o);
        const bool xon = (a.enX ? a.enX[pid] != 0 : true) && !a.lay.x_off;
        double Jp[3][3], gP[3];
        point_rows<true>(o, ctx.cp, xon, Jp, gP);
        // J_pts gram (ba_solver.py:911-924) and J_pts^T W r
        const int pr[6][2] = {{0, 0}, {0, 1}, {0, 2}, {1, 1}, {1, 2}, {2, 2}};
#pragma unroll
        for (int q = 0; q < 6; ++q) {
            int i = pr[q][0], j = pr[q][1];
            c[q] = Jp[0][i] * Jp[0][j] + Jp[1][i] * Jp[1][j] + Jp[2][i] * Jp[2][j];
        }
        c[6] = gP[0]; c[7] = gP[1]; c[8] = gP[2];
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) sh[tid][k] = c[k];
    __syncthreads();
    const int first_ct = a.chunk_meta[4 * chunk + 1], n_ct = a.chunk_meta[4 * chunk + 2];
    double mx = 0.0;
    if (tid < n_ct) {
        const int64_t ct = first_ct + tid;
        const int f = a.ct_first[ct], m = a.ct_m[ct], pid = a.ct_pid[ct];
        double s[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) s[k] = 0.0;
        for (int q = 0; q < m; ++q)
#pragma unroll
            for (int k = 0; k < 9; ++k) s[k] += sh[f + q][k];
#pragma unroll
        for (int k = 0; k < 6; ++k) a.Hpp[6 * ct + k] = s[k];
#pragma unroll
        for (int k = 0; k < 3; ++k) a.gp[3 * ct + k] = s[6 + k];
        const float* X = a.pts3d + 3 * (int64_t)pid;
        reinterpret_cast<float4*>(a.ct_pt)[ct] = make_float4(X[0], X[1], X[2], (a.enX ? a.enX[pid] != 0 : true) ? 1.f : 0.f);
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

// lam_p = dampen * max diag over all tracks (BlockDiagMat.dampen_, ba_solver.py:575-582).
// The maximum of non-negative doubles is the maximum of their bit patterns, so blocks combine with
// an integer atomic max into word n of cmax (cleared by k_lam_clear); the result is order-free.
__global__ void k_lam_clear(double* __restrict__ cmax, int64_t n) { cmax[n] = 0.0; }

__global__ void __launch_bounds__(256) k_lam_reduce(double* __restrict__ cmax, int64_t n) {
    __shared__ double s[256];
    double m = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) m = fmax(m, cmax[i]);
    s[threadIdx.x] = m;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) s[threadIdx.x] = fmax(s[threadIdx.x], s[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0)
        atomicMax(reinterpret_cast<unsigned long long*>(cmax + n), (unsigned long long)__double_as_longlong(s[0]));
}

__global__ void k_lam_final(const double* __restrict__ cmax, int64_t n, double dampen, int adaptive, int x_off,
                            double* __restrict__ out) {
    out[0] = (adaptive && !x_off) ? dampen * cmax[n] : dampen;
}

// ----------------------------------------------------------------------------- camera-pair blocks
//
// k_schur: one workgroup (8 waves, two per SIMD) per batch.  Per chunk of 128 observation slots:
//   A1  waves 0-1, lane per slot: form the weighted camera rows J_c from the slot's linearisation
//       record (rows 4-6 of the slot's LDS block, column 15 = W r / sqrt(W)) and the point rows;
//       wave 2, lane per chunk track: Cholesky factor of the damped point block, its reciprocal
//       pivots and w = L^-1 g_p; coverage masks by ballot.
//   A2  waves 0-1: V = J_c^T J_p L^-T (rows 0-2 of the block, column 15 = w for the first
//       observation of the track in the image, else 0); several observations of one track in one
//       image are then summed into the first one.
//   B   every wave, for each camera-pair slot it owns (accumulator in registers):
//         off-diagonal (a,b):  acc += V_ta^T V_tb        one 16x16x4 fp64 MFMA per covering track
//         diagonal (a,a):      acc += V_ta^T V_ta        per covering track
//                              acc -= J_o^T J_o          per observation o in image a
//       Rows 3 and 7 of a block are zero, so every MFMA reads 4 whole block rows with a uniform
//       base address.  The partial block is -acc; column 15 of a diagonal tile then holds
//       sum J_c^T W r - V w = the image's rhs term, and diag(J_c^T J_c) is summed from the
//       squared B operands of the J MFMAs.
// The next chunk's inputs (slot streams, and the chunk-track state written by k_track_pp) are
// fetched while the current chunk's MFMAs run; every fetch is a single level (no gathers).

__device__ __forceinline__ uint64_t uni64(uint64_t x) {
    uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return ((uint64_t)hi << 32) | lo;
}

struct ObsPre {                 // one observation slot, fetched a chunk ahead
    int info, obs;
    float dep[BA_PRE_C];
};

struct TrkPre {                 // one chunk track, fetched a chunk ahead
    double H[6], g[3];
    float4 X;
    int mask, n_ct;
};

// per chunk track in LDS: the fetched state, then (after the factorisation) the factor
struct TrkStage {
    double L[6];                // H_pp upper, replaced by the Cholesky factor
    double w[3];                // g_p, replaced by L^-1 g_p
    double rp[3];               // reciprocal pivots
    float4 X;                   // point, enable flag
    int mask, pad;
};

__device__ __forceinline__ void obs_fetch(const LinArgs& a, int64_t slot, int C, ObsPre& p) {
    p.info = a.slot_info[slot];
    p.obs = a.chunk_obs[slot];
    const float* dg = a.s_dep + slot * C;
#pragma unroll
    for (int c = 0; c < BA_PRE_C; ++c) p.dep[c] = c < C ? dg[c] : 0.f;
}

__device__ __forceinline__ void trk_fetch(const LinArgs& a, int ck, int first_ct, int lane, TrkPre& p) {
    p.n_ct = a.chunk_meta[4 * ck + 2];
    int64_t ct = (int64_t)first_ct + lane;
    ct = ct < a.n_ctracks ? ct : a.n_ctracks - 1;
    p.mask = a.ct_mask[ct];
#pragma unroll
    for (int k = 0; k < 6; ++k) p.H[k] = a.Hpp[6 * ct + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) p.g[k] = a.gp[3 * ct + k];
    p.X = reinterpret_cast<const float4*>(a.ct_pt)[ct];
}

__device__ __forceinline__ void trk_stage(const TrkPre& p, TrkStage& s) {
#pragma unroll
    for (int k = 0; k < 6; ++k) s.L[k] = p.H[k];
#pragma unroll
    for (int k = 0; k < 3; ++k) s.w[k] = p.g[k];
    s.X = p.X;
    s.mask = p.mask;
}

template <int HK, int HP>
__global__ void __launch_bounds__(BA_WAVES * 64) k_schur(LinArgs a) {
    extern __shared__ double sBlk[];                     // [BA_CHUNK][BA_BLK] observation blocks
    __shared__ TrkStage sTS[BA_MAX_CT];                  // per chunk track
    __shared__ ObsPre sPre[BA_CHUNK];                    // per observation slot
    __shared__ double sDv[BA_MAX_LOCAL][16];             // per local image: diag(J_c^T J_c)
    __shared__ uint64_t sTm[BA_MAX_LOCAL];               // chunk tracks covering each local image
    __shared__ uint64_t sIm[BA_MAX_LOCAL][2];            // slots observed in each local image
    __shared__ uint64_t sLm[BA_MAX_LOCAL][2];            // ... first slot of a (track, image) run
    __shared__ int sInfo[BA_CHUNK];
    __shared__ unsigned char sRowT[BA_MAX_LOCAL * BA_MAX_CT];   // (image, track) -> first slot
    __shared__ CamF sCam[BA_MAX_LOCAL];
    __shared__ unsigned char sEn[BA_MAX_LOCAL * 3];
    __shared__ int sPair[BA_MAX_SLOTS];
    __shared__ int sDup[2];
    __shared__ int sNct;

    const int d = a.lay.d, C = a.lay.C;
    const int batch = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const bool obs_lane = tid < BA_CHUNK;                // waves 0-1: one observation slot per lane
    const bool trk_wave = wave == 2;                     // wave 2: one chunk track per lane
    const int nimg = a.b_nimgs[batch];
    const int s0 = a.b_slot_ptr[batch], ns = a.b_slot_ptr[batch + 1] - s0;
    const double lam = a.lam_p[0];
    const int c_begin = a.b_chunk_ptr[batch], c_end = a.b_chunk_ptr[batch + 1];
    int first_ct = a.chunk_meta[4 * c_begin + 1];

    {
        ObsPre pre;
        TrkPre tpre;
        if (obs_lane) obs_fetch(a, (int64_t)c_begin * BA_CHUNK + tid, C, pre);
        else if (trk_wave) trk_fetch(a, c_begin, first_ct, lane, tpre);
        // local image parameters
        if (tid < nimg) {
            int img = a.b_imgs[(int64_t)batch * a.L + tid];
            int node = a.infos[a.n_imgs + img], cam = a.infos[2 * a.n_imgs + img];
            load_cam(sCam[tid], a.K, a.P_rig2cam, a.P_rig2cam_stride, a.P_w2rig, cam, node);
            sEn[3 * tid + 0] = a.enK ? a.enK[cam] : 1;
            sEn[3 * tid + 1] = a.enP ? a.enP[node] : 1;
            sEn[3 * tid + 2] = a.enZ ? a.enZ[img] : 1;
        }
        // the pair of slot q: (a | b << 8), -1 past the batch's slots
        for (int q = tid; q < BA_MAX_SLOTS; q += BA_WAVES * 64) sPair[q] = q < ns ? a.slot_pair[s0 + q] : -1;
        for (int q = tid; q < BA_MAX_LOCAL * 16; q += BA_WAVES * 64) sDv[q >> 4][q & 15] = 0.0;
        if (obs_lane) sPre[tid] = pre;
        else if (trk_wave) {
            trk_stage(tpre, sTS[lane]);
            if (lane == 0) sNct = tpre.n_ct;
        }
    }
    __syncthreads();

    dbl4 acc[BA_SLOTS_PER_WAVE];
#pragma unroll
    for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) acc[q] = dbl4{0.0, 0.0, 0.0, 0.0};
    // MFMA operand element of this lane inside a 4-row group: row lane/16, column lane%16
    const int loff = (lane >> 4) * 16 + (lane & 15);

    for (int ck = c_begin; ck < c_end; ++ck) {
        if (ck != c_begin) __syncthreads();    // previous chunk consumed; this chunk's inputs staged
        const int n_ct = sNct;

        // ---------------- A1
        const int info = obs_lane ? sPre[tid].info : -1;
        const bool valid = info >= 0;
        const int li = info & 0xff, ct = (info >> 8) & 0xff, leader = info >> 16;
        if (obs_lane) {
            sInfo[tid] = info;
            if (valid) {
                const ObsPre& pr = sPre[tid];
                DepSrc dep;
#pragma unroll
                for (int c = 0; c < BA_PRE_C; ++c) dep.r[c] = pr.dep[c];
                dep.g = a.s_dep + ((int64_t)ck * BA_CHUNK + tid) * C;
                ObsCore o;
                core_load(a.core + (int64_t)ck * BA_CORE * BA_CHUNK, tid, o);
                const bool eK = sEn[3 * li] != 0, eP = sEn[3 * li + 1] != 0, eZ = sEn[3 * li + 2] != 0;
                double* blk = sBlk + tid * BA_BLK;
                emit_jc<HK, HP>(o, a.lay, eK, eP, eZ, pr.obs == 0, dep, [&](int r, int j, double v) {
                    if (j < 15) blk[64 + 16 * r + j] = j < d ? v : 0.0;
                });
#pragma unroll
                for (int r = 0; r < 3; ++r) blk[64 + 16 * r + 15] = o.Rs[r];
#pragma unroll
                for (int j = 0; j < 16; ++j) blk[112 + j] = 0.0;
                // J_p waits in row 0 until A2 overwrites the row with V
                double Jp[3][3], gP[3];
                point_rows<false>(o, sCam[li], sTS[ct].X.w != 0.f && !a.lay.x_off, Jp, gP);
#pragma unroll
                for (int r = 0; r < 3; ++r)
#pragma unroll
                    for (int k = 0; k < 3; ++k) blk[3 * r + k] = Jp[r][k];
                if (leader == tid) sRowT[li * BA_MAX_CT + ct] = (unsigned char)tid;
            }
            uint64_t im = 0, lm = 0;
#pragma unroll
            for (int m = 0; m < BA_MAX_LOCAL; ++m) {
                const uint64_t b = __ballot(valid && li == m);
                const uint64_t bl = __ballot(valid && li == m && leader == tid);
                if (lane == m) { im = b; lm = bl; }
            }
            if (lane < BA_MAX_LOCAL) { sIm[lane][wave] = im; sLm[lane][wave] = lm; }
            const uint64_t dup = __ballot(valid && leader != tid);
            if (lane == 0) sDup[wave] = dup != 0;
        } else if (trk_wave) {
            TrkStage& T = sTS[lane];
            const int mask = T.mask;
            if (lane < n_ct) {
                double H[6], Lf[6];
#pragma unroll
                for (int k = 0; k < 6; ++k) H[k] = T.L[k];
                chol3_factor(H, lam, Lf);
                const double r0 = 1.0 / Lf[0], r1 = 1.0 / Lf[3], r2 = 1.0 / Lf[5];
                const double w0 = T.w[0] * r0;
                const double w1 = (T.w[1] - Lf[1] * w0) * r1;
                const double w2 = (T.w[2] - Lf[2] * w0 - Lf[4] * w1) * r2;
#pragma unroll
                for (int k = 0; k < 6; ++k) T.L[k] = Lf[k];
                T.rp[0] = r0; T.rp[1] = r1; T.rp[2] = r2;
                T.w[0] = w0; T.w[1] = w1; T.w[2] = w2;
            }
            uint64_t tm = 0;
#pragma unroll
            for (int m = 0; m < BA_MAX_LOCAL; ++m) {
                const uint64_t b = __ballot(lane < n_ct && ((mask >> m) & 1));
                if (lane == m) tm = b;
            }
            if (lane < BA_MAX_LOCAL) sTm[lane] = tm;
        }
        __syncthreads();

        // ---------------- A2: V = J_c^T P with P = J_p L^-T, column by column
        if (valid) {
            const TrkStage& T = sTS[ct];
            const double l10 = T.L[1], l20 = T.L[2], l21 = T.L[4], r0 = T.rp[0], r1 = T.rp[1], r2 = T.rp[2];
            double* blk = sBlk + tid * BA_BLK;
            double P[3][3];
#pragma unroll
            for (int r = 0; r < 3; ++r) {
                P[r][0] = blk[3 * r] * r0;
                P[r][1] = (blk[3 * r + 1] - l10 * P[r][0]) * r1;
                P[r][2] = (blk[3 * r + 2] - l20 * P[r][0] - l21 * P[r][1]) * r2;
            }
            const bool lead = leader == tid;
#pragma unroll
            for (int j = 0; j < 15; ++j) {
                const double j0 = blk[64 + j], j1 = blk[80 + j], j2 = blk[96 + j];
#pragma unroll
                for (int c = 0; c < 3; ++c) blk[16 * c + j] = j < d ? j0 * P[0][c] + j1 * P[1][c] + j2 * P[2][c] : 0.0;
            }
#pragma unroll
            for (int c = 0; c < 3; ++c) blk[16 * c + 15] = lead ? T.w[c] : 0.0;
#pragma unroll
            for (int j = 0; j < 16; ++j) blk[48 + j] = 0.0;
        }
        __syncthreads();
        if (sDup[0] | sDup[1]) {
            // several observations of one track in one image: V of the run is summed into its first slot
            if (valid && leader == tid) {
                double* dst = sBlk + tid * BA_BLK;
                for (int f = tid + 1; f < BA_CHUNK; ++f) {
                    const int fi = sInfo[f];
                    if (fi < 0 || (fi >> 16) != tid) break;
                    const double* src = sBlk + f * BA_BLK;
#pragma unroll
                    for (int c = 0; c < 3; ++c)
#pragma unroll
                        for (int j = 0; j < 15; ++j) dst[16 * c + j] += src[16 * c + j];
                }
            }
            __syncthreads();
        }

        // next chunk's inputs: fetched into registers now, staged into LDS after the MFMAs
        const bool more = ck + 1 < c_end;
        ObsPre pre;
        TrkPre tpre;
        if (more) {
            if (obs_lane) {
                obs_fetch(a, (int64_t)(ck + 1) * BA_CHUNK + tid, C, pre);
            } else if (trk_wave) {
                first_ct += n_ct;
                trk_fetch(a, ck + 1, first_ct, lane, tpre);
            }
        }

        // ---------------- B: camera-pair tiles
        // coverage masks and first-slot rows of every owned off-diagonal slot, read together
        int pqs[BA_SLOTS_PER_WAVE];
        uint64_t covs[BA_SLOTS_PER_WAVE];
        int rAs[BA_SLOTS_PER_WAVE], rBs[BA_SLOTS_PER_WAVE];
#pragma unroll
        for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
            const int pq = __builtin_amdgcn_readfirstlane(sPair[wave + BA_WAVES * q]);
            const int la = pq & 0xff, lb = (pq >> 8) & 0xff;
            pqs[q] = pq;
            covs[q] = 0;
            rAs[q] = rBs[q] = 0;
            if (pq >= 0 && la != lb) {
                covs[q] = sTm[la] & sTm[lb];
                rAs[q] = sRowT[la * BA_MAX_CT + lane];
                rBs[q] = sRowT[lb * BA_MAX_CT + lane];
            }
        }
#pragma unroll
        for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
            const int pq = pqs[q];
            if (pq < 0) continue;
            const int la = pq & 0xff, lb = (pq >> 8) & 0xff;
            if (la != lb) {
                uint64_t cov = uni64(covs[q]);
                const int rA = rAs[q], rB = rBs[q];
                // covering tracks in groups of four: the eight operand reads of a group are issued
                // together, then its four MFMAs run as they arrive (a short group re-reads its first
                // track with B = 0, adding exact zeros)
                while (cov) {
                    int t[4];
                    int n = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        if (cov) { t[k] = __builtin_ctzll(cov); cov &= cov - 1; ++n; }
                        else t[k] = t[0];
                    }
                    double A[4], B[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        A[k] = sBlk[__builtin_amdgcn_readlane(rA, t[k]) * BA_BLK + loff];
                        B[k] = sBlk[__builtin_amdgcn_readlane(rB, t[k]) * BA_BLK + loff];
                    }
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        acc[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(A[k], k < n ? B[k] : 0.0, acc[q], 0, 0, 0);
                    // keep the group's LDS reads ahead of its MFMAs (the scheduler would otherwise
                    // pair each read with its MFMA to save registers, serialising on LDS latency)
                    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                }
            } else {
                // J rows (block offset 64) of every observation in the image, subtracted (A = -B) and
                // feeding diag(J_c^T J_c); then V rows (offset 0) of every (track, image) run; both
                // lists in groups of four like the off-diagonal tracks
                double dsq = 0.0;
#pragma unroll
                for (int part = 0; part < 2; ++part) {
                    const bool jr = part == 0;
                    uint64_t w0 = uni64(jr ? sIm[la][0] : sLm[la][0]);
                    uint64_t w1 = uni64(jr ? sIm[la][1] : sLm[la][1]);
                    const int roff = (jr ? 64 : 0) + loff;
                    while (w0 | w1) {
                        int o[4];
                        int n = 0;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            if (w0) { o[k] = __builtin_ctzll(w0); w0 &= w0 - 1; ++n; }
                            else if (w1) { o[k] = 64 + __builtin_ctzll(w1); w1 &= w1 - 1; ++n; }
                            else o[k] = o[0];
                        }
                        double B[4];
#pragma unroll
                        for (int k = 0; k < 4; ++k) B[k] = sBlk[o[k] * BA_BLK + roff];
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const double b = k < n ? B[k] : 0.0;
                            acc[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(jr ? -b : b, b, acc[q], 0, 0, 0);
                            if (jr) dsq += b * b;
                        }
                        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
                        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                    }
                }
                dsq += __shfl_xor(dsq, 16);
                dsq += __shfl_xor(dsq, 32);
                if (lane < 16) sDv[la][lane] += dsq;
            }
        }
        // stage the next chunk's inputs (A1 and A2 of this chunk are past, so the arrays are free)
        if (more) {
            if (obs_lane) sPre[tid] = pre;
            else if (trk_wave) {
                trk_stage(tpre, sTS[lane]);
                if (lane == 0) sNct = tpre.n_ct;
            }
        }
    }

    // flush this batch's partial blocks (-acc, row-major d x d, local orientation);
    // v_mfma_f64_16x16x4f64 accumulator layout: lane l, element v holds D[4v + l/16][l%16]
    const int jc = lane & 15;
#pragma unroll
    for (int q = 0; q < BA_SLOTS_PER_WAVE; ++q) {
        const int pq = __builtin_amdgcn_readfirstlane(sPair[wave + BA_WAVES * q]);
        if (pq >= 0) {
            const int sl = wave + BA_WAVES * q;
            double* P = a.partials + (int64_t)(s0 + sl) * d * d;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = 4 * v + (lane >> 4);
                if (i < d && jc < d) P[i * d + jc] = -acc[q][v];
            }
            const int la = pq & 0xff, lb = (pq >> 8) & 0xff;
            if (la == lb && jc == 15) {
                double* o = a.img_partials + ((int64_t)batch * a.L + la) * 2 * d;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int i = 4 * v + (lane >> 4);
                    if (i < d) o[i] = -acc[q][v];
                }
            }
        }
    }
    __syncthreads();
    {
        const int va = tid >> 4, vj = tid & 15;
        if (va < nimg && vj < d) a.img_partials[((int64_t)batch * a.L + va) * 2 * d + d + vj] = sDv[va][vj];
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
        const int pid = a.s_pid[slot];
        DepSrc dep;
        load_dep(dep, a.s_dep + slot * a.lay.C, a.lay.C);
        ObsCore o;
        core_load(a.core + (int64_t)chunk * BA_CORE * BA_CHUNK, tid, o);
        // t = J_c delta_c, with delta_c of this image gathered through the unknown map
        double xs[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int u = j < d ? a.umap[(int64_t)img * d + j] : -1;
            xs[j] = u >= 0 ? a.dc[u] : 0.0;
        }
        double t[3] = {0.0, 0.0, 0.0};
        emit_jc<HK, HP>(o, a.lay, ctx.enK, ctx.enP, ctx.enZ, obs == 0, dep,
                        [&](int r, int j, double v) { t[r] += v * xs[j]; });
        const bool xon = (a.enX ? a.enX[pid] != 0 : true) && !a.lay.x_off;
        double Jp[3][3], gP[3];
        point_rows<false>(o, ctx.cp, xon, Jp, gP);
#pragma unroll
        for (int k = 0; k < 3; ++k) y[k] = Jp[0][k] * t[0] + Jp[1][k] * t[1] + Jp[2][k] * t[2];
    }
    sh[tid][0] = y[0]; sh[tid][1] = y[1]; sh[tid][2] = y[2];
    __syncthreads();
    const int first_ct = a.chunk_meta[4 * chunk + 1], n_ct = a.chunk_meta[4 * chunk + 2];
    if (tid < n_ct) {
        const int64_t ctk = first_ct + tid;
        int f = a.ct_first[ctk], m = a.ct_m[ctk], pid = a.ct_pid[ctk];
        double s[3] = {0.0, 0.0, 0.0};
        for (int q = 0; q < m; ++q) { s[0] += sh[f + q][0]; s[1] += sh[f + q][1]; s[2] += sh[f + q][2]; }
        double H[6], Lf[6], b[3], z[3], x[3];
#pragma unroll
        for (int k = 0; k < 6; ++k) H[k] = a.Hpp[6 * ctk + k];
#pragma unroll
        for (int k = 0; k < 3; ++k) b[k] = a.gp[3 * ctk + k] - s[k];
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
    BA_REQUIRE(a.lay.d >= 1 && a.lay.d <= 15, "fused path supports 1 <= d <= 15 image-level parameters");
    BA_REQUIRE(a.lay.off_tau == 2 * a.lay.hasK && a.lay.off_zcf == a.lay.off_tau + 6 * a.lay.hasP &&
                   a.lay.d == a.lay.off_zcf + (a.lay.hasZ ? a.lay.C : 0),
               "inconsistent image-level layout");
    BA_REQUIRE(a.lay.C >= 0 && a.lay.C <= BA_MAX_C, "fused path supports at most 24 z-coefficient columns");
    BA_REQUIRE(a.L >= 1 && a.L <= BA_MAX_LOCAL, "bad plan L");
    if (stage == 0) {
        hipLaunchKernelGGL(k_lam_clear, dim3(1), dim3(1), 0, st, a.chunk_max, a.n_chunks);
        if (a.n_chunks > 0) {
            BA_REQUIRE(a.n_ctracks >= 1 && a.ct_pt != nullptr, "chunk-track state missing");
            BA_DISPATCH_KP(a.lay, hipLaunchKernelGGL((k_track_pp<HK_, HP_>), dim3((unsigned)a.n_chunks), dim3(BA_CHUNK), 0,
                                                     st, a));
            const int64_t nb = a.n_chunks < 256 * 256 ? (a.n_chunks + 255) / 256 : 256;
            hipLaunchKernelGGL(k_lam_reduce, dim3((unsigned)nb), dim3(256), 0, st, a.chunk_max, a.n_chunks);
        }
        hipLaunchKernelGGL(k_lam_final, dim3(1), dim3(1), 0, st, a.chunk_max, a.n_chunks, a.lay.dampen, a.lay.adaptive,
                           a.lay.x_off, a.lam_p);
        BA_LAUNCHED();
        return BA_OK;
    }
    if (stage == 1 && a.n_batches > 0) {
        size_t lds = (size_t)BA_CHUNK * BA_BLK * sizeof(double);
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
    BA_REQUIRE(a.lay.d >= 1 && a.lay.d <= 15, "fused path supports 1 <= d <= 15 image-level parameters");
    if (a.n_chunks == 0) return BA_OK;
    hipStream_t st = (hipStream_t)stream;
    BA_DISPATCH_KP(a.lay, hipLaunchKernelGGL((k_backsub<HK_, HP_>), dim3((unsigned)a.n_chunks), dim3(BA_CHUNK), 0, st, a));
    BA_LAUNCHED();
    return BA_OK;
}
