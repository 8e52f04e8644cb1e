// Reduced camera system: unknown-level assembly and Jacobi-preconditioned CG on the device.
//
// Restates the reference's _solve_CG / _pcg (src/blast3r/inference/ba_solver.py:184-206,
// :1197-1238) on the explicit image-pair blocks produced by ba_linearize_schur:
//   S_u = P^T S_img P + diag(damping),  M = clamp(diag(A), 1e-12),
// where P maps image-level parameters [foc(cam) | tau(node) | zcf(img)] to the
// reference's unknown order [foc | tau | zcf] (ba_solver.py:119).  The CG
// iteration, its stopping test, the clamps and the best-so-far return follow
// _pcg line by line; scalars stay on the device (no host synchronisation).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cmath>

#include "ba_common.h"
#include "ba_error.h"

namespace ba {

#define PCG_T 256
// threads of the image-row SpMV: 8 groups of 16 lanes.  Two waves per row keep every row of a
// 1024-image system resident at once (the kernel needs ~112 VGPRs: 4 waves per SIMD).
#define PCG_ST 128
// Block partials of the update launch (nb blocks): r.r and r.z, PCG_NP per block.
#define PCG_NP 2
#define PCG_LF 16           // entries of a long inverse list each lane has in flight
#define PCG_IPF 4           // image partials of p.Ap each update thread requests at launch
enum { PT_RR = 0, PT_RZ = 1 };

// state (working precision): ST_RZ0/1 r.z after n updates and ST_BEST0/1 the best residual norm after n updates,
// both in slot n & 1; ST_BETA the beta of the current direction; ST_LEAF.. the camera-leaf damping.
// ST_LEAFMAX.. (3 words): the per-leaf maxima of |diag(A)| as bit patterns, accumulated by k_leaf_max.
enum { ST_BNORM = 0, ST_RZ0 = 1, ST_RZ1 = 2, ST_BEST0 = 3, ST_BEST1 = 4, ST_BETA = 5, ST_LEAF = 8, ST_LEAFMAX = 11 };
// istate: IS_DONE0 / IS_DONE1 "stopped before update n" in slot n & 1, IS_K iterations run,
// IS_CONV converged, IS_BESTK best iterate, IS_USEBEST the best iterate is returned.
enum { IS_DONE0 = 0, IS_DONE1 = 1, IS_K = 2, IS_CONV = 3, IS_BESTK = 4, IS_USEBEST = 5 };

// The arrays of ba_pcg_args in the working precision Real (double, or float when real32 is set).
template <typename Real>
struct PcgV {
    const Real *S_pairs, *e_img, *dg_img;
    Real *rhs, *diagA, *damp, *x, *xbest, *r, *z, *p, *y_img, *partials, *state, *S_rows, *img_part;
    __device__ __forceinline__ explicit PcgV(const ba_pcg_args& a)
        : S_pairs((const Real*)a.S_pairs), e_img((const Real*)a.e_img), dg_img((const Real*)a.dg_img),
          rhs((Real*)a.rhs), diagA((Real*)a.diagA), damp((Real*)a.damp), x((Real*)a.x), xbest((Real*)a.xbest),
          r((Real*)a.r), z((Real*)a.z), p((Real*)a.p), y_img((Real*)a.y_img), partials((Real*)a.partials),
          state((Real*)a.state), S_rows((Real*)a.S_rows), img_part((Real*)a.img_part) {}
};

// search direction of update n: p_n = z_n + beta_n p_{n-1} (ba_solver.py:1235), written as one
// fused multiply-add so that every kernel that forms it gets the same bits
template <typename Real>
__device__ __forceinline__ Real pdir(Real z, Real pold, Real beta) { return fma(beta, pold, z); }

// Sum over the 64 lanes of a wave; every lane gets the same bits (each butterfly step adds the
// same two values in either lane, and fp addition commutes).
template <typename Real>
__device__ __forceinline__ Real wave_sum(Real v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Sum over a block of NT threads in a fixed order (waves by butterfly, then the wave sums in wave
// order); every thread gets the result.  sh holds at least NT / 64 doubles.
template <int NT, typename Real>
__device__ __forceinline__ Real block_sum(Real v, Real* sh) {
    v = wave_sum(v);
    __syncthreads();                                  // sh may still be read by a previous call
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    Real t = Real(0);
#pragma unroll
    for (int k = 0; k < NT / 64; ++k) t += sh[k];
    return t;
}

// K block sums at once with two barriers; v[k] becomes the sum of every thread's v[k], in the
// same order as block_sum.  sh holds at least K * NT / 64 doubles.
template <int NT, int K, typename Real>
__device__ __forceinline__ void block_sums(Real (&v)[K], Real* sh) {
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = wave_sum(v[k]);
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
#pragma unroll
        for (int k = 0; k < K; ++k) sh[k * (NT / 64) + (threadIdx.x >> 6)] = v[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k) {
        Real t = Real(0);
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) t += sh[k * (NT / 64) + w];
        v[k] = t;
    }
}

// Sums of r.r and r.z over the nb block partials (deterministic, identical in every block of NT
// threads); sh holds at least 2 * NT / 64 doubles.
template <int NT, typename Real>
__device__ __forceinline__ void sum_partials(const Real* __restrict__ part, int nb, Real (&rs)[2], Real* sh) {
    rs[0] = Real(0); rs[1] = Real(0);
    for (int b = threadIdx.x; b < nb; b += NT) { rs[0] += part[PCG_NP * b + PT_RR]; rs[1] += part[PCG_NP * b + PT_RZ]; }
    block_sums<NT, 2>(rs, sh);
}

// unknown-level rhs and diag(H_cc) from the image-level vectors; one wave per unknown so that
// shared unknowns (one focal pair for every image of a camera) reduce in parallel
template <typename Real>
__global__ void __launch_bounds__(PCG_T) k_unk_setup(ba_pcg_args a) {
    const PcgV<Real> av(a);
    const int lane = threadIdx.x & 63;
    if (blockIdx.x == 0 && threadIdx.x < 3)                  // k_leaf_max's accumulators
        av.state[ST_LEAFMAX + threadIdx.x] = Real(0);
    int64_t u = (int64_t)blockIdx.x * (PCG_T / 64) + (threadIdx.x >> 6);
    if (u >= a.n_u) return;
    Real e = Real(0), g = Real(0);
    for (int q = a.inv_ptr[u] + lane; q < a.inv_ptr[u + 1]; q += 64) {
        int src = a.inv_src[q];
        e += av.e_img[src];
        g += av.dg_img[src];
    }
    for (int off = 32; off > 0; off >>= 1) {
        e += __shfl_down(e, off);
        g += __shfl_down(g, off);
    }
    if (lane == 0) { av.rhs[u] = e; av.diagA[u] = g; }
}

// per-leaf damping (BlockDiagMat.dampen_, ba_solver.py:575-582) and the Jacobi preconditioner.
// leaf ids 0..2 = foc, tau, zcf; 3..5 = the same groups switched off (a zero matrix damped by
// dampen * I, ZerosMat.dampen_, ba_solver.py:510-517).
// Two launches over every block of unknowns: the per-leaf maxima (fmax within a block; across blocks
// an integer max of the bit patterns, which orders non-negative doubles as their values, so the
// result does not depend on the order; a block whose maximum is NaN contributes nothing, as fmax
// ignores NaN), then the damping and the clamped preconditioner diagonal per unknown.
template <typename Real>
__global__ void __launch_bounds__(PCG_T) k_leaf_max(ba_pcg_args a) {
    const PcgV<Real> av(a);
    __shared__ Real sh[3][PCG_T];
    Real m[3] = {Real(0), Real(0), Real(0)};
    for (int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x; u < a.n_u; u += (int64_t)gridDim.x * PCG_T) {
        const int l = a.leaf[u];
        if (l < 3) m[l] = fmax(m[l], fabs(av.diagA[u]));
    }
#pragma unroll
    for (int l = 0; l < 3; ++l) sh[l][threadIdx.x] = m[l];
    __syncthreads();
    for (int w = PCG_T / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w)
#pragma unroll
            for (int l = 0; l < 3; ++l) sh[l][threadIdx.x] = fmax(sh[l][threadIdx.x], sh[l][threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x < 3) {
        const Real mv = sh[threadIdx.x][0];
        if (!isnan(mv)) atomic_max_nonneg(av.state + ST_LEAFMAX + threadIdx.x, mv);
    }
}

template <typename Real>
__global__ void __launch_bounds__(PCG_T) k_leaf_damp(ba_pcg_args a) {
    const PcgV<Real> av(a);
    Real lam[6];
#pragma unroll
    for (int l = 0; l < 3; ++l) {
        const Real mx = av.state[ST_LEAFMAX + l];        // the bits k_leaf_max combined are the value's
        lam[l] = a.adaptive ? Real(a.dampen) * mx : Real(a.dampen);
        lam[l + 3] = Real(a.dampen);
    }
    for (int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x; u < a.n_u; u += (int64_t)gridDim.x * PCG_T) {
        Real dmp = lam[a.leaf[u]];
        av.damp[u] = dmp;
        Real dA = av.diagA[u] + dmp;
        av.diagA[u] = dA > Real(1e-12) ? dA : Real(1e-12);          // diagA.clamp(min=1e-12) (ba_solver.py:191-192)
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        for (int l = 0; l < 3; ++l) av.state[ST_LEAF + l] = lam[l];
    }
}

// x = 0, r = b, z = M^-1 r, p_{-1} = 0 (so that p_0 = z_0); partials of b.b and r.z
template <typename Real>
__global__ void __launch_bounds__(PCG_T) k_pcg_init(ba_pcg_args a) {
    const PcgV<Real> av(a);
    __shared__ Real sh[PCG_T];
    int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x;
    Real t[2] = {Real(0), Real(0)};
    if (u < a.n_u) {
        Real b = av.rhs[u];
        Real z = b / av.diagA[u];
        av.x[u] = Real(0); av.xbest[u] = Real(0); av.r[u] = b; av.z[u] = z; av.p[a.n_u + u] = Real(0);
        t[0] = b * b; t[1] = b * z;
    }
    block_sums<PCG_T, 2>(t, sh);
    if (threadIdx.x == 0) { av.partials[PCG_NP * blockIdx.x + PT_RR] = t[0]; av.partials[PCG_NP * blockIdx.x + PT_RZ] = t[1]; }
}

template <typename Real>
__global__ void __launch_bounds__(PCG_T) k_pcg_init2(ba_pcg_args a, int nb) {
    const PcgV<Real> av(a);
    __shared__ Real sh[PCG_T];
    Real rs[2];
    sum_partials<PCG_T>(av.partials, nb, rs, sh);
    const Real bb = rs[0], rz = rs[1];
    if (threadIdx.x == 0) {
        Real bn = sqrt(bb);
        av.state[ST_BNORM] = bn > Real(1e-12) ? bn : Real(1e-12);    // torch.norm(b).clamp(min=1e-12)
        av.state[ST_RZ0] = rz;
        av.state[ST_BEST0] = INFINITY; av.state[ST_BEST1] = INFINITY;
        av.state[ST_BETA] = Real(0);
        a.istate[IS_DONE0] = a.maxiter <= 0; a.istate[IS_DONE1] = 0; a.istate[IS_K] = 0; a.istate[IS_CONV] = 0;
        a.istate[IS_BESTK] = 0;
        a.istate[IS_USEBEST] = 1;
    }
}

// Image-row copies of the pair blocks, column-major: entry q of image row i (pair p, flag tr) holds
// B = S(i, i2) with B[j][j2] at S_rows[q][j2 * d + j], so that the SpMV's lanes (one per output
// row j) read each column of a block contiguously.  S(i, i2) is S_p for tr = 0 and S_p^T for tr = 1.
// row_u[q][j2] = umap[i2][j2] (-1 past d, gw entries per block: 16 for d <= 16, else 32): the unknowns
// the block multiplies.  One wave per destination entry (its d^2 elements and gw unknowns over the
// lanes), so that the entry's indices are resolved once per wave.
template <typename Real>
__global__ void __launch_bounds__(PCG_T) k_rows_build(ba_pcg_args a, int64_t n_ent, int gw) {
    const PcgV<Real> av(a);
    const int d = a.d, dd = d * d;
    const int64_t q = (int64_t)blockIdx.x * (PCG_T / 64) + (threadIdx.x >> 6);      // destination block
    if (q >= n_ent) return;
    const int lane = threadIdx.x & 63;
    int64_t qs = q;                                    // its source entry of row_ent
    if (a.row_cap > 0) {                               // fixed capacity: row i at [i cap, (i + 1) cap)
        const int64_t i = q / a.row_cap, k = q - i * a.row_cap;
        qs = a.row_ptr[i] + k;
        if (qs >= a.row_ptr[i + 1]) {                  // past the row's end: a zero block, no unknowns
            for (int e = lane; e < dd; e += 64) av.S_rows[q * dd + e] = Real(0);
            if (lane < gw) a.row_u[q * gw + lane] = -1;
            return;
        }
    }
    const int ent = a.row_ent[qs];
    const int64_t p = ent >> 1;
    const Real* S = av.S_pairs + p * dd;
    for (int e = lane; e < dd; e += 64) {
        const int j2 = e / d, j = e - j2 * d;
        av.S_rows[q * dd + e] = (ent & 1) ? S[j2 * d + j] : S[j * d + j2];
    }
    if (lane < gw) {
        const int i2 = (ent & 1) ? a.pair_i1[p] : a.pair_i2[p];
        a.row_u[q * gw + lane] = lane < d ? a.umap[(int64_t)i2 * d + lane] : -1;
    }
}

// ----------------------------------------------------------------------------- one CG iteration
// Iteration n (n = 0 .. maxiter - 1; the reference numbers it n + 1, ba_solver.py:1216-1236) is two
// launches:
//   k_pcg_spmv(n)    the stopping decisions after update n - 1 (every block forms them from the same
//                    partial sums, so they agree without a grid barrier), the best-so-far copy, then
//                    y_img = S_img p_n with p_n formed on the fly from z and p_{n-1}, and per image
//                    row i a partial of p.Ap = sum_e p_u(e) y_e + sum_u damp_u p_u^2 (e over the
//                    image-level entries, u over the unknowns, the block of row i taking
//                    u = i, i + n_imgs, ...: A p = P^T y_img + damp p);
//   k_pcg_update(n)  alpha, A p of the block's unknowns (one thread per short inverse list, one
//                    wave per long one), x, r, z, the stored p_n, and the block partials of r.r
//                    and r.z.
// p is Real-buffered (p_n in slot n & 1).  A launch after the stopping point returns at once: the
// flag "stopped before update n" lives in IS_DONE0 + (n & 1) and is written by k_pcg_spmv(n - 1).

// y_img[i][j] = sum over the blocks of image row i of S(i, i2)[j, :] . p(i2): one workgroup of
// PCG_ST threads per image row; its PCG_ST / 16 lane groups (one lane per row j) take every
// (PCG_ST / 16)-th block of the row.  Lane j2 of a group forms p_n at the block's column unknown j2 and the group shares the
// 16 values by shuffles; the group sums are added in LDS in a fixed order.  The operands of the
// first pass, the row's own unknowns and the partial sums are requested before any of them is used.
template <int GW, typename Real>
__global__ void __launch_bounds__(PCG_ST) k_pcg_spmv(ba_pcg_args a, int n, int nb) {
    const PcgV<Real> av(a);
    __shared__ Real sh[PCG_ST];
    __shared__ Real sDamp[PCG_ST / 64];
    const int i = blockIdx.x;
    const int grp = threadIdx.x / GW, j = threadIdx.x % GW;
    const int d = a.d, dd = d * d;
    const Real* __restrict__ pold = av.p + (int64_t)((n + 1) & 1) * a.n_u;
    // operands that depend on nothing are requested first: each thread's first block partials of
    // update n - 1, the scalar state, and (threads 0..d-1) the row's own unknowns with z and p_{n-1}
    Real pr0 = Real(0), pr1 = Real(0);
    if (threadIdx.x < nb) { pr0 = av.partials[PCG_NP * threadIdx.x + PT_RR]; pr1 = av.partials[PCG_NP * threadIdx.x + PT_RZ]; }
    const Real best = av.state[ST_BEST0 + ((n - 1) & 1)], rz_old = av.state[ST_RZ0 + ((n - 1) & 1)];
    const Real bnorm = av.state[ST_BNORM];
    int uo = -1;
    Real zo = Real(0), po = Real(0);
    if (threadIdx.x < GW && j < d) {
        uo = a.umap[(int64_t)i * d + j];
        if (uo >= 0) { zo = av.z[uo]; po = pold[uo]; }
    }
    // the row's blocks: from the fixed capacity when set (no load on this chain), else from row_ptr
    const int q0 = a.row_cap > 0 ? i * a.row_cap : a.row_ptr[i];
    const int q1 = a.row_cap > 0 ? q0 + a.row_cap : a.row_ptr[i + 1];
    auto load = [&](int q, int& u, Real& zv, Real& pv, Real (&bcol)[GW]) {
        const bool live = q < q1;
        u = live ? a.row_u[(int64_t)q * GW + j] : -1;
        zv = Real(0); pv = Real(0);
        if (u >= 0) { zv = av.z[u]; pv = pold[u]; }
        const Real* B = av.S_rows + (int64_t)q * dd;
#pragma unroll
        for (int j2 = 0; j2 < GW; ++j2) bcol[j2] = (live && j < d && j2 < d) ? B[j2 * d + j] : Real(0);
    };
    auto mac = [&](int u, Real zv, Real pv, Real beta, const Real (&bcol)[GW], Real acc) {
        const Real xj = u >= 0 ? pdir(zv, pv, beta) : Real(0);
#pragma unroll
        for (int j2 = 0; j2 < GW; ++j2) acc += bcol[j2] * __shfl(xj, j2, GW);
        return acc;
    };
    int u;
    Real zv, pv, bcol[GW];
    load(q0 + grp, u, zv, pv, bcol);                 // requested before the done flag is known
    // damping term of the unknowns v = i + k n_imgs (thread k): its first operands are requested now
    const int64_t v0 = i + (int64_t)threadIdx.x * a.n_imgs;
    Real dz = Real(0), dpo = Real(0), dd0 = Real(0);
    if (v0 < a.n_u) { dz = av.z[v0]; dpo = pold[v0]; dd0 = av.damp[v0]; }
    if (a.istate[IS_DONE0 + (n & 1)]) {
        if (blockIdx.x == 0 && threadIdx.x == 0) a.istate[IS_DONE0 + ((n + 1) & 1)] = 1;
        return;
    }

    Real beta = Real(0);
    if (n >= 1) {
        // end of update n - 1 (ba_solver.py:1222-1236)
        Real rs[2] = {Real(0), Real(0)};
        if (threadIdx.x < nb) { rs[0] += pr0; rs[1] += pr1; }     // the order of sum_partials
        for (int b = threadIdx.x + PCG_ST; b < nb; b += PCG_ST) { rs[0] += av.partials[PCG_NP * b + PT_RR]; rs[1] += av.partials[PCG_NP * b + PT_RZ]; }
        block_sums<PCG_ST, 2>(rs, sh);
        const Real rr = rs[0], rz_new = rs[1];
        const Real rnorm = sqrt(rr);
        const bool improved = rnorm < best;
        const bool conv = rnorm <= Real(a.tol) * bnorm;
        const bool bad = !isfinite(rz_new);
        const bool stop = conv || bad || n >= a.maxiter;
        beta = rz_new / (rz_old > Real(1e-32) ? rz_old : Real(1e-32));
        if (improved)                                    // best_so_far = r_norm, x, k
            for (int64_t v = (int64_t)blockIdx.x * PCG_ST + threadIdx.x; v < a.n_u; v += (int64_t)gridDim.x * PCG_ST)
                av.xbest[v] = av.x[v];
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            av.state[ST_BEST0 + (n & 1)] = improved ? rnorm : best;
            if (improved) a.istate[IS_BESTK] = n;
            av.state[ST_RZ0 + (n & 1)] = rz_new;
            av.state[ST_BETA] = beta;
            a.istate[IS_K] = n;
            if (conv) { a.istate[IS_CONV] = 1; a.istate[IS_USEBEST] = 0; }
            a.istate[IS_DONE0 + ((n + 1) & 1)] = stop;
        }
        if (stop) return;
    } else if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.istate[IS_DONE0 + 1] = 0;
    }
    Real dsum = Real(0);
    {
        const Real pv0 = pdir(dz, dpo, beta);
        dsum = dd0 * pv0 * pv0;
        for (int64_t v = v0 + (int64_t)PCG_ST * a.n_imgs; v < a.n_u; v += (int64_t)PCG_ST * a.n_imgs) {
            const Real pv2 = pdir(av.z[v], pold[v], beta);
            dsum += av.damp[v] * pv2 * pv2;
        }
        dsum = wave_sum(dsum);
    }
    // the row's further blocks: each block's unknown index is requested one block ahead, so that its z,
    // p and values are requested together (the sum keeps the block order)
    auto index_of = [&](int q) { return q < q1 ? a.row_u[(int64_t)q * GW + j] : -1; };
    int un = index_of(q0 + PCG_ST / GW + grp);
    Real acc = mac(u, zv, pv, beta, bcol, Real(0));
    for (int qb = q0 + PCG_ST / GW; qb < q1; qb += PCG_ST / GW) {
        const int q = qb + grp;
        u = un;
        zv = Real(0); pv = Real(0);
        if (u >= 0) { zv = av.z[u]; pv = pold[u]; }
        const Real* B = av.S_rows + (int64_t)q * dd;
#pragma unroll
        for (int j2 = 0; j2 < GW; ++j2) bcol[j2] = (q < q1 && j < d && j2 < d) ? B[j2 * d + j] : Real(0);
        un = index_of(q + PCG_ST / GW);
        acc = mac(u, zv, pv, beta, bcol, acc);
    }
    __syncthreads();
    sh[threadIdx.x] = acc;
    if ((threadIdx.x & 63) == 0) sDamp[threadIdx.x >> 6] = dsum;
    __syncthreads();
    // y of this image row; the row's share of p.Ap: sum_e p_u(e) y_e over its entries (one wave,
    // 16 rows at most) plus the damping sum of its unknowns
    if (threadIdx.x < 64) {
        Real part = Real(0);
        if (j < d && threadIdx.x < GW) {
            Real t = Real(0);
            for (int g = 0; g < PCG_ST / GW; ++g) t += sh[GW * g + j];
            av.y_img[(int64_t)i * d + j] = t;
            if (uo >= 0) part = pdir(zo, po, beta) * t;
        }
        part = wave_sum(part);
        if (threadIdx.x == 0) {
            Real dt = Real(0);
#pragma unroll
            for (int w = 0; w < PCG_ST / 64; ++w) dt += sDamp[w];
            av.img_part[i] = part + dt;
        }
    }
}

// alpha = rz / max(p.Ap, 1e-32); x += alpha p; r -= alpha Ap; z = M^-1 r (ba_solver.py:1217-1228);
// p_n stored in slot n & 1; block partials r.r, r.z.  A p of
// unknown u is the sum of the image-level rows mapping to u plus damp[u] p_n[u]: one thread sums a
// list of at most BA_PCG_LONG_LIST entries; the block's long lists (a focal pair shared by every
// image of a camera) are summed first, one wave each, 8 entries per lane in flight, into LDS.
template <typename Real>
__global__ void __launch_bounds__(PCG_T) k_pcg_update(ba_pcg_args a, int n) {
    const PcgV<Real> av(a);
    __shared__ Real sh[2 * (PCG_T / 64)];
    __shared__ Real sLong[PCG_T];
    // requested first: the image partials of p.Ap (the first PCG_IPF of each thread) and the scalars
    Real ipf[PCG_IPF];
#pragma unroll
    for (int k = 0; k < PCG_IPF; ++k) {
        const int b = threadIdx.x + k * PCG_T;
        ipf[k] = b < a.n_imgs ? av.img_part[b] : Real(0);
    }
    const Real beta = av.state[ST_BETA], rz = av.state[ST_RZ0 + (n & 1)];
    if (a.istate[IS_DONE0 + ((n + 1) & 1)]) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x;
    const Real* __restrict__ pold = av.p + (int64_t)((n + 1) & 1) * a.n_u;
    Real zu = Real(0), pu = Real(0), xu = Real(0), ru = Real(0), du = Real(1), dmp = Real(0), y1 = Real(0);
    int q0 = 0, q1 = 0, li = -1, s1 = -1;
    if (u < a.n_u) {                                   // operands first, then the reductions
        zu = av.z[u]; pu = pold[u]; xu = av.x[u]; ru = av.r[u]; du = av.diagA[u]; dmp = av.damp[u];
        li = a.long_idx[u];
        if (a.src1 != nullptr) {                       // a one-entry list resolved ahead
            s1 = a.src1[u];
            if (s1 >= 0) y1 = av.y_img[s1];
        }
        if (s1 < 0) { q0 = a.inv_ptr[u]; q1 = a.inv_ptr[u + 1]; }
    }
    const int lk0 = a.long_ptr[blockIdx.x], lk1 = a.long_ptr[blockIdx.x + 1];
    for (int k = lk0 + w; k < lk1; k += PCG_T / 64) {
        int b0, b1;
        if (a.long_rng != nullptr) {
            b0 = a.long_rng[2 * k]; b1 = a.long_rng[2 * k + 1];
        } else {
            const int v = a.long_u[k];
            b0 = a.inv_ptr[v]; b1 = a.inv_ptr[v + 1];
        }
        Real s = Real(0);
        for (int q = b0 + lane; q < b1; q += 64 * PCG_LF) {
            int src[PCG_LF];
#pragma unroll
            for (int t = 0; t < PCG_LF; ++t) src[t] = q + 64 * t < b1 ? a.inv_src[q + 64 * t] : -1;
#pragma unroll
            for (int t = 0; t < PCG_LF; ++t) s += src[t] >= 0 ? av.y_img[src[t]] : Real(0);
        }
        s = wave_sum(s);
        if (lane == 0) sLong[k - lk0] = s;
    }
    // the short lists: y_img is complete at launch, so these sums need nothing from the reductions
    Real ys = Real(0);
    if (s1 >= 0)
        ys = Real(0) + y1;                                 // the same sum as the one-entry loop below
    else if (li < 0)
        for (int q = q0; q < q1; ++q) ys += av.y_img[a.inv_src[q]];
    Real sums[1] = {Real(0)};
#pragma unroll
    for (int k = 0; k < PCG_IPF; ++k)
        if (threadIdx.x + k * PCG_T < a.n_imgs) sums[0] += ipf[k];
    for (int b = threadIdx.x + PCG_IPF * PCG_T; b < a.n_imgs; b += PCG_T) sums[0] += av.img_part[b];
    block_sums<PCG_T, 1>(sums, sh);                    // p.Ap (its barriers also publish sLong)
    const Real pap = sums[0];
    const Real denom = pap > Real(1e-32) ? pap : Real(1e-32);
    const Real alpha = rz / denom;
    Real t[PCG_NP] = {Real(0), Real(0)};
    if (u < a.n_u) {
        const Real pn = pdir(zu, pu, beta);
        const Real apu = (li >= 0 ? sLong[li] : ys) + dmp * pn;
        av.p[(int64_t)(n & 1) * a.n_u + u] = pn;
        const Real x = xu + alpha * pn;
        const Real r = ru - alpha * apu;
        const Real z = r / du;
        av.x[u] = x; av.r[u] = r; av.z[u] = z;
        t[PT_RR] = r * r; t[PT_RZ] = r * z;
    }
    block_sums<PCG_T, PCG_NP>(t, sh);
    if (threadIdx.x < PCG_NP) av.partials[PCG_NP * blockIdx.x + threadIdx.x] = threadIdx.x == 0 ? t[0] : t[1];
}

// the flag "stopped before update n" (read once the launches before it have run) to memory the host reads
// (pinned host memory: a system-scope store)
__global__ void k_pcg_stopped(const int32_t* __restrict__ flag, int32_t* out) {
    if (threadIdx.x == 0) __hip_atomic_store(out, *flag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// result: x if converged else the best iterate
template <typename Real>
__global__ void __launch_bounds__(PCG_T) k_pcg_result(ba_pcg_args a) {
    const PcgV<Real> av(a);
    int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x;
    if (u < a.n_u && a.istate[IS_USEBEST]) av.x[u] = av.xbest[u];
}

}  // namespace ba

using namespace ba;

static inline unsigned nb_of(int64_t n) { return (unsigned)((n + PCG_T - 1) / PCG_T); }

// partial sums: PCG_NP per block of the update launch (one thread per unknown)
extern "C" int64_t ba_pcg_partials_size(int64_t n_u) {
    const int64_t m = n_u < 1 ? 1 : n_u;
    return PCG_NP * ((m + PCG_T - 1) / PCG_T);
}

namespace ba {
// The unknown-level rhs, damping and preconditioner diagonal (the first part of ba_pcg_solve), for
// the direct solve that shares them: rhs = P^T e_img, damp per leaf, diagA = clamp(P^T dg_img + damp).
int unknown_setup(const ba_pcg_args& a, hipStream_t st) {
    if (a.n_u == 0) return BA_OK;
    BA_REQUIRE(!a.real32, "the direct reduced solve runs in fp64 only (real32 = 0)");
    const unsigned nb = nb_of(a.n_u);
    const unsigned nbw = (unsigned)((a.n_u + PCG_T / 64 - 1) / (PCG_T / 64));
    hipLaunchKernelGGL(k_unk_setup<double>, dim3(nbw), dim3(PCG_T), 0, st, a);
    hipLaunchKernelGGL(k_leaf_max<double>, dim3(nb), dim3(PCG_T), 0, st, a);
    hipLaunchKernelGGL(k_leaf_damp<double>, dim3(nb), dim3(PCG_T), 0, st, a);
    BA_LAUNCHED();
    return BA_OK;
}
}  // namespace ba

// the launches of ba_pcg_solve_range in the working precision Real
template <typename Real>
static void pcg_launch(const ba_pcg_args& a, int32_t it0, int32_t it1, int32_t finish, int32_t* stopped_out,
                       int64_t n_ent, unsigned nb, unsigned nbw, hipStream_t st) {
    const int gw = a.d <= 16 ? 16 : 32;               // lanes per block row group of the SpMV (row_u stride)
    if (it0 == 0) {                                  // the setup precedes iteration 0
        if (n_ent > 0)
            hipLaunchKernelGGL(k_rows_build<Real>, dim3((unsigned)((n_ent + PCG_T / 64 - 1) / (PCG_T / 64))),
                               dim3(PCG_T), 0, st, a, n_ent, gw);
        hipLaunchKernelGGL(k_unk_setup<Real>, dim3(nbw), dim3(PCG_T), 0, st, a);
        hipLaunchKernelGGL(k_leaf_max<Real>, dim3(nb), dim3(PCG_T), 0, st, a);
        hipLaunchKernelGGL(k_leaf_damp<Real>, dim3(nb), dim3(PCG_T), 0, st, a);
        hipLaunchKernelGGL(k_pcg_init<Real>, dim3(nb), dim3(PCG_T), 0, st, a);
        hipLaunchKernelGGL(k_pcg_init2<Real>, dim3(1), dim3(PCG_T), 0, st, a, (int)nb);
    }
    auto spmv = [&](int it) {
        if (gw == 16)
            hipLaunchKernelGGL((k_pcg_spmv<16, Real>), dim3((unsigned)a.n_imgs), dim3(PCG_ST), 0, st, a, it, (int)nb);
        else
            hipLaunchKernelGGL((k_pcg_spmv<32, Real>), dim3((unsigned)a.n_imgs), dim3(PCG_ST), 0, st, a, it, (int)nb);
    };
    for (int it = it0; it < it1; ++it) {
        spmv(it);
        hipLaunchKernelGGL(k_pcg_update<Real>, dim3(nb), dim3(PCG_T), 0, st, a, it);
    }
    if (finish) {
        // the decisions after update it1 - 1 (after the last update, or a launch that returns at once once
        // the loop has stopped), then the result
        spmv(it1);
        hipLaunchKernelGGL(k_pcg_result<Real>, dim3(nb), dim3(PCG_T), 0, st, a);
    } else if (stopped_out != nullptr) {
        hipLaunchKernelGGL(k_pcg_stopped, dim3(1), dim3(64), 0, st, a.istate + IS_DONE0 + (it1 & 1), stopped_out);
    }
}

extern "C" int ba_pcg_solve_range(const ba_pcg_args* args, int32_t it0, int32_t it1, int32_t finish,
                                  int32_t* stopped_out, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_pcg_args& a = *args;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.n_u >= 0 && a.d >= 1 && a.d <= 32 && a.maxiter >= 0, "bad sizes (1 <= d <= 32)");
    BA_REQUIRE(a.n_long >= 0 && a.n_long <= a.n_u && a.long_ptr != nullptr && a.long_idx != nullptr &&
                   (a.n_long == 0 || a.long_u != nullptr) && a.img_part != nullptr,
               "bad long-list unknowns or image partials");
    BA_REQUIRE(0 <= it0 && it0 <= it1 && it1 <= a.maxiter, "iteration range outside [0, maxiter]");
    if (a.n_u == 0) return BA_OK;
    {
        const void* need[] = {a.umap, a.inv_ptr, a.inv_src, a.leaf, a.row_ptr, a.row_ent, a.pair_i1, a.pair_i2,
                              a.S_pairs, a.e_img, a.dg_img, a.rhs, a.diagA, a.damp, a.x, a.xbest, a.r, a.z, a.p,
                              a.y_img, a.partials, a.state, a.istate};
        for (const void* q : need) BA_REQUIRE(q != nullptr, "null pointer in ba_pcg_args");
    }
    const unsigned nb = nb_of(a.n_u);
    const unsigned nbw = (unsigned)((a.n_u + PCG_T / 64 - 1) / (PCG_T / 64));        // wave per unknown (setup)
    BA_REQUIRE(a.row_cap >= 0 && a.row_cap % (PCG_ST / 16) == 0, "row_cap must be a multiple of 8");
    const int64_t n_ent = a.row_cap > 0 ? (int64_t)a.n_imgs * a.row_cap : a.n_row_ent;
    BA_REQUIRE(n_ent >= 0 && a.S_rows != nullptr && a.row_u != nullptr, "image-row block workspace missing");
    if (a.real32) pcg_launch<float>(a, it0, it1, finish, stopped_out, n_ent, nb, nbw, st);
    else          pcg_launch<double>(a, it0, it1, finish, stopped_out, n_ent, nb, nbw, st);
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int ba_pcg_solve(const ba_pcg_args* args, void* stream) {
    return ba_pcg_solve_range(args, 0, args != nullptr ? args->maxiter : 0, 1, nullptr, stream);
}

// The device address of host memory that the device can reach (pinned, mapped), or NULL: the target that
// ba_pcg_solve_range's stopped_out needs, checked before any kernel is handed it.
extern "C" void* ba_host_mapped_ptr(const void* host_ptr) {
    if (host_ptr == nullptr) return nullptr;
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, host_ptr) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (at.type != hipMemoryTypeHost || at.devicePointer == nullptr) return nullptr;
    return at.devicePointer;
}
