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

enum { ST_BNORM = 0, ST_RZ0 = 1, ST_RZ1 = 2, ST_BEST0 = 3, ST_BEST1 = 4, ST_LEAF = 8 };
// istate: IS_DONE0 / IS_DONE1 done flags (double-buffered by iteration parity), IS_K iterations,
// IS_CONV converged, IS_BESTK best iterate, IS_USEBEST the best iterate is returned.
enum { IS_DONE0 = 0, IS_DONE1 = 1, IS_K = 2, IS_CONV = 3, IS_BESTK = 4, IS_USEBEST = 5 };

__device__ __forceinline__ double block_sum(double v, double* sh) {
    sh[threadIdx.x] = v;
    __syncthreads();
    for (int w = PCG_T / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
        __syncthreads();
    }
    double r = sh[0];
    __syncthreads();
    return r;
}

// Sum of n block partials at stride 3 (deterministic, identical in every block).
__device__ __forceinline__ double sum_partials(const double* __restrict__ part, int nb, int which, double* sh) {
    double v = 0.0;
    for (int b = threadIdx.x; b < nb; b += PCG_T) v += part[3 * b + which];
    return block_sum(v, sh);
}

// unknown-level rhs and diag(H_cc) from the image-level vectors; one wave per unknown so that
// shared unknowns (one focal pair for every image of a camera) reduce in parallel
__global__ void __launch_bounds__(PCG_T) k_unk_setup(ba_pcg_args a) {
    const int lane = threadIdx.x & 63;
    int64_t u = (int64_t)blockIdx.x * (PCG_T / 64) + (threadIdx.x >> 6);
    if (u >= a.n_u) return;
    double e = 0.0, g = 0.0;
    for (int q = a.inv_ptr[u] + lane; q < a.inv_ptr[u + 1]; q += 64) {
        int src = a.inv_src[q];
        e += a.e_img[src];
        g += a.dg_img[src];
    }
    for (int off = 32; off > 0; off >>= 1) {
        e += __shfl_down(e, off);
        g += __shfl_down(g, off);
    }
    if (lane == 0) { a.rhs[u] = e; a.diagA[u] = g; }
}

// per-leaf damping (BlockDiagMat.dampen_, ba_solver.py:575-582) and the Jacobi preconditioner.
// leaf ids 0..2 = foc, tau, zcf; 3..5 = the same groups switched off (a zero matrix damped by
// dampen * I, ZerosMat.dampen_, ba_solver.py:510-517).
__global__ void __launch_bounds__(PCG_T) k_leaf_damp(ba_pcg_args a) {
    __shared__ double sh[PCG_T];
    double m[3] = {0.0, 0.0, 0.0};
    for (int64_t u = threadIdx.x; u < a.n_u; u += PCG_T) {
        int l = a.leaf[u];
        if (l < 3) m[l] = fmax(m[l], fabs(a.diagA[u]));
    }
    double lam[6];
    for (int l = 0; l < 3; ++l) {
        sh[threadIdx.x] = m[l];
        __syncthreads();
        for (int w = PCG_T / 2; w > 0; w >>= 1) {
            if ((int)threadIdx.x < w) sh[threadIdx.x] = fmax(sh[threadIdx.x], sh[threadIdx.x + w]);
            __syncthreads();
        }
        lam[l] = a.adaptive ? a.dampen * sh[0] : a.dampen;
        lam[l + 3] = a.dampen;
        __syncthreads();
    }
    for (int64_t u = threadIdx.x; u < a.n_u; u += PCG_T) {
        double dmp = lam[a.leaf[u]];
        a.damp[u] = dmp;
        double dA = a.diagA[u] + dmp;
        a.diagA[u] = dA > 1e-12 ? dA : 1e-12;          // diagA.clamp(min=1e-12) (ba_solver.py:191-192)
    }
    if (threadIdx.x == 0) {
        for (int l = 0; l < 3; ++l) a.state[ST_LEAF + l] = lam[l];
    }
}

// x = 0, r = b, z = M^-1 r, p = z; partials of b.b and r.z
__global__ void __launch_bounds__(PCG_T) k_pcg_init(ba_pcg_args a) {
    __shared__ double sh[PCG_T];
    int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x;
    double bb = 0.0, rz = 0.0;
    if (u < a.n_u) {
        double b = a.rhs[u];
        double z = b / a.diagA[u];
        a.x[u] = 0.0; a.xbest[u] = 0.0; a.r[u] = b; a.z[u] = z; a.p[u] = z;
        bb = b * b; rz = b * z;
    }
    double s0 = block_sum(bb, sh), s1 = block_sum(rz, sh);
    if (threadIdx.x == 0) { a.partials[3 * blockIdx.x + 0] = s0; a.partials[3 * blockIdx.x + 1] = s1; }
}

__global__ void __launch_bounds__(PCG_T) k_pcg_init2(ba_pcg_args a, int nb) {
    __shared__ double sh[PCG_T];
    double bb = sum_partials(a.partials, nb, 0, sh);
    double rz = sum_partials(a.partials, nb, 1, sh);
    if (threadIdx.x == 0) {
        double bn = sqrt(bb);
        a.state[ST_BNORM] = bn > 1e-12 ? bn : 1e-12;    // torch.norm(b).clamp(min=1e-12)
        a.state[ST_RZ0] = rz;
        a.state[ST_BEST0] = INFINITY; a.state[ST_BEST1] = INFINITY;
        a.istate[IS_DONE0] = a.maxiter <= 0; a.istate[IS_DONE1] = 0; a.istate[IS_K] = 0; a.istate[IS_CONV] = 0;
        a.istate[IS_BESTK] = 0;
        a.istate[IS_USEBEST] = 1;
    }
}

// Image-row copies of the pair blocks, column-major: entry q of image row i (pair p, flag tr) holds
// B = S(i, i2) with B[j][j2] at S_rows[q][j2 * d + j], so that the SpMV's lanes (one per output
// row j) read each column of a block contiguously.  S(i, i2) is S_p for tr = 0 and S_p^T for tr = 1.
__global__ void __launch_bounds__(PCG_T) k_rows_build(ba_pcg_args a, int64_t n_ent) {
    const int d = a.d, dd = d * d;
    const int64_t tid = (int64_t)blockIdx.x * PCG_T + threadIdx.x;
    if (tid >= n_ent * dd) return;
    const int64_t q = tid / dd;
    const int e = (int)(tid - q * dd);
    const int j2 = e / d, j = e - (e / d) * d;
    const int ent = a.row_ent[q];
    const int64_t p = ent >> 1;
    const double* S = a.S_pairs + p * dd;
    a.S_rows[q * dd + e] = (ent & 1) ? S[j2 * d + j] : S[j * d + j2];
}

// ----------------------------------------------------------------------------- one CG iteration
// Four launches per iteration; a launch whose iteration is past the stopping point returns at
// once (the done flag of iteration k lives in IS_DONE0 + (k & 1), so the kernel that writes the
// flag for k + 1 never races with blocks of the same launch reading the flag for k).

// y_img[i][j] = sum over the blocks of image row i of S(i, i2)[j, :] . p(i2): one workgroup per
// image row; its 16 lane groups (one lane per output row j) take every 16th block of the row, and
// the group sums are added in LDS in a fixed order.  The 16 unknown indices of a block, then the 16
// values, are read as independent loads.
__global__ void __launch_bounds__(PCG_T) k_spmv_img(ba_pcg_args a, int k) {
    __shared__ double sh[PCG_T];
    if (a.istate[IS_DONE0 + (k & 1)]) return;
    const int i = blockIdx.x;
    const int grp = threadIdx.x >> 4, j = threadIdx.x & 15;
    const int d = a.d, dd = d * d;
    double acc = 0.0;
    if (j < d) {
        for (int q = a.row_ptr[i] + grp; q < a.row_ptr[i + 1]; q += PCG_T / 16) {
            const int ent = a.row_ent[q];
            const int pr = ent >> 1;
            const int i2 = (ent & 1) ? a.pair_i1[pr] : a.pair_i2[pr];
            const double* B = a.S_rows + (int64_t)q * dd;
            const int* um = a.umap + (int64_t)i2 * d;
            int u2[16];
#pragma unroll
            for (int j2 = 0; j2 < 16; ++j2) u2[j2] = j2 < d ? um[j2] : -1;
            double xv[16];
#pragma unroll
            for (int j2 = 0; j2 < 16; ++j2) xv[j2] = u2[j2] >= 0 ? a.p[u2[j2]] : 0.0;
#pragma unroll
            for (int j2 = 0; j2 < 16; ++j2)
                if (j2 < d) acc += B[j2 * d + j] * xv[j2];
        }
    }
    sh[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < 16 && j < d) {
        double t = 0.0;
        for (int g = 0; g < PCG_T / 16; ++g) t += sh[16 * g + j];
        a.y_img[(int64_t)i * d + j] = t;
    }
}

// Ap[u] = sum of the image-level rows mapping to u + damp[u] p[u] (one wave per unknown);
// per-block partial of p.Ap
__global__ void __launch_bounds__(PCG_T) k_spmv_unk(ba_pcg_args a, int k) {
    __shared__ double sh[PCG_T / 64];
    if (a.istate[IS_DONE0 + (k & 1)]) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int64_t u = (int64_t)blockIdx.x * (PCG_T / 64) + w;
    double s = 0.0;
    if (u < a.n_u) {
        // a shared unknown (one focal pair for every image of a camera) has a long list: its
        // entries are read 8 per lane at a time as independent loads
        const int q0 = a.inv_ptr[u], q1 = a.inv_ptr[u + 1];
        for (int q = q0 + lane; q < q1; q += 64 * 8) {
            int src[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) src[t] = q + 64 * t < q1 ? a.inv_src[q + 64 * t] : -1;
#pragma unroll
            for (int t = 0; t < 8; ++t) s += src[t] >= 0 ? a.y_img[src[t]] : 0.0;
        }
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off);
    double pap = 0.0;
    if (lane == 0 && u < a.n_u) {
        s += a.damp[u] * a.p[u];
        a.Ap[u] = s;
        pap = a.p[u] * s;
    }
    if (lane == 0) sh[w] = pap;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int q = 0; q < PCG_T / 64; ++q) t += sh[q];
        a.partials[3 * blockIdx.x + 2] = t;
    }
}

// alpha = rz / max(p.Ap, 1e-32); x += alpha p; r -= alpha Ap; z = M^-1 r; partials r.r, r.z
__global__ void __launch_bounds__(PCG_T) k_pcg_update(ba_pcg_args a, int nb, int nbw, int k) {
    __shared__ double sh[PCG_T];
    if (a.istate[IS_DONE0 + (k & 1)]) return;
    double pap = sum_partials(a.partials, nbw, 2, sh);
    double denom = pap > 1e-32 ? pap : 1e-32;
    double alpha = a.state[ST_RZ0 + (k & 1)] / denom;
    int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x;
    double rr = 0.0, rz = 0.0;
    if (u < a.n_u) {
        double x = a.x[u] + alpha * a.p[u];
        double r = a.r[u] - alpha * a.Ap[u];
        double z = r / a.diagA[u];
        a.x[u] = x; a.r[u] = r; a.z[u] = z;
        rr = r * r; rz = r * z;
    }
    __syncthreads();
    double s0 = block_sum(rr, sh), s1 = block_sum(rz, sh);
    if (threadIdx.x == 0) { a.partials[3 * blockIdx.x + 0] = s0; a.partials[3 * blockIdx.x + 1] = s1; }
}

// best-so-far bookkeeping, stopping test, beta and the new search direction
// (ba_solver.py:1222-1236); k counts from 0, the reference numbers the same iteration k + 1.
__global__ void __launch_bounds__(PCG_T) k_pcg_dir(ba_pcg_args a, int nb, int k) {
    __shared__ double sh[PCG_T];
    if (a.istate[IS_DONE0 + (k & 1)]) {
        if (blockIdx.x == 0 && threadIdx.x == 0) a.istate[IS_DONE0 + ((k + 1) & 1)] = 1;
        return;
    }
    double rr = sum_partials(a.partials, nb, 0, sh);
    double rz_new = sum_partials(a.partials, nb, 1, sh);
    double rnorm = sqrt(rr);
    double best = a.state[ST_BEST0 + (k & 1)];
    bool improved = rnorm < best;
    int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x;
    if (improved && u < a.n_u) a.xbest[u] = a.x[u];
    bool conv = rnorm <= a.tol * a.state[ST_BNORM];
    bool bad = !isfinite(rz_new);
    double rz_old = a.state[ST_RZ0 + (k & 1)];
    double beta = rz_new / (rz_old > 1e-32 ? rz_old : 1e-32);
    if (!conv && !bad && u < a.n_u) a.p[u] = a.z[u] + beta * a.p[u];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.state[ST_BEST0 + ((k + 1) & 1)] = improved ? rnorm : best;
        if (improved) a.istate[IS_BESTK] = k + 1;
        a.state[ST_RZ0 + ((k + 1) & 1)] = rz_new;
        a.istate[IS_K] = k + 1;
        int done = 0;
        if (conv) { done = 1; a.istate[IS_CONV] = 1; a.istate[IS_USEBEST] = 0; }
        else if (bad || k + 1 >= a.maxiter) { done = 1; }
        a.istate[IS_DONE0 + ((k + 1) & 1)] = done;
    }
}

// result: x if converged else the best iterate
__global__ void __launch_bounds__(PCG_T) k_pcg_result(ba_pcg_args a) {
    int64_t u = (int64_t)blockIdx.x * PCG_T + threadIdx.x;
    if (u < a.n_u && a.istate[IS_USEBEST]) a.x[u] = a.xbest[u];
}

}  // namespace ba

using namespace ba;

static inline unsigned nb_of(int64_t n) { return (unsigned)((n + PCG_T - 1) / PCG_T); }

// partial sums: 3 per block of the widest launch (one wave per unknown)
extern "C" int64_t ba_pcg_partials_size(int64_t n_u) { return 3 * (((n_u < 1 ? 1 : n_u) + 3) / 4) + 3; }

extern "C" int ba_pcg_solve(const ba_pcg_args* args, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_pcg_args& a = *args;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.n_u >= 0 && a.d >= 1 && a.d <= 16 && a.maxiter >= 0, "bad sizes");
    if (a.n_u == 0) return BA_OK;
    const unsigned nb = nb_of(a.n_u);
    const unsigned nbw = (unsigned)((a.n_u + PCG_T / 64 - 1) / (PCG_T / 64));        // wave per unknown
    const int64_t n_ent = a.n_row_ent;
    BA_REQUIRE(n_ent >= 0 && a.S_rows != nullptr, "image-row block workspace missing");
    if (n_ent > 0)
        hipLaunchKernelGGL(k_rows_build, dim3((unsigned)((n_ent * a.d * a.d + PCG_T - 1) / PCG_T)), dim3(PCG_T), 0, st, a,
                           n_ent);
    hipLaunchKernelGGL(k_unk_setup, dim3(nbw), dim3(PCG_T), 0, st, a);
    hipLaunchKernelGGL(k_leaf_damp, dim3(1), dim3(PCG_T), 0, st, a);
    hipLaunchKernelGGL(k_pcg_init, dim3(nb), dim3(PCG_T), 0, st, a);
    hipLaunchKernelGGL(k_pcg_init2, dim3(1), dim3(PCG_T), 0, st, a, (int)nb);
    BA_LAUNCHED();
    for (int it = 0; it < a.maxiter; ++it) {
        hipLaunchKernelGGL(k_spmv_img, dim3((unsigned)a.n_imgs), dim3(PCG_T), 0, st, a, it);
        hipLaunchKernelGGL(k_spmv_unk, dim3(nbw), dim3(PCG_T), 0, st, a, it);
        hipLaunchKernelGGL(k_pcg_update, dim3(nb), dim3(PCG_T), 0, st, a, (int)nb, (int)nbw, it);
        hipLaunchKernelGGL(k_pcg_dir, dim3(nb), dim3(PCG_T), 0, st, a, (int)nb, it);
    }
    hipLaunchKernelGGL(k_pcg_result, dim3(nb), dim3(PCG_T), 0, st, a);
    BA_LAUNCHED();
    return BA_OK;
}
