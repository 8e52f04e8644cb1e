// Direct solve of the reduced camera system (north-star stage 4: "the reduced-system Cholesky solve
// on the same GPU").  The reference's only definition of a direct reduced solve is
// GaussNewtonSolver._solve_dense_S (src/blast3r/inference/ba_solver.py:208-226): S = A - B D^-1 C,
// rhs = g_c - B D^-1 g_p, delta_c = torch.linalg.solve(S, rhs).  Here S_u = P^T S_img P + diag(damp)
// (the image-pair blocks of ba_linearize_schur mapped onto the reference's unknowns, with the per-leaf
// damping of ba_solver.py:575-582) is symmetric positive definite, so it is factored S_u = L L^T
// (fp64) and solved by two triangular sweeps; delta_c lands in the same x as the PCG's, so the
// back-substitution that follows is unchanged.
//
// Two layouts:
//   dense   S_u assembled as a full lower triangle (n_u padded to 128), factored by right-looking
//           128-column panels: the diagonal block's inverse in LDS (one workgroup, as the cyclic
//           reduction's super-blocks), the panel below as A_ik L_kk^-T and the trailing update
//           A_ij -= L_ik L_jk^T as 128 x 128 blocks of v_mfma_f64_16x16x4f64 tiles; the triangular
//           sweeps go block by block.  Any structure.
//   banded  the image-level blocks of a block-banded structure (every image pair within w images)
//           with the unknowns shared by several images (a mono camera's focal pair) as a dense
//           border.  When s >= w images fit a super-block of 128 unknowns, the super-blocks form a
//           block-tridiagonal system, solved by block cyclic reduction: each level eliminates every
//           other remaining super-block in parallel (a 128 x 128 L L^T and L^-1 per super-block in
//           LDS, then batched MFMA products for the neighbours' Schur updates), ~log2(n_imgs / s)
//           levels; the border enters as extra right-hand sides.  Otherwise one workgroup walks the
//           images, keeping the w + 1 active block rows in LDS, and runs both sweeps in the same
//           launch.  Work ~ n_imgs (w d)^2 d instead of n_u^3.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cmath>

#include "ba_common.h"
#include "ba_error.h"

namespace ba {
int unknown_setup(const ba_pcg_args& a, hipStream_t st);   // ba_pcg.hip

// ba_pcg_args with its working-precision arrays typed as fp64: the direct solve runs in fp64 only
// (ba_reduced_solve refuses real32), so its kernels read the fields through this same-layout view.
struct PcgArgs64 {
    int64_t n_u;
    int32_t n_imgs, d;
    const int32_t *umap, *inv_ptr, *inv_src, *leaf, *row_ptr, *row_ent, *pair_i1, *pair_i2;
    const double *S_pairs, *e_img, *dg_img;
    double dampen; int32_t adaptive;
    int32_t maxiter; double tol;
    double *rhs, *diagA, *damp, *x, *xbest, *r, *z, *p, *y_img, *partials, *state;
    int32_t* istate;
    double* S_rows;
    int64_t n_row_ent;
    int32_t* row_u;
    const int32_t* long_u;
    int64_t n_long;
    const int32_t *long_ptr, *long_idx;
    double* img_part;
    const int32_t *src1, *long_rng;
    int32_t row_cap;
    int32_t real32;
};
static_assert(sizeof(PcgArgs64) == sizeof(ba_pcg_args) && offsetof(PcgArgs64, real32) == offsetof(ba_pcg_args, real32) &&
                  offsetof(PcgArgs64, S_pairs) == offsetof(ba_pcg_args, S_pairs) &&
                  offsetof(PcgArgs64, img_part) == offsetof(ba_pcg_args, img_part) &&
                  offsetof(PcgArgs64, S_rows) == offsetof(ba_pcg_args, S_rows),
              "PcgArgs64 mirrors ba_pcg_args");

#define CH_T 256

typedef double dbl4 __attribute__((ext_vector_type(4)));

// ba_chol_args plus the banded layout's arrays, carved out of the caller's work buffer
struct ChArgs {
    int32_t mode;
    double* A;
    int64_t lda;
    double* Linv;
    const int32_t* pair_idx;
    const int32_t* kind;
    const int32_t* shared_u;
    int32_t n_shared;
    int32_t w;
    int32_t db;                 // banded: block size (the image-level columns that are local somewhere)
    const int32_t* bcol;        // banded: (db) image-level column of each band column
    const int32_t* bpos;        // banded: (d) band column of each image-level column, or -1
    int32_t* info;
    double *Ab, *Bfull, *Cb, *bl, *Lcol, *Lbord, *yv, *xl;
    // banded by block cyclic reduction: nsb super-blocks of s images (CR_MP unknowns each, padded)
    int32_t nsb, s;
    double *crD, *crE, *crR, *crL, *crGa, *crGb, *crY, *crX, *crXb;
    double* ss_part;            // (n_shared (n_shared + 1), 64) partial sums: the shared-shared entries, then
                                // the border products of the cyclic reduction
};

// ------------------------------------------------------------------ assembly
// Unknown classes (host-built from the inverse lists): kind 1 = local (exactly one image-level entry,
// e.g. a pose or z-coefficient), 2 = shared (several entries: a mono camera's focal pair, a rig node),
// 0 = isolated (none: a group switched off, a zero leaf damped by dampen * I).
//
// S_img(a, b) for image-level entries a = (i, r), b = (j, c): the pair block of images (i, j).
__device__ __forceinline__ double s_img(const PcgArgs64& a, const int32_t* __restrict__ pair_idx, int i, int r,
                                        int j, int c) {
    const int d = a.d;
    if (i <= j) {
        const int p = pair_idx[(int64_t)i * a.n_imgs + j];
        return p >= 0 ? a.S_pairs[((int64_t)p * d + r) * d + c] : 0.0;
    }
    const int p = pair_idx[(int64_t)j * a.n_imgs + i];
    return p >= 0 ? a.S_pairs[((int64_t)p * d + c) * d + r] : 0.0;
}

// dense: S_u[u][v] for v <= u where neither is shared (the identity on the padding rows n_u .. N, the
// damping alone on an isolated unknown), one thread per (u, v)
__global__ void __launch_bounds__(CH_T) k_dense_assemble(PcgArgs64 a, ChArgs c, int64_t N) {
    const int64_t u = blockIdx.y;
    const int64_t v = (int64_t)blockIdx.x * CH_T + threadIdx.x;
    if (v > u || u >= N) return;
    double val = 0.0;
    if (u < a.n_u && v < a.n_u) {
        const int ku = c.kind[u], kv = c.kind[v];
        if (ku == 2 || kv == 2) return;                 // k_shared_local / k_shared_part
        if (ku == 1 && kv == 1) {
            const int ea = a.inv_src[a.inv_ptr[u]], eb = a.inv_src[a.inv_ptr[v]];
            const int ia = ea / a.d, ib = eb / a.d;
            val = s_img(a, c.pair_idx, ia, ea - ia * a.d, ib, eb - ib * a.d);
        }
        if (u == v) val += a.damp[u];
    } else if (u == v) {
        val = 1.0;
    }
    c.A[u * c.lda + v] = val;
}

// S_u(s, v) for every shared s (blockIdx.y) and every local v (one wave each; lane l sums the pairs l, l + 64, ..
// of v's image row, the lanes are summed in a fixed tree): written to the dense matrix (mode 0) or to the
// border rows Bfull[s][entry of v] (mode 1)
__global__ void __launch_bounds__(CH_T) k_shared_local(PcgArgs64 a, ChArgs c, int mode) {
    const int lane = threadIdx.x & 63;
    const int64_t v = (int64_t)blockIdx.x * (CH_T / 64) + (threadIdx.x >> 6);
    const int sb = blockIdx.y;
    if (v >= a.n_u || c.kind[v] != 1) return;
    const int s = c.shared_u[sb];
    const int d = a.d;
    const int e = a.inv_src[a.inv_ptr[v]];
    const int j = e / d, cv = e - j * d;
    double val = 0.0;
    for (int q = a.row_ptr[j] + lane; q < a.row_ptr[j + 1]; q += 64) {
        const int ent = a.row_ent[q];
        const int p = ent >> 1, tr = ent & 1;
        const int i = tr ? a.pair_i1[p] : a.pair_i2[p];
        const double* S = a.S_pairs + (int64_t)p * d * d;
        for (int r = 0; r < d; ++r)
            if (a.umap[(int64_t)i * d + r] == s) val += tr ? S[r * d + cv] : S[cv * d + r];
    }
    for (int off = 32; off > 0; off >>= 1) val += __shfl_xor(val, off);
    if (lane != 0) return;
    if (mode == 0) {
        const int64_t r = s > v ? s : v, q = s > v ? v : s;
        c.A[r * c.lda + q] = val;
    } else {
        c.Bfull[(int64_t)sb * a.n_imgs * c.db + (int64_t)j * c.db + c.bpos[cv]] = val;
    }
}

// S_u(s1, s2) for shared s2 <= s1 (by list position): every pair block's entries that carry (s1, s2),
// summed by block (b1 n_s + b2, chunk) over a fixed slice of the image pairs (pair p goes to chunk
// (p / CH_T) mod SS_CHUNKS), then over the chunks in order by k_shared_sum, with the damping on the diagonal
#define SS_CHUNKS 64
__global__ void __launch_bounds__(CH_T) k_shared_part(PcgArgs64 a, ChArgs c, int64_t n_pairs) {
    __shared__ double sh[CH_T / 64];
    const int ns = c.n_shared;
    const int b1 = (int)blockIdx.x / ns, b2 = (int)blockIdx.x - b1 * ns;
    if (b2 > b1) return;
    const int s1 = c.shared_u[b1], s2 = c.shared_u[b2];
    const int d = a.d;
    double val = 0.0;
    for (int64_t p = (int64_t)blockIdx.y * CH_T + threadIdx.x; p < n_pairs; p += (int64_t)SS_CHUNKS * CH_T) {
        const int i1 = a.pair_i1[p], i2 = a.pair_i2[p];
        const double* S = a.S_pairs + p * d * d;
        for (int r = 0; r < d; ++r) {
            const int u1 = a.umap[(int64_t)i1 * d + r];
            if (u1 != s1 && u1 != s2) continue;
            for (int q = 0; q < d; ++q) {
                const int u2 = a.umap[(int64_t)i2 * d + q];
                if (u1 == s1 && u2 == s2) val += S[r * d + q];
                if (i1 != i2 && u2 == s1 && u1 == s2) val += S[r * d + q];
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) val += __shfl_xor(val, off);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = val;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < CH_T / 64; ++w) t += sh[w];
        c.ss_part[(int64_t)blockIdx.x * SS_CHUNKS + blockIdx.y] = t;
    }
}

// written to the dense matrix (mode 0) or to the corner Cb (mode 1)
__global__ void __launch_bounds__(CH_T) k_shared_sum(PcgArgs64 a, ChArgs c, int mode) {
    const int ns = c.n_shared;
    const int e = (int)(blockIdx.x * CH_T + threadIdx.x);
    if (e >= ns * ns) return;
    const int b1 = e / ns, b2 = e - b1 * ns;
    if (b2 > b1) return;
    double t = 0.0;
    for (int k = 0; k < SS_CHUNKS; ++k) t += c.ss_part[(int64_t)e * SS_CHUNKS + k];
    const int s1 = c.shared_u[b1], s2 = c.shared_u[b2];
    if (s1 == s2) t += a.damp[s1];
    if (mode == 0) {
        const int64_t r = s1 > s2 ? s1 : s2, q = s1 > s2 ? s2 : s1;
        c.A[r * c.lda + q] = t;
    } else {
        c.Cb[b1 * ns + b2] = t;
        c.Cb[b2 * ns + b1] = t;
    }
}

__global__ void __launch_bounds__(CH_T) k_copy_pad(const double* __restrict__ src, int64_t n, int64_t N,
                                                   double* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * CH_T + threadIdx.x;
    if (i < N) dst[i] = i < n ? src[i] : 0.0;
}

// unknowns that no image-level entry carries (a parameter group switched off: a zero leaf damped by
// dampen * I, ba_solver.py:510-517) are decoupled: x_u = rhs_u / damp_u (the rhs is zero there)
__global__ void __launch_bounds__(CH_T) k_isolated(PcgArgs64 a, const double* __restrict__ xs) {
    const int64_t u = (int64_t)blockIdx.x * CH_T + threadIdx.x;
    if (u >= a.n_u) return;
    a.x[u] = a.inv_ptr[u + 1] > a.inv_ptr[u] ? xs[u] : a.rhs[u] / a.damp[u];
}

__global__ void k_chol_status(PcgArgs64 a, const int32_t* __restrict__ info) {
    if (threadIdx.x == 0 && a.istate) {
        a.istate[0] = 1; a.istate[1] = 1;
        a.istate[2] = 0;                     // no iterations
        a.istate[3] = info[0] == 0x7fffffff; // "converged": the factorisation found every pivot positive
        a.istate[4] = 0; a.istate[5] = 0;
    }
}

__global__ void k_info_init(int32_t* info) {
    if (threadIdx.x == 0) info[0] = 0x7fffffff;
}


// ------------------------------------------------------------------ banded layout
// Unknown order of the banded factor: the local unknowns image by image (entry (i, c) at i d + c;
// an entry that is inactive or carries a shared unknown is an identity row there), then the n_s
// shared unknowns (the border).  Every image pair (i, j) of the structure has |i - j| <= w, so the
// factor of the local part is block-banded with w sub-diagonal blocks.
#define CB_T 512
#define CB_MAXD 16
#define CB_MAXM 160
#define CB_MAXS 8
#define CB_PF 5                 // new-row entries per thread: (16 x 160) / 512
#define CB_NX 6                 // staged backward entries per thread: (160 + 8) x 16 / 512
#define CB_PK(r, c) ((r) * ((r) + 1) / 2 + (c))

// Ab[i][k] (db x db) = the local block of S_u at images (i, i - k), k = 0..w (zero for i - k < 0), in
// band columns (the image-level columns that carry a local unknown in some image: a mono camera's focal
// columns, shared by every image, are left out), the damping on a local diagonal entry, 1 on a
// non-local one; bl[i db + r] = the local rhs entries; the border rows Bfull cleared.
__global__ void __launch_bounds__(CH_T) k_band_assemble(PcgArgs64 a, ChArgs c) {
    const int d = a.d, db = c.db, w1 = c.w + 1;
    const int64_t e = (int64_t)blockIdx.x * CH_T + threadIdx.x;
    const int64_t per = (int64_t)w1 * db * db;
    if (e >= (int64_t)a.n_imgs * per) return;
    const int i = (int)(e / per);
    int rem = (int)(e - (int64_t)i * per);
    const int k = rem / (db * db);
    rem -= k * db * db;
    const int r = rem / db, q = rem - r * db;
    const int j = i - k;
    const int cr = c.bcol[r], cq = c.bcol[q];
    double val = 0.0;
    const int ua = a.umap[(int64_t)i * d + cr];
    const bool la = ua >= 0 && c.kind[ua] == 1;
    if (j >= 0) {
        const int ub = a.umap[(int64_t)j * d + cq];
        const bool lb = ub >= 0 && c.kind[ub] == 1;
        if (la && lb) val = s_img(a, c.pair_idx, i, cr, j, cq);
        if (k == 0 && r == q) val = la ? val + a.damp[ua] : 1.0;
    }
    c.Ab[e] = val;
    if (k == 0 && q == 0) {
        c.bl[(int64_t)i * db + r] = la ? a.rhs[ua] : 0.0;
        // border couplings: k_shared_local (launched next) writes those of the local entries; the
        // other entries are identity rows, uncoupled
        for (int b = 0; b < c.n_shared; ++b) c.Bfull[(int64_t)b * a.n_imgs * db + (int64_t)i * db + r] = 0.0;
    }
}

// LDS of k_band_solve (dynamic): two packed lower triangles of the window (M (M + 1) / 2 doubles
// each), two copies of the border rows (n_s x M), the corner (n_s^2), two copies of the rhs window (M),
// the border rhs (n_s), the diagonal block's y / reciprocal pivots (2 x 16) and x_b (n_s).
__host__ __device__ inline int64_t band_lds_doubles(int M, int ns) {
    return (int64_t)M * (M + 1) + 2 * (int64_t)ns * M + (int64_t)ns * ns + 2 * M + ns + 2 * CB_MAXD + ns;
}

// One workgroup factors the banded system and runs both triangular sweeps.  LDS holds the active
// window: block rows i .. i + w of the local part as a packed lower triangle (M = (w + 1) d rows), the
// border rows restricted to those columns, the corner and the rhs window, in two copies: each step
// reads one and writes the next, so the window moves down an image as a side effect of its update.
// Per image i:
//   1. wave 0 factors the diagonal block in registers (lane r holds row r; the columns' values move by
//      lane shuffles), keeps the reciprocal pivots, and forms y_i = L_ii^-1 b_i (the forward sweep
//      rides along);
//   2. one thread per panel row (and per border row) solves its row against L_ii^T, stores it to the
//      factor, and subtracts its share of y_i from the rhs window;
//   3. the trailing window takes - P P^T as 16 x 16 tiles of v_mfma_f64_16x16x4f64 (K = d padded to a
//      multiple of 4), written one image up into the other copy; the border rows and the corner
//      their own products; the next image's block row, border columns and rhs (prefetched into
//      registers at the start of the step) fill the last rows of the other copy.
// Then thread 0 factors the corner, and the backward sweep walks the images in reverse, reading each
// column panel of L (prefetched one step ahead) against the solved x of the following images.
__global__ void __launch_bounds__(CB_T) k_band_solve(PcgArgs64 a, ChArgs c) {
    extern __shared__ double lds[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int d = c.db, w1 = c.w + 1, M = w1 * d, Md = M - d, ns = c.n_shared, n_imgs = a.n_imgs;
    const int64_t nl = (int64_t)n_imgs * d;
    const int PK = M * (M + 1) / 2;
    double* Wbuf[2] = {lds, lds + PK};
    double* Bbuf[2] = {lds + 2 * PK, lds + 2 * PK + ns * M};
    double* Cw = lds + 2 * PK + 2 * ns * M;
    double* bwbuf[2] = {Cw + ns * ns, Cw + ns * ns + M};
    double* bw = bwbuf[0];
    double* bb = bwbuf[1] + M;
    double* yd = bb + ns;
    double* rp = yd + CB_MAXD;
    double* xb = rp + CB_MAXD;
    // block (image ir, image ic) entry (r, q) of the local part, identity past the last image
    auto band_at = [&](int ir, int ic, int r, int q) -> double {
        if (ir >= n_imgs) return (ir == ic && r == q) ? 1.0 : 0.0;
        return c.Ab[(((int64_t)ir * w1 + (ir - ic)) * d + r) * d + q];
    };
    auto row_of = [&](int e) -> int {          // the packed row of index e
        int r = (int)((sqrt(8.0 * e + 1.0) - 1.0) * 0.5);
        while (CB_PK(r + 1, 0) <= e) ++r;
        while (CB_PK(r, 0) > e) --r;
        return r;
    };
    // ---- initial window: images 0 .. w
    for (int e = t; e < PK; e += CB_T) {
        const int r = row_of(e), q = e - CB_PK(r, 0);
        Wbuf[0][e] = band_at(r / d, q / d, r % d, q % d);
    }
    for (int e = t; e < ns * M; e += CB_T) {
        const int bq = e % M;
        Bbuf[0][e] = bq < nl ? c.Bfull[(int64_t)(e / M) * nl + bq] : 0.0;
    }
    for (int e = t; e < ns * ns; e += CB_T) Cw[e] = c.Cb[e];
    for (int e = t; e < M; e += CB_T) bw[e] = e < nl ? c.bl[e] : 0.0;
    if (t < ns) bb[t] = a.rhs[c.shared_u[t]];
    // this thread's entries of the window's last block row (new rows Md .. M - 1, packed order)
    const int n_new = PK - CB_PK(Md, 0);
    int nr_r[CB_PF], nr_q[CB_PF];
#pragma unroll
    for (int k = 0; k < CB_PF; ++k) {
        const int e = t + k * CB_T;
        nr_r[k] = -1; nr_q[k] = 0;
        if (e < n_new) {
            const int g = CB_PK(Md, 0) + e;
            nr_r[k] = row_of(g);
            nr_q[k] = g - CB_PK(nr_r[k], 0);
        }
    }
    // this wave's tiles of the trailing window
    const int n16 = (Md + 15) >> 4, ntile = n16 * (n16 + 1) / 2, nk = (d + 3) >> 2;
    const int l16 = lane & 15, lk = lane >> 4;
    __syncthreads();
    for (int i = 0; i < n_imgs; ++i) {
        double* W = Wbuf[i & 1];
        double* Wn = Wbuf[(i + 1) & 1];
        double* Bw = Bbuf[i & 1];
        double* Bn = Bbuf[(i + 1) & 1];
        bw = bwbuf[i & 1];
        double* bwn = bwbuf[(i + 1) & 1];
        // prefetch the block row of image i + w + 1 (the last rows of the next window)
        const int inew = i + w1;
        double pf[CB_PF], pfb = 0.0, pfr = 0.0;
#pragma unroll
        for (int k = 0; k < CB_PF; ++k)
            pf[k] = nr_r[k] >= 0 ? band_at(inew, i + 1 + nr_q[k] / d, nr_r[k] - Md, nr_q[k] % d) : 0.0;
        if (t < ns * d) {
            const int q = t % d;
            pfb = (int64_t)inew * d + q < nl ? c.Bfull[(int64_t)(t / d) * nl + (int64_t)inew * d + q] : 0.0;
        }
        if (t < d) pfr = (int64_t)inew * d + t < nl ? c.bl[(int64_t)inew * d + t] : 0.0;

        // 1. diagonal block (wave 0): L_ii in registers, reciprocal pivots, y_i = L_ii^-1 b_i
        if (wave == 0) {
            double row[CB_MAXD];
#pragma unroll
            for (int q = 0; q < CB_MAXD; ++q) row[q] = (lane < d && q <= lane) ? W[CB_PK(lane, q)] : 0.0;
            double rinv = 0.0;
#pragma unroll
            for (int j = 0; j < CB_MAXD; ++j) {
                if (j < d) {
                    double pj = __shfl(row[j], j);
                    if (!(pj > 0.0)) {
                        if (lane == 0) atomicMin(c.info, (int32_t)((int64_t)i * d + j + 1));
                        pj = 1.0;
                    }
                    const double ljj = sqrt(pj), rj = 1.0 / ljj;
                    if (lane == j) { row[j] = ljj; rinv = rj; }
                    else if (lane > j) row[j] = row[j] * rj;
                    const double lj = row[j];
#pragma unroll
                    for (int q = j + 1; q < CB_MAXD; ++q) {
                        const double lqj = __shfl(lj, q);
                        if (q < d && lane >= q && lane < d) row[q] -= lj * lqj;
                    }
                }
            }
            double acc = lane < d ? bw[lane] : 0.0, y = 0.0;
#pragma unroll
            for (int m = 0; m < CB_MAXD; ++m) {
                if (m < d) {
                    if (lane == m) y = acc * rinv;
                    const double ym = __shfl(y, m);
                    if (lane > m) acc -= row[m] * ym;
                }
            }
            if (lane < d) {
                double* Lc = c.Lcol + ((int64_t)i * M + lane) * d;
#pragma unroll
                for (int q = 0; q < CB_MAXD; ++q)
                    if (q < d) Lc[q] = q <= lane ? row[q] : 0.0;
                rp[lane] = rinv;
                yd[lane] = y;
                c.yv[(int64_t)i * d + lane] = y;
            }
            // L_ii for the panel rows of step 2 (read from W: rows 0..d-1 are not read by anything else)
            if (lane < d) {
#pragma unroll
                for (int q = 0; q < CB_MAXD; ++q)
                    if (q <= lane) W[CB_PK(lane, q)] = row[q];
            }
        }
        __syncthreads();
        // 2. panel rows and border rows against L_ii^T; their share of y_i leaves the rhs window
        if (t < Md + ns) {
            const bool pr = t < Md;
            const int r = d + t, b = t - Md;
            double x[CB_MAXD];
            double dot = 0.0;
#pragma unroll
            for (int q = 0; q < CB_MAXD; ++q) {
                x[q] = 0.0;
                if (q < d) {
                    double v = pr ? W[CB_PK(r, q)] : Bw[b * M + q];
#pragma unroll
                    for (int m = 0; m < CB_MAXD; ++m)
                        if (m < q) v -= x[m] * W[CB_PK(q, m)];
                    x[q] = v * rp[q];
                    dot += x[q] * yd[q];
                }
            }
            double* dst = pr ? c.Lcol + ((int64_t)i * M + r) * d : c.Lbord + ((int64_t)i * ns + b) * d;
            double* wrow = pr ? W + CB_PK(r, 0) : Bw + b * M;
#pragma unroll
            for (int q = 0; q < CB_MAXD; ++q)
                if (q < d) { wrow[q] = x[q]; dst[q] = x[q]; }
            if (pr) bw[r] -= dot;
            else bb[b] -= dot;
        }
        __syncthreads();
        // 3. next window = trailing window - P P^T (one image up), border rows and corner, new last rows
        for (int tile = wave; tile < ntile; tile += CB_T / 64) {
            int ti = (int)((sqrt(8.0 * tile + 1.0) - 1.0) * 0.5);
            while ((ti + 1) * (ti + 2) / 2 <= tile) ++ti;
            while (ti * (ti + 1) / 2 > tile) --ti;
            const int tj = tile - ti * (ti + 1) / 2;
            const int ra = 16 * ti + l16, rb = 16 * tj + l16;
            dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
            for (int kk = 0; kk < nk; ++kk) {
                const int k = 4 * kk + lk;
                const double av = (ra < Md && k < d) ? W[CB_PK(d + ra, k)] : 0.0;
                const double bv = (rb < Md && k < d) ? W[CB_PK(d + rb, k)] : 0.0;
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = 16 * ti + 4 * v + lk, q = 16 * tj + l16;
                if (r < Md && q <= r) Wn[CB_PK(r, q)] = W[CB_PK(d + r, d + q)] - acc[v];
            }
        }
        for (int e = t; e < ns * Md + ns * ns; e += CB_T) {
            if (e < ns * Md) {
                const int b = e / Md, q = e - b * Md;
                double sum = 0.0;
                for (int m = 0; m < d; ++m) sum += Bw[b * M + m] * W[CB_PK(d + q, m)];
                Bn[b * M + q] = Bw[b * M + d + q] - sum;
            } else {
                const int f = e - ns * Md, b1 = f / ns, b2 = f - b1 * ns;
                double sum = 0.0;
                for (int m = 0; m < d; ++m) sum += Bw[b1 * M + m] * Bw[b2 * M + m];
                Cw[f] -= sum;
            }
        }
#pragma unroll
        for (int k = 0; k < CB_PF; ++k)
            if (nr_r[k] >= 0) Wn[CB_PK(nr_r[k], nr_q[k])] = pf[k];
        if (t < ns * d) Bn[(t / d) * M + Md + t % d] = pfb;
        // the rhs window moves down one image (its entries d.. took this step's share in step 2)
        if (t < Md) bwn[t] = bw[t + d];
        if (t < d) bwn[Md + t] = pfr;
        __syncthreads();
    }
    bw = bwbuf[n_imgs & 1];
    // ---- border: factor the corner in place, finish the forward sweep, start the backward one
    if (t == 0) {
        for (int r = 0; r < ns; ++r)
            for (int q = 0; q <= r; ++q) {
                double v = Cw[r * ns + q];
                for (int m = 0; m < q; ++m) v -= Cw[r * ns + m] * Cw[q * ns + m];
                if (r == q) {
                    if (!(v > 0.0)) {
                        atomicMin(c.info, (int32_t)(nl + r + 1));
                        v = 1.0;
                    }
                    Cw[r * ns + r] = sqrt(v);
                } else {
                    Cw[r * ns + q] = v / Cw[q * ns + q];
                }
            }
        for (int r = 0; r < ns; ++r) {
            double v = bb[r];
            for (int m = 0; m < r; ++m) v -= Cw[r * ns + m] * bb[m];
            bb[r] = v / Cw[r * ns + r];
        }
        for (int r = ns - 1; r >= 0; --r) {
            double v = bb[r];
            for (int m = r + 1; m < ns; ++m) v -= Cw[m * ns + r] * xb[m];
            xb[r] = v / Cw[r * ns + r];
        }
        for (int r = 0; r < ns; ++r) a.x[c.shared_u[r]] = xb[r];
    }
    // backward sweep: x_i = L_ii^-T (y_i - sum_r L(r, i)^T x_r - L_b,i^T x_b).  xw holds x of the
    // window's images circularly (image j at slot j mod (w + 1)); images past the last one stay zero
    // (their panel rows of L are zero anyway).  The column panel of L (M x d) and the border rows
    // (n_s x d) of image i are staged in LDS (two slots over the free window buffers, w >= 1), the
    // next image's loaded into registers while this one is used.  Wave g forms the dots of columns g and
    // g + 8; wave 0 holds column q of L_ii in lane q, so the back substitution only broadcasts x_m.
    double* xw = bw;                          // the rhs window is free now
    const int slot_sz = M * d + ns * d, n_sl = (slot_sz + CB_T - 1) / CB_T;
    double* Lp[2] = {lds, lds + slot_sz};     // over the window buffers (2 slot_sz <= M (M + 1) + 2 ns M)
    __syncthreads();
    if (t < M) xw[t] = 0.0;
    auto stage_val = [&](int i, int e) -> double {
        if (e < M * d) return c.Lcol[(int64_t)i * M * d + e];
        return c.Lbord[(int64_t)i * ns * d + (e - M * d)];
    };
    for (int e = t; e < slot_sz; e += CB_T) Lp[(n_imgs - 1) & 1][e] = stage_val(n_imgs - 1, e);
    __syncthreads();
    const int g = t >> 6;                     // column group: columns g, g + 8
    int rq[3], rm[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int r = d + lane + 64 * k;
        rq[k] = r / d;
        rm[k] = r - rq[k] * d;
    }
    for (int i = n_imgs - 1; i >= 0; --i) {
        double nx[CB_NX];
#pragma unroll
        for (int k = 0; k < CB_NX; ++k) {
            const int e = t + k * CB_T;
            nx[k] = (i >= 1 && k < n_sl && e < slot_sz) ? stage_val(i - 1, e) : 0.0;
        }
        const double* P = Lp[i & 1];
        // columns g and g + 8 of this image's panel against the solved x of the following images
#pragma unroll
        for (int h = 0; h < CB_MAXD; h += CB_T / 64) {
            const int col = g + h;
            double sum = 0.0;
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                const int r = d + lane + 64 * k;
                if (col < d && r < M) sum += P[r * d + col] * xw[((i + rq[k]) % w1) * d + rm[k]];
            }
            if (col < d && lane < ns) sum += P[M * d + lane * d + col] * xb[lane];
            for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
            if (col < d && lane == 0) yd[col] = c.yv[(int64_t)i * d + col] - sum;
        }
        __syncthreads();
        if (wave == 0) {
            double lc[CB_MAXD];
#pragma unroll
            for (int m = 0; m < CB_MAXD; ++m) lc[m] = (lane < d && m < d && m >= lane) ? P[m * d + lane] : 0.0;
            double acc = lane < d ? yd[lane] : 0.0, xv = 0.0;
#pragma unroll
            for (int m = CB_MAXD - 1; m >= 0; --m) {
                if (m < d) {
                    if (lane == m) xv = acc / lc[m];
                    const double xm = __shfl(xv, m);
                    if (lane < m) acc -= lc[m] * xm;
                }
            }
            if (lane < d) {
                xw[(i % w1) * d + lane] = xv;
                c.xl[(int64_t)i * d + lane] = xv;
            }
        }
#pragma unroll
        for (int k = 0; k < CB_NX; ++k) {
            const int e = t + k * CB_T;
            if (i >= 1 && k < n_sl && e < slot_sz) Lp[(i - 1) & 1][e] = nx[k];
        }
        __syncthreads();
    }
}

// x of the local unknowns from the banded solution (shared ones were written by k_band_solve);
// isolated unknowns: rhs / damp
__global__ void __launch_bounds__(CH_T) k_band_scatter(PcgArgs64 a, ChArgs c) {
    const int64_t u = (int64_t)blockIdx.x * CH_T + threadIdx.x;
    if (u >= a.n_u) return;
    const int k = c.kind[u];
    if (k == 1) {
        const int e = a.inv_src[a.inv_ptr[u]], i = e / a.d;
        a.x[u] = c.xl[(int64_t)i * c.db + c.bpos[e - i * a.d]];
    }
    else if (k == 0) a.x[u] = a.rhs[u] / a.damp[u];
}

// ------------------------------------------------------------------ banded layout, block cyclic reduction
// Super-block I holds the local unknowns of images I s .. I s + s - 1 (entry (i, r) at (i - I s) db + r),
// padded to CR_MP with identity rows; images past the last one are identity rows too.  Since s >= w, only
// neighbouring super-blocks couple: S = tridiag(E_I (block (I, I - 1)), D_I, E_{I+1}^T).
//
// Level h = 1, 2, 4, ...: the remaining super-blocks are I = h - 1 (mod h); those at I = h - 1 (mod 2h)
// are eliminated, each against its remaining neighbours a = I - h and b = I + h (when they exist):
//   D_I = L L^T,  Ga = L^-1 E_I,  Gb = L^-1 E_b^T,  Y_I = L^-1 R_I
//   D_a -= Ga^T Ga,  D_b -= Gb^T Gb,  E_b <- -Gb^T Ga (b now couples to a),  R_a -= Ga^T Y_I,  R_b -= Gb^T Y_I
// and, levels in reverse, X_I = L^-T (Y_I - Ga X_a - Gb X_b).  This is L L^T of S in the odd-even
// order of the super-blocks, so it is as stable as the sequential factor.  R carries CR_NR right-hand
// sides: the local rhs, then the border columns (the couplings of the n_s shared unknowns), so that
// X = S_loc^-1 [b | B] and the border is solved from its n_s x n_s Schur complement.
#define CR_MP 128                       // unknowns per super-block
#define CR_MP2 (CR_MP * CR_MP)
#define CR_NR 16                        // right-hand sides per super-block (n_s <= 15)
#define CR_T 512                        // threads of the super-block factor
#define CR_LD (CR_MP + 1)               // LDS row pitch of the factor
#define CR_LDS_DOUBLES (CR_MP * CR_LD + 8 * 256 + 16)

// images per super-block, or 0 when the cyclic reduction does not apply (a super-block of s >= w images
// must fit CR_MP unknowns, the border CR_NR - 1 columns)
__host__ __device__ inline int cr_images(int db, int w, int ns) {
    if (db < 1 || w < 1 || ns < 0 || ns > CR_NR - 1 || w * db > CR_MP) return 0;
    const int s = CR_MP / db;
    return s > w ? s : w;
}

__global__ void __launch_bounds__(CH_T) k_cr_assemble(PcgArgs64 a, ChArgs c) {
    const int64_t e = (int64_t)blockIdx.x * CH_T + threadIdx.x;
    if (e >= (int64_t)c.nsb * CR_MP2) return;
    const int I = (int)(e / CR_MP2);
    const int rem = (int)(e - (int64_t)I * CR_MP2);
    const int u = rem / CR_MP, v = rem - u * CR_MP;
    const int db = c.db, w = c.w, w1 = c.w + 1, n = a.n_imgs, m = c.s * db;
    const int iu = I * c.s + u / db, ru = u % db;
    auto band = [&](int i, int k, int r, int q) { return c.Ab[(((int64_t)i * w1 + k) * db + r) * db + q]; };
    double dv = u == v ? 1.0 : 0.0;       // padding and images past the last one: identity
    if (u < m && v < m && iu < n) {
        const int iv = I * c.s + v / db, rv = v % db;
        if (iv < n) {
            dv = 0.0;
            if (iu >= iv) {
                if (iu - iv <= w) dv = band(iu, iu - iv, ru, rv);
            } else if (iv - iu <= w) {
                dv = band(iv, iv - iu, rv, ru);
            }
        }
    }
    c.crD[e] = dv;
    double ev = 0.0;                      // block (I, I - 1)
    if (I >= 1 && u < m && v < m && iu < n) {
        const int iv = (I - 1) * c.s + v / db, k = iu - iv;
        if (k <= w) ev = band(iu, k, ru, v % db);
    }
    c.crE[e] = ev;
    if (v < CR_NR) {
        double rv = 0.0;
        if (u < m && iu < n) {
            if (v == 0) rv = c.bl[(int64_t)iu * db + ru];
            else if (v <= c.n_shared) rv = c.Bfull[(int64_t)(v - 1) * n * db + (int64_t)iu * db + ru];
        }
        c.crR[((int64_t)I * CR_MP + u) * CR_NR + v] = rv;
    }
}

// acc += A B over k in [kb, ke) (multiples of 16) for one 16 x 16 tile of a wave: fa(r, k) = A[r][k],
// fb(k, c) = B[k][c] relative to the tile's corner (v_mfma_f64_16x16x4f64 operand lane l: row / column
// l % 16, k = l / 16; accumulator element v of lane l: row 4 v + l / 16, column l % 16).  The operands of
// 16 k are loaded before their MFMAs.
template <class FA, class FB>
__device__ __forceinline__ void cr_mma(dbl4& acc, int kb, int ke, FA fa, FB fb, int l16, int lk) {
    for (int k = kb; k < ke; k += 16) {
        double av[4], bv[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            av[kk] = fa(l16, k + 4 * kk + lk);
            bv[kk] = fb(k + 4 * kk + lk, l16);
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av[kk], bv[kk], acc, 0, 0, 0);
    }
}

// sum over the 64 lanes of a wave (butterfly; every lane gets the same bits)
__device__ __forceinline__ double wave_sum64(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// lane src's v in every lane (src uniform)
__device__ __forceinline__ double lane_bcast(double v, int src) {
    const int2 b = __builtin_bit_cast(int2, v);
    return __builtin_bit_cast(double, make_int2(__builtin_amdgcn_readlane(b.x, src), __builtin_amdgcn_readlane(b.y, src)));
}

// 1 / sqrt(x) for x > 0: the hardware estimate refined by two Newton steps y (3 - x y^2) / 2
__device__ __forceinline__ double rsqrt_nr(double x) {
    double y = __builtin_amdgcn_rsq(x);
    const double hx = 0.5 * x;
    y = y * fma(-hx * y, y, 1.5);
    y = y * fma(-hx * y, y, 1.5);
    return y;
}

// Diagonal block p of the super-block factor, by wave 0: L_pp and L_pp^-1 (to Inv[p]; the block of S keeps
// L_pp below its diagonal and garbage above).  Lane r (mod 16) holds row r.  Step j sends the unscaled
// column j through LDS (Inv[p] serves as staging) while the pivot's reciprocal square root is formed, and
// updates row r by a_rj a_qj / a_jj; entries above the diagonal take updates too (no predication) and are
// never read.  A pivot that is not positive is recorded in info and replaced by 1.
__device__ __forceinline__ void cr_diag_block(double* __restrict__ S, double* __restrict__ Inv, int p, int lane,
                                              int32_t* __restrict__ info, int32_t pos0) {
    const int r = lane & 15;
    double* B = S + 16 * p * CR_LD + 16 * p;
    double* col = Inv + p * 256;
    double row[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) row[q] = q <= r ? B[r * CR_LD + q] : 0.0;
    double rinv = 0.0;
    int first_bad = -1;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        // every lane writes (lanes 16-63 the same values as 0-15); a wave's LDS accesses complete in order
        if (j < 15) col[16 * j + r] = row[j];
        double pj = lane_bcast(row[j], j);
        const bool bad = !(pj > 0.0);
        first_bad = (first_bad < 0 && bad) ? j : first_bad;
        pj = bad ? 1.0 : pj;
        const double rs = rsqrt_nr(pj);
        if (j < 15) {
            const double tj = row[j] * (rs * rs);
#pragma unroll
            for (int q = j + 1; q < 16; ++q) row[q] = fma(-tj, col[16 * j + q], row[q]);
        }
        row[j] = r == j ? pj * rs : row[j] * rs;
        rinv = r == j ? rs : rinv;
    }
    if (first_bad >= 0 && lane == 0) atomicMin(info, pos0 + first_bad + 1);
    // the factored rows through LDS (B); lane c (mod 16) forms column c of L_pp^-1 by forward substitution,
    // reading the rows at uniform addresses
#pragma unroll
    for (int q = 0; q < 16; ++q) B[r * CR_LD + q] = row[q];     // lanes 16-63: the same values
    double x[16];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
        const double ri = lane_bcast(rinv, rr);
        double sum = 0.0;
#pragma unroll
        for (int mm = 0; mm < rr; ++mm) sum = fma(B[rr * CR_LD + mm], x[mm], sum);
        x[rr] = rr == r ? ri : (rr > r ? -ri * sum : 0.0);
    }
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) col[rr * 16 + r] = x[rr];       // lanes 16-63: the same values
}

// D = L L^T in LDS by 16-column panels (wave 0 factors and inverts the 16 x 16 diagonal block; the panel
// below and the trailing blocks are MFMA products; wave 0 takes the next diagonal block's trailing update
// first and factors it while the other waves finish the trailing blocks), then L^-1 in place by block
// columns from the right (L^-1_ij = - sum_{k = j+1..i} L^-1_ik L_kj L_jj^-1).
// The factor of one 128 x 128 SPD block by a workgroup of CR_T threads: the lower triangle of D (row pitch
// ld; the whole block is read, the part above the diagonal ignored) in, L^-1 (row pitch CR_MP, zero above
// the diagonal) out; lds holds CR_LDS_DOUBLES.  A pivot that is
// not positive goes to info as pos0 + its column + 1.
__device__ __forceinline__ void factor128(const double* __restrict__ D, int64_t ld, double* __restrict__ Lo,
                                          int32_t* __restrict__ info, int32_t pos0, double* lds) {
    double* S = lds;                          // [CR_MP][CR_LD]
    double* Inv = lds + CR_MP * CR_LD;        // [8][16][16] inverses of the diagonal blocks
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, lk = lane >> 4;
    {
        // the whole block (every load in flight at once), then its lower triangle into LDS
        double v[CR_MP2 / CR_T];
#pragma unroll
        for (int k = 0; k < CR_MP2 / CR_T; ++k) {
            const int e = t + k * CR_T, r = e / CR_MP, q = e - r * CR_MP;
            v[k] = D[r * ld + q];
        }
#pragma unroll
        for (int k = 0; k < CR_MP2 / CR_T; ++k) {
            const int e = t + k * CR_T, r = e / CR_MP, q = e - r * CR_MP;
            S[r * CR_LD + q] = q <= r ? v[k] : 0.0;
        }
    }
    __syncthreads();
    if (wave == 0) cr_diag_block(S, Inv, 0, lane, info, pos0);
    __syncthreads();
    for (int p = 0; p < 7; ++p) {
        // panel: L_ip = A_ip L_pp^-T for the block rows below
        if (wave < 7 - p) {
            double* Ab = S + 16 * (p + 1 + wave) * CR_LD + 16 * p;
            const double* Ip = Inv + p * 256;
            dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(Ab[l16 * CR_LD + 4 * kk + lk], Ip[l16 * 16 + 4 * kk + lk],
                                                           acc, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) Ab[(4 * v + lk) * CR_LD + l16] = acc[v];
        }
        __syncthreads();
        // trailing blocks (ib, jb), p < jb <= ib: A_ij -= L_ip L_jp^T; wave 0 takes (p + 1, p + 1) and then
        // factors it, waves 1-7 the others
        int tc = 0;
        for (int ib = p + 1; ib < 8; ++ib)
            for (int jb = p + 1; jb <= ib; ++jb) {
                const bool mine = (ib == p + 1) ? wave == 0 : (wave != 0 && tc++ % 7 == wave - 1);
                if (!mine) continue;
                const double* Li = S + 16 * ib * CR_LD + 16 * p;
                const double* Lj = S + 16 * jb * CR_LD + 16 * p;
                dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(Li[l16 * CR_LD + 4 * kk + lk],
                                                               Lj[l16 * CR_LD + 4 * kk + lk], acc, 0, 0, 0);
                double* C = S + 16 * ib * CR_LD + 16 * jb;
#pragma unroll
                for (int v = 0; v < 4; ++v) C[(4 * v + lk) * CR_LD + l16] -= acc[v];
            }
        if (wave == 0) cr_diag_block(S, Inv, p + 1, lane, info, pos0 + 16 * (p + 1));
        __syncthreads();
    }
    // L^-1 in place, block columns from the right
    for (int j = 7; j >= 0; --j) {
        const double* Ij = Inv + j * 256;
        if (j < 7) {
            // W_k = L_kj L_jj^-1 over L_kj
            if (wave < 7 - j) {
                double* Lk = S + 16 * (j + 1 + wave) * CR_LD + 16 * j;
                dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    acc = __builtin_amdgcn_mfma_f64_16x16x4f64(Lk[l16 * CR_LD + 4 * kk + lk],
                                                               Ij[(4 * kk + lk) * 16 + l16], acc, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v) Lk[(4 * v + lk) * CR_LD + l16] = acc[v];
            }
            __syncthreads();
            // L^-1_ij = - sum_{k = j+1..i} L^-1_ik W_k
            dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
            const int ib = j + 1 + wave;
            if (wave < 7 - j) {
                for (int k = j + 1; k <= ib; ++k) {
                    const double* Lik = S + 16 * ib * CR_LD + 16 * k;
                    const double* Wk = S + 16 * k * CR_LD + 16 * j;
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk)
                        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(Lik[l16 * CR_LD + 4 * kk + lk],
                                                                   Wk[(4 * kk + lk) * CR_LD + l16], acc, 0, 0, 0);
                }
            }
            __syncthreads();
            if (wave < 7 - j) {
                double* Q = S + 16 * ib * CR_LD + 16 * j;
#pragma unroll
                for (int v = 0; v < 4; ++v) Q[(4 * v + lk) * CR_LD + l16] = -acc[v];
            }
        }
        if (t < 256) S[(16 * j + (t >> 4)) * CR_LD + 16 * j + (t & 15)] = Ij[t];
        __syncthreads();
    }
    for (int e = t; e < CR_MP2; e += CR_T) {
        const int r = e / CR_MP, q = e - r * CR_MP;
        Lo[e] = q <= r ? S[r * CR_LD + q] : 0.0;
    }
}

__global__ void __launch_bounds__(CR_T) k_cr_factor(ChArgs c, int h) {
    extern __shared__ double lds[];
    const int I = (2 * (int)blockIdx.x + 1) * h - 1;
    factor128(c.crD + (int64_t)I * CR_MP2, CR_MP, c.crL + (int64_t)I * CR_MP2, c.info, I * CR_MP, lds);
}

// Ga = L^-1 E_I, Gb = L^-1 E_b^T and Y_I = L^-1 R_I for the eliminated super-block I = (2 blockIdx.x + 1) h - 1,
// one 16 x 16 tile per wave: blockIdx.y 0-15 Ga (tile row y / 2, tile columns 4 (y % 2) + wave), 16-31 Gb,
// 32-33 Y (tile row 4 (y - 32) + wave)
__global__ void __launch_bounds__(256) k_cr_elim(ChArgs c, int h) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lk = lane >> 4;
    const int I = (2 * (int)blockIdx.x + 1) * h - 1, y = blockIdx.y;
    const double* Li = c.crL + (int64_t)I * CR_MP2;
    dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
    if (y < 32) {
        const bool left = y < 16;
        const int nb = left ? I - h : I + h;
        if (nb < 0 || nb >= c.nsb) return;
        const int r0 = 16 * ((y & 15) >> 1), c0 = 16 * (4 * (y & 1) + wave);
        const double* La = Li + (int64_t)r0 * CR_MP;
        auto fa = [&](int r, int k) { return La[r * CR_MP + k]; };
        if (left) {
            const double* E = c.crE + (int64_t)I * CR_MP2 + c0;
            cr_mma(acc, 0, r0 + 16, fa, [&](int k, int q) { return E[k * CR_MP + q]; }, l16, lk);
        } else {
            const double* E = c.crE + (int64_t)nb * CR_MP2 + (int64_t)c0 * CR_MP;
            cr_mma(acc, 0, r0 + 16, fa, [&](int k, int q) { return E[q * CR_MP + k]; }, l16, lk);
        }
        double* G = (left ? c.crGa : c.crGb) + (int64_t)I * CR_MP2 + (int64_t)r0 * CR_MP + c0;
#pragma unroll
        for (int v = 0; v < 4; ++v) G[(4 * v + lk) * CR_MP + l16] = acc[v];
    } else {
        const int r0 = 16 * (4 * (y - 32) + wave);
        const double* La = Li + (int64_t)r0 * CR_MP;
        const double* R = c.crR + (int64_t)I * CR_MP * CR_NR;
        cr_mma(acc, 0, r0 + 16, [&](int r, int k) { return La[r * CR_MP + k]; },
               [&](int k, int q) { return R[k * CR_NR + q]; }, l16, lk);
        double* Y = c.crY + ((int64_t)I * CR_MP + r0) * CR_NR;
#pragma unroll
        for (int v = 0; v < 4; ++v) Y[(4 * v + lk) * CR_NR + l16] = acc[v];
    }
}

// Schur updates of the remaining super-block K = (2 blockIdx.x + 2) h - 1 from its eliminated neighbours
// p = K - h and q = K + h (if any), one 16 x 16 tile per wave: D_K (blockIdx.y 0-15), the new coupling
// E_K = -Gb_p^T Ga_p to p - h (16-31, when p - h exists), R_K (32-33)
__global__ void __launch_bounds__(256) k_cr_update(ChArgs c, int h) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lk = lane >> 4;
    const int K = (2 * (int)blockIdx.x + 2) * h - 1, y = blockIdx.y;
    const int p = K - h, q = K + h;
    const bool hq = q < c.nsb;
    const double* Gbp = c.crGb + (int64_t)p * CR_MP2;
    const double* Gaq = c.crGa + (int64_t)q * CR_MP2;
    dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
    if (y < 32) {
        const bool dblk = y < 16;
        if (!dblk && p - h < 0) return;
        const int r0 = 16 * ((y & 15) >> 1), c0 = 16 * (4 * (y & 1) + wave);
        const double* Bm = dblk ? Gbp : c.crGa + (int64_t)p * CR_MP2;
        cr_mma(acc, 0, CR_MP, [&](int r, int k) { return Gbp[k * CR_MP + r0 + r]; },
               [&](int k, int cc) { return Bm[k * CR_MP + c0 + cc]; }, l16, lk);
        if (dblk && hq)
            cr_mma(acc, 0, CR_MP, [&](int r, int k) { return Gaq[k * CR_MP + r0 + r]; },
                   [&](int k, int cc) { return Gaq[k * CR_MP + c0 + cc]; }, l16, lk);
        double* O = (dblk ? c.crD : c.crE) + (int64_t)K * CR_MP2 + (int64_t)r0 * CR_MP + c0;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            double* o = O + (4 * v + lk) * CR_MP + l16;
            *o = dblk ? *o - acc[v] : -acc[v];
        }
    } else {
        const int r0 = 16 * (4 * (y - 32) + wave);
        const double* Yp = c.crY + (int64_t)p * CR_MP * CR_NR;
        const double* Yq = c.crY + (int64_t)q * CR_MP * CR_NR;
        cr_mma(acc, 0, CR_MP, [&](int r, int k) { return Gbp[k * CR_MP + r0 + r]; },
               [&](int k, int cc) { return Yp[k * CR_NR + cc]; }, l16, lk);
        if (hq)
            cr_mma(acc, 0, CR_MP, [&](int r, int k) { return Gaq[k * CR_MP + r0 + r]; },
                   [&](int k, int cc) { return Yq[k * CR_NR + cc]; }, l16, lk);
        double* R = c.crR + ((int64_t)K * CR_MP + r0) * CR_NR;
#pragma unroll
        for (int v = 0; v < 4; ++v) R[(4 * v + lk) * CR_NR + l16] -= acc[v];
    }
}

// back substitution of the super-blocks eliminated at level h: X_I = L^-T (Y_I - Ga X_a - Gb X_b), wave w
// the rows 16 w ..
__global__ void __launch_bounds__(512) k_cr_back(ChArgs c, int h) {
    __shared__ double sT[CR_MP][CR_NR + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, lk = lane >> 4;
    const int I = (2 * (int)blockIdx.x + 1) * h - 1, a = I - h, b = I + h;
    const int r0 = 16 * wave;
    dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
    if (a >= 0) {
        const double* G = c.crGa + (int64_t)I * CR_MP2 + (int64_t)r0 * CR_MP;
        const double* X = c.crX + (int64_t)a * CR_MP * CR_NR;
        cr_mma(acc, 0, CR_MP, [&](int r, int k) { return G[r * CR_MP + k]; },
               [&](int k, int q) { return X[k * CR_NR + q]; }, l16, lk);
    }
    if (b < c.nsb) {
        const double* G = c.crGb + (int64_t)I * CR_MP2 + (int64_t)r0 * CR_MP;
        const double* X = c.crX + (int64_t)b * CR_MP * CR_NR;
        cr_mma(acc, 0, CR_MP, [&](int r, int k) { return G[r * CR_MP + k]; },
               [&](int k, int q) { return X[k * CR_NR + q]; }, l16, lk);
    }
    const double* Y = c.crY + (int64_t)I * CR_MP * CR_NR;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int r = r0 + 4 * v + lk;
        sT[r][l16] = Y[r * CR_NR + l16] - acc[v];
    }
    __syncthreads();
    const double* Li = c.crL + (int64_t)I * CR_MP2;
    acc = (dbl4){0.0, 0.0, 0.0, 0.0};
    cr_mma(acc, r0, CR_MP, [&](int r, int k) { return Li[k * CR_MP + r0 + r]; },
           [&](int k, int q) { return sT[k][q]; }, l16, lk);
    double* X = c.crX + ((int64_t)I * CR_MP + r0) * CR_NR;
#pragma unroll
    for (int v = 0; v < 4; ++v) X[(4 * v + lk) * CR_NR + l16] = acc[v];
}

// X of local entry u = i db + r (image i) and right-hand side col
__device__ __forceinline__ double cr_x(const ChArgs& c, int64_t u, int col) {
    const int i = (int)(u / c.db), r = (int)(u - (int64_t)i * c.db);
    const int I = i / c.s;
    return c.crX[((int64_t)I * CR_MP + (i - I * c.s) * c.db + r) * CR_NR + col];
}

// border: the corner's Schur complement C - B^T S_loc^-1 B and rhs b_s - B^T S_loc^-1 b_loc.  k_cr_bpart sums
// B[b1] . X[:, col] over a fixed slice of the local entries (block (chunk, b1 (n_s + 1) + col)), lanes and
// waves in a fixed tree; k_cr_border adds the chunks in order, factors the corner and solves (thread 0).
#define BP_CHUNKS 64
static_assert(BP_CHUNKS <= SS_CHUNKS, "the border products share the shared-shared partial-sum buffer");
__global__ void __launch_bounds__(CH_T) k_cr_bpart(PcgArgs64 a, ChArgs c) {
    __shared__ double sh[CH_T / 64];
    const int ns = c.n_shared, combo = blockIdx.y, b1 = combo / (ns + 1), col = combo - b1 * (ns + 1);
    const int64_t nl = (int64_t)a.n_imgs * c.db;
    double s = 0.0;
    for (int64_t u = (int64_t)blockIdx.x * CH_T + threadIdx.x; u < nl; u += (int64_t)BP_CHUNKS * CH_T)
        s += c.Bfull[(int64_t)b1 * nl + u] * cr_x(c, u, col);
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < CH_T / 64; ++w) t += sh[w];
        c.ss_part[(int64_t)combo * BP_CHUNKS + blockIdx.x] = t;
    }
}

__global__ void k_cr_border(PcgArgs64 a, ChArgs c) {
    double Cc[(CR_NR - 1) * (CR_NR - 1)], rb[CR_NR - 1], xb[CR_NR - 1];
    if (threadIdx.x != 0) return;
    const int ns = c.n_shared;
    const int64_t nl = (int64_t)a.n_imgs * c.db;
    for (int b1 = 0; b1 < ns; ++b1)
        for (int col = 0; col <= ns; ++col) {
            double s = 0.0;
            for (int k = 0; k < BP_CHUNKS; ++k) s += c.ss_part[(int64_t)(b1 * (ns + 1) + col) * BP_CHUNKS + k];
            if (col == 0) rb[b1] = a.rhs[c.shared_u[b1]] - s;
            else Cc[b1 * ns + col - 1] = c.Cb[b1 * ns + col - 1] - s;
        }
    for (int r = 0; r < ns; ++r)
        for (int q = 0; q <= r; ++q) {
            double v = Cc[r * ns + q];
            for (int m = 0; m < q; ++m) v -= Cc[r * ns + m] * Cc[q * ns + m];
            if (r == q) {
                if (!(v > 0.0)) {
                    atomicMin(c.info, (int32_t)(nl + r + 1));
                    v = 1.0;
                }
                Cc[r * ns + r] = sqrt(v);
            } else {
                Cc[r * ns + q] = v / Cc[q * ns + q];
            }
        }
    for (int r = 0; r < ns; ++r) {
        double v = rb[r];
        for (int m = 0; m < r; ++m) v -= Cc[r * ns + m] * rb[m];
        rb[r] = v / Cc[r * ns + r];
    }
    for (int r = ns - 1; r >= 0; --r) {
        double v = rb[r];
        for (int m = r + 1; m < ns; ++m) v -= Cc[m * ns + r] * xb[m];
        xb[r] = v / Cc[r * ns + r];
    }
    for (int r = 0; r < ns; ++r) {
        a.x[c.shared_u[r]] = xb[r];
        c.crXb[r] = xb[r];
    }
}

// the local solution: x_loc = S_loc^-1 b_loc - S_loc^-1 B x_s
__global__ void __launch_bounds__(CH_T) k_cr_local(PcgArgs64 a, ChArgs c) {
    const int64_t u = (int64_t)blockIdx.x * CH_T + threadIdx.x;
    if (u >= (int64_t)a.n_imgs * c.db) return;
    double v = cr_x(c, u, 0);
    for (int b = 0; b < c.n_shared; ++b) v -= cr_x(c, u, 1 + b) * c.crXb[b];
    c.xl[u] = v;
}

// ------------------------------------------------------------------ dense layout, 128-column panels
// Right-looking L L^T of S_u (lower triangle, row pitch lda = n_u rounded up to 128) by block columns of 128:
// the diagonal block's L^-1 by factor128 (one workgroup), the panel below as L_ik = A_ik L_kk^-T (in place,
// and into the panel copy P), the trailing blocks as A_ij -= L_ik L_jk^T from P.  Triangular sweeps by
// block with the diagonal blocks' inverses.
#define DN_NB CR_MP
#define DN_KC 16                     // K columns of P staged in LDS at a time by the trailing update

__global__ void __launch_bounds__(CR_T) k_dn_factor(const double* __restrict__ A, int64_t lda, int k,
                                                    double* __restrict__ Linv, int32_t* __restrict__ info) {
    extern __shared__ double lds[];
    const int64_t o = (int64_t)k * DN_NB;
    factor128(A + o * lda + o, lda, Linv + (int64_t)k * CR_MP2, info, (int32_t)o, lds);
}

// the 16-row strip blockIdx.x below block k: L = A_strip L_kk^-T, wave w the columns 16 w ..; the strip is in
// LDS before anything is written.  L goes to A and to P (rows below block k, row pitch DN_NB).
__global__ void __launch_bounds__(512) k_dn_panel(double* __restrict__ A, int64_t lda, int k,
                                                  const double* __restrict__ Linv, double* __restrict__ P) {
    __shared__ double sA[16][DN_NB + 1];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l16 = lane & 15, lk = lane >> 4;
    const int64_t o = (int64_t)k * DN_NB, rp = 16 * (int64_t)blockIdx.x, r0 = o + DN_NB + rp;
    for (int e = t; e < 16 * DN_NB; e += 512) {
        const int r = e / DN_NB, q = e - r * DN_NB;
        sA[r][q] = A[(r0 + r) * lda + o + q];
    }
    __syncthreads();
    const double* Li = Linv + (int64_t)k * CR_MP2;
    const int c0 = 16 * wave;
    dbl4 acc = (dbl4){0.0, 0.0, 0.0, 0.0};
    // B[q][c] = L^-1[c0 + c][q], zero for q > c0 + c
    cr_mma(acc, 0, c0 + 16, [&](int r, int q) { return sA[r][q]; },
           [&](int q, int cc) { return Li[(c0 + cc) * CR_MP + q]; }, l16, lk);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int r = 4 * v + lk, c = c0 + l16;
        A[(r0 + r) * lda + o + c] = acc[v];
        P[(rp + r) * DN_NB + c] = acc[v];
    }
}

// trailing blocks (i, j), k < j <= i, from the triangular index blockIdx.x: A_ij -= P_i P_j^T.  Four waves, each
// a 64 x 64 quadrant as 4 x 4 tiles of v_mfma_f64_16x16x4f64 over K = 128, the operands staged in LDS DN_KC
// columns at a time (rows padded to DN_KC + 1 doubles); two workgroups fit a CU.
__global__ void __launch_bounds__(256) k_dn_syrk(double* __restrict__ A, int64_t lda, int k,
                                                 const double* __restrict__ P) {
    __shared__ double sa[DN_NB][DN_KC + 1];
    __shared__ double sb[DN_NB][DN_KC + 1];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l16 = lane & 15, lk = lane >> 4;
    const int64_t q = blockIdx.x;
    int bi = (int)((sqrt(8.0 * (double)q + 1.0) - 1.0) * 0.5);
    while ((int64_t)(bi + 1) * (bi + 2) / 2 <= q) ++bi;
    while ((int64_t)bi * (bi + 1) / 2 > q) --bi;
    const int bj = (int)(q - (int64_t)bi * (bi + 1) / 2);
    const double* Pi = P + (int64_t)bi * DN_NB * DN_NB;
    const double* Pj = P + (int64_t)bj * DN_NB * DN_NB;
    const int qi = (wave >> 1) * 64, qj = (wave & 1) * 64;
    dbl4 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int nj = 0; nj < 4; ++nj) acc[mi][nj] = (dbl4){0.0, 0.0, 0.0, 0.0};
    // the next chunk's operands are loaded into registers while this one's MFMAs run
    constexpr int PER = DN_NB * DN_KC / 256;          // operands of one matrix per thread and chunk
    double ra[PER], rb[PER];
    auto fetch = [&](int kc) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = t + 256 * i, r = e / DN_KC, c = e - r * DN_KC;
            ra[i] = Pi[r * DN_NB + kc + c];
            rb[i] = Pj[r * DN_NB + kc + c];
        }
    };
    fetch(0);
    for (int kc = 0; kc < DN_NB; kc += DN_KC) {
        if (kc) __syncthreads();                      // the previous chunk is consumed
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = t + 256 * i, r = e / DN_KC, c = e - r * DN_KC;
            sa[r][c] = ra[i];
            sb[r][c] = rb[i];
        }
        __syncthreads();
        if (kc + DN_KC < DN_NB) fetch(kc + DN_KC);
#pragma unroll 2
        for (int kk = 0; kk < DN_KC / 4; ++kk) {
            double av[4], bv[4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) av[mi] = sa[qi + 16 * mi + l16][4 * kk + lk];
#pragma unroll
            for (int nj = 0; nj < 4; ++nj) bv[nj] = sb[qj + 16 * nj + l16][4 * kk + lk];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int nj = 0; nj < 4; ++nj)
                    acc[mi][nj] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[mi], bv[nj], acc[mi][nj], 0, 0, 0);
        }
    }
    const int64_t ro = (int64_t)(k + 1 + bi) * DN_NB, co = (int64_t)(k + 1 + bj) * DN_NB;
    // C -= acc, sixteen elements' loads in flight at a time
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        double cv[4][4];
#pragma unroll
        for (int nj = 0; nj < 4; ++nj)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                cv[nj][v] = __builtin_nontemporal_load(A + (ro + qi + 16 * mi + 4 * v + lk) * lda + co + qj + 16 * nj + l16);
#pragma unroll
        for (int nj = 0; nj < 4; ++nj)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                A[(ro + qi + 16 * mi + 4 * v + lk) * lda + co + qj + 16 * nj + l16] = cv[nj][v] - acc[mi][nj][v];
    }
}

// Forward sweep, block k: y_k = L_kk^-1 b_k (every workgroup forms it from b_k, which this launch does not
// write; workgroup 0 stores it), workgroup w >= 1: b_i -= L_ik y_k for i = k + w.  A row product by two
// threads, each over 64 contiguous columns (16-byte loads, all in flight), the halves added by a shuffle.
__global__ void __launch_bounds__(256) k_dn_fwd(const double* __restrict__ A, int64_t lda, int k,
                                                const double* __restrict__ Linv, double* __restrict__ b,
                                                double* __restrict__ y) {
    __shared__ double sb[DN_NB], sy[DN_NB];
    const int t = threadIdx.x, r = t >> 1, h = t & 1;
    const int64_t o = (int64_t)k * DN_NB;
    if (t < DN_NB) sb[t] = b[o + t];
    __syncthreads();
    // row r of M (row pitch ld) times v (LDS), by the thread pair (r, h)
    auto row = [&](const double* M, int64_t ld, const double* v) {
        const double2* Mr = reinterpret_cast<const double2*>(M + (int64_t)r * ld + 64 * h);
        double2 m[32];
#pragma unroll
        for (int q = 0; q < 32; ++q) m[q] = Mr[q];
        double s = 0.0;
#pragma unroll
        for (int q = 0; q < 32; ++q) s += m[q].x * v[64 * h + 2 * q] + m[q].y * v[64 * h + 2 * q + 1];
        return s + __shfl_xor(s, 1);
    };
    const double yr = row(Linv + (int64_t)k * CR_MP2, CR_MP, sb);
    if (h == 0) sy[r] = yr;
    __syncthreads();
    if (blockIdx.x == 0) {
        if (t < DN_NB) y[o + t] = sy[t];
        return;
    }
    const int64_t ro = o + (int64_t)blockIdx.x * DN_NB;
    const double s = row(A + ro * lda + o, lda, sy);
    if (h == 0) b[ro + r] -= s;
}

// Backward sweep, block k: x_k = L_kk^-T y_k (workgroup 0 stores it), workgroup w >= 1: y_i -= L_ki^T x_k for
// i = w - 1 < k; thread r forms output r, reading the rows of L_ki (coalesced across threads).
__global__ void __launch_bounds__(DN_NB) k_dn_bwd(const double* __restrict__ A, int64_t lda, int k,
                                                  const double* __restrict__ Linv, double* __restrict__ y,
                                                  double* __restrict__ x) {
    __shared__ double sy[DN_NB], sx[DN_NB];
    const int t = threadIdx.x;
    const int64_t o = (int64_t)k * DN_NB;
    sy[t] = y[o + t];
    __syncthreads();
    const double* Li = Linv + (int64_t)k * CR_MP2;
    double s = 0.0;                           // L^-1[q][t] is zero for q < t
#pragma unroll 16
    for (int q = 0; q < DN_NB; ++q) s += Li[q * CR_MP + t] * sy[q];
    sx[t] = s;
    __syncthreads();
    if (blockIdx.x == 0) {
        x[o + t] = s;
        return;
    }
    const int64_t io = (int64_t)(blockIdx.x - 1) * DN_NB;
    double acc = 0.0;
#pragma unroll 16
    for (int q = 0; q < DN_NB; ++q) acc += A[(o + q) * lda + io + t] * sx[q];
    y[io + t] -= acc;
}

}  // namespace ba

using namespace ba;

extern "C" int64_t ba_chol_dense_lda(int64_t n_u) {
    const int64_t m = n_u < 1 ? 1 : n_u;
    return (m + DN_NB - 1) / DN_NB * DN_NB;
}

extern "C" int64_t ba_chol_work_doubles(int32_t mode, int64_t n_u, int32_t n_imgs, int32_t d, int32_t w,
                                        int32_t n_shared) {
    // banded: d is the band block size db
    const int64_t ss = (int64_t)n_shared * (n_shared + 1) * SS_CHUNKS;     // also BP_CHUNKS per border product
    if (mode == 0) return (3 + DN_NB) * ba_chol_dense_lda(n_u) + ss;
    const int64_t M = (int64_t)(w + 1) * d, nl = (int64_t)n_imgs * d;
    int64_t n = (int64_t)n_imgs * (w + 1) * d * d + (int64_t)n_shared * nl + (int64_t)n_shared * n_shared + nl +
                (int64_t)n_imgs * M * d + (int64_t)n_imgs * n_shared * d + 2 * nl;
    const int32_t nsb = mode == 1 ? ba_chol_band_superblocks(d, w, n_shared, n_imgs) : 0;
    if (nsb > 0) n += (int64_t)nsb * (5 * CR_MP2 + 3 * CR_MP * CR_NR) + CR_NR;
    return n + ss;
}

extern "C" int32_t ba_chol_band_superblocks(int32_t d, int32_t w, int32_t n_shared, int32_t n_imgs) {
    const int s = cr_images(d, w, n_shared);
    if (s == 0 || n_imgs < 1) return 0;
    return (n_imgs + s - 1) / s;
}

extern "C" int64_t ba_chol_band_lds_bytes(int32_t d, int32_t w, int32_t n_shared) {
    return band_lds_doubles((w + 1) * d, n_shared) * (int64_t)sizeof(double);
}

extern "C" int ba_reduced_solve(const ba_pcg_args* args, const ba_chol_args* cargs, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr && cargs != nullptr, "ba_reduced_solve: null args");
    BA_REQUIRE(!args->real32, "ba_reduced_solve: the direct solve runs in fp64 only (real32 must be 0)");
    const PcgArgs64& a = *reinterpret_cast<const PcgArgs64*>(args);
    const ba_chol_args& ca = *cargs;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.n_u >= 0 && a.d >= 1 && a.d <= 32, "ba_reduced_solve: bad sizes (1 <= d <= 32)");
    if (a.n_u == 0) return BA_OK;
    {
        const void* need[] = {a.umap, a.inv_ptr, a.inv_src, a.leaf, a.S_pairs, a.e_img, a.dg_img, a.rhs, a.diagA,
                              a.damp, a.x, a.state, a.row_ptr, a.row_ent, a.pair_i1, a.pair_i2, ca.pair_idx, ca.info,
                              ca.work, ca.kind};
        for (const void* q : need) BA_REQUIRE(q != nullptr, "ba_reduced_solve: null pointer in the arguments");
    }
    BA_REQUIRE(ca.n_shared >= 0 && (ca.n_shared == 0 || ca.shared_u != nullptr),
               "ba_reduced_solve: shared unknowns missing");
    ChArgs c{};
    c.mode = ca.mode; c.A = ca.A; c.lda = ca.lda; c.Linv = ca.Linv; c.pair_idx = ca.pair_idx; c.kind = ca.kind;
    c.shared_u = ca.shared_u; c.n_shared = ca.n_shared; c.w = ca.w; c.info = ca.info;
    c.db = ca.db; c.bcol = ca.bcol; c.bpos = ca.bpos;
    const int64_t n_pairs = ca.n_pairs;
    int rc = unknown_setup(*args, st);
    if (rc != BA_OK) return rc;
    hipLaunchKernelGGL(k_info_init, dim3(1), dim3(64), 0, st, c.info);
    const unsigned nbu = (unsigned)((a.n_u + CH_T - 1) / CH_T);
    const unsigned nbw = (unsigned)((a.n_u + CH_T / 64 - 1) / (CH_T / 64));     // one wave per unknown
    if (ca.mode == 1 || ca.mode == 2) {
        BA_REQUIRE(ca.db >= 1 && ca.db <= a.d && ca.bcol != nullptr && ca.bpos != nullptr,
                   "ba_reduced_solve: the banded layout needs 1 <= db <= d, bcol, bpos");
        const int d = ca.db, M = (ca.w + 1) * d;
        const int s_cr = ca.mode == 1 ? cr_images(d, ca.w, ca.n_shared) : 0;
        BA_REQUIRE(ca.w >= 1 && (s_cr > 0 || (d <= CB_MAXD && M <= CB_MAXM && ca.n_shared <= CB_MAXS)),
                   "ba_reduced_solve: the banded layout needs w >= 1 and either w db <= 128 with at most 15 shared "
                   "unknowns (mode 1) or db <= 16, (w + 1) db <= 160 and at most 8 shared unknowns");
        const int64_t nl = (int64_t)a.n_imgs * d;
        double* w = ca.work;
        c.Ab = w; w += (int64_t)a.n_imgs * (ca.w + 1) * d * d;
        c.Bfull = w; w += (int64_t)ca.n_shared * nl;
        c.Cb = w; w += (int64_t)ca.n_shared * ca.n_shared;
        c.bl = w; w += nl;
        c.Lcol = w; w += (int64_t)a.n_imgs * M * d;
        c.Lbord = w; w += (int64_t)a.n_imgs * ca.n_shared * d;
        c.yv = w; w += nl;
        c.xl = w; w += nl;
        if (s_cr > 0) {
            c.s = s_cr;
            c.nsb = (a.n_imgs + s_cr - 1) / s_cr;
            const int64_t big = (int64_t)c.nsb * CR_MP2, rhs = (int64_t)c.nsb * CR_MP * CR_NR;
            c.crD = w; w += big;
            c.crE = w; w += big;
            c.crL = w; w += big;
            c.crGa = w; w += big;
            c.crGb = w; w += big;
            c.crR = w; w += rhs;
            c.crY = w; w += rhs;
            c.crX = w; w += rhs;
            c.crXb = w; w += CR_NR;
        }
        c.ss_part = w;
        const int64_t nab = (int64_t)a.n_imgs * (ca.w + 1) * d * d;
        hipLaunchKernelGGL(k_band_assemble, dim3((unsigned)((nab + CH_T - 1) / CH_T)), dim3(CH_T), 0, st, a, c);
        if (ca.n_shared > 0) {
            hipLaunchKernelGGL(k_shared_local, dim3(nbw, (unsigned)ca.n_shared), dim3(CH_T), 0, st, a, c, 1);
            hipLaunchKernelGGL(k_shared_part, dim3((unsigned)(ca.n_shared * ca.n_shared), SS_CHUNKS), dim3(CH_T), 0,
                               st, a, c, n_pairs);
            hipLaunchKernelGGL(k_shared_sum, dim3((unsigned)((ca.n_shared * ca.n_shared + CH_T - 1) / CH_T)),
                               dim3(CH_T), 0, st, a, c, 1);
        }
        if (s_cr > 0) {
            const int nsb = c.nsb;
            const int64_t big = (int64_t)nsb * CR_MP2;
            hipLaunchKernelGGL(k_cr_assemble, dim3((unsigned)((big + CH_T - 1) / CH_T)), dim3(CH_T), 0, st, a, c);
            const size_t cr_lds = (size_t)CR_LDS_DOUBLES * sizeof(double);
            BA_HIP(hipFuncSetAttribute((const void*)k_cr_factor, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)cr_lds));
            int levels = 0;
            for (int h = 1; h <= nsb; h *= 2, ++levels) {
                const int n_elim = (nsb / h + 1) / 2, n_kept = nsb / (2 * h);
                hipLaunchKernelGGL(k_cr_factor, dim3((unsigned)n_elim), dim3(CR_T), cr_lds, st, c, h);
                hipLaunchKernelGGL(k_cr_elim, dim3((unsigned)n_elim, 34), dim3(256), 0, st, c, h);
                if (n_kept > 0) hipLaunchKernelGGL(k_cr_update, dim3((unsigned)n_kept, 34), dim3(256), 0, st, c, h);
            }
            for (int l = levels - 1; l >= 0; --l) {
                const int h = 1 << l;
                hipLaunchKernelGGL(k_cr_back, dim3((unsigned)((nsb / h + 1) / 2)), dim3(512), 0, st, c, h);
            }
            if (ca.n_shared > 0) {
                hipLaunchKernelGGL(k_cr_bpart, dim3(BP_CHUNKS, (unsigned)(ca.n_shared * (ca.n_shared + 1))), dim3(CH_T),
                                   0, st, a, c);
                hipLaunchKernelGGL(k_cr_border, dim3(1), dim3(64), 0, st, a, c);
            }
            hipLaunchKernelGGL(k_cr_local, dim3((unsigned)((nl + CH_T - 1) / CH_T)), dim3(CH_T), 0, st, a, c);
            hipLaunchKernelGGL(k_band_scatter, dim3(nbu), dim3(CH_T), 0, st, a, c);
            hipLaunchKernelGGL(k_chol_status, dim3(1), dim3(64), 0, st, a, c.info);
            BA_LAUNCHED();
            return BA_OK;
        }
        const size_t lds_bytes = (size_t)band_lds_doubles(M, ca.n_shared) * sizeof(double);
        BA_REQUIRE(lds_bytes <= 160 * 1024, "ba_reduced_solve: the banded window does not fit LDS (use mode 0)");
        BA_HIP(hipFuncSetAttribute((const void*)k_band_solve, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)lds_bytes));
        hipLaunchKernelGGL(k_band_solve, dim3(1), dim3(CB_T), lds_bytes, st, a, c);
        hipLaunchKernelGGL(k_band_scatter, dim3(nbu), dim3(CH_T), 0, st, a, c);
        hipLaunchKernelGGL(k_chol_status, dim3(1), dim3(64), 0, st, a, c.info);
        BA_LAUNCHED();
        return BA_OK;
    }
    BA_REQUIRE(ca.mode == 0, "ba_reduced_solve: unknown mode");
    const int64_t N = ba_chol_dense_lda(a.n_u);
    BA_REQUIRE(c.A != nullptr && c.lda >= N && c.Linv != nullptr, "ba_reduced_solve: dense workspace missing");
    const int nt = (int)(N / DN_NB);
    double* b = ca.work;
    double* y = b + N;
    double* xs = y + N;
    double* P = xs + N;                      // panel copy: (N - DN_NB) x DN_NB
    c.ss_part = P + N * DN_NB;
    hipLaunchKernelGGL(k_dense_assemble, dim3((unsigned)((N + CH_T - 1) / CH_T), (unsigned)N), dim3(CH_T), 0, st, a,
                       c, N);
    if (ca.n_shared > 0) {
        hipLaunchKernelGGL(k_shared_local, dim3(nbw, (unsigned)ca.n_shared), dim3(CH_T), 0, st, a, c, 0);
        hipLaunchKernelGGL(k_shared_part, dim3((unsigned)(ca.n_shared * ca.n_shared), SS_CHUNKS), dim3(CH_T), 0, st,
                           a, c, n_pairs);
        hipLaunchKernelGGL(k_shared_sum, dim3((unsigned)((ca.n_shared * ca.n_shared + CH_T - 1) / CH_T)), dim3(CH_T),
                           0, st, a, c, 0);
    }
    const size_t f_lds = (size_t)CR_LDS_DOUBLES * sizeof(double);
    BA_HIP(hipFuncSetAttribute((const void*)k_dn_factor, hipFuncAttributeMaxDynamicSharedMemorySize, (int)f_lds));
    for (int k = 0; k < nt; ++k) {
        hipLaunchKernelGGL(k_dn_factor, dim3(1), dim3(CR_T), f_lds, st, c.A, c.lda, k, c.Linv, c.info);
        const int below = nt - 1 - k;
        if (below > 0) {
            hipLaunchKernelGGL(k_dn_panel, dim3((unsigned)(below * (DN_NB / 16))), dim3(512), 0, st, c.A, c.lda, k, c.Linv, P);
            const int64_t tri = (int64_t)below * (below + 1) / 2;
            hipLaunchKernelGGL(k_dn_syrk, dim3((unsigned)tri), dim3(256), 0, st, c.A, c.lda, k, P);
        }
    }
    hipLaunchKernelGGL(k_copy_pad, dim3((unsigned)((N + CH_T - 1) / CH_T)), dim3(CH_T), 0, st, a.rhs, a.n_u, N, b);
    for (int k = 0; k < nt; ++k)
        hipLaunchKernelGGL(k_dn_fwd, dim3((unsigned)(nt - k)), dim3(256), 0, st, c.A, c.lda, k, c.Linv, b, y);
    for (int k = nt - 1; k >= 0; --k)
        hipLaunchKernelGGL(k_dn_bwd, dim3((unsigned)(k + 1)), dim3(DN_NB), 0, st, c.A, c.lda, k, c.Linv, y, xs);
    hipLaunchKernelGGL(k_isolated, dim3(nbu), dim3(CH_T), 0, st, a, xs);
    hipLaunchKernelGGL(k_chol_status, dim3(1), dim3(64), 0, st, a, c.info);
    BA_LAUNCHED();
    return BA_OK;
}
