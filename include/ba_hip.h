/*
 * libba_hip.so -- C ABI of the MI355X bundle-adjustment linearize + Schur path.
 *
 * Drop-in boundary for the reference's native module `ba_with_rigs_cuda_kernels`
 * (src/blast3r/extensions/cujac/sfm_jacobian_rigs.cu, pybind table at :1254-1275,
 * Python aliases at src/blast3r/extensions/cujac/__init__.py:18-22) and for the
 * solver work the reference does in PyTorch (src/blast3r/inference/ba_solver.py).
 *
 * Conventions for every entry point:
 *   - returns 0 on success, nonzero on error; ba_last_error() holds a message
 *     (thread-local), the Python layer raises RuntimeError with it;
 *   - all pointers are device pointers unless the name says host; the caller
 *     owns every buffer (the library allocates no caller-visible memory);
 *   - `stream` is a hipStream_t; work is enqueued asynchronously and never
 *     synchronised, like the reference's getCurrentCUDAStream launches (.cu:293);
 *   - entry points are stateless and reentrant; calls that share output or
 *     workspace buffers must not overlap.
 */
#ifndef BA_HIP_H
#define BA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ misc */
const char* ba_last_error(void);
int ba_version(void);
/* sizeof(name) for every argument struct below ("ba_lin_args", ...), -1 for an unknown name: lets a
 * binding check its own struct layout against the library's before the first launch.  Host only. */
int64_t ba_abi_sizeof(const char* name);

/* ------------------------------------------------------------------ operator-level (cujac) API */

/* residuals_with_rigs (sfm_jacobian_rigs.cu:1048-1101, kernel :129-259).
 * out: (n_out, n_obs) fp32 with n_out = 9 when pnorm > 0 else 3, rows
 * [r0 r1 r2 | err0 err1 err2 | w0 w1 w2]; every element is written. */
int ba_residuals(const int32_t* infos, int32_t n_imgs, const float* K, const float* P_rig2cam,
                 int64_t P_rig2cam_stride, const float* P_w2rig, const float* z_coefs, const float* pts3d,
                 const int32_t* pids, const float* pix2d, const float* pix2d_std, const float* pix2d_dep,
                 int64_t n_obs, int32_t C, int32_t is_depth_log, float weight_z, float pnorm,
                 float max_pix_err, float huber_delta, float w_pts_null, float* out, void* stream);

/* jacobians_with_rigs (sfm_jacobian_rigs.cu:1105-1148, kernel :323-509).
 * J_cam (n_obs,3,8), J_zcf (n_obs,1,C), J_pts (n_obs,3,3): fp64 if float64 else fp32. */
int ba_jacobians(const int32_t* infos, int32_t n_imgs, const float* K, const float* P_rig2cam,
                 int64_t P_rig2cam_stride, const float* P_w2rig, const float* z_coefs, const float* pts3d,
                 const int32_t* pids, const float* pix2d_std, const float* pix2d_dep, int64_t n_obs, int32_t C,
                 int32_t is_depth_log, int32_t float64, void* J_cam, void* J_zcf, void* J_pts, void* stream);

/* chol3x3_solve (sfm_jacobian_rigs.cu:1151-1169, kernel :560-634). dtype 0 = fp32, 1 = fp64. */
int ba_chol3x3_solve(const void* blocks, const void* rhs, void* out, int64_t n, double jitter, int32_t dtype,
                     void* stream);

/* blockcoo_matvec (sfm_jacobian_rigs.cu:1171-1219); any (bh, bw); every element of y is written.  Blocks may
 * come in any order and repeat; each output element sums its blocks in ascending block order (stable radix
 * sort of the block ids by output block, then one thread per output element), so the result is
 * deterministic.  Block indices outside [0, HB1) / [0, WB1) are ignored.  workspace: at least
 * ba_blockcoo_workspace_size(n_blocks, transpose ? WB1 : HB1) bytes of device memory, 256-byte aligned. */
int64_t ba_blockcoo_workspace_size(int64_t n_blocks, int64_t n_out_blocks);
int ba_blockcoo_matvec(const void* blocks, int32_t bh, int32_t bw, const void* row_idx, const void* col_idx,
                       int32_t index_int64, int64_t n_blocks, const void* x, void* y, int64_t HB1, int64_t WB1,
                       int32_t transpose, int32_t dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* fused_einsum_bki_bkj (sfm_jacobian_rigs.cu:1222-1250); any (I, J, K), strides in elements. */
int ba_einsum_bki_bkj(const void* left, int64_t l_bs, int64_t l_ks, const void* right, int64_t r_bs, int64_t r_ks,
                      void* out, int64_t B, int32_t K, int32_t I, int32_t J, int32_t dtype, void* stream);

/* exp_se3 (cujac/__init__.py:56-58): xi (n,6) = [w|v] -> (n,4,4) fp32. */
int ba_exp_se3(const float* xi, float* out, int64_t n, void* stream);

/* ------------------------------------------------------------------ structure plan (host) */
/* Built once per observation structure; replaces the per-iteration torch.unique /
 * index bookkeeping of ba_solver.py:51-56, :877-909, :968-974.  Host pointers. */
void* ba_plan_create(const int32_t* cum_nkpts, int32_t n_imgs, const int32_t* pids, int64_t n_obs,
                     int32_t n_tracks, int32_t max_local_imgs, int32_t max_slots, int64_t max_batch_obs);
int ba_plan_query(const void* plan, int64_t* scalars, int64_t* array_sizes);
int ba_plan_export(const void* plan, int32_t which, int32_t* host_dst);
void ba_plan_destroy(void* plan);
const char* ba_plan_last_error(void);
/* The plan of prev's structure with one image and new tracks appended (`old | new`, tracks.py:84-102:
 * per image, prev's observations, then add_cnt[i] of the new tracks, whose ids add_pids lists image by
 * image); byte-identical to ba_plan_create on the merged structure, but only the batches from the first
 * new track's place in the track order on are planned again.  prev is consumed on success (no counterpart
 * in the reference, which rebuilds its structure with torch.unique on every iteration, ba_solver.py:877-909). */
void* ba_plan_append(void* prev, const int32_t* add_cnt, int32_t n_imgs_new, const int32_t* add_pids, int64_t n_add,
                     int32_t n_tracks_new);
/* array `which` of the plan in place (host memory, valid until the plan is destroyed or appended to) */
const int32_t* ba_plan_array(const void* plan, int32_t which);
/* per array, the leading elements equal to the parent plan's (chunk_obs / slot_src after adding shift[image]);
 * per image (n_imgs of the plan), that shift.  All 0 for a plan made by ba_plan_create. */
int ba_plan_stable(const void* plan, int64_t* stable, int32_t* shift);
/* device: ids[q] += shift[img[q]], q < n (a device copy of a parent plan's chunk_obs / slot_src brought to the
 * appended structure's observation ids; no counterpart in the reference) */
int ba_plan_shift_ids(int32_t* ids, const int32_t* img, const int32_t* shift, int64_t n, void* stream);

/* ------------------------------------------------------------------ fused linearize + Schur */
typedef struct {
    float weight_z, pnorm, max_pix_err, huber_delta, w_pts_null;
    int32_t is_depth_log;
} ba_huber;

typedef struct {
    int32_t d, C, off_tau, off_zcf, hasK, hasP, hasZ;     /* image-level block layout [foc|tau|zcf] */
    int32_t no_grad_f_from_rz, optim_Z0, optim_Z_1st_cam;  /* ba_solver.py:38-39, :59-60 */
    float wmin, wmax;                                       /* clamp_w (ba_solver.py:123-124) */
    double dampen;                                          /* 1e-12 (engine.py:490) */
    int32_t adaptive, x_off;                                /* adaptive_dampen; optim_X is False */
} ba_layout;

typedef struct {
    /* structure */
    const int32_t* infos; int32_t n_imgs;
    const int32_t *chunk_obs, *chunk_meta, *slot_info;
    const int32_t *ct_pid, *ct_first, *ct_m, *ct_mask;
    const int32_t *b_chunk_ptr, *b_imgs, *b_nimgs, *b_slot_ptr, *slot_pair;
    int32_t L;
    /* observations in plan slot order */
    const float *s_pix, *s_std, *s_dep;
    const int32_t *s_pid, *s_img;
    /* parameters */
    const float* K; const float* P_rig2cam; int64_t P_rig2cam_stride; const float* P_w2rig;
    const float* z_coefs; const float* pts3d;
    /* optional uint8 enable masks per cam / node / image / track (NULL = all on) */
    const uint8_t *enK, *enP, *enZ, *enX;
    ba_huber hp;
    ba_layout lay;
    /* (R) = elements of the working precision: double, or float when real32 is set */
    /* per-track state in chunk-track order (the plan's ct_* arrays): H_pp upper (n_ctracks,6) and
     * g_p (n_ctracks,3) (R), the point and its enable flag (n_ctracks,4) in fp32 */
    void *Hpp, *gp;      /* (R) Hpp 16-byte aligned */
    void *chunk_max;     /* (R) (n_chunks + 1) scratch */
    void *lam_p;         /* (R) (1) point-leaf damping value, written by ba_linearize_schur */
    /* partial blocks: (n_slots, d, d) and (n_batches, L, 2, d) scratch (R) */
    void *partials, *img_partials;
    /* back-substitution inputs/outputs: dc (R), dX fp32, dX64 (R) */
    const void* dc; const int32_t* umap; float* dX; void* dX64;
    /* sizes and reductions */
    int64_t n_chunks, n_batches, n_pairs;
    const int32_t *pair_ptr, *pair_src, *img_ptr, *img_src;
    /* outputs (R): image-pair blocks of S (n_pairs,d,d), rhs (n_imgs,d), diag(H_cc) (n_imgs,d) */
    void *S_pairs, *e_img, *dg_img;
    /* optional given residuals / IRLS weights, element (obs, k) at r_in[obs*r_s0 + k*r_s1]
     * (the `residuals`, `w_pts` arguments of solve_delta, ba_solver.py:110); NULL = recompute */
    const float *r_in, *w_in;
    int64_t r_s0, r_s1, w_s0, w_s1;
    float* ct_pt;         /* (n_ctracks,4) scratch written by stage 0: x, y, z, enable */
    int64_t n_ctracks;
    double* core;         /* scratch: per-observation linearisation record (stage 0), the Jacobian core evaluated
                             in fp64: (n_chunks,20,128) doubles, or with real32 (n_chunks,24,128) floats (the
                             same fields rounded to fp32; the pointer is then read as float*) */
    const int32_t *chunk_slots, *chunk_ent, *chunk_eptr;   /* plan: MFMA entry lists of every chunk */
    const int32_t *b_pos_slot;                             /* plan: batch slot at each Schur-kernel place */
    void* pfac;           /* (R) (n_ctracks,12) 16-byte aligned scratch written by stage 0: Cholesky factor L of H_pp +
                             lam_p I (upper storage), w = L^-1 g_p, reciprocal pivots */
    const int32_t* b_order;  /* plan: batches in dispatch order (most expensive first); NULL = 0, 1, ... */
    int32_t* work_ctr;       /* 1 int of device scratch: the camera-pair kernel's batch queue (one
                                workgroup per CU); NULL = one workgroup per batch */
    const void* dc_img;      /* optional (R) (n_imgs, d): delta_c at image level (dc[umap], 0 where umap is
                                -1), read by the back-substitution instead of dc through umap */
    /* 0: every (R) array is fp64 (the reference's dtype=torch.float64 solver, engine.py:490); 1: fp32 (its
     * dtype=torch.float32 default, ba_solver.py:22, :37, :128): the Jacobian core and the weighted rows of
     * an observation are evaluated in fp64 and rounded, every product, sum and factor after them is fp32 */
    int32_t real32;
} ba_lin_args;

/* Stages 1-3: point blocks, camera-pair Schur blocks, rhs and diag(H_cc) at image level.
 * Requires d <= 15 and C <= 24. */
int ba_linearize_schur(const ba_lin_args* args, void* stream);

/* The same work split in its three launch groups (callers that time the camera-pair
 * kernel on its own): 0 point blocks + damping, 1 camera-pair batches, 2 reductions. */
int ba_linearize_stage(const ba_lin_args* args, int32_t stage, void* stream);

/* Stage 4b: delta_p = (H_pp + lam_p I)^-1 (g_p - H_pc delta_c) per track, written to dX
 * (n_tracks,3) fp32 (and dX64 if not NULL); dc is the reduced solution, umap the
 * (n_imgs, d) image-parameter -> unknown index map (-1 = inactive). */
int ba_backsubstitute(const ba_lin_args* args, void* stream);

/* ------------------------------------------------------------------ pair-major linearize + Schur */
/* The same reduced system as ba_linearize_schur (S blocks per image pair, rhs and diag(H_cc) per
 * image, point blocks per track), built without chunks or batches, so that tracks of any length, up
 * to 31 image-level parameters and any co-visibility pattern are handled (the batched path needs
 * d <= 15, tracks within 13 images and 128 observations, and is slow on random co-visibility).
 * Structure from ba_pm_plan_create (host) or ba_pm_dplan_create (device); a run is the observations of
 * one track in one image:
 *   per observation       J_p^T J_p and J_p^T W r (pobs); per wave of BA_PM_SPAN observations and
 *                         image, sum J_c^T J_c and J_c^T W r (jslots, MFMA)
 *   per track             H_pp, g_p in image order; the point-leaf damping; L, L^-1 g_p
 *   per run (t, i)        V_ti = (sum J_c^T J_p) L^-T (V, 3 x dp per run); per wave of BA_PM_SPAN
 *                         runs and image, sum V V^T and V L^-1 g_p (vslots, MFMA)
 *   per image i           S_ii, rhs and diag(H_cc) from its slots, summed in wave order
 *   per image pair (i, j) S_ij = - sum_t V_ti V_tj^T over the pair's terms (one wave, MFMA)
 * Replaces the same reference work as ba_linearize_schur (ba_solver.py:110-206). */
void* ba_pm_plan_create(const int32_t* cum_nkpts, int32_t n_imgs, const int32_t* pids, int64_t n_obs,
                        int32_t n_tracks);
int ba_pm_plan_query(const void* plan, int64_t* scalars, int64_t* array_sizes);
int ba_pm_plan_export(const void* plan, int32_t which, int32_t* host_dst);
void ba_pm_plan_destroy(void* plan);
/* The same plan built on the device, array for array equal to ba_pm_plan_create's (the reference derives
 * this structure with torch.unique / index_add_ on every solve, ba_solver.py:877-909): cum_nkpts (n_imgs)
 * and pids (n_obs) are device arrays; the plan owns its device arrays (hipMalloc) until
 * ba_pm_dplan_destroy.  Runs on `stream` and synchronises it while it sizes its arrays (once per
 * structure, never inside a solve).  NULL on error: ba_pm_dplan_last_error() says why. */
void* ba_pm_dplan_create(const int32_t* cum_nkpts, int32_t n_imgs, const int32_t* pids, int64_t n_obs,
                         int32_t n_tracks, void* stream);
int ba_pm_dplan_query(const void* plan, int64_t* scalars, int64_t* array_sizes);
const int32_t* ba_pm_dplan_array(const void* plan, int32_t which);
/* array `which` (BA_PM_* order) into a device buffer of at least its length, on `stream` */
int ba_pm_dplan_copy(const void* plan, int32_t which, int32_t* dst, void* stream);
void ba_pm_dplan_destroy(void* plan);
const char* ba_pm_dplan_last_error(void);

typedef struct {
    /* structure: the pair-major plan's arrays (device) */
    const int32_t* infos; int32_t n_imgs; int32_t n_tracks;
    const int32_t *run_ptr, *run_obs, *run_trk, *run_img, *img_run_ptr, *trk_run_ptr, *trk_run, *trk_obs_ptr,
        *trk_obs, *obs_img, *pair_i1, *pair_i2, *diag_pair, *term_ptr, *term;
    const int32_t* pair_sched;               /* optional: the order k_pm_pairs takes the pairs in (NULL = pair order) */
    int64_t n_obs, n_runs, n_pairs;
    /* observations in their own (image-major) order */
    const int32_t* pids; const float *pix2d, *pix2d_std, *pix2d_dep;
    /* parameters */
    const float* K; const float* P_rig2cam; int64_t P_rig2cam_stride; const float* P_w2rig;
    const float* z_coefs; const float* pts3d;
    const uint8_t *enK, *enP, *enZ, *enX;    /* optional enable masks (NULL = all on) */
    ba_huber hp;
    ba_layout lay;                           /* d <= 31 */
    const float *r_in, *w_in;                /* optional given residuals / weights, as in ba_lin_args */
    int64_t r_s0, r_s1, w_s0, w_s1;
    /* workspace; (R) = elements of the working precision: double, or float when real32 is set */
    void* pobs;                              /* (R) (n_obs, 9) */
    float* wobs;                             /* (n_obs, 4) 16-byte aligned: sqrt(W) per residual row */
    void *jslots, *vslots;                   /* (R) per-wave image sums: ba_pm_slot_doubles(n_obs | n_runs, n_imgs, d) */
    void* yrun;                              /* unused (may be NULL): kept so that the layout stays the same */
    void *Hpp, *gp;                          /* (R) (n_tracks, 6) 16-byte aligned, (n_tracks, 3) */
    void* tmax;                              /* (R) (ceil(n_tracks / 256) + 1) */
    void* lam_p;                             /* (R) (1) point-leaf damping value */
    void* pfac;                              /* (R) (n_tracks, 16) 32-byte aligned (16 in fp32): L, L^-1 g_p, reciprocal
                                              * pivots and the point, per track */
    void* V;                                 /* (R) (n_runs, 3, dp), dp = 16 for d <= 15 else 32 */
    /* outputs (R): (n_pairs, d, d), (n_imgs, d), (n_imgs, d) */
    void *S_pairs, *e_img, *dg_img;
    /* back-substitution: delta_c at image level (R) (n_imgs, d), point steps (n_tracks, 3) in fp32 and,
     * optionally, in the working precision (R) */
    const void* dc_img; float* dX; void* dX64;
    /* 0: every (R) array is fp64 (the reference's dtype=torch.float64 solver, engine.py:490); 1: fp32
     * throughout (its dtype=torch.float32 default, ba_solver.py:22, :37, :128): the Jacobian core is
     * evaluated in fp64 and rounded, every product, sum and factor after it is fp32 */
    int32_t real32;
} ba_pm_args;

int ba_pm_linearize_schur(const ba_pm_args* args, void* stream);
/* the same in two launches sequences: stage 0 = observations, tracks, damping, point factors, runs and
 * per-image blocks; stage 1 = the off-diagonal pair blocks (k_pm_pairs), for timing them apart */
int ba_pm_linearize_stage(const ba_pm_args* args, int stage, void* stream);
/* doubles of one slot array of ba_pm_args (n_items = n_obs for jslots, n_runs for vslots); -1 for d
 * outside 1..31 */
int64_t ba_pm_slot_doubles(int64_t n_items, int32_t n_imgs, int32_t d);
/* delta_p = L^-T (L^-1 g_p - sum_i V_ti^T delta_c(i)) per track (= (H_pp + lam_p I)^-1 (g_p - H_pc delta_c)) */
int ba_pm_backsubstitute(const ba_pm_args* args, void* stream);

/* ------------------------------------------------------------------ reduced system (PCG) */
typedef struct {
    int64_t n_u;                       /* active unknowns */
    int32_t n_imgs, d;                 /* d <= 32 */
    const int32_t *umap;               /* (n_imgs, d) -> unknown or -1 */
    const int32_t *inv_ptr, *inv_src;  /* unknown -> list of image-level entries (i*d + j) */
    const int32_t *leaf;               /* (n_u) 0 foc, 1 tau, 2 zcf */
    const int32_t *row_ptr, *row_ent;  /* image rows of the pair structure: (pair << 1) | transposed */
    const int32_t *pair_i1, *pair_i2;
    const void *S_pairs, *e_img, *dg_img; /* (R) */
    double dampen; int32_t adaptive;
    int32_t maxiter; double tol;
    /* workspace, (R) = the working precision (double, or float when real32 is set); p holds 2 * n_u
     * (the search direction, double-buffered) */
    void *rhs, *diagA, *damp, *x, *xbest, *r, *z, *p, *y_img;   /* (R) */
    void *partials;                    /* (R) ba_pcg_partials_size(n_u) elements */
    void *state;                       /* (R) 16 elements */
    int32_t *istate;                   /* 8 ints: [0], [1] done flags, [2] iterations, [3] converged,
                                          [4] best iteration, [5] best iterate returned */
    void *S_rows;                      /* (R) (n_row_ent, d, d): the pair blocks copied per image row */
    int64_t n_row_ent;                 /* row_ptr[n_imgs] */
    int32_t *row_u;                    /* (n_row_ent, 16 if d <= 16 else 32) workspace: the unknowns each image-row
                                          block multiplies */
    const int32_t *long_u;             /* the unknowns whose inv list has more than BA_PCG_LONG_LIST entries,
                                          every one of them, ascending (e.g. a focal pair shared by many images) */
    int64_t n_long;
    const int32_t *long_ptr;           /* (ceil(n_u / 256) + 1): long_u[long_ptr[b] .. long_ptr[b + 1]) lie in
                                          [256 b, 256 b + 256) */
    const int32_t *long_idx;           /* (n_u): k - long_ptr[u / 256] for u = long_u[k], else -1 */
    void *img_part;                    /* (R) (n_imgs) workspace: per image row partial of p.Ap */
    /* optional (NULL = follow inv_ptr / inv_src): the lists pre-resolved, one dependent load fewer */
    const int32_t *src1;               /* (n_u): the only entry of u's inv list when it has exactly one,
                                          else -1 */
    const int32_t *long_rng;           /* (2 n_long): the inv-list bounds of long_u[k] */
    int32_t row_cap;                   /* 0: S_rows / row_u hold row i's blocks at [row_ptr[i], row_ptr[i+1]);
                                          > 0 (a multiple of 8, at least every row's length): at
                                          [i row_cap, (i+1) row_cap), the rest zero blocks with unknown -1,
                                          and S_rows / row_u sized for n_imgs * row_cap blocks */
    int32_t real32;                    /* 0: (R) = double; 1: (R) = float, the reference's fp32 _pcg
                                          (ba_solver.py:1197-1238 on its dtype=torch.float32 operator);
                                          ba_reduced_solve takes 0 only */
} ba_pcg_args;

#define BA_PCG_LONG_LIST 32

/* Builds the unknown-level rhs, diag(A) with per-leaf damping (ba_solver.py:575-582,
 * :1188-1191) and runs Jacobi-PCG (ba_solver.py:184-206, :1197-1238) on
 * S = P^T S_img P + damping, entirely on the device (two launches per iteration, no host
 * synchronisation).  The result (the converged iterate, else the best one) is left in x;
 * istate holds the loop's outcome. */
int ba_pcg_solve(const ba_pcg_args* args, void* stream);
/* ba_pcg_solve in parts, for a caller that stops launching once the loop has stopped (the reference's loop
 * checks its stopping rule on the host after every iteration, ba_solver.py:1216-1236; launched in full, the
 * iterations after the stop return at once but still cost a launch each): the setup when it0 == 0, then
 * iterations [it0, it1) (0 <= it0 <= it1 <= maxiter); with finish, the decisions after update it1 - 1 and the
 * result (valid when it1 == maxiter or when the loop has stopped before update it1); else, when stopped_out
 * is not NULL, a last kernel stores the flag "stopped before update it1" (0 or 1) to *stopped_out with a
 * system-scope store (pinned host memory).  ba_pcg_solve(a) = ba_pcg_solve_range(a, 0, maxiter, 1, NULL). */
int ba_pcg_solve_range(const ba_pcg_args* args, int32_t it0, int32_t it1, int32_t finish, int32_t* stopped_out,
                       void* stream);
/* The device address of pinned, mapped host memory (hipPointerGetAttributes), or NULL when the device cannot
 * reach it: the stopped_out target of ba_pcg_solve_range (no counterpart in the reference). */
void* ba_host_mapped_ptr(const void* host_ptr);
int64_t ba_pcg_partials_size(int64_t n_u);

/* ------------------------------------------------------------------ reduced system (direct solve) */
/* Direct solve of S_u delta_c = rhs with S_u = P^T S_img P + diag(damp), the system ba_pcg_solve
 * iterates on.  Replaces the reference's explicit-Schur solve GaussNewtonSolver._solve_dense_S
 * (ba_solver.py:208-226: S = A - B D^-1 C, torch.linalg.solve(S, rhs) at :220).  S_u is symmetric
 * positive definite (fp64, damped), so it is factored L L^T: densely (mode 0, any structure), or, when
 * every image pair lies within w images and few unknowns are shared, as a block band of width w with
 * the shared unknowns as a dense border (mode 1: by block cyclic reduction over super-blocks of
 * 128 unknowns when w db <= 128 and n_shared <= 15, else by one workgroup walking the images;
 * mode 2: always the one-workgroup walk). */
typedef struct {
    int32_t mode;                /* 0: dense (any structure); 1: banded with a dense border (cyclic reduction
                                    where it applies); 2: banded, one workgroup */
    double* A;                   /* dense: (lda, lda) workspace; the lower triangle of S_u, then L below the
                                    diagonal blocks */
    int64_t lda;                 /* dense: ba_chol_dense_lda(n_u) (n_u rounded up to 128) */
    double* Linv;                /* dense: (lda / 128, 128, 128) inverses of the diagonal blocks of L */
    const int32_t* pair_idx;     /* (n_imgs, n_imgs): the pair id of images (i, j), i <= j, or -1 */
    const int32_t* kind;         /* (n_u): 1 local (one image-level entry), 2 shared (several: a mono
                                    camera's focal pair, a rig node), 0 isolated (none) */
    const int32_t* shared_u;     /* (n_shared): the shared unknowns */
    int32_t n_shared;            /* banded: at most 15 (cyclic reduction) or 8 (one workgroup) */
    int32_t w;                   /* banded: every image pair (i, j) has |i - j| <= w (>= 1); cyclic reduction:
                                    w db <= 128; one workgroup: (w + 1) db <= 160 and
                                    ba_chol_band_lds_bytes(db, w, n_shared) <= 160 KB */
    int32_t db;                  /* banded: block size, the number of image-level columns that carry a
                                    local unknown in some image (a mono camera's focal pair is left out) */
    const int32_t* bcol;         /* banded: (db) image-level column of each band column */
    const int32_t* bpos;         /* banded: (d) band column of each image-level column, or -1 */
    int64_t n_pairs;             /* image pairs of the structure (pair_i1 / pair_i2 of ba_pcg_args) */
    int32_t* info;               /* (1): INT32_MAX when every pivot was positive, else the first column
                                    (1-based) whose pivot was not (replaced by 1 to keep the sweep finite) */
    double* work;                /* ba_chol_work_doubles(mode, n_u, n_imgs, d (db when banded), w, n_shared) */
} ba_chol_args;

int64_t ba_chol_dense_lda(int64_t n_u);
/* LDS bytes of the banded layout's workgroup (d = db); mode 1 requires at most 160 KB */
int64_t ba_chol_band_lds_bytes(int32_t d, int32_t w, int32_t n_shared);
int64_t ba_chol_work_doubles(int32_t mode, int64_t n_u, int32_t n_imgs, int32_t d, int32_t w, int32_t n_shared);
/* super-blocks of mode 1's cyclic reduction for this structure (d = db), or 0 when mode 1 runs the
 * one-workgroup factor (no counterpart in the reference: a layout query) */
int32_t ba_chol_band_superblocks(int32_t d, int32_t w, int32_t n_shared, int32_t n_imgs);

/* Uses every field of ba_pcg_args that the unknown-level setup of ba_pcg_solve uses (umap, inv lists,
 * leaf, S_pairs, e_img, dg_img, dampen / adaptive, rhs, diagA, damp, state) and writes delta_c to
 * args->x, like the PCG; istate (if set) reports 0 iterations and "converged" = every pivot positive. */
int ba_reduced_solve(const ba_pcg_args* args, const ba_chol_args* chol, void* stream);

/* ------------------------------------------------------------------ LM step (update + line search) */

/* One trial of the lm_step update (engine.py:310-313, :347-354, cujac/__init__.py:56-58):
 *   K_out = K with fx, fy <- max(f - scale*dK, min_f)     dK (n_cams,2)
 *   P_out = exp_se3(-scale*dP) @ P_w2rig                   dP (n_nodes,6) = [w|v]
 *   z_out = z_coefs - scale*dZ                             dZ (n_imgs,C)
 *   X_out = pts3d - scale*dX                               dX (n_tracks,3)
 * fp32 in and out; the outputs may not alias the inputs. */
int ba_apply_update(const float* K, const float* P_w2rig, const float* z_coefs, const float* pts3d,
                    const float* dK, const float* dP, const float* dZ, const float* dX, float scale, float min_f,
                    int32_t n_cams, int32_t n_nodes, int32_t n_imgs, int32_t C, int64_t n_tracks, float* K_out,
                    float* P_out, float* z_out, float* X_out, void* stream);

/* Bytes of device workspace ba_objective needs for n_obs observations. */
int64_t ba_objective_workspace_bytes(int64_t n_obs);

/* Line-search objective of lm_step (engine.py:263-278, :357-361) from the residual buffer of
 * ba_residuals (has_err != 0: (9,n_obs) rows r|err|w; else (3,n_obs) rows r):
 *   out[0] = mean(err) (fp32 result of an fp64 sum), out[1] = reproj_score = mean of the lowest
 *   80% of ||(r0,r1)|| (exact selection on the fp32 values, no sort).  out is device memory. */
int ba_objective(const float* res, int64_t n_obs, int32_t has_err, void* workspace, float* out, void* stream);

/* ba_objective without a workspace argument and without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The passes recompute each observation's
 * key from res instead of storing it, and keep their partial sums (at most 2048 blocks) in a static
 * per-GPU scratch array of 42 KB, so every n_obs fits (up to the 32-bit rank limit that
 * ba_objective shares: n_obs <= 5368709119, rejected with an error beyond).  Outputs equal
 * ba_objective's bit for bit.  All calls on one GPU share its scratch array: calls that overlap on
 * one GPU (other streams, other threads) race and must be serialised by the caller. */
int ba_objective_noalloc(const float* res, int64_t n_obs, int32_t has_err, float* out, void* stream);

/* lm_step's input checks, `assert tensor.isfinite().all()` on every input (engine.py:340-344), for up
 * to BA_NONFINITE_MAX_SPANS fp32 arrays in one launch: flags[t] (device, int32) = 1 when
 * ptrs[t][0 .. counts[t]) holds a NaN or an infinity, else 0.  int32 inputs are finite by type. */
#define BA_NONFINITE_MAX_SPANS 16
int ba_nonfinite_flags(const float* const* ptrs, const int64_t* counts, int32_t n_spans, int32_t* flags,
                       void* stream);

/* Measurement helper with no counterpart in the reference: STREAM triad a = b + s c over n fp64
 * values (16-byte aligned device arrays), whose bandwidth the benchmark reports as the achievable
 * HBM figure beside the roofline fractions. */
int ba_stream_triad(double* a, const double* b, const double* c, double s, int64_t n, void* stream);

/* ------------------------------------------------------------------ F sampling */

/* Multi-depth values at the observations (replaces the per-image bilinear_sampling calls of
 * gather_data_from_dense_tracks, src/blast3r/inference/tracks.py:865-872, and
 * src/blast3r/utils/geometry.py:167-198: grid_sample bilinear, padding 'border',
 * align_corners=False, pixel (i, j) centred at (i + .5, j + .5)).
 * Observation o belongs to image img(o) = upper bound of o in cum_nppi (image-major order,
 * rigs.py:50-51); its row of out is the bilinear sample of that image's map at pix2d[o]. */
typedef struct {
    const int64_t* map_addr;   /* (n_imgs,) device addresses of the maps, each (H, W, Cm) fp32 row-major */
    const int32_t* map_hw;     /* (n_imgs, 2) per-image H, W; null when every map is H x W */
    int32_t H, W;              /* map size when map_hw is null */
    int32_t Cm;                /* channels sampled per map, 1..1024 */
    int32_t pix_stride;        /* floats from one pixel to the next (rows are W * pix_stride apart);
                                  0 means Cm.  A channel slice of a wider map, e.g. raw[..., 2:], is
                                  sampled in place with map_addr at its first channel */
    int32_t insert_ones;       /* 1: out column 1 is a sampled constant-one channel and map channel c >= 1
                                  goes to column c + 1 (the stack [F0, 1, F1, ...] of multidepth.py:53-54) */
    const int32_t* cum_nppi;   /* (n_imgs,) inclusive cumulative observation counts (infos row 0) */
    int64_t n_imgs;
    const float* pix2d;        /* (n_obs, 2) pixel coordinates x, y */
    int64_t n_obs;
    float* out;                /* (n_obs, Cm + insert_ones) fp32 */
} ba_sample_args;

int ba_sample_depth(const ba_sample_args* args, void* stream);

/* ------------------------------------------------------------------ observation structure (layout builder) */

/* One image-major observation set (ObservedTracks, src/blast3r/inference/tracks.py:19-57):
 * rows of image i follow those of image i - 1; nppi[i] rows per image. */
typedef struct {
    const int32_t* pids;       /* (n_rows,) track ids */
    const float* pix2d;        /* (n_rows, 2) */
    const float* pix2d_std;    /* (n_rows, 2) */
    const float* pix2d_dep;    /* (n_rows, C) */
    const int32_t* nppi;       /* (n_imgs,) rows per image */
    int64_t n_imgs;
} ba_obs_set;

/* Image-wise gather.  Output image j holds the rows of image sel_a[j] of set a, then the rows of
 * image sel_b[j] of set b with pid_shift_b added to their track ids (-1 or an index past the set's
 * images selects nothing).  Replaces `old | new` (tracks.py:84-102: sel_a[j] = j for the old images,
 * -1 for the new last one, sel_b[j] = j, shift = old n_tracks) and `tracks[idx]` for an index tensor
 * (tracks.py:66-74: sel_a = idx, sel_b = null).  Output buffers hold n_rows rows, the total the
 * caller expects; *total (device, may be null) receives the total the selection really has, and
 * rows past n_rows are not written. */
typedef struct {
    ba_obs_set a, b;
    const int32_t* sel_a;      /* (n_out,) or null */
    const int32_t* sel_b;      /* (n_out,) or null (then set b is not read) */
    int32_t pid_shift_b;
    int32_t C;                 /* depth channels of both sets */
    int64_t n_out;             /* output images */
    int64_t n_rows;
    int32_t* pids;             /* outputs: (n_rows,), (n_rows, 2), (n_rows, 2), (n_rows, C), (n_out,) */
    float* pix2d;
    float* pix2d_std;
    float* pix2d_dep;
    int32_t* nppi;
    int64_t* total;
    void* workspace;           /* ba_tracks_workspace_bytes(n_rows, 0, max(n_out, images of a and b)) */
} ba_gather_args;

int ba_tracks_gather(const ba_gather_args* args, void* stream);

/* Track removal (ObservedTracks.remove, tracks.py:116-127): rows whose track id is listed in bad
 * (int32 or int64 ids, any order, repeats allowed; ids matching no row are ignored, as torch.isin)
 * are dropped; the remaining rows keep their order, nppi counts them per image, and each kept
 * track is renumbered by its rank among the tracks that still have a row (torch.unique's sorted
 * values and inverse).  old_to_keep[k] = old id of new track k.  counts (device) = {tracks kept,
 * rows kept}; the outputs are sized for the input (every row / track kept). */
typedef struct {
    ba_obs_set in;
    int64_t n_rows;            /* rows of the input set */
    int64_t n_tracks;
    int32_t C;
    int32_t bad_int64;         /* bad holds int64 ids (else int32) */
    const void* bad;
    int64_t n_bad;
    int32_t* pids;             /* outputs: (n_rows,), (n_rows, 2), (n_rows, 2), (n_rows, C), (n_imgs,), (n_tracks,), (2,) */
    float* pix2d;
    float* pix2d_std;
    float* pix2d_dep;
    int32_t* nppi;
    int32_t* old_to_keep;
    int64_t* counts;
    void* workspace;           /* ba_tracks_workspace_bytes(n_rows, n_tracks, n_imgs) */
} ba_remove_args;

int ba_tracks_remove(const ba_remove_args* args, void* stream);

/* ObservedTracks.to_dense(n_imgs_out) (tracks.py:104-114): out (n_imgs_out, n_tracks, 2) fp32 is
 * NaN except out[i, pids[o]] = pix2d[o] for the rows o of image i (the caller views it transposed). */
int ba_tracks_to_dense(const int32_t* pids, const float* pix2d, const int32_t* nppi, int64_t n_imgs, int64_t n_rows,
                       int64_t n_tracks, int64_t n_imgs_out, float* out, void* workspace, void* stream);

/* ObservedTracks.img_id (tracks.py:45-49): out[o] = number of distinct delimiters cumsum(nppi)[:-1]
 * at or before row o (int64).  Delimiters that coincide (empty images) count once, as in the
 * reference's assignment res[delims] = 1; the caller rejects a delimiter equal to n_rows, which the
 * reference's indexing rejects. */
int ba_tracks_img_id(const int32_t* nppi, int64_t n_imgs, int64_t n_rows, int64_t* out, void* workspace, void* stream);

/* Workspace of the four calls above (bytes). */
int64_t ba_tracks_workspace_bytes(int64_t n_rows, int64_t n_tracks, int64_t n_imgs);

/* ------------------------------------------------------------------ dense tangent prior */

/* _dense_tangent_prior_terms (src/blast3r/inference/engine.py:15-179) for every image at once:
 * the combined log-depth exp(min(sum_c z_c L_c, 80)) of the image's maps and its reference
 * pointmap, both sampled at rows / columns s//2 + s k, give unit-tangent residuals along rows and
 * columns weighted by the planar confidence of the pointmap's depth (engine.py:182-200).
 *   loss (1,): sum over images of weight * mean(w r^2) per direction, in the working precision;
 *   g_z (n_imgs, C), H_z (n_imgs, C, C): Gauss-Newton terms w.r.t. z_coefs (compute_gn), with
 *   column / row 0 zeroed when optim_Z0 is 0.
 * Images whose subsampled width or channel count is below 2 contribute nothing (engine.py:75).
 * fp64 selects the working precision (the reference's dtype argument); the pointmap tangents and
 * the confidence stay fp32 either way, as in the reference; sums are fp64. */
typedef struct {
    const int64_t* depth_addr; /* (n_imgs,) device address of each image's log-depth map (H_i, W_i, >= C) fp32,
                                  pixels depth_pix_stride floats apart, rows W_i pixels apart; channel c at +c */
    const int64_t* ref_addr;   /* (n_imgs,) address of each image's reference pointmap (H_i, W_i, 3) fp32,
                                  pixels ref_pix_stride floats apart */
    const int32_t* map_hw;     /* (n_imgs, 2) per-image H_i, W_i, or null when every map is H x W */
    int32_t H, W;              /* the map size, or the largest H_i and W_i when map_hw is given */
    int32_t depth_pix_stride;
    int32_t ref_pix_stride;
    const float* K;            /* (n_cams, 3, 3) */
    const int32_t* cam_ids;    /* (n_imgs,) camera of each image (rigs row 2) */
    const float* z_coefs;      /* (n_imgs, C) */
    int64_t n_imgs;            /* 1..65535 */
    int32_t C;                 /* z-coefficients (channels used), <= 16 with compute_gn */
    int32_t tan_stride;
    int32_t normalize;         /* normalize_tangents */
    int32_t optim_Z0;
    int32_t fp64;              /* working precision of loss / g_z / H_z: 0 fp32, 1 fp64 */
    int32_t compute_gn;
    double weight;             /* weight_tan */
    double eps;
    void* loss;
    void* g_z;
    void* H_z;
    void* workspace;
    int64_t workspace_bytes;   /* >= ba_tangent_workspace_bytes(n_imgs, C, H, W, tan_stride, normalize, compute_gn) */
} ba_tangent_args;

int ba_tangent_prior(const ba_tangent_args* args, void* stream);
int64_t ba_tangent_workspace_bytes(int64_t n_imgs, int32_t C, int32_t H, int32_t W, int32_t tan_stride,
                                   int32_t normalize, int32_t compute_gn);

/* confident_in_planar_regions (engine.py:182-200) of one (H, W) fp32 map: exp(-alpha (lx^2 + ly^2)) with
 * lx, ly the row / column Laplacians (one-sided at the borders) divided by the 3x3 minimum
 * (at least 1e-12). */
int ba_planar_confidence(const float* D0, int32_t H, int32_t W, float alpha, float* out, void* stream);

/* z_prior injection (ba_solver.py:141-173) into the image-level reduced system before damping:
 * S_pairs[diag_pair[i]][o + c][o + d] += H_z[i][c][d], e_img[i][o + c] += g_z[i][c],
 * dg_img[i][o + c] += H_z[i][c][c], for the n_imgs images (d x d blocks, o = d - C); every array fp64, or
 * fp32 when real32 is set (the reduced system of the pair-major path's fp32 solver). */
int ba_add_z_prior(void* S_pairs, const int32_t* diag_pair, void* e_img, void* dg_img, const void* H_z,
                   const void* g_z, int64_t n_imgs, int32_t d, int32_t C, int32_t real32, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* BA_HIP_H */
