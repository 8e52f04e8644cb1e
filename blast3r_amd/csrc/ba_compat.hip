// Operator-level entry points with the semantics of the reference cujac module
// (src/blast3r/extensions/cujac/sfm_jacobian_rigs.cu, ".cu" below; Python
// aliases in src/blast3r/extensions/cujac/__init__.py:18-22, :56-58).
// These let the reference's own solver run on MI355X unchanged; the fused
// linearize + Schur path lives in ba_schur.hip.
#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>
#include <cmath>
#include <string>

#include "ba_common.h"
#include "ba_error.h"

namespace ba {
static thread_local std::string g_err;
void set_error(const std::string& msg) { g_err = msg; }
void clear_error() { g_err.clear(); }
}  // namespace ba

using namespace ba;

extern "C" const char* ba_last_error(void) { return ba::g_err.c_str(); }
extern "C" int ba_version(void) { return 1; }

static inline hipStream_t S(void* s) { return (hipStream_t)s; }
static inline unsigned nblk(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

// ----------------------------------------------------------------------------- residuals
// One block per RES_T * RES_K consecutive observations (RES_K per thread, RES_T apart, so every load
// and store is coalesced).  The observations of a block are image-sorted, so its images form the range
// [lo, hi], found by two searches per block; the cameras and z-coefficients of the first RES_NI images
// of that range are staged in LDS (blocks over more images read the rest from memory).  All loads of a
// thread's RES_K observations are issued before any of them is evaluated.  The per-observation
// arithmetic is eval_residual's, in the reference's order (.cu:129-259).
constexpr int RES_T = 256, RES_K = 4, RES_NI = 4, RES_ZC = 32;

__device__ __forceinline__ int obs_image_in(const int* __restrict__ cum, int lo, int hi, int idx) {
    int a = lo, b = hi + 1;                  // cum[a - 1] <= idx < cum[a], a in [lo, hi]
    while (b - a > 1) {
        int m = (a + b) >> 1;
        if (idx < cum[m - 1]) b = m; else a = m;
    }
    return a;
}

__global__ void __launch_bounds__(RES_T) k_residuals(const int* __restrict__ infos, int n_imgs, const float* __restrict__ K,
                                                     const float* __restrict__ Prc, int64_t prc_stride,
                                                     const float* __restrict__ Pwr, const float* __restrict__ zc,
                                                     const float* __restrict__ pts, const int* __restrict__ pids,
                                                     const float* __restrict__ pix, const float* __restrict__ sd,
                                                     const float* __restrict__ dep, int64_t n_obs, int C, HuberParams hp,
                                                     float* __restrict__ out) {
    __shared__ int s_rng[2];
    __shared__ CamF s_cam[RES_NI];
    __shared__ float s_zc[RES_NI * RES_ZC];
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * (RES_T * RES_K);
    const int64_t last = (base + RES_T * RES_K < n_obs ? base + RES_T * RES_K : n_obs) - 1;
    if (tid == 0) s_rng[0] = obs_image(infos, n_imgs, (int)base);
    if (tid == 64) s_rng[1] = obs_image(infos, n_imgs, (int)last);
    __syncthreads();
    const int lo = s_rng[0], hi = s_rng[1];
    const int nst = hi - lo + 1 < RES_NI ? hi - lo + 1 : RES_NI;
    const bool zc_lds = C <= RES_ZC;
    if (tid < nst) {
        CamF c;
        load_cam(c, K, Prc, prc_stride, Pwr, infos[2 * n_imgs + lo + tid], infos[n_imgs + lo + tid]);
        s_cam[tid] = c;
    }
    if (zc_lds && tid < nst * C) s_zc[tid] = zc[(int64_t)lo * C + tid];
    // every load of the thread's observations (indices clamped into range; only stores are guarded)
    int64_t idx[RES_K];
    int pid[RES_K], img[RES_K];
    float2 uv[RES_K], sv[RES_K];
    float X[RES_K][3];
#pragma unroll
    for (int k = 0; k < RES_K; ++k) {
        const int64_t i = base + k * RES_T + tid;
        idx[k] = i < n_obs ? i : n_obs - 1;
        pid[k] = pids[idx[k]];
        uv[k] = reinterpret_cast<const float2*>(pix)[idx[k]];
        sv[k] = reinterpret_cast<const float2*>(sd)[idx[k]];
        img[k] = lo == hi ? lo : obs_image_in(infos, lo, hi, (int)idx[k]);
    }
#pragma unroll
    for (int k = 0; k < RES_K; ++k) {
        const float* x = pts + 3 * (int64_t)pid[k];
        X[k][0] = x[0]; X[k][1] = x[1]; X[k][2] = x[2];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < RES_K; ++k) {
        const int li = img[k] - lo;
        CamF cp;
        if (li < RES_NI) cp = s_cam[li];
        else load_cam(cp, K, Prc, prc_stride, Pwr, infos[2 * n_imgs + img[k]], infos[n_imgs + img[k]]);
        const float* zi = zc_lds && li < RES_NI ? s_zc + li * C : zc + (int64_t)img[k] * C;
        float g = 0.f;
        for (int c = 0; c < C; ++c) g += zi[c] * dep[idx[k] * C + c];
        ResOut o;
        eval_residual(cp, X[k], uv[k].x, uv[k].y, sv[k].x, sv[k].y, g, hp, o);
        if (base + k * RES_T + tid < n_obs) {
            const int64_t i = idx[k];
#pragma unroll
            for (int r = 0; r < 3; ++r) __builtin_nontemporal_store(o.r[r], out + r * n_obs + i);
            if (hp.pnorm > 0.f) {
#pragma unroll
                for (int r = 0; r < 3; ++r) {
                    __builtin_nontemporal_store(o.err[r], out + (3 + r) * n_obs + i);
                    __builtin_nontemporal_store(o.w[r], out + (6 + r) * n_obs + i);
                }
            }
        }
    }
}

// Replaces residuals_with_rigs (.cu:1048-1101).  out is (n_out, n_obs) fp32, n_out = 9 if
// pnorm > 0 else 3; every element is written (rows with z <= 1e-3 get zeros, .cu:212).
extern "C" int ba_residuals(const int32_t* infos, int32_t n_imgs, const float* K, const float* P_rig2cam,
                            int64_t P_rig2cam_stride, const float* P_w2rig, const float* z_coefs, const float* pts3d,
                            const int32_t* pids, const float* pix2d, const float* pix2d_std, const float* pix2d_dep,
                            int64_t n_obs, int32_t C, int32_t is_depth_log, float weight_z, float pnorm,
                            float max_pix_err, float huber_delta, float w_pts_null, float* out, void* stream) {
    clear_error();
    BA_REQUIRE(pnorm == -1.f || (pnorm > 0.f && pnorm <= 2.f), "pnorm must be in {-1} U ]0,2]");
    BA_REQUIRE(n_imgs > 0 && C >= 0 && n_obs >= 0, "bad sizes");
    if (n_obs == 0) return BA_OK;
    HuberParams hp{weight_z, pnorm, max_pix_err, huber_delta, w_pts_null, is_depth_log};
    hipLaunchKernelGGL(k_residuals, dim3(nblk(n_obs, RES_T * RES_K)), dim3(RES_T), 0, S(stream), infos, n_imgs, K, P_rig2cam,
                       P_rig2cam_stride, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std, pix2d_dep, n_obs, C, hp, out);
    BA_LAUNCHED();
    return BA_OK;
}

// ----------------------------------------------------------------------------- jacobians
template <typename T>
__global__ void __launch_bounds__(256) k_jacobians(const int* __restrict__ infos, int n_imgs, const float* __restrict__ K,
                                                   const float* __restrict__ Prc, int64_t prc_stride,
                                                   const float* __restrict__ Pwr, const float* __restrict__ zc,
                                                   const float* __restrict__ pts, const int* __restrict__ pids,
                                                   const float* __restrict__ sd, const float* __restrict__ dep,
                                                   int64_t n_obs, int C, int is_depth_log, T* __restrict__ Jcam,
                                                   T* __restrict__ Jz, T* __restrict__ Jp) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_obs) return;
    int img = obs_image(infos, n_imgs, (int)idx);
    int node = infos[n_imgs + img];
    int cam = infos[2 * n_imgs + img];
    int pid = pids[idx];
    CamF cp;
    load_cam(cp, K, Prc, prc_stride, Pwr, cam, node);
    float X[3] = {pts[3 * (int64_t)pid], pts[3 * (int64_t)pid + 1], pts[3 * (int64_t)pid + 2]};
    double g = 0.0;   // Tfloat guidance (.cu:466-468): float products accumulated in double
    for (int c = 0; c < C; ++c) {
        float pr = zc[(int64_t)img * C + c] * dep[idx * C + c];
        g += (double)pr;
    }
    float2 sv = reinterpret_cast<const float2*>(sd)[idx];
    JacOut J;
    eval_jacobian(cp, X, sv.x, sv.y, g, is_depth_log, J);
#pragma unroll
    for (int k = 0; k < 24; ++k) Jcam[idx * 24 + k] = (T)J.Jcam[k];
    for (int c = 0; c < C; ++c) Jz[idx * C + c] = J.valid ? (T)(J.zscale * (double)dep[idx * C + c]) : (T)0;
#pragma unroll
    for (int k = 0; k < 9; ++k) Jp[idx * 9 + k] = (T)J.Jp[k];
}

// Replaces jacobians_with_rigs (.cu:1105-1148): J_cam (N,3,8), J_zcf (N,1,C), J_pts (N,3,3),
// fp64 when float64 != 0 else fp32; every element is written.
extern "C" int ba_jacobians(const int32_t* infos, int32_t n_imgs, const float* K, const float* P_rig2cam,
                            int64_t P_rig2cam_stride, const float* P_w2rig, const float* z_coefs, const float* pts3d,
                            const int32_t* pids, const float* pix2d_std, const float* pix2d_dep, int64_t n_obs,
                            int32_t C, int32_t is_depth_log, int32_t float64, void* J_cam, void* J_zcf, void* J_pts,
                            void* stream) {
    clear_error();
    BA_REQUIRE(n_imgs > 0 && C >= 0 && n_obs >= 0, "bad sizes");
    if (n_obs == 0) return BA_OK;
    if (float64)
        hipLaunchKernelGGL(k_jacobians<double>, dim3(nblk(n_obs, 256)), dim3(256), 0, S(stream), infos, n_imgs, K,
                           P_rig2cam, P_rig2cam_stride, P_w2rig, z_coefs, pts3d, pids, pix2d_std, pix2d_dep, n_obs, C,
                           is_depth_log, (double*)J_cam, (double*)J_zcf, (double*)J_pts);
    else
        hipLaunchKernelGGL(k_jacobians<float>, dim3(nblk(n_obs, 256)), dim3(256), 0, S(stream), infos, n_imgs, K,
                           P_rig2cam, P_rig2cam_stride, P_w2rig, z_coefs, pts3d, pids, pix2d_std, pix2d_dep, n_obs, C,
                           is_depth_log, (float*)J_cam, (float*)J_zcf, (float*)J_pts);
    BA_LAUNCHED();
    return BA_OK;
}

// ----------------------------------------------------------------------------- chol3x3
template <typename T>
__device__ __forceinline__ T bsqrt(T x) { return sqrt(x); }
template <>
__device__ __forceinline__ float bsqrt<float>(float x) { return sqrtf(x); }

template <typename T>
__global__ void __launch_bounds__(256) k_chol3x3(const T* __restrict__ A, const T* __restrict__ b, T* __restrict__ y,
                                                 int64_t n, T jitter) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const T* a = A + i * 9;
    T a00 = a[0] + jitter, a11 = a[4] + jitter, a22 = a[8] + jitter;     // .cu:578-595
    T a01 = (a[1] + a[3]) * T(0.5), a02 = (a[2] + a[6]) * T(0.5), a12 = (a[5] + a[7]) * T(0.5);
    a00 = a00 > T(0) ? a00 : a00 + jitter;                               // .cu:600
    T l00 = bsqrt(a00);
    T l10 = a01 / l00, l20 = a02 / l00;
    T t11 = a11 - l10 * l10;
    t11 = t11 > T(0) ? t11 : t11 + jitter;
    T l11 = bsqrt(t11);
    T l21 = (a12 - l10 * l20) / l11;
    T t22 = a22 - l20 * l20 - l21 * l21;
    t22 = t22 > T(0) ? t22 : t22 + jitter;
    T l22 = bsqrt(t22);
    const T* r = b + i * 3;
    T z0 = r[0] / l00;                                                   // .cu:621-628
    T z1 = (r[1] - l10 * z0) / l11;
    T z2 = (r[2] - l20 * z0 - l21 * z1) / l22;
    T x2 = z2 / l22;
    T x1 = (z1 - l21 * x2) / l11;
    T x0 = (z0 - l10 * x1 - l20 * x2) / l00;
    y[i * 3 + 0] = x0; y[i * 3 + 1] = x1; y[i * 3 + 2] = x2;
}

// Replaces chol3x3_solve (.cu:1151-1169). dtype: 0 fp32, 1 fp64.
extern "C" int ba_chol3x3_solve(const void* blocks, const void* rhs, void* out, int64_t n, double jitter, int32_t dtype,
                                void* stream) {
    clear_error();
    BA_REQUIRE(n >= 0, "bad size");
    if (n == 0) return BA_OK;
    if (dtype == 1)
        hipLaunchKernelGGL(k_chol3x3<double>, dim3(nblk(n, 256)), dim3(256), 0, S(stream), (const double*)blocks,
                           (const double*)rhs, (double*)out, n, jitter);
    else
        hipLaunchKernelGGL(k_chol3x3<float>, dim3(nblk(n, 256)), dim3(256), 0, S(stream), (const float*)blocks,
                           (const float*)rhs, (float*)out, n, (float)jitter);
    BA_LAUNCHED();
    return BA_OK;
}

// ----------------------------------------------------------------------------- block-COO matvec
// y = A x (or A^T x) for A given as n (bh x bw) blocks at block positions (row_idx, col_idx), in any order
// and with repeats.  Output-driven, deterministic and free of atomics:
//   1. each block's output block index becomes a sort key (an index outside [0, n_out) becomes the
//      sentinel n_out, which no output reads);
//   2. the block ids are sorted by key with a stable radix sort over the bits of [0, n_out];
//   3. seg[k] = first sorted position with key >= k (one thread per sorted position writes the keys
//      between its predecessor's and its own), so output block k owns the sorted range [seg[k], seg[k+1]);
//   4. one thread per output element sums its blocks' contributions in ascending block id, then stores y
//      (every element is written, so no clearing pass).
// The sum order is fixed by the input, so repeated calls give bit-identical results.
struct BcooWs {
    uint32_t *keys_in, *keys_out, *ids_in, *ids_out;
    int32_t* seg;
    void* sort_tmp;
    size_t sort_bytes;
    int64_t total;
};

static inline size_t bcoo_align(size_t b) { return (b + 255) & ~(size_t)255; }

static inline unsigned bcoo_bits(int64_t n_out) {
    unsigned b = 1;
    while (b < 32 && ((int64_t)1 << b) <= n_out) ++b;      // keys are in [0, n_out]
    return b;
}

// layout of the caller's workspace; base == nullptr only sizes it
static hipError_t bcoo_layout(void* base, int64_t n, int64_t n_out, hipStream_t st, BcooWs& w) {
    size_t tmp = 0;
    hipError_t e = rocprim::radix_sort_pairs((void*)nullptr, tmp, (uint32_t*)nullptr, (uint32_t*)nullptr,
                                             (uint32_t*)nullptr, (uint32_t*)nullptr, (unsigned)n, 0u,
                                             bcoo_bits(n_out), st);
    if (e != hipSuccess) return e;
    const size_t v = bcoo_align((size_t)n * 4);
    char* p = (char*)base;
    w.keys_in = (uint32_t*)p; w.keys_out = (uint32_t*)(p + v);
    w.ids_in = (uint32_t*)(p + 2 * v); w.ids_out = (uint32_t*)(p + 3 * v);
    w.seg = (int32_t*)(p + 4 * v);
    const size_t segb = bcoo_align((size_t)(n_out + 1) * 4);
    w.sort_tmp = p + 4 * v + segb;
    w.sort_bytes = tmp;
    w.total = (int64_t)(4 * v + segb + bcoo_align(tmp));
    return hipSuccess;
}

template <typename I>
__global__ void __launch_bounds__(256) k_bcoo_keys(const I* __restrict__ out_idx, int64_t n, int64_t n_out,
                                                   uint32_t* __restrict__ keys, uint32_t* __restrict__ ids) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t k = (int64_t)out_idx[i];
    keys[i] = (uint32_t)(k >= 0 && k < n_out ? k : n_out);
    ids[i] = (uint32_t)i;
}

__global__ void __launch_bounds__(256) k_bcoo_bounds(const uint32_t* __restrict__ skeys, int64_t n, int64_t n_out,
                                                     int32_t* __restrict__ seg) {
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s > n) return;
    const int64_t lo = s ? (int64_t)skeys[s - 1] + 1 : 0;
    const int64_t hi = s < n ? (int64_t)skeys[s] : n_out;
    for (int64_t k = lo; k <= hi; ++k) seg[k] = (int32_t)s;
}

template <typename T, typename I>
__global__ void __launch_bounds__(256) k_bcoo_rows(const T* __restrict__ blocks, int bh, int bw,
                                                   const I* __restrict__ in_idx, int64_t n_in,
                                                   const uint32_t* __restrict__ sid, const int32_t* __restrict__ seg,
                                                   int64_t n_out, const T* __restrict__ x, T* __restrict__ y,
                                                   int transpose) {
    const int per = transpose ? bw : bh;             // outputs per output block
    const int len = transpose ? bh : bw;             // inputs per input block
    const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= n_out * per) return;
    const int64_t k = o / per;
    const int e = (int)(o - k * per);
    // element (e, j) of the block as seen from the output side: A[e][j] or A[j][e]
    const int es = transpose ? 1 : bw, js = transpose ? bw : 1;
    T acc = T(0);
    for (int32_t s = seg[k], s1 = seg[k + 1]; s < s1; ++s) {
        const int64_t b = sid[s];
        const int64_t c = (int64_t)in_idx[b];
        if (c < 0 || c >= n_in) continue;            // the reference reads out of bounds here; skip instead
        const T* A = blocks + b * (int64_t)bh * bw + (int64_t)e * es;
        const T* xs = x + c * len;
        for (int j = 0; j < len; ++j) acc = fma(A[(int64_t)j * js], xs[j], acc);
    }
    y[o] = acc;
}

extern "C" int64_t ba_blockcoo_workspace_size(int64_t n_blocks, int64_t n_out_blocks) {
    clear_error();
    if (n_blocks < 0 || n_blocks >= ((int64_t)1 << 31) || n_out_blocks < 0 || n_out_blocks >= ((int64_t)1 << 31)) {
        set_error("blockcoo_matvec: block counts must be in [0, 2^31)");
        return -1;
    }
    BcooWs w;
    if (bcoo_layout(nullptr, n_blocks, n_out_blocks, nullptr, w) != hipSuccess) {
        set_error("blockcoo_matvec: sort workspace query failed");
        return -1;
    }
    return w.total;
}

// Replaces blockcoo_matvec (.cu:1171-1219) for any block shape; every element of y is written.
extern "C" int ba_blockcoo_matvec(const void* blocks, int32_t bh, int32_t bw, const void* row_idx, const void* col_idx,
                                  int32_t index_int64, int64_t n_blocks, const void* x, void* y, int64_t HB1,
                                  int64_t WB1, int32_t transpose, int32_t dtype, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
    clear_error();
    BA_REQUIRE(bh > 0 && bw > 0 && n_blocks >= 0 && HB1 >= 0 && WB1 >= 0, "bad block shape");
    BA_REQUIRE(n_blocks < ((int64_t)1 << 31) && HB1 < ((int64_t)1 << 31) && WB1 < ((int64_t)1 << 31),
               "block counts must be below 2^31");
    const int64_t n_out = transpose ? WB1 : HB1, n_in = transpose ? HB1 : WB1;
    const int per = transpose ? bw : bh;
    if (n_out == 0) return BA_OK;
    hipStream_t st = S(stream);
    BcooWs w;
    BA_HIP(bcoo_layout(workspace, n_blocks, n_out, st, w));
    BA_REQUIRE(workspace != nullptr && workspace_bytes >= w.total, "workspace too small (ba_blockcoo_workspace_size)");
    const void* out_idx = transpose ? col_idx : row_idx;
    const void* in_idx = transpose ? row_idx : col_idx;
    if (n_blocks > 0) {
        if (index_int64)
            hipLaunchKernelGGL(k_bcoo_keys<int64_t>, dim3(nblk(n_blocks, 256)), dim3(256), 0, st,
                               (const int64_t*)out_idx, n_blocks, n_out, w.keys_in, w.ids_in);
        else
            hipLaunchKernelGGL(k_bcoo_keys<int32_t>, dim3(nblk(n_blocks, 256)), dim3(256), 0, st,
                               (const int32_t*)out_idx, n_blocks, n_out, w.keys_in, w.ids_in);
        BA_LAUNCHED();
        size_t tb = w.sort_bytes;
        BA_HIP(rocprim::radix_sort_pairs(w.sort_tmp, tb, w.keys_in, w.keys_out, w.ids_in, w.ids_out,
                                         (unsigned)n_blocks, 0u, bcoo_bits(n_out), st));
    }
    hipLaunchKernelGGL(k_bcoo_bounds, dim3(nblk(n_blocks + 1, 256)), dim3(256), 0, st, w.keys_out, n_blocks, n_out,
                       w.seg);
    BA_LAUNCHED();
    const unsigned g = nblk(n_out * per, 256);
#define BA_BCOO(T, I)                                                                                          \
    hipLaunchKernelGGL((k_bcoo_rows<T, I>), dim3(g), dim3(256), 0, st, (const T*)blocks, bh, bw, (const I*)in_idx, \
                       n_in, w.ids_out, w.seg, n_out, (const T*)x, (T*)y, transpose)
    if (dtype == 1) { if (index_int64) BA_BCOO(double, int64_t); else BA_BCOO(double, int32_t); }
    else            { if (index_int64) BA_BCOO(float, int64_t);  else BA_BCOO(float, int32_t); }
#undef BA_BCOO
    BA_LAUNCHED();
    return BA_OK;
}

// ----------------------------------------------------------------------------- einsum bki,bkj->bij
template <typename T>
__global__ void __launch_bounds__(256) k_einsum(const T* __restrict__ L, int64_t l_bs, int64_t l_ks,
                                                const T* __restrict__ R, int64_t r_bs, int64_t r_ks,
                                                T* __restrict__ out, int64_t B, int K, int I, int J) {
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t total = B * I * J;
    if (tid >= total) return;
    int64_t b = tid / (I * J);
    int ij = (int)(tid - b * I * J);
    int i = ij / J, j = ij - (ij / J) * J;
    const T* lb = L + b * l_bs;
    const T* rb = R + b * r_bs;
    T acc = T(0);
    for (int k = 0; k < K; ++k) acc += lb[k * l_ks + i] * rb[k * r_ks + j];
    out[tid] = acc;
}

// Replaces fused_einsum_bki_bkj (.cu:1222-1250) for every (I, J, K): the reference dispatch
// list (.cu:969-1007) lacks (C,6,1) for C=5, which the pose/depth-coefficient cross term needs.
extern "C" int ba_einsum_bki_bkj(const void* left, int64_t l_bs, int64_t l_ks, const void* right, int64_t r_bs,
                                 int64_t r_ks, void* out, int64_t B, int32_t K, int32_t I, int32_t J, int32_t dtype,
                                 void* stream) {
    clear_error();
    BA_REQUIRE(B >= 0 && K >= 0 && I > 0 && J > 0, "bad sizes");
    int64_t total = B * I * J;
    if (total == 0) return BA_OK;
    if (dtype == 1)
        hipLaunchKernelGGL(k_einsum<double>, dim3(nblk(total, 256)), dim3(256), 0, S(stream), (const double*)left, l_bs,
                           l_ks, (const double*)right, r_bs, r_ks, (double*)out, B, K, I, J);
    else
        hipLaunchKernelGGL(k_einsum<float>, dim3(nblk(total, 256)), dim3(256), 0, S(stream), (const float*)left, l_bs,
                           l_ks, (const float*)right, r_bs, r_ks, (float*)out, B, K, I, J);
    BA_LAUNCHED();
    return BA_OK;
}

// ----------------------------------------------------------------------------- SE(3) exponential
// Closed form: R = I + A [w]x + B [w]x^2, t = (I + B [w]x + Cc [w]x^2) v, with
// A = sin(th)/th, B = (1-cos th)/th^2, Cc = (th - sin th)/th^3 (Taylor series below 1e-4 rad),
// evaluated in fp64 and rounded once to fp32.  Same map as torch.matrix_exp of the hat matrix
// (cujac/__init__.py:43-58).
__device__ __forceinline__ void se3_exp(const double xi[6], double Rt[12]) {
    double wx = xi[0], wy = xi[1], wz = xi[2];
    double th2 = wx * wx + wy * wy + wz * wz;
    double th = sqrt(th2);
    double A, B, Cc;
    if (th < 1e-4) {
        A = 1.0 - th2 / 6.0 + th2 * th2 / 120.0;
        B = 0.5 - th2 / 24.0 + th2 * th2 / 720.0;
        Cc = 1.0 / 6.0 - th2 / 120.0 + th2 * th2 / 5040.0;
    } else {
        double s = sin(th), c = cos(th);
        A = s / th;
        B = (1.0 - c) / th2;
        Cc = (th - s) / (th2 * th);
    }
    double W[9] = {0, -wz, wy, wz, 0, -wx, -wy, wx, 0};
    double W2[9];
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c) {
            double s = 0;
            for (int k = 0; k < 3; ++k) s += W[3 * r + k] * W[3 * k + c];
            W2[3 * r + c] = s;
        }
    for (int r = 0; r < 3; ++r) {
        double t = 0;
        for (int c = 0; c < 3; ++c) {
            double I = (r == c) ? 1.0 : 0.0;
            Rt[4 * r + c] = I + A * W[3 * r + c] + B * W2[3 * r + c];
            double V = I + B * W[3 * r + c] + Cc * W2[3 * r + c];
            t += V * xi[3 + c];
        }
        Rt[4 * r + 3] = t;
    }
}

__global__ void __launch_bounds__(256) k_exp_se3(const float* __restrict__ xi, float* __restrict__ out, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    double x[6];
    for (int k = 0; k < 6; ++k) x[k] = xi[i * 6 + k];
    double Rt[12];
    se3_exp(x, Rt);
    float* o = out + i * 16;
    for (int k = 0; k < 12; ++k) o[k] = (float)Rt[k];
    o[12] = 0.f; o[13] = 0.f; o[14] = 0.f; o[15] = 1.f;
}

// Replaces exp_se3 (cujac/__init__.py:56-58): xi (B,6) = [w | v] -> (B,4,4) fp32.
extern "C" int ba_exp_se3(const float* xi, float* out, int64_t n, void* stream) {
    clear_error();
    BA_REQUIRE(n >= 0, "bad size");
    if (n == 0) return BA_OK;
    hipLaunchKernelGGL(k_exp_se3, dim3(nblk(n, 256)), dim3(256), 0, S(stream), xi, out, n);
    BA_LAUNCHED();
    return BA_OK;
}
