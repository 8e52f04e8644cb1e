// Dense tangent prior on the z-coefficients (src/blast3r/inference/engine.py:15-179) and the
// planar confidence it weights by (engine.py:182-200).
//
// For every image: the log-depth channels and the reference pointmap are sampled on the grid of
// rows / columns s//2 + s k; the combined depth D = exp(min(sum_c a_c L_c, 80)) gives points
// X = D K_s^-1 (u + .5, v + .5, 1) with the subsampled intrinsics K_s; neighbouring points along
// rows (x) and columns (y) give tangents t, the pointmap X0 gives t0, and the residual is
// r = t / |t| - t0 / |t0| (|.| clamped below by eps; without normalisation both use |t0| and X0 is
// first rescaled by the lower median of D / z0).  Weights w = sqrt(max(Cw Cw', 0)) with Cw the
// planar confidence of X0's depth.  Per image: loss terms weight * mean(w r^2) per direction, and
// Gauss-Newton terms g = sum scale w J^T r, H = sum scale w J^T J w.r.t. the image's
// z-coefficients, scale = weight / (3 n_pairs) of the direction.
//
// Layout: one workgroup per (image, tile of TR x TG_TC pair origins; TR = 16 rows for the loss alone,
// 8 with the Gauss-Newton terms, 4 with more than 8 coefficients; each thread takes TR x TG_TC / 256
// origins).  The tile's points and
// the row / column after it are computed once into LDS (X, X0, Cw, the channel values), the depth
// halo the planar confidence needs is staged before that; each thread then takes one origin and
// its x and y pairs.  The derivative of a pair difference is rank two in the channel values:
//   dt/da_c = L_c(q) U + L_c(p) V,  U = P X(q) / |t|,  V = -P X(p) / |t|,  P = I - t_hat t_hat^T
// (P = I and |t0| without normalisation), so per pair five dot products and the channel values
// give g and H.  Partials go to a workspace in tile order and are summed per image in that order.
// Up to 16 coefficients one workgroup holds the whole upper triangle of H in registers; above that
// (up to 24) the rows of H are split over TG_RB-row groups (grid z), each group recomputing the
// tile and holding only its rows.
//
// Precision: fp32 or fp64 working type T (the reference's dtype argument), with the pointmap
// tangents and the confidence in fp32 as the reference keeps them; sums in fp64.  The fp32 parts
// follow torch's unfused operation order (no contraction).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cmath>

#include "ba_common.h"
#include "ba_error.h"
#include "ba_hip.h"

#pragma clang fp contract(off)

namespace ba {

#define TG_T 256
#define TG_TC 64                // tile columns (pair origins)
#define TG_RC (TG_TC + 1)
#define TG_HC (TG_TC + 3)
#define TG_CMAX 24              // z-coefficients with the Gauss-Newton terms
#define TG_RB 4                 // rows of H per workgroup above 16 coefficients
// tile rows: 16 for the loss alone, 8 with the Gauss-Newton terms, 4 with more than 8 coefficients
// (the channel values then fill LDS)
template <int CMAX, bool GN> struct TgRows { static constexpr int TR = !GN ? 16 : (CMAX > 8 ? 4 : 8); };

static inline int64_t tg_div_up(int64_t a, int64_t b) { return (a + b - 1) / b; }
static inline int64_t tg_align(int64_t b) { return (b + 255) & ~int64_t(255); }

__host__ __device__ static inline int grid_len(int n, int s) { return n > s / 2 ? (n - s / 2 + s - 1) / s : 0; }

template <typename T> __device__ __forceinline__ T dexp(T x);
template <> __device__ __forceinline__ float dexp<float>(float x) { return expf(x); }
template <> __device__ __forceinline__ double dexp<double>(double x) { return exp(x); }
template <typename T> __device__ __forceinline__ T dsqrt(T x);
template <> __device__ __forceinline__ float dsqrt<float>(float x) { return sqrtf(x); }
template <> __device__ __forceinline__ double dsqrt<double>(double x) { return sqrt(x); }

struct TgImage {
    const float* dep;
    const float* ref;
    int Hi, Wi, Hs, Ws;
};

__device__ __forceinline__ TgImage tg_image(const ba_tangent_args& a, int img) {
    TgImage m;
    m.dep = reinterpret_cast<const float*>(a.depth_addr[img]);
    m.ref = reinterpret_cast<const float*>(a.ref_addr[img]);
    m.Hi = a.map_hw ? a.map_hw[2 * img] : a.H;
    m.Wi = a.map_hw ? a.map_hw[2 * img + 1] : a.W;
    m.Hs = grid_len(m.Hi, a.tan_stride);
    m.Ws = grid_len(m.Wi, a.tan_stride);
    return m;
}

__device__ __forceinline__ int64_t tg_pix(const TgImage& m, int s, int gr, int gc) {
    return (int64_t)(s / 2 + s * gr) * m.Wi + (s / 2 + s * gc);
}

// K_s^-1 of the subsampled intrinsics (principal point minus s//2, rows 0-1 divided by s), in T,
// by the adjugate; the reference inverts the same matrix with LU (last-bit differences only)
template <typename T>
__device__ __forceinline__ void tg_invK(const ba_tangent_args& a, int img, T (&iK)[3][3]) {
    const float* Kc = a.K + 9 * (int64_t)a.cam_ids[img];
    T k[3][3];
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c) k[r][c] = (T)Kc[3 * r + c];
    const T o = (T)(a.tan_stride / 2), s = (T)a.tan_stride;
    k[0][2] = k[0][2] - o;
    k[1][2] = k[1][2] - o;
    for (int c = 0; c < 3; ++c) { k[0][c] = k[0][c] / s; k[1][c] = k[1][c] / s; }
    const T c00 = k[1][1] * k[2][2] - k[1][2] * k[2][1];
    const T c01 = k[1][2] * k[2][0] - k[1][0] * k[2][2];
    const T c02 = k[1][0] * k[2][1] - k[1][1] * k[2][0];
    const T det = k[0][0] * c00 + k[0][1] * c01 + k[0][2] * c02;
    const T id = (T)1 / det;
    iK[0][0] = c00 * id;
    iK[0][1] = (k[0][2] * k[2][1] - k[0][1] * k[2][2]) * id;
    iK[0][2] = (k[0][1] * k[1][2] - k[0][2] * k[1][1]) * id;
    iK[1][0] = c01 * id;
    iK[1][1] = (k[0][0] * k[2][2] - k[0][2] * k[2][0]) * id;
    iK[1][2] = (k[0][2] * k[1][0] - k[0][0] * k[1][2]) * id;
    iK[2][0] = c02 * id;
    iK[2][1] = (k[0][1] * k[2][0] - k[0][0] * k[2][1]) * id;
    iK[2][2] = (k[0][0] * k[1][1] - k[0][1] * k[1][0]) * id;
}

// combined depth of grid point (gr, gc): exp(min(sum_c a_c L_c, 80)) in T
template <typename T>
__device__ __forceinline__ T tg_depth(const ba_tangent_args& a, const TgImage& m, int img, int gr, int gc, float* Lout) {
    const float* p = m.dep + tg_pix(m, a.tan_stride, gr, gc) * a.depth_pix_stride;
    const float* zc = a.z_coefs + (int64_t)img * a.C;
    T acc = 0;
    for (int c = 0; c < a.C; ++c) {
        const float l = p[c];
        if (Lout) Lout[c] = l;
        acc = acc + (T)zc[c] * (T)l;
    }
    return dexp<T>(acc < (T)80 ? acc : (T)80);
}

// ---------------------------------------------------------------- lower median of D / z0
// One workgroup per image; keys are the bit patterns of the positive ratios (order-preserving),
// ~0 for masked points.  Radix select from the most significant byte.
template <typename T>
__global__ void __launch_bounds__(TG_T) k_tan_median(ba_tangent_args a, uint64_t* __restrict__ keys, int64_t key_stride,
                                                      double* __restrict__ scale) {
    __shared__ uint32_t hist[256];
    __shared__ uint64_t sPrefix;
    __shared__ int64_t sRank, sCount;
    const int img = blockIdx.x;
    const TgImage m = tg_image(a, img);
    // (the host sizes key_stride for the largest image; the clamp only keeps accesses in bounds)
    const int n = (int)((int64_t)m.Hs * m.Ws < key_stride ? (int64_t)m.Hs * m.Ws : key_stride);
    uint64_t* kk = keys + (int64_t)img * key_stride;
    int64_t cnt = 0;
    for (int i = threadIdx.x; i < n; i += TG_T) {
        const int gr = i / m.Ws, gc = i - gr * m.Ws;
        const float z0 = m.ref[tg_pix(m, a.tan_stride, gr, gc) * a.ref_pix_stride + 2];
        uint64_t key = ~(uint64_t)0;
        if (z0 > 1e-6f) {
            const T r = tg_depth<T>(a, m, img, gr, gc, nullptr) / (T)z0;
            if (sizeof(T) == 4) key = (uint64_t)__float_as_uint((float)r);
            else key = (uint64_t)__double_as_longlong((double)r);
            ++cnt;
        }
        kk[i] = key;
    }
    // count of unmasked points
    if (threadIdx.x == 0) sCount = 0;
    __syncthreads();
    atomicAdd((unsigned long long*)&sCount, (unsigned long long)cnt);
    __syncthreads();
    const int64_t total = sCount;
    if (total == 0) {
        if (threadIdx.x == 0) scale[img] = 1.0;
        return;
    }
    if (threadIdx.x == 0) { sPrefix = 0; sRank = (total - 1) / 2; }     // torch.median: lower median
    uint64_t mask = 0;
    for (int byte = (int)sizeof(T) - 1; byte >= 0; --byte) {
        hist[threadIdx.x] = 0;
        __syncthreads();
        const uint64_t prefix = sPrefix;
        for (int i = threadIdx.x; i < n; i += TG_T) {
            const uint64_t k = kk[i];
            if (k != ~(uint64_t)0 && (k & mask) == prefix) atomicAdd(&hist[(k >> (8 * byte)) & 255], 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int64_t r = sRank, acc = 0;
            int b = 0;
            for (; b < 255; ++b) {
                if (acc + hist[b] > r) break;
                acc += hist[b];
            }
            sRank = r - acc;
            sPrefix = prefix | ((uint64_t)b << (8 * byte));
        }
        mask |= (uint64_t)255 << (8 * byte);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const uint64_t k = sPrefix;
        scale[img] = sizeof(T) == 4 ? (double)__uint_as_float((uint32_t)k) : __longlong_as_double((long long)k);
    }
}

// ---------------------------------------------------------------- tiles
// RB = 0: the whole upper triangle of H; RB > 0: rows c0 .. c0 + RB - 1 of H (c0 = RB blockIdx.z),
// full rows, of which the entries on and right of the diagonal are written
template <typename T, int CMAX, bool GN, bool NORM, int RB = 0>
__global__ void __launch_bounds__(TG_T) k_tan_tile(ba_tangent_args a, const double* __restrict__ scale,
                                                    double* __restrict__ part, int n_tc, int n_acc) {
    constexpr int NR = RB > 0 ? RB : CMAX;
    constexpr int E = RB > 0 ? RB * CMAX : CMAX * (CMAX + 1) / 2;
    const int c0 = RB > 0 ? (int)blockIdx.z * RB : 0;
    constexpr int TG_TR = TgRows<CMAX, GN>::TR, TG_RR = TG_TR + 1, TG_HR = TG_TR + 3;
    __shared__ float sD0[TG_HR][TG_HC];
    __shared__ T sX[3][TG_RR * TG_RC];
    __shared__ float sX0[3][TG_RR * TG_RC];
    __shared__ float sCw[TG_RR * TG_RC];
    __shared__ float sL[GN ? CMAX : 1][TG_RR * TG_RC];
    __shared__ double sRed[TG_T / 64];
    // an image's tiles on one XCD, so that the halo rows neighbouring tiles share are fetched into one L2
    const unsigned lb = xcd_block(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x * gridDim.y);
    const int img = (int)(lb / gridDim.x), tile = (int)(lb % gridDim.x);
    const TgImage m = tg_image(a, img);
    const int tr0 = (tile / n_tc) * TG_TR, tc0 = (tile % n_tc) * TG_TC;
    double* out = part + ((int64_t)img * gridDim.x + tile) * n_acc;
    const int C = a.C;
    if (m.Ws < 2 || C < 2 || tr0 >= m.Hs || tc0 >= m.Ws) {       // skipped image (engine.py:75) or empty tile
        for (int j = threadIdx.x; j < n_acc; j += TG_T) out[j] = 0.0;
        return;
    }
    const int s = a.tan_stride;
    float s32 = 1.0f;
    if (!NORM) s32 = (float)scale[img];
    // depth of X0 on the halo (grid rows tr0-1 .. tr0+TR+1, columns tc0-1 .. tc0+TC+1)
    for (int i = threadIdx.x; i < TG_HR * TG_HC; i += TG_T) {
        const int hr = i / TG_HC, hc = i - hr * TG_HC;
        const int gr = tr0 - 1 + hr, gc = tc0 - 1 + hc;
        float z = 0.0f;
        if (gr >= 0 && gr < m.Hs && gc >= 0 && gc < m.Ws) {
            z = m.ref[tg_pix(m, s, gr, gc) * a.ref_pix_stride + 2];
            if (!NORM) z = s32 * z;
        }
        sD0[hr][hc] = z;
    }
    T iK[3][3];
    tg_invK<T>(a, img, iK);
    __syncthreads();
    // region points: X, X0, Cw, channel values
    for (int i = threadIdx.x; i < TG_RR * TG_RC; i += TG_T) {
        const int rr = i / TG_RC, rc = i - rr * TG_RC;
        const int gr = tr0 + rr, gc = tc0 + rc;
        if (gr >= m.Hs || gc >= m.Ws) continue;
        float Lv[GN ? CMAX : 1];
        const T D = tg_depth<T>(a, m, img, gr, gc, GN ? Lv : nullptr);
        if (GN)
            for (int c = 0; c < C; ++c) sL[c][i] = Lv[c];
        const T u = (T)gc + (T)0.5, v = (T)gr + (T)0.5;
        for (int k = 0; k < 3; ++k) sX[k][i] = ((u * iK[k][0] + v * iK[k][1]) + iK[k][2]) * D;
        const float* pr = m.ref + tg_pix(m, s, gr, gc) * a.ref_pix_stride;
        for (int k = 0; k < 3; ++k) sX0[k][i] = NORM ? pr[k] : s32 * pr[k];
        // planar confidence (engine.py:182-200) of X0's depth at (gr, gc)
        const int hr = rr + 1, hc = rc + 1;
        const float d = sD0[hr][hc];
        float lx = 2.0f * d, ly = 2.0f * d;
        if (gc >= 1) lx = lx - sD0[hr][hc - 1];
        if (gc + 1 < m.Ws) lx = lx - sD0[hr][hc + 1];
        if (gr >= 1) ly = ly - sD0[hr - 1][hc];
        if (gr + 1 < m.Hs) ly = ly - sD0[hr + 1][hc];
        float mn = INFINITY;
        for (int dr = -1; dr <= 1; ++dr)
            for (int dc = -1; dc <= 1; ++dc) {
                const int r2 = gr + dr, c2 = gc + dc;
                if (r2 >= 0 && r2 < m.Hs && c2 >= 0 && c2 < m.Ws) mn = fminf(mn, sD0[hr + dr][hc + dc]);
            }
        mn = fmaxf(mn, 1e-12f);
        lx = lx / mn;
        ly = ly / mn;
        sCw[i] = expf(-10000.0f * (lx * lx + ly * ly));
    }
    __syncthreads();

    double lsum[2] = {0.0, 0.0};
    double g[GN ? NR : 1];
    double Hacc[GN ? E : 1];
    if (GN) {
#pragma unroll
        for (int c = 0; c < NR; ++c) g[c] = 0.0;
#pragma unroll
        for (int e = 0; e < E; ++e) Hacc[e] = 0.0;
    }
    const float eps_f = (float)a.eps;
    const T eps_t = (T)a.eps;
#pragma unroll 1
    for (int po = threadIdx.x; po < TG_TR * TG_TC; po += TG_T) {
    const int tr = po / TG_TC, tc = po - tr * TG_TC;
    const int gr = tr0 + tr, gc = tc0 + tc;
    const int p = tr * TG_RC + tc;
#pragma unroll 1
    for (int dir = 0; dir < 2; ++dir) {
        const bool ok = dir == 0 ? (gr + 1 < m.Hs && gc < m.Ws) : (gr < m.Hs && gc + 1 < m.Ws);
        if (!ok) continue;
        const int q = dir == 0 ? p + TG_RC : p + 1;
        T t[3];
        float t0[3];
        for (int k = 0; k < 3; ++k) { t[k] = sX[k][q] - sX[k][p]; t0[k] = sX0[k][q] - sX0[k][p]; }
        const float n0 = sqrtf((t0[0] * t0[0] + t0[1] * t0[1]) + t0[2] * t0[2]);
        const float is0 = 1.0f / fmaxf(n0, eps_f);
        T is;
        if (NORM) {
            const T nt = dsqrt<T>((t[0] * t[0] + t[1] * t[1]) + t[2] * t[2]);
            is = (T)1 / (nt > eps_t ? nt : eps_t);
        } else {
            is = (T)is0;
        }
        T th[3], r[3];
        for (int k = 0; k < 3; ++k) { th[k] = t[k] * is; r[k] = th[k] - (T)(t0[k] * is0); }
        const float w = sqrtf(fmaxf(sCw[q] * sCw[p], 0.0f));
        for (int k = 0; k < 3; ++k) {
            const T r2 = r[k] * r[k];
            lsum[dir] += (double)((T)w * r2);
        }
        if (GN) {
            const int np = dir == 0 ? (m.Hs - 1) * m.Ws : m.Hs * (m.Ws - 1);
            const double ww = a.weight / (3.0 * (double)np) * (double)w;
            double U[3], V[3];
            if (NORM) {
                double dq = 0.0, dp = 0.0;
                for (int k = 0; k < 3; ++k) { dq += (double)th[k] * (double)sX[k][q]; dp += (double)th[k] * (double)sX[k][p]; }
                for (int k = 0; k < 3; ++k) {
                    U[k] = (double)is * ((double)sX[k][q] - (double)th[k] * dq);
                    V[k] = -(double)is * ((double)sX[k][p] - (double)th[k] * dp);
                }
            } else {
                for (int k = 0; k < 3; ++k) { U[k] = (double)is * (double)sX[k][q]; V[k] = -(double)is * (double)sX[k][p]; }
            }
            double uu = 0, uv = 0, vv = 0, ur = 0, vr = 0;
            for (int k = 0; k < 3; ++k) {
                uu += U[k] * U[k]; uv += U[k] * V[k]; vv += V[k] * V[k];
                ur += U[k] * (double)r[k]; vr += V[k] * (double)r[k];
            }
            // channel values of q (alpha) and p (beta), read from LDS as needed
            // (entries past C accumulate zeros: the channel values are read as 0 there)
            double al[CMAX], be[CMAX];
#pragma unroll
            for (int c = 0; c < CMAX; ++c) {
                al[c] = c < C ? (double)sL[c][q] : 0.0;
                be[c] = c < C ? (double)sL[c][p] : 0.0;
            }
            if (RB == 0) {
#pragma unroll
                for (int c = 0; c < CMAX; ++c) {
                    g[c] += ww * (al[c] * ur + be[c] * vr);
                    const double s1 = ww * (al[c] * uu + be[c] * uv);
                    const double s2 = ww * (al[c] * uv + be[c] * vv);
#pragma unroll
                    for (int d2 = c; d2 < CMAX; ++d2) Hacc[c * CMAX - c * (c - 1) / 2 + (d2 - c)] += s1 * al[d2] + s2 * be[d2];
                }
            } else {
#pragma unroll
                for (int r2 = 0; r2 < NR; ++r2) {
                    // the group's row c (uniform over the workgroup) read from LDS: a register array
                    // indexed at run time would live in scratch memory
                    const int c = c0 + r2;
                    const double ac = c < C ? (double)sL[c][q] : 0.0, bc = c < C ? (double)sL[c][p] : 0.0;
                    g[r2] += ww * (ac * ur + bc * vr);
                    const double s1 = ww * (ac * uu + bc * uv);
                    const double s2 = ww * (ac * uv + bc * vv);
#pragma unroll
                    for (int d2 = 0; d2 < CMAX; ++d2) Hacc[r2 * CMAX + d2] += s1 * al[d2] + s2 * be[d2];
                }
            }
        }
    }
    }
    // block sums in a fixed order: waves by butterfly, then the wave sums in wave order
    auto bsum = [&](double v) -> double {
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) sRed[threadIdx.x >> 6] = v;
        __syncthreads();
        double t2 = 0.0;
        for (int w2 = 0; w2 < TG_T / 64; ++w2) t2 += sRed[w2];
        return t2;
    };
    double v;
    if (RB > 0) {
        // (bsum synchronises the workgroup: every condition below is uniform over it)
        if (c0 == 0) {
            v = bsum(lsum[0]); if (threadIdx.x == 0) out[0] = v;
            v = bsum(lsum[1]); if (threadIdx.x == 0) out[1] = v;
        }
#pragma unroll
        for (int r2 = 0; r2 < NR; ++r2) {
            const int c = c0 + r2;
            if (c >= C) break;
            v = bsum(g[r2]);
            if (threadIdx.x == 0) out[2 + c] = v;
            // entry (c, d2) of the upper triangle, row by row: sum_{c' < c} (C - c') + (d2 - c)
            const int row0 = 2 + C + c * C - c * (c - 1) / 2 - c;
#pragma unroll
            for (int d2 = 0; d2 < CMAX; ++d2) {
                if (d2 >= c && d2 < C) {
                    v = bsum(Hacc[r2 * CMAX + d2]);
                    if (threadIdx.x == 0) out[row0 + d2] = v;
                }
            }
        }
        return;
    }
    v = bsum(lsum[0]); if (threadIdx.x == 0) out[0] = v;
    v = bsum(lsum[1]); if (threadIdx.x == 0) out[1] = v;
    if (GN) {
#pragma unroll
        for (int c = 0; c < CMAX; ++c) {
            if (c < C) {
                v = bsum(g[c]);
                if (threadIdx.x == 0) out[2 + c] = v;
            }
        }
        int j = 2 + C;
#pragma unroll
        for (int c = 0; c < CMAX; ++c) {
#pragma unroll
            for (int d2 = c; d2 < CMAX; ++d2) {
                if (c < C && d2 < C) {
                    v = bsum(Hacc[c * CMAX - c * (c - 1) / 2 + (d2 - c)]);
                    if (threadIdx.x == 0) out[j] = v;
                    ++j;
                }
            }
        }
    }
}

// per image: sum of the tile partials in tile order; g_z, H_z (symmetric, in T) and the image's
// two loss terms weight * mean(w r^2) (x, y; 0 where the reference adds nothing), in T
template <typename T>
__global__ void __launch_bounds__(TG_T) k_tan_reduce(ba_tangent_args a, const double* __restrict__ part, int n_tiles,
                                                      int n_acc, T* __restrict__ img_loss) {
    const int img = blockIdx.x, C = a.C;
    for (int j = threadIdx.x; j < n_acc; j += TG_T) {
        double s = 0.0;
        for (int t = 0; t < n_tiles; ++t) s += part[((int64_t)img * n_tiles + t) * n_acc + j];
        if (j < 2) {
            const TgImage m = tg_image(a, img);
            const int64_t np = j == 0 ? (int64_t)(m.Hs - 1) * m.Ws : (int64_t)m.Hs * (m.Ws - 1);
            T term = 0;
            if (m.Ws >= 2 && C >= 2 && np > 0) term = (T)a.weight * (T)(s / (3.0 * (double)np));
            img_loss[2 * img + j] = term;
            continue;
        }
        if (!a.compute_gn) continue;
        if (j < 2 + C) {
            const int c = j - 2;
            if (!a.optim_Z0 && c == 0) s = 0.0;
            static_cast<T*>(a.g_z)[(int64_t)img * C + c] = (T)s;
            continue;
        }
        // entry j - 2 - C of the upper triangle, row by row
        int e = j - 2 - C, c = 0;
        while (e >= C - c) { e -= C - c; ++c; }
        const int d2 = c + e;
        if (!a.optim_Z0 && (c == 0 || d2 == 0)) s = 0.0;
        T* Hz = static_cast<T*>(a.H_z) + (int64_t)img * C * C;
        Hz[c * C + d2] = (T)s;
        Hz[d2 * C + c] = (T)s;
    }
}

// tan_loss = the images' terms added one by one in image order, x then y (engine.py:132-135): the
// terms are staged through LDS in coalesced chunks and one thread adds them in order
template <typename T>
__global__ void __launch_bounds__(TG_T) k_tan_loss(ba_tangent_args a, const T* __restrict__ img_loss) {
    __shared__ T sT[2 * 1024];
    T loss = 0;
    const int64_t n = 2 * a.n_imgs;
    for (int64_t c0 = 0; c0 < n; c0 += 2 * 1024) {
        const int64_t m = n - c0 < 2 * 1024 ? n - c0 : 2 * 1024;
        __syncthreads();
        for (int64_t i = threadIdx.x; i < m; i += TG_T) sT[i] = img_loss[c0 + i];
        __syncthreads();
        if (threadIdx.x == 0)
            for (int64_t i = 0; i < m; ++i) loss = loss + sT[i];
    }
    if (threadIdx.x == 0) *static_cast<T*>(a.loss) = loss;
}

// planar confidence of one (H, W) fp32 map (engine.py:182-200)
__global__ void __launch_bounds__(TG_T) k_planar_conf(const float* __restrict__ D0, int H, int W, float alpha,
                                                       float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * TG_T + threadIdx.x;
    if (i >= (int64_t)H * W) return;
    const int r = (int)(i / W), c = (int)(i - (int64_t)r * W);
    const float d = D0[i];
    float lx = 2.0f * d, ly = 2.0f * d;
    if (c >= 1) lx = lx - D0[i - 1];
    if (c + 1 < W) lx = lx - D0[i + 1];
    if (r >= 1) ly = ly - D0[i - W];
    if (r + 1 < H) ly = ly - D0[i + W];
    float mn = INFINITY;
    for (int dr = -1; dr <= 1; ++dr)
        for (int dc = -1; dc <= 1; ++dc) {
            const int r2 = r + dr, c2 = c + dc;
            if (r2 >= 0 && r2 < H && c2 >= 0 && c2 < W) mn = fminf(mn, D0[(int64_t)r2 * W + c2]);
        }
    mn = fmaxf(mn, 1e-12f);
    lx = lx / mn;
    ly = ly / mn;
    out[i] = expf(-alpha * (lx * lx + ly * ly));
}

}  // namespace ba

using namespace ba;

struct TgLayout {
    int n_tr, n_tc, n_tiles, n_acc;
    int64_t key_stride;
    int64_t off_scale, off_keys, off_part, off_loss, total;
};

// tile rows of the kernel instantiation chosen for C (see launch_all)
static int tg_tile_rows(int C, int compute_gn) {
    return !compute_gn ? TgRows<1, false>::TR
                       : (C > 16 ? TgRows<TG_CMAX, true>::TR : C > 8 ? TgRows<16, true>::TR : TgRows<8, true>::TR);
}

static TgLayout tg_layout(int64_t n_imgs, int C, int H, int W, int s, int normalize, int compute_gn) {
    TgLayout L;
    const int Hs = grid_len(H, s), Ws = grid_len(W, s);
    L.n_tr = (int)tg_div_up(Hs > 0 ? Hs : 1, tg_tile_rows(C, compute_gn));
    L.n_tc = (int)tg_div_up(Ws > 0 ? Ws : 1, TG_TC);
    L.n_tiles = L.n_tr * L.n_tc;
    L.n_acc = 2 + (compute_gn ? C + C * (C + 1) / 2 : 0);
    L.key_stride = normalize ? 0 : (int64_t)Hs * Ws;
    const int64_t n = n_imgs > 0 ? n_imgs : 1;
    L.off_scale = 0;
    L.off_keys = tg_align(L.off_scale + n * 8);
    L.off_part = tg_align(L.off_keys + n * L.key_stride * 8);
    L.off_loss = tg_align(L.off_part + n * L.n_tiles * L.n_acc * 8);
    L.total = tg_align(L.off_loss + n * 2 * 8);
    return L;
}

extern "C" int64_t ba_tangent_workspace_bytes(int64_t n_imgs, int32_t C, int32_t H, int32_t W, int32_t tan_stride,
                                              int32_t normalize, int32_t compute_gn) {
    if (tan_stride < 1) return -1;
    return tg_layout(n_imgs, C, H, W, tan_stride, normalize, compute_gn).total;
}

template <typename T, int CMAX, bool GN, bool NORM, int RB = 0>
static void launch_tiles(const ba_tangent_args& a, const TgLayout& L, char* ws, hipStream_t st) {
    const unsigned groups = RB > 0 ? (unsigned)((a.C + RB - 1) / RB) : 1u;
    hipLaunchKernelGGL((k_tan_tile<T, CMAX, GN, NORM, RB>), dim3((unsigned)L.n_tiles, (unsigned)a.n_imgs, groups),
                       dim3(TG_T), 0, st, a, (const double*)(ws + L.off_scale), (double*)(ws + L.off_part), L.n_tc,
                       L.n_acc);
}

template <typename T>
static void launch_all(const ba_tangent_args& a, const TgLayout& L, char* ws, hipStream_t st) {
    if (!a.normalize)
        hipLaunchKernelGGL(k_tan_median<T>, dim3((unsigned)a.n_imgs), dim3(TG_T), 0, st, a, (uint64_t*)(ws + L.off_keys),
                           L.key_stride, (double*)(ws + L.off_scale));
    if (a.compute_gn) {
        if (a.C <= 4) {
            if (a.normalize) launch_tiles<T, 4, true, true>(a, L, ws, st);
            else launch_tiles<T, 4, true, false>(a, L, ws, st);
        } else if (a.C <= 6) {
            if (a.normalize) launch_tiles<T, 6, true, true>(a, L, ws, st);
            else launch_tiles<T, 6, true, false>(a, L, ws, st);
        } else if (a.C <= 8) {
            if (a.normalize) launch_tiles<T, 8, true, true>(a, L, ws, st);
            else launch_tiles<T, 8, true, false>(a, L, ws, st);
        } else if (a.C <= 12) {
            if (a.normalize) launch_tiles<T, 12, true, true>(a, L, ws, st);
            else launch_tiles<T, 12, true, false>(a, L, ws, st);
        } else if (a.C <= 16) {
            if (a.normalize) launch_tiles<T, 16, true, true>(a, L, ws, st);
            else launch_tiles<T, 16, true, false>(a, L, ws, st);
        } else {
            if (a.normalize) launch_tiles<T, TG_CMAX, true, true, TG_RB>(a, L, ws, st);
            else launch_tiles<T, TG_CMAX, true, false, TG_RB>(a, L, ws, st);
        }
    } else {
        if (a.normalize) launch_tiles<T, 1, false, true>(a, L, ws, st);
        else launch_tiles<T, 1, false, false>(a, L, ws, st);
    }
    hipLaunchKernelGGL(k_tan_reduce<T>, dim3((unsigned)a.n_imgs), dim3(TG_T), 0, st, a, (const double*)(ws + L.off_part),
                       L.n_tiles, L.n_acc, (T*)(ws + L.off_loss));
    hipLaunchKernelGGL(k_tan_loss<T>, dim3(1), dim3(TG_T), 0, st, a, (const T*)(ws + L.off_loss));
}

extern "C" int ba_tangent_prior(const ba_tangent_args* args, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_tangent_args& a = *args;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.n_imgs >= 1 && a.n_imgs <= 65535, "n_imgs must be in [1, 65535]");
    BA_REQUIRE(a.C >= 1 && a.tan_stride >= 1 && a.H >= 0 && a.W >= 0, "bad sizes");
    BA_REQUIRE(!a.compute_gn || a.C <= TG_CMAX, "the Gauss-Newton terms support at most 24 z-coefficients");
    BA_REQUIRE(a.depth_pix_stride >= a.C && a.ref_pix_stride >= 3, "pixel strides below the channel counts");
    BA_REQUIRE(a.depth_addr && a.ref_addr && a.K && a.cam_ids && a.z_coefs && a.loss && a.workspace, "missing arrays");
    BA_REQUIRE(!a.compute_gn || (a.g_z && a.H_z), "g_z / H_z missing");
    BA_REQUIRE(a.eps > 0.0, "eps must be positive");
    const TgLayout L = tg_layout(a.n_imgs, a.C, a.H, a.W, a.tan_stride, a.normalize, a.compute_gn);
    BA_REQUIRE(a.workspace_bytes >= L.total, "workspace too small");
    char* ws = (char*)a.workspace;
    if (a.fp64) launch_all<double>(a, L, ws, st);
    else launch_all<float>(a, L, ws, st);
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int ba_planar_confidence(const float* D0, int32_t H, int32_t W, float alpha, float* out, void* stream) {
    clear_error();
    BA_REQUIRE(D0 && out && H >= 0 && W >= 0, "bad arguments");
    const int64_t n = (int64_t)H * W;
    if (n == 0) return BA_OK;
    hipLaunchKernelGGL(k_planar_conf, dim3((unsigned)tg_div_up(n, TG_T)), dim3(TG_T), 0, (hipStream_t)stream, D0, H, W,
                       alpha, out);
    BA_LAUNCHED();
    return BA_OK;
}

namespace ba {
template <typename Real>
__global__ void __launch_bounds__(TG_T) k_add_z_prior(Real* __restrict__ S, const int32_t* __restrict__ diag_pair,
                                                       Real* __restrict__ e_img, Real* __restrict__ dg_img,
                                                       const Real* __restrict__ Hz, const Real* __restrict__ gz,
                                                       int64_t n_imgs, int d, int C) {
    const int64_t t = (int64_t)blockIdx.x * TG_T + threadIdx.x;
    const int per = C * C + C;
    if (t >= n_imgs * per) return;
    const int64_t i = t / per;
    const int e = (int)(t - i * per);
    const int o = d - C;
    if (e < C * C) {
        const int c = e / C, dd = e - c * C;
        const Real h = Hz[i * C * C + e];
        S[(int64_t)diag_pair[i] * d * d + (o + c) * d + (o + dd)] += h;
        if (c == dd) dg_img[i * d + o + c] += h;
    } else {
        const int c = e - C * C;
        e_img[i * d + o + c] += gz[i * C + c];
    }
}
}  // namespace ba

extern "C" int ba_add_z_prior(void* S_pairs, const int32_t* diag_pair, void* e_img, void* dg_img, const void* H_z,
                              const void* g_z, int64_t n_imgs, int32_t d, int32_t C, int32_t real32, void* stream) {
    clear_error();
    BA_REQUIRE(S_pairs && diag_pair && e_img && dg_img && H_z && g_z, "missing arrays");
    BA_REQUIRE(n_imgs >= 0 && C >= 1 && d >= C, "bad sizes");
    const int64_t n = n_imgs * (C * C + C);
    if (n == 0) return BA_OK;
    const dim3 g((unsigned)tg_div_up(n, TG_T));
    if (real32)
        hipLaunchKernelGGL(k_add_z_prior<float>, g, dim3(TG_T), 0, (hipStream_t)stream, (float*)S_pairs, diag_pair,
                           (float*)e_img, (float*)dg_img, (const float*)H_z, (const float*)g_z, n_imgs, d, C);
    else
        hipLaunchKernelGGL(k_add_z_prior<double>, g, dim3(TG_T), 0, (hipStream_t)stream, (double*)S_pairs, diag_pair,
                           (double*)e_img, (double*)dg_img, (const double*)H_z, (const double*)g_z, n_imgs, d, C);
    BA_LAUNCHED();
    return BA_OK;
}
