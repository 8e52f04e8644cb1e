// LM step helpers on the device: parameter update and the line-search objective.
//
//   ba_apply_update  K <- clip(K - s dK, 100), P <- exp_se3(-s dP) P, z <- z - s dZ, X <- X - s dX
//                    (src/blast3r/inference/engine.py:310-313, :347-354; cujac/__init__.py:56-58)
//   ba_objective     loss = mean(err) (engine.py:268) and reproj_score = mean of the lowest
//                    80% of ||r[:, :2]|| (engine.py:357-361), the latter by an exact radix
//                    select on the fp32 bit patterns instead of a full sort.
//   ba_nonfinite_flags  the `tensor.isfinite().all()` input checks of lm_step (engine.py:340-344)
//                    for every fp32 input in one launch.
//   ba_stream_triad  a = b + s c in fp64 (STREAM triad): the achievable HBM bandwidth that the
//                    benchmark reports beside the roofline fractions (no counterpart in the reference).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cmath>
#include <mutex>

#include "ba_common.h"
#include "ba_error.h"

namespace ba {

__device__ __forceinline__ void se3_exp_local(const double xi[6], double Rt[12]) {
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
            t += (I + B * W[3 * r + c] + Cc * W2[3 * r + c]) * xi[3 + c];
        }
        Rt[4 * r + 3] = t;
    }
}

// one thread per camera / node / image / track item, flattened
__global__ void __launch_bounds__(256) k_apply_update(const float* __restrict__ K, const float* __restrict__ P,
                                                      const float* __restrict__ Z, const float* __restrict__ X,
                                                      const float* __restrict__ dK, const float* __restrict__ dP,
                                                      const float* __restrict__ dZ, const float* __restrict__ dX,
                                                      float scale, float min_f, int n_cams, int n_nodes, int n_imgs,
                                                      int C, int64_t n_tracks, float* __restrict__ Ko,
                                                      float* __restrict__ Po, float* __restrict__ Zo,
                                                      float* __restrict__ Xo) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n_cams) {
        const float* k = K + t * 9;
        float* o = Ko + t * 9;
        for (int e = 0; e < 9; ++e) o[e] = k[e];
        float fx = k[0] - dK[2 * t] * scale, fy = k[4] - dK[2 * t + 1] * scale;   // update_K (engine.py:347-354)
        o[0] = fx < min_f ? min_f : fx;
        o[4] = fy < min_f ? min_f : fy;
        return;
    }
    t -= n_cams;
    if (t < n_nodes) {
        double xi[6], Rt[12];
        for (int e = 0; e < 6; ++e) xi[e] = -(double)(dP[6 * t + e] * scale);
        se3_exp_local(xi, Rt);
        float E[16];
        for (int e = 0; e < 12; ++e) E[e] = (float)Rt[e];
        E[12] = 0.f; E[13] = 0.f; E[14] = 0.f; E[15] = 1.f;
        const float* p = P + t * 16;
        float* o = Po + t * 16;
        for (int r = 0; r < 4; ++r)
            for (int c = 0; c < 4; ++c) {
                float s = 0.f;
                for (int k = 0; k < 4; ++k) s += E[4 * r + k] * p[4 * k + c];
                o[4 * r + c] = s;
            }
        return;
    }
    t -= n_nodes;
    if (t < (int64_t)n_imgs * C) { Zo[t] = Z[t] - dZ[t] * scale; return; }
    t -= (int64_t)n_imgs * C;
    if (t < 3 * n_tracks) { Xo[t] = X[t] - dX[t] * scale; }
}

// ------------------------------------------------------------------ objective
#define OBJ_T 256
#define OBJ_NBMAX 2048

__global__ void k_obj_init(uint32_t* __restrict__ hist, uint32_t* __restrict__ sel, uint32_t k) {
    hist[threadIdx.x] = 0;
    if (threadIdx.x == 0) { sel[0] = 0; sel[1] = 0; sel[2] = k; sel[3] = 0; }
}

// the selection key of observation i: the bit pattern of ||(r0, r1)|| (non-negative, so the pattern
// orders as the value).  Every kernel forms it through this one function, so a key stored by
// k_obj_prep and a key recomputed from res (ebits == nullptr) are the same bits.
__device__ __forceinline__ uint32_t obj_key(const float* __restrict__ res, int64_t n, int64_t i) {
    const float r0 = res[i], r1 = res[n + i];
    return __float_as_uint(sqrtf(r0 * r0 + r1 * r1));
}

__global__ void __launch_bounds__(OBJ_T) k_obj_prep(const float* __restrict__ res, int64_t n, int has_err,
                                                   uint32_t* __restrict__ ebits, double* __restrict__ part) {
    __shared__ double sh[OBJ_T];
    double s = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * OBJ_T + threadIdx.x; i < n; i += (int64_t)gridDim.x * OBJ_T) {
        if (ebits) ebits[i] = obj_key(res, n, i);
        if (has_err) s += (double)res[3 * n + i] + (double)res[4 * n + i] + (double)res[5 * n + i];
    }
    sh[threadIdx.x] = s;
    __syncthreads();
    for (int w = OBJ_T / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = sh[0];
}

// histogram of the next 8 bits among values whose higher bits equal the prefix.  The values cluster
// in few bins (the top byte is the exponent), so each block keeps 8 sub-histograms (lane & 7; rows
// 257 words apart, so a bin's copies lie in different LDS banks) to spread the atomic increments.
#define OBJ_SUBH 8
__global__ void __launch_bounds__(OBJ_T) k_obj_hist(const uint32_t* __restrict__ ebits, const float* __restrict__ res,
                                                   int64_t n, const uint32_t* __restrict__ sel, int shift,
                                                   uint32_t* __restrict__ hist) {
    __shared__ uint32_t h[OBJ_SUBH][257];
#pragma unroll
    for (int k = 0; k < OBJ_SUBH; ++k) h[k][threadIdx.x] = 0;
    __syncthreads();
    uint32_t prefix = sel[0], pmask = sel[1];
    uint32_t* mine = h[threadIdx.x & (OBJ_SUBH - 1)];
    for (int64_t i = (int64_t)blockIdx.x * OBJ_T + threadIdx.x; i < n; i += (int64_t)gridDim.x * OBJ_T) {
        uint32_t b = ebits ? ebits[i] : obj_key(res, n, i);
        if ((b & pmask) == prefix) atomicAdd(&mine[(b >> shift) & 0xffu], 1u);
    }
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int k = 0; k < OBJ_SUBH; ++k) t += h[k][threadIdx.x];
    if (t) atomicAdd(&hist[threadIdx.x], t);
}

// pick the bin holding the k-th smallest (k in sel[2], 1-based); clear hist for the next pass
// One wave: lane l holds bins 4l .. 4l + 3; an inclusive scan of the lane sums finds the lane, then
// the bin, where the running count first reaches k (the same bin and count as a sequential walk;
// when no bin reaches k: bin 255 with the full count, as that walk leaves them).
__global__ void __launch_bounds__(64) k_obj_pick(uint32_t* __restrict__ hist, uint32_t* __restrict__ sel, int shift) {
    const int l = threadIdx.x;
    const uint32_t k = sel[2];
    uint32_t h[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) h[q] = hist[4 * l + q];
    const uint32_t s = h[0] + h[1] + h[2] + h[3];
    uint32_t inc = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(inc, off);
        if (l >= off) inc += t;
    }
    const uint64_t ball = __ballot(inc >= k);
    int b = 255;
    uint32_t cum = __shfl(inc, 63);
    if (ball) {
        const int L = __ffsll((unsigned long long)ball) - 1;
        uint32_t c = __shfl(inc - s, L);
        uint32_t hl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) hl[q] = __shfl(h[q], L);
        int q = 0;
        for (; q < 3; ++q) {
            if (c + hl[q] >= k) break;
            c += hl[q];
        }
        b = 4 * L + q;
        cum = c;
    }
    if (l == 0) {
        sel[0] |= (uint32_t)b << shift;
        sel[1] |= 0xffu << shift;
        sel[2] = k - cum;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) hist[4 * l + q] = 0;
}

__global__ void __launch_bounds__(OBJ_T) k_obj_below(const uint32_t* __restrict__ ebits, const float* __restrict__ res,
                                                    int64_t n, const uint32_t* __restrict__ sel,
                                                    double* __restrict__ psum, uint32_t* __restrict__ pcnt) {
    __shared__ double sh[OBJ_T];
    __shared__ uint32_t sc[OBJ_T];
    uint32_t T = sel[0];
    double s = 0.0;
    uint32_t c = 0;
    for (int64_t i = (int64_t)blockIdx.x * OBJ_T + threadIdx.x; i < n; i += (int64_t)gridDim.x * OBJ_T) {
        uint32_t b = ebits ? ebits[i] : obj_key(res, n, i);
        if (b < T) { s += (double)__uint_as_float(b); c += 1; }
    }
    sh[threadIdx.x] = s; sc[threadIdx.x] = c;
    __syncthreads();
    for (int w = OBJ_T / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) { sh[threadIdx.x] += sh[threadIdx.x + w]; sc[threadIdx.x] += sc[threadIdx.x + w]; }
        __syncthreads();
    }
    if (threadIdx.x == 0) { psum[blockIdx.x] = sh[0]; pcnt[blockIdx.x] = sc[0]; }
}

__global__ void __launch_bounds__(OBJ_T) k_obj_final(const double* __restrict__ lpart, const double* __restrict__ psum,
                                                    const uint32_t* __restrict__ pcnt, int nb, int64_t n,
                                                    int64_t n80, const uint32_t* __restrict__ sel, int has_err,
                                                    float* __restrict__ out) {
    __shared__ double sh[OBJ_T], sl[OBJ_T];
    __shared__ uint64_t sc[OBJ_T];
    double s = 0.0, l = 0.0;
    uint64_t c = 0;
    for (int b = threadIdx.x; b < nb; b += OBJ_T) { s += psum[b]; l += lpart[b]; c += pcnt[b]; }
    sh[threadIdx.x] = s; sl[threadIdx.x] = l; sc[threadIdx.x] = c;
    __syncthreads();
    for (int w = OBJ_T / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) {
            sh[threadIdx.x] += sh[threadIdx.x + w]; sl[threadIdx.x] += sl[threadIdx.x + w]; sc[threadIdx.x] += sc[threadIdx.x + w];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        float T = __uint_as_float(sel[0]);
        double tot = sh[0] + (double)(n80 - (int64_t)sc[0]) * (double)T;
        out[0] = has_err ? (float)(sl[0] / (3.0 * (double)n)) : NAN;
        out[1] = n80 > 0 ? (float)(tot / (double)n80) : NAN;
    }
}

// ------------------------------------------------------------------ input checks
struct NfSpans {
    const float* p[BA_NONFINITE_MAX_SPANS];
    int64_t n[BA_NONFINITE_MAX_SPANS];
};

__global__ void __launch_bounds__(64) k_nf_clear(int32_t* flags, int n) {
    if ((int)threadIdx.x < n) flags[threadIdx.x] = 0;
}

// blockIdx.y = span; every block strides over its span, 16-byte loads where the span's first element is
// 16-byte aligned (the 0-3 leading elements before that boundary and the tail are read singly).  A
// non-finite value (exponent bits all ones) sets the span's flag; every writer stores the same 1.
#define NF_T 256
__global__ void __launch_bounds__(NF_T) k_nonfinite(NfSpans sp, int32_t* flags) {
    const int t = blockIdx.y;
    const float* __restrict__ p = sp.p[t];
    const int64_t n = sp.n[t];
    const uint32_t E = 0x7f800000u;
    const int64_t mis = (int64_t)(((16 - ((uintptr_t)p & 15)) & 15) >> 2);   // elements before the 16-byte boundary
    const int64_t lead = mis < n ? mis : n;
    bool bad = false;
    const int64_t gtid = (int64_t)blockIdx.x * NF_T + threadIdx.x, gstride = (int64_t)gridDim.x * NF_T;
    if (((uintptr_t)p & 3) == 0) {
        const int64_t nv = (n - lead) >> 2;
        const uint4* __restrict__ v = (const uint4*)(p + lead);
        for (int64_t k = gtid; k < nv; k += gstride) {
            const uint4 q = v[k];
            bad |= ((q.x & E) == E) | ((q.y & E) == E) | ((q.z & E) == E) | ((q.w & E) == E);
        }
        for (int64_t k = gtid; k < lead; k += gstride) bad |= (__float_as_uint(p[k]) & E) == E;
        for (int64_t k = lead + 4 * nv + gtid; k < n; k += gstride) bad |= (__float_as_uint(p[k]) & E) == E;
    } else {
        for (int64_t k = gtid; k < n; k += gstride) bad |= (__float_as_uint(p[k]) & E) == E;
    }
    if (bad) flags[t] = 1;
}

// ------------------------------------------------------------------ STREAM triad
__global__ void __launch_bounds__(256) k_triad(double* __restrict__ a, const double* __restrict__ b,
                                               const double* __restrict__ c, double s, int64_t n) {
    const int64_t n2 = n >> 1;
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x, gs = (int64_t)gridDim.x * 256;
    for (int64_t i = g; i < n2; i += gs) {
        const double2 x = reinterpret_cast<const double2*>(b)[i], y = reinterpret_cast<const double2*>(c)[i];
        reinterpret_cast<double2*>(a)[i] = make_double2(x.x + s * y.x, x.y + s * y.y);
    }
    if (g == 0 && (n & 1)) a[n - 1] = b[n - 1] + s * c[n - 1];
}

}  // namespace ba

using namespace ba;

static inline unsigned nbk(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

// a[i] = b[i] + s * c[i], i < n (fp64, 16-byte aligned arrays)
extern "C" int ba_stream_triad(double* a, const double* b, const double* c, double s, int64_t n, void* stream) {
    clear_error();
    BA_REQUIRE(n >= 0, "bad size");
    if (n == 0) return BA_OK;
    BA_REQUIRE(a && b && c, "null array");
    BA_REQUIRE((((uintptr_t)a | (uintptr_t)b | (uintptr_t)c) & 15) == 0, "arrays must be 16-byte aligned");
    // a large grid with few elements per thread streams best (measured on MI355X over 3 x 1 GiB:
    // 5.5 TB/s at 65536 blocks against 4.6-5.0 TB/s at 2048-16384 blocks or with unrolled loads)
    int64_t nb = (n / 2 + 255) / 256;
    nb = nb < 1 ? 1 : (nb > 65536 ? 65536 : nb);
    hipLaunchKernelGGL(k_triad, dim3((unsigned)nb), dim3(256), 0, (hipStream_t)stream, a, b, c, s, n);
    BA_LAUNCHED();
    return BA_OK;
}

// flags[t] = 1 when ptrs[t][0 .. counts[t]) holds a NaN or an infinity (fp32), else 0.
extern "C" int ba_nonfinite_flags(const float* const* ptrs, const int64_t* counts, int32_t n_spans, int32_t* flags,
                                  void* stream) {
    clear_error();
    BA_REQUIRE(n_spans >= 0 && n_spans <= BA_NONFINITE_MAX_SPANS, "ba_nonfinite_flags: 0 to 16 arrays");
    BA_REQUIRE(n_spans == 0 || (ptrs != nullptr && counts != nullptr && flags != nullptr), "null argument");
    if (n_spans == 0) return BA_OK;
    NfSpans sp{};
    int64_t most = 0;
    for (int t = 0; t < n_spans; ++t) {
        BA_REQUIRE(counts[t] >= 0 && (counts[t] == 0 || ptrs[t] != nullptr), "bad array");
        sp.p[t] = ptrs[t];
        sp.n[t] = counts[t];
        most = counts[t] > most ? counts[t] : most;
    }
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_nf_clear, dim3(1), dim3(64), 0, st, flags, (int)n_spans);
    // enough blocks to stream the largest array at full bandwidth: 4 floats per thread per pass
    int64_t nbx = (most / 4 + NF_T - 1) / NF_T;
    nbx = nbx < 1 ? 1 : (nbx > 2048 ? 2048 : nbx);
    hipLaunchKernelGGL(k_nonfinite, dim3((unsigned)nbx, (unsigned)n_spans), dim3(NF_T), 0, st, sp, flags);
    BA_LAUNCHED();
    return BA_OK;
}

// Replaces the update block of lm_step (engine.py:310-313): one launch for every parameter group.
extern "C" int ba_apply_update(const float* K, const float* P_w2rig, const float* z_coefs, const float* pts3d,
                               const float* dK, const float* dP, const float* dZ, const float* dX, float scale,
                               float min_f, int32_t n_cams, int32_t n_nodes, int32_t n_imgs, int32_t C,
                               int64_t n_tracks, float* K_out, float* P_out, float* z_out, float* X_out,
                               void* stream) {
    clear_error();
    int64_t total = (int64_t)n_cams + n_nodes + (int64_t)n_imgs * C + 3 * n_tracks;
    if (total == 0) return BA_OK;
    hipLaunchKernelGGL(k_apply_update, dim3(nbk(total, 256)), dim3(256), 0, (hipStream_t)stream, K, P_w2rig, z_coefs,
                       pts3d, dK, dP, dZ, dX, scale, min_f, n_cams, n_nodes, n_imgs, C, n_tracks, K_out, P_out, z_out,
                       X_out);
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int64_t ba_objective_workspace_bytes(int64_t n_obs) {
    int64_t nb = (n_obs + OBJ_T - 1) / OBJ_T;
    if (nb < 1) nb = 1;
    return 4 * n_obs + 8 * nb * 2 + 4 * nb + 4 * 256 + 4 * 4 + 64;
}

namespace ba {

// The launch sequence of ba_objective.  ebits (4 bytes per observation) keeps each observation's
// key between the passes; when it is null the passes recompute the key from res instead.  lpart,
// psum (fp64) and pcnt hold one partial per block of the grid-stride passes (at most OBJ_NBMAX),
// hist 256 counters, sel 4 words; k_obj_init clears hist and sel, every partial is written before
// it is read.
static int objective_launch(const float* res, int64_t n_obs, int32_t has_err, uint32_t* ebits, double* lpart,
                            double* psum, uint32_t* pcnt, uint32_t* hist, uint32_t* sel, float* out, hipStream_t st) {
    int64_t nb = (n_obs + OBJ_T - 1) / OBJ_T;
    if (nb < 1) nb = 1;
    int64_t n80 = n_obs * 80 / 100;
    BA_REQUIRE(n80 <= (int64_t)UINT32_MAX, "ba_objective: the 80% rank of n_obs must fit 32 bits "
                                          "(n_obs <= 5368709119)");
    // the per-block partials of prep and below: at most OBJ_NBMAX blocks (grid-stride loops), so the
    // one-block final sum stays short
    const int64_t nbp = nb < OBJ_NBMAX ? nb : OBJ_NBMAX;
    hipLaunchKernelGGL(k_obj_init, dim3(1), dim3(256), 0, st, hist, sel, (uint32_t)(n80 > 0 ? n80 : 1));
    if (n_obs > 0) {
        hipLaunchKernelGGL(k_obj_prep, dim3((unsigned)nbp), dim3(OBJ_T), 0, st, res, n_obs, has_err, ebits, lpart);
        unsigned hb = (unsigned)(nb < 1024 ? nb : 1024);
        for (int pass = 0; pass < 4; ++pass) {
            int shift = 24 - 8 * pass;
            hipLaunchKernelGGL(k_obj_hist, dim3(hb), dim3(OBJ_T), 0, st, ebits, res, n_obs, sel, shift, hist);
            hipLaunchKernelGGL(k_obj_pick, dim3(1), dim3(64), 0, st, hist, sel, shift);
        }
        hipLaunchKernelGGL(k_obj_below, dim3((unsigned)nbp), dim3(OBJ_T), 0, st, ebits, res, n_obs, sel, psum, pcnt);
    } else {
        hipLaunchKernelGGL(k_obj_prep, dim3(1), dim3(OBJ_T), 0, st, res, (int64_t)0, has_err, ebits, lpart);
        hipLaunchKernelGGL(k_obj_below, dim3(1), dim3(OBJ_T), 0, st, ebits, res, (int64_t)0, sel, psum, pcnt);
    }
    hipLaunchKernelGGL(k_obj_final, dim3(1), dim3(OBJ_T), 0, st, lpart, psum, pcnt, n_obs > 0 ? (int)nbp : 1, n_obs,
                       n80, sel, has_err, out);
    BA_LAUNCHED();
    return BA_OK;
}

// Scratch of ba_objective_noalloc: the fixed-size part of the objective's workspace (the per-block
// partials, histogram and selection state; no per-observation keys), one copy per GPU for the life
// of the process.  Host code never uses the symbol itself: each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current.
#define OBJ_SCRATCH_BYTES (OBJ_NBMAX * (8 + 8 + 4) + 256 * 4 + 4 * 4)
static __device__ __align__(256) unsigned char scratch[(OBJ_SCRATCH_BYTES + 255) / 256 * 256];

#define OBJ_MAX_DEVICES 64
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[OBJ_MAX_DEVICES];

static int scratch_of_current_device(unsigned char** out) {
    int dev = -1;
    BA_HIP(hipGetDevice(&dev));
    BA_REQUIRE(dev >= 0 && dev < OBJ_MAX_DEVICES, "ba_objective_noalloc: device index beyond 64");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        BA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        BA_REQUIRE(p != nullptr, "ba_objective_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *out = (unsigned char*)g_scratch_ptr[dev];
    return BA_OK;
}

}  // namespace ba

// loss = mean(err) and reproj_score from the (9 or 3, n_obs) residual buffer; out[0] = loss,
// out[1] = reproj_score (fp32, device).  Workspace of ba_objective_workspace_bytes(n_obs).
extern "C" int ba_objective(const float* res, int64_t n_obs, int32_t has_err, void* workspace, float* out,
                            void* stream) {
    clear_error();
    BA_REQUIRE(n_obs >= 0, "ba_objective: n_obs < 0");
    int64_t nb = (n_obs + OBJ_T - 1) / OBJ_T;
    if (nb < 1) nb = 1;
    char* w = (char*)workspace;
    uint32_t* ebits = (uint32_t*)w; w += 4 * n_obs;
    w = (char*)(((uintptr_t)w + 7) & ~(uintptr_t)7);
    double* lpart = (double*)w; w += 8 * nb;
    double* psum = (double*)w; w += 8 * nb;
    uint32_t* pcnt = (uint32_t*)w; w += 4 * nb;
    uint32_t* hist = (uint32_t*)w; w += 4 * 256;
    uint32_t* sel = (uint32_t*)w;
    return objective_launch(res, n_obs, has_err, ebits, lpart, psum, pcnt, hist, sel, out, (hipStream_t)stream);
}

// ba_objective with no workspace argument and no allocation: the passes recompute each key from res
// and keep their partials in the library's per-GPU scratch array.  Calls that overlap on one GPU
// share that array and race; the results equal ba_objective's bit for bit.
extern "C" int ba_objective_noalloc(const float* res, int64_t n_obs, int32_t has_err, float* out, void* stream) {
    clear_error();
    BA_REQUIRE(n_obs >= 0, "ba_objective_noalloc: n_obs < 0");
    unsigned char* sp = nullptr;
    int rc = scratch_of_current_device(&sp);
    if (rc != BA_OK) return rc;
    double* lpart = (double*)sp;
    double* psum = lpart + OBJ_NBMAX;
    uint32_t* pcnt = (uint32_t*)(psum + OBJ_NBMAX);
    uint32_t* hist = pcnt + OBJ_NBMAX;
    uint32_t* sel = hist + 256;
    return objective_launch(res, n_obs, has_err, nullptr, lpart, psum, pcnt, hist, sel, out, (hipStream_t)stream);
}
