// Pair-major structure plan built on the device.
//
// The arrays of ba_pm_plan_create (ba_plan.cpp: runs, the tracks' runs and observations in image order,
// the image pairs with their (run, run) terms, the image rows of the pair structure), equal to them
// element for element, from the structure of src/blast3r/inference/tracks.py:19-57 (image-major
// observations, rigs.py:50-51).  Every ordering the host planner produces by a stable sort or a
// bucket fill is produced here by a stable radix sort (rocPRIM) over a composite key:
//   runs        observations by (image, track id), stable: the observation order within a run;
//   track runs  runs by track, stable: the image order within a track;
//   terms       (run r, run rb) of one track with image(r) < image(rb), by (image(r), image(rb), r):
//               the pair order (i1, i2), and within a pair the run order of image i1;
//   image rows  (pair, role) items in pair order, by row image, stable.
// Segment bounds come from flag / scan kernels; counts are exact integer sums.  The arrays live in
// device memory the plan owns (hipMalloc); the caller copies what it keeps and destroys the plan.
#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <algorithm>
#include <cstdint>
#include <string>
#include <vector>

#include "ba_error.h"
#include "ba_plan.h"

namespace ba {

namespace {

constexpr int PT = 256;

inline unsigned grid_of(int64_t n) { return (unsigned)std::max<int64_t>(1, (n + PT - 1) / PT); }

// bits to hold every value in [0, x]
inline unsigned bits_for(uint64_t x) {
    unsigned b = 1;
    while (b < 64 && (x >> b) != 0) ++b;
    return b;
}

// ---------------------------------------------------------------------------- kernels
// input checks: bit 0 cum decreasing, bit 1 cum[F-1] != n_obs, bit 2 pid out of range
__global__ void __launch_bounds__(PT) k_check(const int32_t* __restrict__ cum, int32_t F, const int32_t* __restrict__ pids,
                                              int64_t n, int32_t T, int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * PT + threadIdx.x;
    int e = 0;
    if (i < F && i > 0 && cum[i] < cum[i - 1]) e |= 1;
    if (i == 0 && (int64_t)cum[F - 1] != n) e |= 2;
    if (i < n && (pids[i] < 0 || pids[i] >= T)) e |= 4;
    if (e) atomicOr(err, e);
}

// observation o -> its image (the first i with cum[i] > o); sort key (image, pid) and value o
__global__ void __launch_bounds__(PT) k_obs_keys(const int32_t* __restrict__ cum, int32_t F, const int32_t* __restrict__ pids,
                                                 int64_t n, unsigned pbits, int32_t* __restrict__ obs_img,
                                                 uint64_t* __restrict__ key, int32_t* __restrict__ val) {
    const int64_t o = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (o >= n) return;
    int lo = 0, hi = F - 1;                             // cum[hi] > o holds (cum[F - 1] = n)
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((int64_t)cum[mid] > o) hi = mid; else lo = mid + 1;
    }
    obs_img[o] = lo;
    key[o] = ((uint64_t)lo << pbits) | (uint64_t)(uint32_t)pids[o];
    val[o] = (int32_t)o;
}

// 1 where a sorted key differs from its predecessor (after masking off `shift` low bits)
__global__ void __launch_bounds__(PT) k_flags64(const uint64_t* __restrict__ key, int64_t n, unsigned shift,
                                                int32_t* __restrict__ flag) {
    const int64_t k = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (k >= n) return;
    flag[k] = k == 0 || (key[k] >> shift) != (key[k - 1] >> shift);
}

// runs from the flagged sorted observations: run_ptr, run_trk, run_img (rid = inclusive scan of the flags)
__global__ void __launch_bounds__(PT) k_runs(const uint64_t* __restrict__ key, const int32_t* __restrict__ flag,
                                             const int32_t* __restrict__ rid, int64_t n, unsigned pbits,
                                             int32_t* __restrict__ run_ptr, int32_t* __restrict__ run_trk,
                                             int32_t* __restrict__ run_img) {
    const int64_t k = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (k >= n || !flag[k]) return;
    const int32_t r = rid[k] - 1;
    run_ptr[r] = (int32_t)k;
    run_trk[r] = (int32_t)(key[k] & ((1ull << pbits) - 1));
    run_img[r] = (int32_t)(key[k] >> pbits);
}

// ptr[v] = first position s of the ascending sequence seq[0..m) with seq[s] >= v, for v in [0, nv]
// (one thread per position writes the values between its predecessor's and its own)
__global__ void __launch_bounds__(PT) k_bounds(const int32_t* __restrict__ seq, int64_t m, int64_t nv,
                                               int32_t* __restrict__ ptr) {
    const int64_t s = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (s > m) return;
    const int64_t lo = s ? (int64_t)seq[s - 1] + 1 : 0;
    const int64_t hi = s < m ? (int64_t)seq[s] : nv;
    for (int64_t v = lo; v <= hi; ++v) ptr[v] = (int32_t)s;
}

__global__ void __launch_bounds__(PT) k_iota(int32_t* __restrict__ v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (i < n) v[i] = (int32_t)i;
}

// observations per run, in track-run order
__global__ void __launch_bounds__(PT) k_run_lens(const int32_t* __restrict__ trk_run, const int32_t* __restrict__ run_ptr,
                                                 int64_t R, int32_t* __restrict__ len) {
    const int64_t k = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (k >= R) return;
    const int32_t r = trk_run[k];
    len[k] = run_ptr[r + 1] - run_ptr[r];
}

// trk_obs_ptr[t] = offs[trk_run_ptr[t]] (offs: exclusive scan of the lengths, offs[R] = n_obs); the
// tracks' observations; the runs per track (for the term counts) and their maximum
__global__ void __launch_bounds__(PT) k_trk_obs(const int32_t* __restrict__ trk_run_ptr, const int32_t* __restrict__ offs,
                                                const int32_t* __restrict__ trk_run, const int32_t* __restrict__ run_ptr,
                                                const int32_t* __restrict__ run_obs, int32_t T, int64_t R,
                                                int32_t* __restrict__ trk_obs_ptr, int32_t* __restrict__ trk_obs,
                                                int64_t* __restrict__ tcnt, int32_t* __restrict__ max_runs) {
    const int64_t t = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (t > T) return;
    const int32_t q0 = trk_run_ptr[t];
    trk_obs_ptr[t] = offs[q0];
    if (t == T) return;
    const int32_t q1 = trk_run_ptr[t + 1];
    const int64_t m = q1 - q0;
    tcnt[t] = m * (m - 1) / 2;
    atomicMax(max_runs, (int32_t)m);
    for (int32_t q = q0; q < q1; ++q) {
        const int32_t r = trk_run[q], o0 = offs[q];
        for (int32_t j = run_ptr[r]; j < run_ptr[r + 1]; ++j) trk_obs[o0 + (j - run_ptr[r])] = run_obs[j];
    }
}

// terms of each (track, position q): (r, rb) for every later run rb of the track, key (a, b, r)
__global__ void __launch_bounds__(PT) k_terms(const int32_t* __restrict__ strk, const int32_t* __restrict__ trk_run,
                                              const int32_t* __restrict__ trk_run_ptr, const int64_t* __restrict__ toff,
                                              const int32_t* __restrict__ run_img, int64_t R, int64_t F, unsigned rbits,
                                              uint64_t* __restrict__ key, int32_t* __restrict__ val) {
    const int64_t k = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (k >= R) return;
    const int32_t t = strk[k];
    const int64_t q0 = trk_run_ptr[t], m = trk_run_ptr[t + 1] - q0, q = k - q0;
    const int32_t r = trk_run[k];
    const uint64_t a = (uint64_t)run_img[r];
    int64_t pos = toff[t] + q * (2 * m - q - 1) / 2;
    for (int64_t q2 = q + 1; q2 < m; ++q2, ++pos) {
        const int32_t rb = trk_run[q0 + q2];
        key[pos] = ((a * (uint64_t)F + (uint64_t)run_img[rb]) << rbits) | (uint64_t)(uint32_t)r;
        val[pos] = rb;
    }
}

// the off-diagonal pairs (distinct (a, b) of the sorted terms): first term and (a, b) of each
__global__ void __launch_bounds__(PT) k_off_pairs(const uint64_t* __restrict__ key, const int32_t* __restrict__ flag,
                                                  const int32_t* __restrict__ pid1, int64_t M, unsigned rbits, int64_t F,
                                                  int32_t* __restrict__ off_start, int32_t* __restrict__ off_a,
                                                  int32_t* __restrict__ off_b) {
    const int64_t s = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (s >= M || !flag[s]) return;
    const int32_t j = pid1[s] - 1;
    const uint64_t ab = key[s] >> rbits;
    off_start[j] = (int32_t)s;
    off_a[j] = (int32_t)(ab / (uint64_t)F);
    off_b[j] = (int32_t)(ab % (uint64_t)F);
}

// pairs per image row: the diagonal one when the image has runs, then its off-diagonal ones
__global__ void __launch_bounds__(PT) k_row_count(const int32_t* __restrict__ img_run_ptr,
                                                  const int32_t* __restrict__ offp_ptr, int32_t F, int32_t* __restrict__ c) {
    const int64_t a = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (a >= F) return;
    c[a] = (img_run_ptr[a + 1] > img_run_ptr[a]) + (offp_ptr[a + 1] - offp_ptr[a]);
}

__global__ void __launch_bounds__(PT) k_diag_pairs(const int32_t* __restrict__ img_run_ptr, const int32_t* __restrict__ pbase,
                                                   const int32_t* __restrict__ offp_ptr, const int32_t* __restrict__ off_start,
                                                   int32_t F, int64_t n_off, int64_t M, int32_t* __restrict__ pair_i1,
                                                   int32_t* __restrict__ pair_i2, int32_t* __restrict__ diag_pair,
                                                   int32_t* __restrict__ term_ptr) {
    const int64_t a = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (a >= F) return;
    if (img_run_ptr[a + 1] > img_run_ptr[a]) {
        const int32_t p = pbase[a];
        pair_i1[p] = (int32_t)a; pair_i2[p] = (int32_t)a;
        diag_pair[a] = p;
        // no terms: it starts where the row's first off-diagonal pair (or any later one) starts
        const int32_t j = offp_ptr[a];
        term_ptr[p] = j < n_off ? off_start[j] : (int32_t)M;
    } else {
        diag_pair[a] = -1;
    }
}

__global__ void __launch_bounds__(PT) k_fill_off(const int32_t* __restrict__ off_start, const int32_t* __restrict__ off_a,
                                                 const int32_t* __restrict__ off_b, const int32_t* __restrict__ offp_ptr,
                                                 const int32_t* __restrict__ pbase, const int32_t* __restrict__ img_run_ptr,
                                                 int64_t n_off, int64_t M, int32_t* __restrict__ pair_i1,
                                                 int32_t* __restrict__ pair_i2, int32_t* __restrict__ term_ptr,
                                                 int32_t* __restrict__ max_terms) {
    const int64_t j = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (j >= n_off) return;
    const int32_t a = off_a[j];
    const int32_t p = pbase[a] + (img_run_ptr[a + 1] > img_run_ptr[a]) + (int32_t)(j - offp_ptr[a]);
    pair_i1[p] = a; pair_i2[p] = off_b[j];
    term_ptr[p] = off_start[j];
    const int64_t e = j + 1 < n_off ? off_start[j + 1] : M;
    atomicMax(max_terms, (int32_t)(e - off_start[j]));
}

// term (r, rb) pairs from the sorted keys and values
__global__ void __launch_bounds__(PT) k_term_out(const uint64_t* __restrict__ key, const int32_t* __restrict__ val, int64_t M,
                                                 unsigned rbits, int32_t* __restrict__ term) {
    const int64_t s = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (s >= M) return;
    term[2 * s] = (int32_t)(key[s] & ((1ull << rbits) - 1));
    term[2 * s + 1] = val[s];
}

// image-row items in pair order: (i1, p << 1) and, off the diagonal, (i2, (p << 1) | 1); position of pair
// p's first item = p + (off-diagonal pairs before p) (= ipos, an exclusive scan of the off flags)
__global__ void __launch_bounds__(PT) k_off_flag(const int32_t* __restrict__ pair_i1, const int32_t* __restrict__ pair_i2,
                                                 int64_t P, int32_t* __restrict__ f) {
    const int64_t p = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (p < P) f[p] = pair_i1[p] != pair_i2[p];
}

__global__ void __launch_bounds__(PT) k_row_items(const int32_t* __restrict__ pair_i1, const int32_t* __restrict__ pair_i2,
                                                  const int32_t* __restrict__ ipos, int64_t P, uint32_t* __restrict__ key,
                                                  int32_t* __restrict__ val) {
    const int64_t p = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (p >= P) return;
    const int64_t q = p + ipos[p];
    key[q] = (uint32_t)pair_i1[p];
    val[q] = (int32_t)(p << 1);
    if (pair_i2[p] != pair_i1[p]) {
        key[q + 1] = (uint32_t)pair_i2[p];
        val[q + 1] = (int32_t)((p << 1) | 1);
    }
}

// per track: the images of its first and last run (0 for a track without runs, which no term names)
__global__ void __launch_bounds__(PT) k_track_span(const int32_t* __restrict__ trk_run_ptr,
                                                   const int32_t* __restrict__ trk_run, const int32_t* __restrict__ run_img,
                                                   int64_t T, int32_t* __restrict__ tlo, int32_t* __restrict__ thi) {
    const int64_t t = (int64_t)blockIdx.x * PT + threadIdx.x;
    if (t >= T) return;
    const int32_t r0 = trk_run_ptr[t], r1 = trk_run_ptr[t + 1];
    tlo[t] = r1 > r0 ? run_img[trk_run[r0]] : 0;
    thi[t] = r1 > r0 ? run_img[trk_run[r1 - 1]] : 0;
}

// per pair (one wave each): the sort key of the pair schedule, lo * (F + 1) + hi with lo / hi the smallest
// first / largest last image of its terms' tracks (F, F without terms), and the pair id as its value
__global__ void __launch_bounds__(PT) k_pair_keys(const int32_t* __restrict__ term_ptr, const int32_t* __restrict__ term,
                                                  const int32_t* __restrict__ run_trk, const int32_t* __restrict__ tlo,
                                                  const int32_t* __restrict__ thi, int64_t NP, int32_t F,
                                                  uint64_t* __restrict__ key, int32_t* __restrict__ val) {
    const int64_t p = (int64_t)blockIdx.x * (PT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (p >= NP) return;                                // p is the same for the whole wave
    const int32_t q0 = term_ptr[p], q1 = term_ptr[p + 1];
    int32_t lo = INT32_MAX, hi = -1;
    for (int32_t q = q0 + lane; q < q1; q += 64) {
        const int32_t t = run_trk[term[2 * (int64_t)q]];
        lo = min(lo, tlo[t]);
        hi = max(hi, thi[t]);
    }
    for (int off = 32; off > 0; off >>= 1) {
        lo = min(lo, __shfl_xor(lo, off));
        hi = max(hi, __shfl_xor(hi, off));
    }
    if (lane == 0) {
        if (q1 == q0) { lo = F; hi = F; }
        key[p] = (uint64_t)lo * (uint64_t)(F + 1) + (uint64_t)hi;
        val[p] = (int32_t)p;
    }
}

// ---------------------------------------------------------------------------- the plan object
struct DevPmPlan {
    int32_t* v[BA_PM_NARRAYS] = {nullptr};
    int64_t size[BA_PM_NARRAYS] = {0};
    int64_t scalars[BA_PM_NSCALARS] = {0};
    ~DevPmPlan() {
        for (auto* p : v)
            if (p) (void)hipFree(p);
    }
};

// temporaries of one build, freed when it returns
struct Temps {
    std::vector<void*> ptrs;
    ~Temps() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <typename T>
    T* get(int64_t n, hipError_t& e) {
        void* p = nullptr;
        if (e == hipSuccess) e = hipMalloc(&p, (size_t)std::max<int64_t>(n, 1) * sizeof(T));
        if (p) ptrs.push_back(p);
        return (T*)p;
    }
};

thread_local std::string g_pm_err;

}  // namespace

}  // namespace ba

using namespace ba;

#define PM_TRY(call)                                                            \
    do {                                                                        \
        hipError_t e_ = (call);                                                 \
        if (e_ != hipSuccess) {                                                 \
            g_pm_err = std::string(#call) + ": " + hipGetErrorString(e_);      \
            delete P;                                                           \
            return nullptr;                                                     \
        }                                                                       \
    } while (0)
#define PM_FAIL(msg)                                                            \
    do {                                                                        \
        g_pm_err = (msg);                                                       \
        delete P;                                                               \
        return nullptr;                                                         \
    } while (0)

namespace {
// stable radix sort of (key, value) pairs over bits [0, end_bit), out of place
template <typename K>
hipError_t sort_pairs(Temps& tmp, const K* kin, K* kout, const int32_t* vin, int32_t* vout, int64_t n, unsigned end_bit,
                      hipStream_t st) {
    if (n == 0) return hipSuccess;
    size_t bytes = 0;
    hipError_t e = rocprim::radix_sort_pairs(nullptr, bytes, kin, kout, vin, vout, (size_t)n, 0u, end_bit, st);
    if (e != hipSuccess) return e;
    void* t = tmp.get<char>((int64_t)bytes, e);
    if (e != hipSuccess) return e;
    return rocprim::radix_sort_pairs(t, bytes, kin, kout, vin, vout, (size_t)n, 0u, end_bit, st);
}

template <typename T>
hipError_t scan(Temps& tmp, const T* in, T* out, int64_t n, bool inclusive, hipStream_t st) {
    if (n == 0) return hipSuccess;
    size_t bytes = 0;
    hipError_t e = inclusive ? rocprim::inclusive_scan(nullptr, bytes, in, out, (size_t)n, rocprim::plus<T>(), st)
                             : rocprim::exclusive_scan(nullptr, bytes, in, out, T(0), (size_t)n, rocprim::plus<T>(), st);
    if (e != hipSuccess) return e;
    void* t = tmp.get<char>((int64_t)bytes, e);
    if (e != hipSuccess) return e;
    return inclusive ? rocprim::inclusive_scan(t, bytes, in, out, (size_t)n, rocprim::plus<T>(), st)
                     : rocprim::exclusive_scan(t, bytes, in, out, T(0), (size_t)n, rocprim::plus<T>(), st);
}

template <typename T>
hipError_t read1(const T* dptr, T& host, hipStream_t st) {
    hipError_t e = hipMemcpyAsync(&host, dptr, sizeof(T), hipMemcpyDeviceToHost, st);
    return e != hipSuccess ? e : hipStreamSynchronize(st);
}
}  // namespace

// Builds the pair-major plan of (cum_nkpts, pids) on the device: both are device arrays (int32), the plan's
// arrays are allocated and owned by the returned handle (NULL on error, see ba_pm_dplan_last_error).  Runs
// on `stream` and synchronises it a few times to size its arrays.
extern "C" void* ba_pm_dplan_create(const int32_t* cum, int32_t F, const int32_t* pids, int64_t n, int32_t T,
                                    void* stream) {
    g_pm_err.clear();
    DevPmPlan* P = nullptr;
    if (F <= 0 || n < 0 || T < 0 || cum == nullptr || (n > 0 && pids == nullptr)) PM_FAIL("bad sizes");
    if (n >= ((int64_t)1 << 30)) PM_FAIL("more than 2^30 observations");
    P = new DevPmPlan();
    hipStream_t st = (hipStream_t)stream;
    Temps tmp;
    hipError_t e = hipSuccess;
    auto alloc_out = [&](int which, int64_t len) -> int32_t* {
        void* p = nullptr;
        if (e == hipSuccess) e = hipMalloc(&p, (size_t)std::max<int64_t>(len, 1) * sizeof(int32_t));
        P->v[which] = (int32_t*)p;
        P->size[which] = len;
        return (int32_t*)p;
    };
    // ---- checks
    int32_t* err = tmp.get<int32_t>(1, e);
    PM_TRY(e);
    PM_TRY(hipMemsetAsync(err, 0, sizeof(int32_t), st));
    hipLaunchKernelGGL(k_check, dim3(grid_of(std::max<int64_t>(n, F))), dim3(PT), 0, st, cum, F, pids, n, T, err);
    int32_t herr = 0;
    PM_TRY(read1(err, herr, st));
    if (herr & 1) PM_FAIL("infos[0] must be non-decreasing");
    if (herr & 2) PM_FAIL("infos[0][-1] != number of observations");
    if (herr & 4) PM_FAIL("pid out of range");
    const unsigned pbits = bits_for(T > 0 ? (uint64_t)T - 1 : 0), ibits = bits_for((uint64_t)F - 1);
    // ---- runs: observations by (image, pid), stable
    int32_t* obs_img = alloc_out(BA_PM_OBS_IMG, n);
    int32_t* run_obs = alloc_out(BA_PM_RUN_OBS, n);
    uint64_t* k1 = tmp.get<uint64_t>(n, e);
    uint64_t* k2 = tmp.get<uint64_t>(n, e);
    int32_t* v1 = tmp.get<int32_t>(n, e);
    int32_t* flag = tmp.get<int32_t>(n, e);
    int32_t* rid = tmp.get<int32_t>(n, e);
    PM_TRY(e);
    if (n > 0) {
        hipLaunchKernelGGL(k_obs_keys, dim3(grid_of(n)), dim3(PT), 0, st, cum, F, pids, n, pbits, obs_img, k1, v1);
        PM_TRY(sort_pairs<uint64_t>(tmp, k1, k2, v1, run_obs, n, pbits + ibits, st));
        hipLaunchKernelGGL(k_flags64, dim3(grid_of(n)), dim3(PT), 0, st, k2, n, 0u, flag);
        PM_TRY(scan<int32_t>(tmp, flag, rid, n, true, st));
    }
    int32_t R32 = 0;
    if (n > 0) PM_TRY(read1(rid + (n - 1), R32, st));
    const int64_t R = R32;
    int32_t* run_ptr = alloc_out(BA_PM_RUN_PTR, R + 1);
    int32_t* run_trk = alloc_out(BA_PM_RUN_TRK, R);
    int32_t* run_img = alloc_out(BA_PM_RUN_IMG, R);
    int32_t* img_run_ptr = alloc_out(BA_PM_IMG_RUN_PTR, (int64_t)F + 1);
    PM_TRY(e);
    if (n > 0)
        hipLaunchKernelGGL(k_runs, dim3(grid_of(n)), dim3(PT), 0, st, k2, flag, rid, n, pbits, run_ptr, run_trk, run_img);
    {
        const int32_t nn = (int32_t)n;
        PM_TRY(hipMemcpyAsync(run_ptr + R, &nn, sizeof(int32_t), hipMemcpyHostToDevice, st));
        PM_TRY(hipStreamSynchronize(st));                  // nn lives on this frame
    }
    hipLaunchKernelGGL(k_bounds, dim3(grid_of(R + 1)), dim3(PT), 0, st, run_img, R, (int64_t)F, img_run_ptr);
    // ---- the tracks' runs (stable by track: image order within a track) and observations
    int32_t* trk_run = alloc_out(BA_PM_TRK_RUN, R);
    int32_t* trk_run_ptr = alloc_out(BA_PM_TRK_RUN_PTR, (int64_t)T + 1);
    int32_t* trk_obs_ptr = alloc_out(BA_PM_TRK_OBS_PTR, (int64_t)T + 1);
    int32_t* trk_obs = alloc_out(BA_PM_TRK_OBS, n);
    int32_t* rids = tmp.get<int32_t>(R, e);
    int32_t* strk = tmp.get<int32_t>(R, e);
    int32_t* lens = tmp.get<int32_t>(R + 1, e);
    int32_t* offs = tmp.get<int32_t>(R + 1, e);
    int64_t* tcnt = tmp.get<int64_t>((int64_t)T + 1, e);
    int64_t* toff = tmp.get<int64_t>((int64_t)T + 1, e);
    int32_t* mx = tmp.get<int32_t>(2, e);
    PM_TRY(e);
    PM_TRY(hipMemsetAsync(mx, 0, 2 * sizeof(int32_t), st));
    PM_TRY(hipMemsetAsync(lens + R, 0, sizeof(int32_t), st));
    PM_TRY(hipMemsetAsync(tcnt + T, 0, sizeof(int64_t), st));
    if (R > 0) {
        hipLaunchKernelGGL(k_iota, dim3(grid_of(R)), dim3(PT), 0, st, rids, R);
        PM_TRY(sort_pairs<int32_t>(tmp, run_trk, strk, rids, trk_run, R, pbits, st));
        hipLaunchKernelGGL(k_run_lens, dim3(grid_of(R)), dim3(PT), 0, st, trk_run, run_ptr, R, lens);
    }
    hipLaunchKernelGGL(k_bounds, dim3(grid_of(R + 1)), dim3(PT), 0, st, strk, R, (int64_t)T, trk_run_ptr);
    PM_TRY(scan<int32_t>(tmp, lens, offs, R + 1, false, st));
    hipLaunchKernelGGL(k_trk_obs, dim3(grid_of((int64_t)T + 1)), dim3(PT), 0, st, trk_run_ptr, offs, trk_run, run_ptr,
                       run_obs, T, R, trk_obs_ptr, trk_obs, tcnt, mx);
    // ---- terms, sorted by (image a, image b, run r)
    PM_TRY(scan<int64_t>(tmp, tcnt, toff, (int64_t)T + 1, false, st));
    int64_t M = 0;
    PM_TRY(read1(toff + T, M, st));
    if (M >= ((int64_t)1 << 30)) PM_FAIL("too many pair terms");
    const unsigned rbits = bits_for(R > 0 ? (uint64_t)R - 1 : 0);
    const unsigned abits = bits_for((uint64_t)F * (uint64_t)F - 1);
    if (rbits + abits > 64) PM_FAIL("image pair and run ids exceed a 64-bit sort key");
    uint64_t* tk1 = tmp.get<uint64_t>(M, e);
    uint64_t* tk2 = tmp.get<uint64_t>(M, e);
    int32_t* tv1 = tmp.get<int32_t>(M, e);
    int32_t* tv2 = tmp.get<int32_t>(M, e);
    int32_t* tflag = tmp.get<int32_t>(M, e);
    int32_t* tpid = tmp.get<int32_t>(M, e);
    PM_TRY(e);
    int32_t n_off32 = 0;
    if (M > 0) {
        hipLaunchKernelGGL(k_terms, dim3(grid_of(R)), dim3(PT), 0, st, strk, trk_run, trk_run_ptr, toff, run_img, R,
                           (int64_t)F, rbits, tk1, tv1);
        PM_TRY(sort_pairs<uint64_t>(tmp, tk1, tk2, tv1, tv2, M, rbits + abits, st));
        hipLaunchKernelGGL(k_flags64, dim3(grid_of(M)), dim3(PT), 0, st, tk2, M, rbits, tflag);
        PM_TRY(scan<int32_t>(tmp, tflag, tpid, M, true, st));
        PM_TRY(read1(tpid + (M - 1), n_off32, st));
    }
    const int64_t n_off = n_off32;
    int32_t* off_start = tmp.get<int32_t>(n_off, e);
    int32_t* off_a = tmp.get<int32_t>(n_off, e);
    int32_t* off_b = tmp.get<int32_t>(n_off, e);
    int32_t* offp_ptr = tmp.get<int32_t>((int64_t)F + 1, e);
    int32_t* rc = tmp.get<int32_t>((int64_t)F + 1, e);
    int32_t* pbase = tmp.get<int32_t>((int64_t)F + 1, e);
    PM_TRY(e);
    if (M > 0)
        hipLaunchKernelGGL(k_off_pairs, dim3(grid_of(M)), dim3(PT), 0, st, tk2, tflag, tpid, M, rbits, (int64_t)F,
                           off_start, off_a, off_b);
    hipLaunchKernelGGL(k_bounds, dim3(grid_of(n_off + 1)), dim3(PT), 0, st, off_a, n_off, (int64_t)F, offp_ptr);
    // ---- pairs: per image row the diagonal pair (an image with runs), then the off-diagonal ones
    PM_TRY(hipMemsetAsync(rc + F, 0, sizeof(int32_t), st));
    hipLaunchKernelGGL(k_row_count, dim3(grid_of(F)), dim3(PT), 0, st, img_run_ptr, offp_ptr, F, rc);
    PM_TRY(scan<int32_t>(tmp, rc, pbase, (int64_t)F + 1, false, st));
    int32_t P32 = 0;
    PM_TRY(read1(pbase + F, P32, st));
    const int64_t NP = P32;
    int32_t* pair_i1 = alloc_out(BA_PM_PAIR_I1, NP);
    int32_t* pair_i2 = alloc_out(BA_PM_PAIR_I2, NP);
    int32_t* diag_pair = alloc_out(BA_PM_DIAG_PAIR, F);
    int32_t* term_ptr = alloc_out(BA_PM_TERM_PTR, NP + 1);
    int32_t* term = alloc_out(BA_PM_TERM, 2 * M);
    PM_TRY(e);
    hipLaunchKernelGGL(k_diag_pairs, dim3(grid_of(F)), dim3(PT), 0, st, img_run_ptr, pbase, offp_ptr, off_start, F, n_off,
                       M, pair_i1, pair_i2, diag_pair, term_ptr);
    if (n_off > 0)
        hipLaunchKernelGGL(k_fill_off, dim3(grid_of(n_off)), dim3(PT), 0, st, off_start, off_a, off_b, offp_ptr, pbase,
                           img_run_ptr, n_off, M, pair_i1, pair_i2, term_ptr, mx + 1);
    {
        const int32_t m32 = (int32_t)M;
        PM_TRY(hipMemcpyAsync(term_ptr + NP, &m32, sizeof(int32_t), hipMemcpyHostToDevice, st));
        PM_TRY(hipStreamSynchronize(st));
    }
    if (M > 0) hipLaunchKernelGGL(k_term_out, dim3(grid_of(M)), dim3(PT), 0, st, tk2, tv2, M, rbits, term);
    // ---- the order k_pm_pairs takes the pairs in (BA_PM_PAIR_SCHED): a stable sort of the pairs by the
    // co-visibility window of their terms' tracks, as the host planner's two counting sorts
    {
        int32_t* pair_sched = alloc_out(BA_PM_PAIR_SCHED, NP);
        int32_t* tlo = tmp.get<int32_t>(T, e);
        int32_t* thi = tmp.get<int32_t>(T, e);
        uint64_t* sk1 = tmp.get<uint64_t>(NP, e);
        uint64_t* sk2 = tmp.get<uint64_t>(NP, e);
        int32_t* sv1 = tmp.get<int32_t>(NP, e);
        PM_TRY(e);
        if (NP > 0) {
            if (T > 0)
                hipLaunchKernelGGL(k_track_span, dim3(grid_of(T)), dim3(PT), 0, st, trk_run_ptr, trk_run, run_img,
                                   (int64_t)T, tlo, thi);
            hipLaunchKernelGGL(k_pair_keys, dim3(grid_of(NP * 64)), dim3(PT), 0, st, term_ptr, term, run_trk, tlo, thi,
                               NP, F, sk1, sv1);
            PM_TRY(sort_pairs<uint64_t>(tmp, sk1, sk2, sv1, pair_sched, NP,
                                        bits_for((uint64_t)F * (uint64_t)(F + 1) + (uint64_t)F), st));
        }
    }
    // ---- image rows: (pair, role) items in pair order, stably by row image
    int32_t* offf = tmp.get<int32_t>(NP + 1, e);
    int32_t* ipos = tmp.get<int32_t>(NP + 1, e);
    PM_TRY(e);
    PM_TRY(hipMemsetAsync(offf + NP, 0, sizeof(int32_t), st));
    if (NP > 0) hipLaunchKernelGGL(k_off_flag, dim3(grid_of(NP)), dim3(PT), 0, st, pair_i1, pair_i2, NP, offf);
    PM_TRY(scan<int32_t>(tmp, offf, ipos, NP + 1, false, st));
    const int64_t NI = NP + n_off;                        // every off-diagonal pair adds one item
    int32_t* row_ptr = alloc_out(BA_PM_ROW_PTR, (int64_t)F + 1);
    int32_t* row_ent = alloc_out(BA_PM_ROW_ENT, NI);
    uint32_t* rk1 = tmp.get<uint32_t>(NI, e);
    uint32_t* rk2 = tmp.get<uint32_t>(NI, e);
    int32_t* rv1 = tmp.get<int32_t>(NI, e);
    PM_TRY(e);
    if (NP > 0) {
        hipLaunchKernelGGL(k_row_items, dim3(grid_of(NP)), dim3(PT), 0, st, pair_i1, pair_i2, ipos, NP, rk1, rv1);
        PM_TRY(sort_pairs<uint32_t>(tmp, rk1, rk2, rv1, row_ent, NI, ibits, st));
    }
    hipLaunchKernelGGL(k_bounds, dim3(grid_of(NI + 1)), dim3(PT), 0, st, (const int32_t*)rk2, NI, (int64_t)F, row_ptr);
    PM_TRY(hipGetLastError());
    int32_t hmx[2] = {0, 0};
    PM_TRY(hipMemcpyAsync(hmx, mx, sizeof(hmx), hipMemcpyDeviceToHost, st));
    PM_TRY(hipStreamSynchronize(st));                    // every temporary is released after the last kernel
    P->scalars[BA_PMS_N_RUNS] = R;
    P->scalars[BA_PMS_N_PAIRS] = NP;
    P->scalars[BA_PMS_N_TERMS] = M;
    P->scalars[BA_PMS_MAX_TERMS] = hmx[1];
    P->scalars[BA_PMS_MAX_TRACK_RUNS] = hmx[0];
    return P;
}

// scalars (BA_PMS_*) and array lengths (BA_PM_* order) of a device plan
extern "C" int ba_pm_dplan_query(const void* plan, int64_t* scalars, int64_t* array_sizes) {
    const DevPmPlan* P = (const DevPmPlan*)plan;
    if (!P) return 1;
    for (int k = 0; k < BA_PM_NSCALARS; ++k) scalars[k] = P->scalars[k];
    for (int k = 0; k < BA_PM_NARRAYS; ++k) array_sizes[k] = P->size[k];
    return 0;
}

// device address of array `which` (valid until ba_pm_dplan_destroy)
extern "C" const int32_t* ba_pm_dplan_array(const void* plan, int32_t which) {
    const DevPmPlan* P = (const DevPmPlan*)plan;
    if (!P || which < 0 || which >= BA_PM_NARRAYS) return nullptr;
    return P->v[which];
}

extern "C" void ba_pm_dplan_destroy(void* plan) { delete (DevPmPlan*)plan; }

extern "C" const char* ba_pm_dplan_last_error(void) { return g_pm_err.c_str(); }

// array `which` copied into the caller's device buffer dst (at least its length), on `stream`
extern "C" int ba_pm_dplan_copy(const void* plan, int32_t which, int32_t* dst, void* stream) {
    const DevPmPlan* P = (const DevPmPlan*)plan;
    if (!P || which < 0 || which >= BA_PM_NARRAYS || dst == nullptr) return 1;
    if (P->size[which] == 0) return 0;
    return hipMemcpyAsync(dst, P->v[which], (size_t)P->size[which] * sizeof(int32_t), hipMemcpyDeviceToDevice,
                          (hipStream_t)stream) == hipSuccess ? 0 : 1;
}
