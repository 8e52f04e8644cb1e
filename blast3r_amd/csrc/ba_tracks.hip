// Observation-structure edits on the device: the ObservedTracks operations of
// src/blast3r/inference/tracks.py:19-127 that build a new image-major observation set.
//
//   ba_tracks_gather   `old | new` (tracks.py:84-102) and `tracks[idx]` (tracks.py:66-74): output
//                      image j = rows of image sel_a[j] of set a, then rows of image sel_b[j] of set b
//                      with a pid shift.  Output-driven copy, one thread per output row.
//   ba_tracks_remove   `remove(bad)` (tracks.py:116-127): drop the rows of the listed tracks, count
//                      the rows kept per image, and renumber the remaining tracks by rank (the
//                      sorted-unique + inverse of torch.unique).
//   ba_tracks_to_dense `to_dense(n_imgs)` (tracks.py:104-114): (n_imgs, n_tracks, 2) NaN-filled.
//   ba_tracks_img_id   `img_id` (tracks.py:45-49), including its treatment of empty images (the
//                      delimiters are set, not added, so coinciding delimiters count once).
//
// All of it is integer / byte movement bounded by HBM; the only non-trivial piece is the
// exclusive scan used for offsets, flags and ranks (three launches: block sums, one-block scan
// of the block sums, block rescans).  Row and track counts must stay below 2^31 (int32 offsets,
// as in the reference's int32 infos row).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cmath>

#include "ba_error.h"
#include "ba_hip.h"

namespace ba {

#define TR_T 256                       // threads of the row/track kernels
#define SC_T 256                       // threads of a scan block
#define SC_I 16                        // elements per thread in a scan block
#define SC_E (SC_T * SC_I)             // elements per scan block
#define SC_TOP 1024                    // threads of the one-block scan of block sums

static inline int64_t div_up(int64_t a, int64_t b) { return (a + b - 1) / b; }
static inline int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

// inclusive scan over a wave (64 lanes)
__device__ __forceinline__ int64_t wave_incl(int64_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t t = __shfl_up(v, d);
        if (lane >= d) v += t;
    }
    return v;
}

// exclusive scan over a block of NT threads; *total gets the block sum
template <int NT>
__device__ __forceinline__ int64_t block_excl(int64_t v, int64_t* sh, int64_t* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t inc = wave_incl(v);
    __syncthreads();
    if (lane == 63) sh[w] = inc;
    __syncthreads();
    int64_t base = 0, all = 0;
#pragma unroll
    for (int k = 0; k < NT / 64; ++k) {
        base += k < w ? sh[k] : 0;
        all += sh[k];
    }
    *total = all;
    return base + inc - v;
}

// in[i] (int32, i < n; 0 past n) summed per block of SC_E
__global__ void __launch_bounds__(SC_T) k_scan_up(const int32_t* __restrict__ in, int64_t n, int64_t* __restrict__ bsum) {
    __shared__ int64_t sh[SC_T / 64];
    const int64_t i0 = (int64_t)blockIdx.x * SC_E + (int64_t)threadIdx.x * SC_I;
    int64_t s = 0;
#pragma unroll
    for (int k = 0; k < SC_I; ++k)
        if (i0 + k < n) s += in[i0 + k];
    int64_t tot;
    block_excl<SC_T>(s, sh, &tot);
    if (threadIdx.x == 0) bsum[blockIdx.x] = tot;
}

// exclusive scan of the nb block sums in place; bsum[nb] = total
__global__ void __launch_bounds__(SC_TOP) k_scan_top(int64_t* __restrict__ bsum, int64_t nb) {
    __shared__ int64_t sh[SC_TOP / 64];
    int64_t run = 0;
    for (int64_t c = 0; c < nb; c += SC_TOP) {
        const int64_t i = c + threadIdx.x;
        const int64_t v = i < nb ? bsum[i] : 0;
        int64_t tot;
        const int64_t ex = block_excl<SC_TOP>(v, sh, &tot);
        if (i < nb) bsum[i] = run + ex;
        run += tot;
    }
    if (threadIdx.x == 0) bsum[nb] = run;
}

// out[i] = sum of in[0..i) for i <= n (out has n + 1 entries).  Each thread reads its elements
// before writing the same positions, so out may alias in.
__global__ void __launch_bounds__(SC_T) k_scan_down(const int32_t* in, int64_t n, const int64_t* __restrict__ bsum,
                                                     int64_t nb, int32_t* out) {
    __shared__ int64_t sh[SC_T / 64];
    const int64_t i0 = (int64_t)blockIdx.x * SC_E + (int64_t)threadIdx.x * SC_I;
    int32_t v[SC_I];
    int64_t s = 0;
#pragma unroll
    for (int k = 0; k < SC_I; ++k) {
        v[k] = i0 + k < n ? in[i0 + k] : 0;
        s += v[k];
    }
    int64_t tot;
    int64_t run = bsum[blockIdx.x] + block_excl<SC_T>(s, sh, &tot);
#pragma unroll
    for (int k = 0; k < SC_I; ++k) {
        if (i0 + k < n) out[i0 + k] = (int32_t)run;
        run += v[k];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) out[n] = (int32_t)bsum[nb];
}

// exclusive scan of n int32 values into out[0..n]; bsum holds scan_blocks(n) + 1 int64
static inline int64_t scan_blocks(int64_t n) { return div_up(n > 0 ? n : 1, SC_E); }

static void scan_i32(const int32_t* in, int64_t n, int32_t* out, int64_t* bsum, hipStream_t st) {
    const int64_t nb = scan_blocks(n);
    hipLaunchKernelGGL(k_scan_up, dim3((unsigned)nb), dim3(SC_T), 0, st, in, n, bsum);
    hipLaunchKernelGGL(k_scan_top, dim3(1), dim3(SC_TOP), 0, st, bsum, nb);
    hipLaunchKernelGGL(k_scan_down, dim3((unsigned)nb), dim3(SC_T), 0, st, in, n, bsum, nb, out);
}

__global__ void __launch_bounds__(TR_T) k_fill_i32(int32_t* __restrict__ p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void __launch_bounds__(TR_T) k_fill_f32(float* __restrict__ p, int64_t n, float v) {
    const int64_t i = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (i < n) p[i] = v;
}

// number of rows of output image j: rows of image sel_a[j] of a plus rows of image sel_b[j] of b
__global__ void __launch_bounds__(TR_T) k_gather_counts(ba_gather_args a, int32_t* __restrict__ cnt) {
    const int64_t j = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (j >= a.n_out) return;
    int32_t c = 0;
    const int32_t ia = a.sel_a ? a.sel_a[j] : -1;
    if (ia >= 0 && ia < a.a.n_imgs) c += a.a.nppi[ia];
    const int32_t ib = a.sel_b ? a.sel_b[j] : -1;
    if (ib >= 0 && ib < a.b.n_imgs) c += a.b.nppi[ib];
    cnt[j] = c;
}

// largest j in [0, n) with off[j] <= o (off ascending, off[0] = 0 <= o)
__device__ __forceinline__ int64_t find_segment(const int32_t* __restrict__ off, int64_t n, int64_t o) {
    int64_t lo = 0, hi = n;                 // off[lo] <= o < off[hi] (off[n] = total > o)
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (off[mid] <= o) lo = mid;
        else hi = mid;
    }
    return lo;
}

struct GatherWs {
    const int32_t* off_a;
    const int32_t* off_b;
    const int32_t* out_off;
    const int32_t* blk_seg;
};

// blk_seg[b] = the output image holding row b * TR_T (the first row of block b of k_gather_rows), for
// the blocks whose first row is below min(total, n_rows): one thread per output image writes the
// blocks that start inside its rows
__global__ void __launch_bounds__(TR_T) k_block_seg(const int32_t* __restrict__ out_off, int64_t n_out, int64_t n_rows,
                                                     int32_t* __restrict__ blk_seg) {
    const int64_t j = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (j >= n_out) return;
    const int64_t s = out_off[j], e = out_off[j + 1] < n_rows ? out_off[j + 1] : n_rows;
    for (int64_t b = (s + TR_T - 1) / TR_T; b * TR_T < e; ++b) blk_seg[b] = (int32_t)j;
}

// one thread per output row; C depth channels copied per row.  The row's image is found from its
// block's first image by stepping forward (a block of rows spans few images), not by a binary
// search of all the offsets: one dependent load instead of about log2(n_out).
__global__ void __launch_bounds__(TR_T) k_gather_rows(ba_gather_args a, GatherWs w) {
    const int64_t o = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (o >= a.n_rows || o >= w.out_off[a.n_out]) return;
    int64_t j = w.blk_seg[blockIdx.x];
    while (w.out_off[j + 1] <= o) ++j;
    int64_t k = o - w.out_off[j];
    const int32_t ia = a.sel_a ? a.sel_a[j] : -1;
    const int32_t na = (ia >= 0 && ia < a.a.n_imgs) ? a.a.nppi[ia] : 0;
    const bool from_a = k < na;                        // (k >= na only when image sel_b[j] of b is valid)
    const int64_t r = from_a ? w.off_a[ia] + k : w.off_b[a.sel_b[j]] + (k - na);
    const int32_t* pids = from_a ? a.a.pids : a.b.pids;
    const float* pix = from_a ? a.a.pix2d : a.b.pix2d;
    const float* sd = from_a ? a.a.pix2d_std : a.b.pix2d_std;
    const float* dep = from_a ? a.a.pix2d_dep : a.b.pix2d_dep;
    a.pids[o] = pids[r] + (from_a ? 0 : a.pid_shift_b);
    reinterpret_cast<float2*>(a.pix2d)[o] = reinterpret_cast<const float2*>(pix)[r];
    reinterpret_cast<float2*>(a.pix2d_std)[o] = reinterpret_cast<const float2*>(sd)[r];
    for (int c = 0; c < a.C; ++c) a.pix2d_dep[o * a.C + c] = dep[r * a.C + c];
}

__global__ void __launch_bounds__(TR_T) k_copy_counts(const int32_t* __restrict__ cnt, int64_t n, int32_t* __restrict__ nppi,
                                                       const int32_t* __restrict__ off, int64_t* __restrict__ total) {
    const int64_t j = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (j < n) nppi[j] = cnt[j];
    if (j == 0 && total) *total = off[n];
}

// ---- remove
__global__ void __launch_bounds__(TR_T) k_mark_bad(ba_remove_args a, int32_t* __restrict__ bad) {
    const int64_t i = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (i >= a.n_bad) return;
    const int64_t t = a.bad_int64 ? reinterpret_cast<const int64_t*>(a.bad)[i]
                                  : (int64_t) reinterpret_cast<const int32_t*>(a.bad)[i];
    if (t >= 0 && t < a.n_tracks) bad[t] = 1;            // ids that match no pid are ignored (torch.isin)
}

// keep[o] = pid not removed; present[pid] = 1 for every kept row (all writers store the same value)
__global__ void __launch_bounds__(TR_T) k_keep_rows(ba_remove_args a, const int32_t* __restrict__ bad,
                                                     int32_t* __restrict__ keep, int32_t* __restrict__ present,
                                                     int64_t n_rows) {
    const int64_t o = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (o >= n_rows) return;
    const int32_t p = a.in.pids[o];
    const bool ok = p >= 0 && p < a.n_tracks && !bad[p];
    keep[o] = ok;
    if (ok) present[p] = 1;
}

// old_to_keep[rank(t)] = t for every track with a kept row (rank = exclusive scan of the present
// flags, so track t is present exactly when rank[t + 1] > rank[t])
__global__ void __launch_bounds__(TR_T) k_old_to_keep(ba_remove_args a, const int32_t* __restrict__ rank) {
    const int64_t t = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (t == 0) a.counts[0] = rank[a.n_tracks];
    if (t >= a.n_tracks) return;
    if (rank[t + 1] > rank[t]) a.old_to_keep[rank[t]] = (int32_t)t;
}

__global__ void __launch_bounds__(TR_T) k_compact_rows(ba_remove_args a, const int32_t* __restrict__ keep,
                                                        const int32_t* __restrict__ pos, const int32_t* __restrict__ rank,
                                                        int64_t n_rows) {
    const int64_t o = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (o == 0) a.counts[1] = pos[n_rows];
    if (o >= n_rows || !keep[o]) return;
    const int64_t q = pos[o];
    a.pids[q] = rank[a.in.pids[o]];
    reinterpret_cast<float2*>(a.pix2d)[q] = reinterpret_cast<const float2*>(a.in.pix2d)[o];
    reinterpret_cast<float2*>(a.pix2d_std)[q] = reinterpret_cast<const float2*>(a.in.pix2d_std)[o];
    for (int c = 0; c < a.C; ++c) a.pix2d_dep[q * a.C + c] = a.in.pix2d_dep[o * a.C + c];
}

// rows kept in image i = pos[end_i] - pos[begin_i]
__global__ void __launch_bounds__(TR_T) k_kept_per_image(ba_remove_args a, const int32_t* __restrict__ off,
                                                          const int32_t* __restrict__ pos) {
    const int64_t i = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (i >= a.in.n_imgs) return;
    auto cl = [&](int32_t v) { return v < 0 ? (int64_t)0 : (v > a.n_rows ? a.n_rows : (int64_t)v); };
    a.nppi[i] = pos[cl(off[i + 1])] - pos[cl(off[i])];     // (clamped: nppi must sum to n_rows)
}

// ---- to_dense / img_id
__global__ void __launch_bounds__(TR_T) k_dense_scatter(const int32_t* __restrict__ pids, const float* __restrict__ pix2d,
                                                         const int32_t* __restrict__ off, int64_t n_imgs, int64_t n_rows,
                                                         int64_t n_tracks, float* __restrict__ out) {
    const int64_t o = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (o >= n_rows || o >= off[n_imgs]) return;
    const int64_t i = find_segment(off, n_imgs, o);
    const int32_t p = pids[o];
    if (p < 0 || p >= n_tracks) return;
    reinterpret_cast<float2*>(out)[i * n_tracks + p] = reinterpret_cast<const float2*>(pix2d)[o];
}

__global__ void __launch_bounds__(TR_T) k_mark_delims(const int32_t* __restrict__ off, int64_t n_imgs, int64_t n_rows,
                                                       int32_t* __restrict__ mark) {
    const int64_t i = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (i + 1 >= n_imgs) return;                       // delimiters cumsum(nppi)[:-1] = off[1..n_imgs-1]
    const int64_t c = off[i + 1];
    if (c >= 0 && c < n_rows) mark[c] = 1;
}

__global__ void __launch_bounds__(TR_T) k_incl_i64(const int32_t* __restrict__ excl, int64_t n, int64_t* __restrict__ out) {
    const int64_t o = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (o < n) out[o] = excl[o + 1];
}

}  // namespace ba

using namespace ba;

static inline unsigned grid_of(int64_t n) { return (unsigned)div_up(n > 0 ? n : 1, TR_T); }

// workspace carving: every piece 256-byte aligned
struct Carve {
    char* p;
    int64_t used = 0;
    template <typename T>
    T* take(int64_t n) {
        T* r = reinterpret_cast<T*>(p ? p + used : nullptr);
        used += align256((n > 0 ? n : 1) * (int64_t)sizeof(T));
        return r;
    }
};

// one layout serves every entry point: [bsum | i32 n_tracks+1 x2 | i32 n_rows+1 x2 | i32 n_imgs+1 x4]
static int64_t carve(void* ws, int64_t n_rows, int64_t n_tracks, int64_t n_imgs, int64_t** bsum, int32_t** t0,
                     int32_t** t1, int32_t** r0, int32_t** r1, int32_t** i0, int32_t** i1, int32_t** i2, int32_t** i3) {
    Carve c{(char*)ws};
    const int64_t nmax = n_rows > n_tracks ? (n_rows > n_imgs ? n_rows : n_imgs) : (n_tracks > n_imgs ? n_tracks : n_imgs);
    *bsum = c.take<int64_t>(scan_blocks(nmax) + 1);
    *t0 = c.take<int32_t>(n_tracks + 1);
    *t1 = c.take<int32_t>(n_tracks + 1);
    *r0 = c.take<int32_t>(n_rows + 1);
    *r1 = c.take<int32_t>(n_rows + 1);
    *i0 = c.take<int32_t>(n_imgs + 1);
    *i1 = c.take<int32_t>(n_imgs + 1);
    *i2 = c.take<int32_t>(n_imgs + 1);
    *i3 = c.take<int32_t>(n_imgs + 1);
    return c.used;
}

extern "C" int64_t ba_tracks_workspace_bytes(int64_t n_rows, int64_t n_tracks, int64_t n_imgs) {
    int64_t* b;
    int32_t *t0, *t1, *r0, *r1, *i0, *i1, *i2, *i3;
    return carve(nullptr, n_rows, n_tracks, n_imgs, &b, &t0, &t1, &r0, &r1, &i0, &i1, &i2, &i3);
}

static bool set_ok(const ba_obs_set& s, int32_t C) {
    return s.n_imgs == 0 || (s.nppi && s.pids && s.pix2d && s.pix2d_std && (C == 0 || s.pix2d_dep));
}

extern "C" int ba_tracks_gather(const ba_gather_args* args, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_gather_args& a = *args;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.n_out >= 0 && a.n_rows >= 0 && a.C >= 0 && a.a.n_imgs >= 0 && a.b.n_imgs >= 0, "bad sizes");
    BA_REQUIRE(a.n_rows < INT32_MAX && a.n_out < INT32_MAX, "too many rows or images (int32 offsets)");
    BA_REQUIRE(set_ok(a.a, a.C) && (a.sel_b == nullptr || set_ok(a.b, a.C)), "missing source arrays");
    BA_REQUIRE(a.sel_a != nullptr || a.sel_b != nullptr, "no source selected");
    BA_REQUIRE(a.nppi && (a.n_rows == 0 || (a.pids && a.pix2d && a.pix2d_std && (a.C == 0 || a.pix2d_dep))),
               "missing output arrays");
    BA_REQUIRE(a.workspace != nullptr, "workspace missing");
    const int64_t n_img_ws = a.a.n_imgs > a.b.n_imgs ? (a.a.n_imgs > a.n_out ? a.a.n_imgs : a.n_out)
                                                     : (a.b.n_imgs > a.n_out ? a.b.n_imgs : a.n_out);
    int64_t* bsum;
    int32_t *t0, *t1, *r0, *r1, *off_a, *off_b, *cnt, *out_off;
    carve(a.workspace, a.n_rows, 0, n_img_ws, &bsum, &t0, &t1, &r0, &r1, &off_a, &off_b, &cnt, &out_off);
    if (a.a.n_imgs > 0) scan_i32(a.a.nppi, a.a.n_imgs, off_a, bsum, st);
    if (a.sel_b && a.b.n_imgs > 0) scan_i32(a.b.nppi, a.b.n_imgs, off_b, bsum, st);
    if (a.n_out > 0) hipLaunchKernelGGL(k_gather_counts, dim3(grid_of(a.n_out)), dim3(TR_T), 0, st, a, cnt);
    scan_i32(cnt, a.n_out, out_off, bsum, st);
    hipLaunchKernelGGL(k_copy_counts, dim3(grid_of(a.n_out)), dim3(TR_T), 0, st, cnt, a.n_out, a.nppi, out_off, a.total);
    if (a.n_rows > 0 && a.n_out > 0) {
        // r0 (n_rows + 1 ints, unused by the gather) holds the per-block first image
        hipLaunchKernelGGL(k_block_seg, dim3(grid_of(a.n_out)), dim3(TR_T), 0, st, out_off, a.n_out, a.n_rows, r0);
        hipLaunchKernelGGL(k_gather_rows, dim3(grid_of(a.n_rows)), dim3(TR_T), 0, st, a,
                           GatherWs{off_a, off_b, out_off, r0});
    }
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int ba_tracks_remove(const ba_remove_args* args, void* stream) {
    clear_error();
    BA_REQUIRE(args != nullptr, "null args");
    const ba_remove_args& a = *args;
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(a.in.n_imgs >= 0 && a.n_tracks >= 0 && a.n_bad >= 0 && a.C >= 0 && a.n_rows >= 0, "bad sizes");
    BA_REQUIRE(a.n_rows < INT32_MAX && a.n_tracks < INT32_MAX, "too many rows or tracks (int32 offsets)");
    BA_REQUIRE(set_ok(a.in, a.C) && (a.n_bad == 0 || a.bad), "missing input arrays");
    BA_REQUIRE(a.nppi && a.old_to_keep && a.counts && a.workspace, "missing outputs or workspace");
    int64_t* bsum;
    int32_t *bad, *rank, *keep, *pos, *off, *i1, *i2, *i3;
    carve(a.workspace, a.n_rows, a.n_tracks, a.in.n_imgs, &bsum, &bad, &rank, &keep, &pos, &off, &i1, &i2, &i3);
    // removed-track flags; present-track flags (written into rank, then scanned in place)
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_of(a.n_tracks + 1)), dim3(TR_T), 0, st, bad, a.n_tracks + 1, 0);
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_of(a.n_tracks + 1)), dim3(TR_T), 0, st, rank, a.n_tracks + 1, 0);
    if (a.n_bad > 0) hipLaunchKernelGGL(k_mark_bad, dim3(grid_of(a.n_bad)), dim3(TR_T), 0, st, a, bad);
    if (a.n_rows > 0)
        hipLaunchKernelGGL(k_keep_rows, dim3(grid_of(a.n_rows)), dim3(TR_T), 0, st, a, bad, keep, rank, a.n_rows);
    scan_i32(rank, a.n_tracks, rank, bsum, st);
    hipLaunchKernelGGL(k_old_to_keep, dim3(grid_of(a.n_tracks + 1)), dim3(TR_T), 0, st, a, rank);
    scan_i32(keep, a.n_rows, pos, bsum, st);
    hipLaunchKernelGGL(k_compact_rows, dim3(grid_of(a.n_rows)), dim3(TR_T), 0, st, a, keep, pos, rank, a.n_rows);
    if (a.in.n_imgs > 0) {
        scan_i32(a.in.nppi, a.in.n_imgs, off, bsum, st);
        hipLaunchKernelGGL(k_kept_per_image, dim3(grid_of(a.in.n_imgs)), dim3(TR_T), 0, st, a, off, pos);
    }
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int ba_tracks_to_dense(const int32_t* pids, const float* pix2d, const int32_t* nppi, int64_t n_imgs,
                                  int64_t n_rows, int64_t n_tracks, int64_t n_imgs_out, float* out, void* workspace,
                                  void* stream) {
    clear_error();
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(n_imgs >= 0 && n_rows >= 0 && n_tracks >= 0 && n_imgs_out >= n_imgs, "bad sizes");
    BA_REQUIRE(n_rows < INT32_MAX, "too many rows (int32 offsets)");
    BA_REQUIRE(out != nullptr && workspace != nullptr && (n_imgs == 0 || nppi != nullptr), "missing arrays");
    int64_t* bsum;
    int32_t *t0, *t1, *r0, *r1, *off, *i1, *i2, *i3;
    carve(workspace, n_rows, 0, n_imgs, &bsum, &t0, &t1, &r0, &r1, &off, &i1, &i2, &i3);
    const int64_t n_out = n_imgs_out * n_tracks * 2;
    if (n_out > 0) hipLaunchKernelGGL(k_fill_f32, dim3(grid_of(n_out)), dim3(TR_T), 0, st, out, n_out, NAN);
    if (n_imgs > 0 && n_rows > 0 && n_tracks > 0) {
        scan_i32(nppi, n_imgs, off, bsum, st);
        hipLaunchKernelGGL(k_dense_scatter, dim3(grid_of(n_rows)), dim3(TR_T), 0, st, pids, pix2d, off, n_imgs, n_rows,
                           n_tracks, out);
    }
    BA_LAUNCHED();
    return BA_OK;
}

extern "C" int ba_tracks_img_id(const int32_t* nppi, int64_t n_imgs, int64_t n_rows, int64_t* out, void* workspace,
                                void* stream) {
    clear_error();
    hipStream_t st = (hipStream_t)stream;
    BA_REQUIRE(n_imgs >= 0 && n_rows >= 0 && n_rows < INT32_MAX, "bad sizes");
    BA_REQUIRE(workspace != nullptr && (n_rows == 0 || out != nullptr) && (n_imgs == 0 || nppi != nullptr),
               "missing arrays");
    if (n_rows == 0) return BA_OK;
    int64_t* bsum;
    int32_t *t0, *t1, *mark, *excl, *off, *i1, *i2, *i3;
    carve(workspace, n_rows, 0, n_imgs, &bsum, &t0, &t1, &mark, &excl, &off, &i1, &i2, &i3);
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_of(n_rows)), dim3(TR_T), 0, st, mark, n_rows, 0);
    if (n_imgs > 1) {
        scan_i32(nppi, n_imgs, off, bsum, st);
        hipLaunchKernelGGL(k_mark_delims, dim3(grid_of(n_imgs)), dim3(TR_T), 0, st, off, n_imgs, n_rows, mark);
    }
    scan_i32(mark, n_rows, excl, bsum, st);
    hipLaunchKernelGGL(k_incl_i64, dim3(grid_of(n_rows)), dim3(TR_T), 0, st, excl, n_rows, out);
    BA_LAUNCHED();
    return BA_OK;
}

// ------------------------------------------------------------------ structure plan after an append
// ids[q] += shift[img[q]] for q < n: the observation ids of a structure plan's chunk slots (chunk_obs, slot_src)
// after ba_plan_append inserted the new tracks' observations into the image blocks (img: each slot's image, 0 for
// an empty slot; shift[0] = 0, so an empty slot's -1 or 0 stays)
__global__ void __launch_bounds__(TR_T) k_plan_shift_ids(int32_t* __restrict__ ids, const int32_t* __restrict__ img,
                                                       const int32_t* __restrict__ shift, int64_t n) {
    const int64_t q = (int64_t)blockIdx.x * TR_T + threadIdx.x;
    if (q < n) ids[q] += shift[img[q]];
}

extern "C" int ba_plan_shift_ids(int32_t* ids, const int32_t* img, const int32_t* shift, int64_t n, void* stream) {
    clear_error();
    BA_REQUIRE(n >= 0 && (n == 0 || (ids != nullptr && img != nullptr && shift != nullptr)), "bad arguments");
    if (n > 0) hipLaunchKernelGGL(k_plan_shift_ids, dim3(grid_of(n)), dim3(TR_T), 0, (hipStream_t)stream, ids, img, shift, n);
    BA_LAUNCHED();
    return BA_OK;
}
