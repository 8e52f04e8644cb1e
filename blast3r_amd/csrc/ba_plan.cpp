// Host-side structure plan for the fused linearize + Schur kernels.
//
// Built once per observation structure (infos + pids), reused by every LM
// iteration: the reference re-derives the same structure with torch.unique on
// every iteration (src/blast3r/inference/ba_solver.py:877-909, :968-974).
//
// Layout produced here:
//   * tracks are ordered by (first image, last image, track id) and packed,
//     whole, into CHUNKs of BA_CHUNK observation slots (a track never straddles
//     a chunk; the unused tail slots hold -1);
//   * consecutive chunks form a BATCH whose tracks together touch at most
//     max_local_imgs images and at most max_slots image pairs; one workgroup
//     owns a batch and accumulates its camera-pair blocks on chip;
//   * every (batch, local pair) "slot" writes one partial block; a CSR maps each
//     global image pair (i1 <= i2) to its slots in batch order, so the final
//     reduction is a deterministic sum.
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include <sys/mman.h>

#include "ba_plan.h"
#include "ba_hip.h"

namespace ba {

// Allocator of the planner's large arrays: blocks of 2 MB and more are 2 MB aligned and advised onto
// transparent huge pages, since the page faults of first touch on fresh memory were a large share of a
// plan build (hundreds of MB of plan and planning state at 8 M observations).
template <class T>
struct HugeAlloc : std::allocator<T> {
    static constexpr size_t kHuge = (size_t)2 << 20;
    template <class U> struct rebind { using other = HugeAlloc<U>; };
    HugeAlloc() = default;
    template <class U> HugeAlloc(const HugeAlloc<U>&) noexcept {}
    T* allocate(size_t n) {
        const size_t bytes = n * sizeof(T);
        if (bytes < kHuge) return std::allocator<T>::allocate(n);
        const size_t sz = (bytes + kHuge - 1) / kHuge * kHuge;
        void* p = std::aligned_alloc(kHuge, sz);
        if (!p) throw std::bad_alloc();
        madvise(p, sz, MADV_HUGEPAGE);       // advice only: without huge pages the memory is the same
        return static_cast<T*>(p);
    }
    void deallocate(T* p, size_t n) {
        if (n * sizeof(T) < kHuge) std::allocator<T>::deallocate(p, n);
        else std::free(p);
    }
};
template <class T, class U> bool operator==(const HugeAlloc<T>&, const HugeAlloc<U>&) { return true; }
template <class T, class U> bool operator!=(const HugeAlloc<T>&, const HugeAlloc<U>&) { return false; }
template <class T> using HugeVec = std::vector<T, HugeAlloc<T>>;

// The same, with a construct without a value that leaves the element uninitialised, so that resize does
// not first zero-fill the plan arrays that emit then writes element by element (about 420 MB at
// 8 M observations).
template <class T>
struct NoInitAlloc : HugeAlloc<T> {
    template <class U> struct rebind { using other = NoInitAlloc<U>; };
    NoInitAlloc() = default;
    template <class U> NoInitAlloc(const NoInitAlloc<U>&) noexcept {}
    template <class U> void construct(U* p) noexcept { ::new ((void*)p) U; }
    template <class U, class... A> void construct(U* p, A&&... a) { ::new ((void*)p) U(std::forward<A>(a)...); }
};
typedef std::vector<int32_t, NoInitAlloc<int32_t>> PlanArray;

static std::string g_plan_err;

// a batch: a contiguous range of the track order, its images and its touched local pairs
struct BatchDesc {
    int32_t k0, k1;                    // range of `order`
    std::vector<int32_t> imgs;         // local image -> global image
    std::vector<uint32_t> rows;        // rows[a] bit b: local pair (a, b), a <= b, is touched
};

// What the planner keeps of a structure so that an appended one (old | new: per image, the old
// observations, then the new tracks' ones) is planned by redoing only the batches it changes.
// Observations are kept as (image, position in the image's block), which an append does not move.
struct PlanState {
    std::vector<int64_t> base;                 // n_imgs + 1: first observation of each image, then n_obs
    HugeVec<int64_t> tptr;                     // n_tracks + 1
    HugeVec<int32_t> tob_img, tob_pos;         // each track's observations, in observation order
    HugeVec<int32_t> tmin, tmax, tdist;        // per track: first and last image, distinct images
    HugeVec<int32_t> order;                    // observed tracks by (first image, last image, track id)
    HugeVec<int64_t> oimg_ptr;                 // per position of `order`: its distinct images in oimg
    HugeVec<int32_t> oimg;
    std::vector<BatchDesc> batches;
    std::vector<int64_t> o_ch, o_ct, o_sl, o_en;   // per batch (and one past the last): first chunk,
                                                   // chunk track, slot and MFMA entry
    int64_t ncov = 0;                          // sum over tracks of m (m + 1) / 2, m distinct images
};

struct Plan {
    int32_t n_imgs = 0, n_tracks = 0, L = 0, max_slots = 0;
    int64_t n_obs = 0, max_batch_obs = 0;
    PlanArray v[BA_PLAN_NARRAYS];             // every element is written by emit (resize leaves them unset)
    int64_t scalars[BA_PLAN_NSCALARS] = {0};
    PlanState st;
    // for a plan made by ba_plan_append: per array, the leading elements equal to the parent plan's (the
    // observation ids of chunk_obs / slot_src after adding shift[image]); per image, that shift
    int64_t stable[BA_PLAN_NARRAYS] = {0};
    std::vector<int32_t> shift;
};

// one batch's arrays, with chunk-track ids and entry offsets local to the batch
struct BatchOut {
    std::vector<int32_t> chunk_obs, slot_info, s_pid, s_img, chunk_meta, ct_pid, ct_first, ct_m, ct_mask, slot_pair,
        chunk_slots, chunk_eptr, pos_slot;
    std::vector<uint32_t> ents;
    bool overflow = false;
};

}  // namespace ba

using namespace ba;

// Runs fn(begin, end) over [0, n) on up to 16 host threads (contiguous ranges).
template <typename F>
static void parallel_for(int64_t n, F fn, int64_t min_per_thread = 65536) {
    unsigned nth = std::thread::hardware_concurrency();
    nth = std::max(1u, std::min(nth == 0 ? 1u : nth, 16u));
    nth = (unsigned)std::max<int64_t>(1, std::min<int64_t>(nth, n / std::max<int64_t>(1, min_per_thread)));
    if (nth <= 1) { fn((int64_t)0, n); return; }
    std::vector<std::thread> pool;
    const int64_t step = (n + nth - 1) / nth;
    for (unsigned w = 1; w < nth; ++w) {
        const int64_t b = w * step, e = std::min(n, b + step);
        if (b < e) pool.emplace_back(fn, b, e);
    }
    fn((int64_t)0, std::min(n, step));
    for (auto& th : pool) th.join();
}

static bool tracks_ok(const PlanState& S, int64_t t0, int64_t t1, int L) {
    int32_t worst_m = 0, worst_d = 0;
    for (int64_t t = t0; t < t1; ++t) {
        worst_m = std::max<int32_t>(worst_m, (int32_t)(S.tptr[t + 1] - S.tptr[t]));
        worst_d = std::max(worst_d, S.tdist[t]);
    }
    if (worst_m > BA_CHUNK) {
        g_plan_err = "a track has more observations than one chunk holds (" + std::to_string(BA_CHUNK) + ")";
        return false;
    }
    if (worst_d > L) {
        g_plan_err = "a track spans more images (" + std::to_string(worst_d) + ") than max_local_imgs (" +
                     std::to_string(L) + ")";
        return false;
    }
    return true;
}

// first / last / distinct images of tracks [t0, t1) from their observation lists
static void track_extent(PlanState& S, int64_t t0, int64_t t1) {
    parallel_for(t1 - t0, [&](int64_t a, int64_t b) {
        for (int64_t t = t0 + a; t < t0 + b; ++t) {
            int last = -1, mn = INT32_MAX, mx = -1, nd = 0;
            for (int64_t k = S.tptr[t]; k < S.tptr[t + 1]; ++k) {
                const int i = S.tob_img[k];
                if (i != last) { nd++; last = i; }
                mn = std::min(mn, i);
                mx = std::max(mx, i);
            }
            S.tmin[t] = mn; S.tmax[t] = mx; S.tdist[t] = nd;
        }
    });
}

// distinct image lists of the order positions [k_begin, end)
static void order_images(PlanState& S, int64_t k_begin) {
    const int64_t n = (int64_t)S.order.size();
    S.oimg_ptr.resize(n + 1);
    for (int64_t k = k_begin; k < n; ++k) S.oimg_ptr[k + 1] = S.oimg_ptr[k] + S.tdist[S.order[k]];
    S.oimg.resize(S.oimg_ptr[n]);
    parallel_for(n - k_begin, [&](int64_t a, int64_t b) {
        for (int64_t k = k_begin + a; k < k_begin + b; ++k) {
            const int t = S.order[k];
            int64_t q = S.oimg_ptr[k];
            int last = -1;
            for (int64_t j = S.tptr[t]; j < S.tptr[t + 1]; ++j) {
                const int i = S.tob_img[j];
                if (i != last) { S.oimg[q++] = i; last = i; }
            }
        }
    });
}

// The batch that opens at order position k: tracks are taken in order until the next one would exceed
// L images, max_slots pairs or max_batch_obs observations.  Returns the batch's end (> k) and fills
// *out, or -1 when the track at k alone needs more pair slots than max_slots.  limg_of (n_imgs, all -1)
// is returned all -1.
static int64_t one_batch(const PlanState& S, int64_t k, int L, int max_slots, int64_t max_batch_obs,
                         std::vector<int32_t>& limg_of, BatchDesc* out) {
    std::vector<int32_t> cur_imgs;
    std::vector<uint32_t> rows(L, 0);
    int cur_nslots = 0, n_cur = 0;
    int64_t cur_obs = 0, kk = k;
    const int64_t n = (int64_t)S.order.size();
    for (; kk < n; ++kk) {
        if (kk + 8 < n) __builtin_prefetch(&S.tptr[S.order[kk + 8]]);   // reached through the track id
        const int t = S.order[kk];
        const int32_t* timgs = S.oimg.data() + S.oimg_ptr[kk];
        const int nti = (int)(S.oimg_ptr[kk + 1] - S.oimg_ptr[kk]);
        const int m = (int)(S.tptr[t + 1] - S.tptr[t]);
        // local ids of the track's images (images not yet local get provisional ids)
        int prov = (int)cur_imgs.size();
        uint32_t M = 0;
        for (int q = 0; q < nti; ++q) {
            const int l = limg_of[timgs[q]];
            M |= 1u << (l >= 0 ? l : prov++);
        }
        bool ok = prov <= L && (max_batch_obs <= 0 || cur_obs + m <= max_batch_obs || n_cur == 0);
        int add_slots = 0;
        if (ok) {
            // local pairs (x <= y) within M that no earlier track of the batch touched
            for (uint32_t r = M; r; r &= r - 1) {
                const int x = __builtin_ctz(r);
                add_slots += __builtin_popcount(M & ~((1u << x) - 1u) & ~rows[x]);
            }
            ok = cur_nslots + add_slots <= max_slots;
        }
        if (!ok) break;
        for (int q = 0; q < nti; ++q)
            if (limg_of[timgs[q]] < 0) { limg_of[timgs[q]] = (int)cur_imgs.size(); cur_imgs.push_back(timgs[q]); }
        for (uint32_t r = M; r; r &= r - 1) {
            const int x = __builtin_ctz(r);
            rows[x] |= M & ~((1u << x) - 1u);
        }
        cur_nslots += add_slots;
        cur_obs += m;
        n_cur++;
    }
    for (int i : cur_imgs) limg_of[i] = -1;
    if (n_cur == 0) return -1;
    *out = BatchDesc{(int32_t)k, (int32_t)kk, std::move(cur_imgs), std::move(rows)};
    return kk;
}

// Greedy batching from order position k_begin (a batch opens there): each batch is the longest run of
// tracks, in order, that fits the limits (one_batch), and the next one opens where it ends.  Appends to
// S.batches.  A batch depends only on where it opens, so the order is cut into segments and, for each
// segment, threads run the greedy as if a batch opened at its start, and again from a few positions
// inside its first batch (a second run stops where it meets the first), until past the next segment's
// start.  The exact chain is then followed from k_begin: wherever it reaches a position at which one of
// its segment's runs opens a batch, it takes that run's batches from there on (they are the ones the
// chain would compute); elsewhere it computes its batches itself.  The result does not depend on the
// segmentation.  Several start positions matter where batches advance in a period: on config 2 each
// batch takes the rest of one first image, the next image and part of the one after, so a run started
// one image off the chain's phase never meets it.
static bool greedy(PlanState& S, int64_t k_begin, int n_imgs, int L, int max_slots, int64_t max_batch_obs) {
    struct Run {
        std::vector<BatchDesc> b;       // b[j] opens at b[j].k0; the run stops at the end of the last one
        bool fail = false;              // the run stopped at a track that alone exceeds max_slots (at its end)
    };
    constexpr int kRuns = 4;            // runs per segment
    const int64_t n = (int64_t)S.order.size();
    const int64_t span = n - k_begin;
    unsigned hw = std::thread::hardware_concurrency();
    const int64_t nth = std::max(1u, std::min(hw == 0 ? 1u : hw, 16u));
    const int64_t nseg = std::max<int64_t>(1, std::min<int64_t>(nth, span / 32768));
    std::vector<int64_t> seg(nseg + 1);
    for (int64_t w = 0; w <= nseg; ++w) seg[w] = k_begin + span * w / nseg;
    std::vector<Run> runs(nseg * kRuns);
    // run r of segment w: r = 0 from the segment's start; r > 0 from r / kRuns of the way into run 0's
    // first batch, until it opens a batch where run 0 does (from there on it is run 0)
    auto one_run = [&](int64_t w, int r, std::vector<int32_t>& limg_of) {
        Run& R = runs[w * kRuns + r];
        const Run& R0 = runs[w * kRuns];
        int64_t p = seg[w];
        if (r > 0) {
            if (R0.b.empty() || R0.fail) return;
            p += (R0.b[0].k1 - R0.b[0].k0) * r / kRuns;
            if (p == seg[w]) return;
        }
        size_t j0 = 0;                                      // run 0's batches opening before p
        while (p < seg[w + 1]) {                            // seg[nseg] = n
            if (r > 0) {
                while (j0 < R0.b.size() && R0.b[j0].k0 < p) ++j0;
                if (j0 < R0.b.size() && R0.b[j0].k0 == p) return;   // met run 0
            }
            BatchDesc bd;
            const int64_t e = one_batch(S, p, L, max_slots, max_batch_obs, limg_of, &bd);
            if (e < 0) { R.fail = true; R.b.push_back(BatchDesc{(int32_t)p, (int32_t)p, {}, {}}); return; }
            R.b.push_back(std::move(bd));
            p = e;
        }
    };
    if (nseg > 1) {
        std::vector<std::thread> pool;
        auto seg_runs = [&](int64_t w) {
            std::vector<int32_t> limg_of(n_imgs, -1);
            for (int r = 0; r < kRuns; ++r) one_run(w, r, limg_of);
        };
        for (int64_t w = 1; w < nseg; ++w) pool.emplace_back(seg_runs, w);
        seg_runs(0);
        for (auto& th : pool) th.join();
    }
    std::vector<int32_t> limg_of(n_imgs, -1);
    int64_t p = k_begin;
    int64_t w = 0;
    while (p < n) {
        while (w + 1 < nseg && seg[w + 1] <= p) ++w;
        // does one of segment w's runs open a batch at p?
        bool taken = false;
        for (int r = 0; r < kRuns && nseg > 1 && !taken; ++r) {
            std::vector<BatchDesc>& rb = runs[w * kRuns + r].b;
            auto it = std::lower_bound(rb.begin(), rb.end(), p, [](const BatchDesc& x, int64_t v) { return x.k0 < v; });
            if (it == rb.end() || it->k0 != p) continue;
            const bool fail = runs[w * kRuns + r].fail;
            const auto stop = fail ? rb.end() - 1 : rb.end();
            for (auto jt = it; jt != stop; ++jt) { p = jt->k1; S.batches.push_back(std::move(*jt)); }
            if (fail) {                // the chain has reached the track the run stopped at
                g_plan_err = "a single track needs more pair slots than max_slots";
                return false;
            }
            taken = true;
        }
        if (taken) continue;
        BatchDesc bd;
        const int64_t e = one_batch(S, p, L, max_slots, max_batch_obs, limg_of, &bd);
        if (e < 0) {
            g_plan_err = "a single track needs more pair slots than max_slots";
            return false;
        }
        S.batches.push_back(std::move(bd));
        p = e;
    }
    return true;
}

// One batch's chunks, MFMA entry lists and wave placement (chunk-track ids and entry offsets local to it).
static void build_batch(const PlanState& S, int batch, std::vector<int32_t>& limg_of, BatchOut& R) {
    const BatchDesc& bd = S.batches[batch];
    for (int a = 0; a < (int)bd.imgs.size(); ++a) limg_of[bd.imgs[a]] = a;
    // local pair slots in (b, a) order
    for (int b = 0; b < (int)bd.imgs.size(); ++b)
        for (int a = 0; a <= b; ++a)
            if ((bd.rows[a] >> b) & 1u) R.slot_pair.push_back(a | (b << 8));
    const int nsl = (int)R.slot_pair.size();
    int k = bd.k0;
    while (k < bd.k1) {                                   // chunks: tracks packed whole, in order
        int used = 0, ntr = 0;
        const size_t base = R.chunk_obs.size();
        R.chunk_obs.resize(base + BA_CHUNK, -1);
        R.slot_info.resize(base + BA_CHUNK, -1);
        R.s_pid.resize(base + BA_CHUNK, 0);
        R.s_img.resize(base + BA_CHUNK, 0);
        const int first_ct = (int)R.ct_pid.size();
        int16_t lead[BA_MAX_CT][BA_MAX_LOCAL];            // per chunk track and local image: its run's first slot
        uint64_t img_trk[BA_MAX_LOCAL] = {0};             // per local image: the chunk tracks seen in it
        while (k < bd.k1) {
            // the track lists are reached through the track id: request them a few tracks ahead
            if (k + 8 < bd.k1) __builtin_prefetch(&S.tptr[S.order[k + 8]]);
            if (k + 4 < bd.k1) {
                const int64_t q = S.tptr[S.order[k + 4]];
                __builtin_prefetch(&S.tob_img[q]);
                __builtin_prefetch(&S.tob_pos[q]);
            }
            const int t = S.order[k];
            const int m = (int)(S.tptr[t + 1] - S.tptr[t]);
            if (used + m > BA_CHUNK || ntr == BA_MAX_CT) break;
            uint32_t mask = 0;
            int last_img = -1, leader = -1;
            for (int j = 0; j < m; ++j) {
                const int i = S.tob_img[S.tptr[t] + j];
                const int lim = limg_of[i];
                if (i != last_img) {
                    leader = used + j;
                    last_img = i;
                    lead[ntr][lim] = (int16_t)leader;
                }
                mask |= 1u << lim;
                R.chunk_obs[base + used + j] = (int32_t)(S.base[i] + S.tob_pos[S.tptr[t] + j]);
                R.slot_info[base + used + j] = lim | (ntr << 8) | (leader << 16);
                R.s_pid[base + used + j] = t;
                R.s_img[base + used + j] = i;
            }
            for (uint32_t r = mask; r; r &= r - 1) img_trk[__builtin_ctz(r)] |= (uint64_t)1 << ntr;
            R.ct_pid.push_back(t);
            R.ct_first.push_back(used);
            R.ct_m.push_back(m);
            R.ct_mask.push_back((int32_t)mask);
            used += m;
            ntr++;
            k++;
        }
        R.chunk_meta.push_back(batch);
        R.chunk_meta.push_back(first_ct);
        R.chunk_meta.push_back(ntr);
        R.chunk_meta.push_back(used);

        // MFMA entry lists of the chunk, slot by slot: an off-diagonal slot (a, b) pairs the
        // first observation of each covering track in a with the one in b (chunk-track order);
        // a diagonal slot (a, a) lists the J rows of every observation in a (slot order, padded
        // to whole groups), then the V rows of the first observation of each (track, image) run
        // in a (slot order)
        int16_t by_img[BA_CHUNK];                          // the chunk's slots grouped by local image
        int img_ptr[BA_MAX_LOCAL + 1] = {0};
        for (int sidx = 0; sidx < used; ++sidx) img_ptr[(R.slot_info[base + sidx] & 0xff) + 1]++;
        for (int a = 0; a < BA_MAX_LOCAL; ++a) img_ptr[a + 1] += img_ptr[a];
        {
            int fill[BA_MAX_LOCAL];
            std::copy(img_ptr, img_ptr + BA_MAX_LOCAL, fill);
            for (int sidx = 0; sidx < used; ++sidx) by_img[fill[R.slot_info[base + sidx] & 0xff]++] = (int16_t)sidx;
        }
        const size_t e0 = R.ents.size();
        R.chunk_eptr.push_back((int32_t)(e0 / 4));
        auto ent = [&](int oa, int ob) { R.ents.push_back((uint32_t)oa | ((uint32_t)ob << 16)); };
        auto pad = [&](size_t from) { while ((R.ents.size() - from) % 4) ent(BA_ZERO, BA_ZERO); };
        for (int q = 0; q < BA_MAX_SLOTS; ++q) {
            if (q >= nsl) { R.chunk_slots.push_back(0); continue; }
            const int a = R.slot_pair[q] & 0xff, bq = (R.slot_pair[q] >> 8) & 0xff;
            const size_t off = R.ents.size() - e0;
            int njg = 0;
            if (a != bq) {
                for (uint64_t r = img_trk[a] & img_trk[bq]; r; r &= r - 1) {
                    const int tt = __builtin_ctzll(r);
                    ent(lead[tt][a] * BA_BLK, lead[tt][bq] * BA_BLK);
                }
            } else {
                for (int x = img_ptr[a]; x < img_ptr[a + 1]; ++x) ent(by_img[x] * BA_BLK + BA_JROW, by_img[x] * BA_BLK + BA_JROW);
                pad(e0 + off);
                njg = (int)((R.ents.size() - e0 - off) / 4);
                for (int x = img_ptr[a]; x < img_ptr[a + 1]; ++x) {
                    const int sidx = by_img[x];
                    if ((R.slot_info[base + sidx] >> 16) == sidx) ent(sidx * BA_BLK, sidx * BA_BLK);
                }
            }
            pad(e0 + off);
            const size_t len = R.ents.size() - e0 - off;
            R.chunk_slots.push_back(BA_TAB(off, len / 4, njg));
        }
        if (R.ents.size() - e0 > BA_LIST_CAP) R.overflow = true;
        while ((R.ents.size() - e0) % 4) R.ents.push_back(0);
    }
    // place the batch's slots on the Schur kernel's waves (place wave + BA_WAVES * k, at most
    // BA_SLOTS_PER_WAVE per wave).  The MFMA phase of a chunk lasts as long as its busiest SIMD
    // (BA_WAVES / 4 waves share one MFMA pipe) and its busiest wave, so slots are taken by
    // decreasing total work and each goes where the summed per-chunk maxima grow least.  A chunk in
    // which the slot has no entries adds the same to every wave's cost (each maximum stays), so only
    // the chunks where it has entries are summed.
    {
        const int nc = (int)(R.chunk_meta.size() / 4);
        std::vector<int32_t> sptr(nsl + 1, 0), sc, sx;   // per slot: its chunks with entries, and their MFMAs
        std::vector<int64_t> tot(nsl, 0);
        for (int c = 0; c < nc; ++c)
            for (int q = 0; q < nsl; ++q)
                if (BA_TAB_NG(R.chunk_slots[(size_t)c * BA_MAX_SLOTS + q]) > 0) sptr[q + 1]++;
        for (int q = 0; q < nsl; ++q) sptr[q + 1] += sptr[q];
        sc.resize(sptr[nsl]);
        sx.resize(sptr[nsl]);
        {
            std::vector<int32_t> fill(sptr.begin(), sptr.end() - 1);
            for (int c = 0; c < nc; ++c)
                for (int q = 0; q < nsl; ++q) {
                    const int x = 3 * BA_TAB_NG(R.chunk_slots[(size_t)c * BA_MAX_SLOTS + q]);
                    if (x > 0) { sc[fill[q]] = c; sx[fill[q]++] = x; tot[q] += x; }
                }
        }
        std::vector<int> sorder(nsl);
        std::iota(sorder.begin(), sorder.end(), 0);
        std::stable_sort(sorder.begin(), sorder.end(), [&](int x, int y) { return tot[x] > tot[y]; });
        constexpr int NS = 4;
        std::vector<int64_t> ls((size_t)nc * NS, 0), lw((size_t)nc * BA_WAVES, 0), ms(nc, 0), mw(nc, 0);
        int cnt[BA_WAVES] = {0};
        R.pos_slot.assign(BA_MAX_SLOTS, -1);
        for (int q : sorder) {
            int64_t simd_cost[NS];
            for (int sd = 0; sd < NS; ++sd) {
                int64_t cost = 0;
                for (int e = sptr[q]; e < sptr[q + 1]; ++e) {
                    const int c = sc[e];
                    cost += NS * std::max(ls[(size_t)c * NS + sd] + sx[e], ms[c]);
                }
                simd_cost[sd] = cost;
            }
            int best = -1;
            int64_t best_cost = 0;
            for (int w = 0; w < BA_WAVES; ++w) {
                if (cnt[w] >= BA_SLOTS_PER_WAVE) continue;
                int64_t cost = simd_cost[w % NS];
                for (int e = sptr[q]; e < sptr[q + 1]; ++e) {
                    const int c = sc[e];
                    cost += std::max(lw[(size_t)c * BA_WAVES + w] + sx[e], mw[c]);
                }
                if (best < 0 || cost < best_cost) { best = w; best_cost = cost; }
            }
            R.pos_slot[best + BA_WAVES * cnt[best]] = q;
            cnt[best]++;
            const int sd = best % NS;
            for (int e = sptr[q]; e < sptr[q + 1]; ++e) {
                const int c = sc[e];
                ls[(size_t)c * NS + sd] += sx[e];
                lw[(size_t)c * BA_WAVES + best] += sx[e];
                ms[c] = std::max(ms[c], ls[(size_t)c * NS + sd]);
                mw[c] = std::max(mw[c], lw[(size_t)c * BA_WAVES + best]);
            }
        }
    }
    for (int i : bd.imgs) limg_of[i] = -1;
}

// Batches [b0, n_batches): their arrays (built in parallel) replace whatever the plan's batch-ordered arrays
// hold from batch b0 on; then the arrays that depend on every batch (dispatch order, global pairs, image rows,
// per-image partial sources) and the scalars.
static bool emit(Plan* P, int b0) {
    PlanState& S = P->st;
    const int n_batches = (int)S.batches.size(), L = P->L, n_imgs = P->n_imgs;
    std::vector<BatchOut> outs(n_batches - b0);
    {
        unsigned nth = std::thread::hardware_concurrency();
        nth = std::max(1u, std::min(nth == 0 ? 1u : nth, 16u));
        nth = (unsigned)std::min<int64_t>(nth, std::max(1, n_batches - b0));
        std::atomic<int> next(b0);
        auto work = [&]() {
            std::vector<int32_t> limg_of(n_imgs, -1);
            for (int b = next++; b < n_batches; b = next++) build_batch(S, b, limg_of, outs[b - b0]);
        };
        std::vector<std::thread> pool;
        for (unsigned w = 1; w < nth; ++w) pool.emplace_back(work);
        work();
        for (auto& th : pool) th.join();
    }
    auto& chunk_obs = P->v[BA_PA_CHUNK_OBS];      // n_chunks * BA_CHUNK obs index or -1
    auto& chunk_meta = P->v[BA_PA_CHUNK_META];    // n_chunks * 4: batch, first ctrack, n ctracks, n slots used
    auto& slot_info = P->v[BA_PA_SLOT_INFO];      // n_chunks * BA_CHUNK: local img | ctrack<<8 | leader_slot<<16 (-1 pad)
    auto& ct_pid = P->v[BA_PA_CT_PID];            // per chunk-track: track id
    auto& ct_first = P->v[BA_PA_CT_FIRST];        // first slot inside the chunk
    auto& ct_m = P->v[BA_PA_CT_M];                // number of observations
    auto& ct_mask = P->v[BA_PA_CT_MASK];          // local-image bit mask
    auto& b_chunk_ptr = P->v[BA_PA_B_CHUNK_PTR];  // n_batches + 1
    auto& b_imgs = P->v[BA_PA_B_IMGS];            // n_batches * L global image ids (-1 pad)
    auto& b_nimgs = P->v[BA_PA_B_NIMGS];          // n_batches
    auto& b_slot_ptr = P->v[BA_PA_B_SLOT_PTR];    // n_batches + 1
    auto& slot_pair = P->v[BA_PA_SLOT_PAIR];      // per slot: a | b << 8  (a <= b local)
    auto& slot_gpair = P->v[BA_PA_SLOT_GPAIR];    // per slot: global pair id
    auto& chunk_slots = P->v[BA_PA_CHUNK_SLOTS];  // n_chunks * BA_MAX_SLOTS
    auto& chunk_ent = P->v[BA_PA_CHUNK_ENT];      // 32-bit entries
    auto& chunk_eptr = P->v[BA_PA_CHUNK_EPTR];    // n_chunks + 1
    auto& b_pos_slot = P->v[BA_PA_B_POS_SLOT];    // n_batches * BA_MAX_SLOTS
    auto& slot_src = P->v[BA_PA_SLOT_SRC];
    auto& s_pid = P->v[BA_PA_S_PID];
    auto& s_img = P->v[BA_PA_S_IMG];
    bool list_overflow = false;
    // offsets of each batch in the concatenated arrays, then a parallel copy
    S.o_ch.resize(n_batches + 1); S.o_ct.resize(n_batches + 1); S.o_sl.resize(n_batches + 1); S.o_en.resize(n_batches + 1);
    if (b0 == 0) { S.o_ch[0] = S.o_ct[0] = S.o_sl[0] = S.o_en[0] = 0; }
    for (int b = b0; b < n_batches; ++b) {
        const BatchOut& R = outs[b - b0];
        S.o_ch[b + 1] = S.o_ch[b] + (int64_t)R.chunk_meta.size() / 4;
        S.o_ct[b + 1] = S.o_ct[b] + (int64_t)R.ct_pid.size();
        S.o_sl[b + 1] = S.o_sl[b] + (int64_t)R.slot_pair.size();
        S.o_en[b + 1] = S.o_en[b] + (int64_t)R.ents.size();
        list_overflow |= R.overflow;
    }
    if (list_overflow) {
        g_plan_err = "a chunk needs more than BA_LIST_CAP MFMA entries";
        return false;
    }
    const auto& o_ch = S.o_ch;
    const auto& o_ct = S.o_ct;
    const auto& o_sl = S.o_sl;
    const auto& o_en = S.o_en;
    const int64_t nch = o_ch[n_batches];
    if (b0 == 0) {
        // room for appended structures (ba_plan_append grows these arrays in place)
        auto room = [](PlanArray& v, int64_t n) { v.reserve((size_t)(n + n / 8 + 4096)); };
        for (auto* v : {&chunk_obs, &slot_info, &slot_src, &s_pid, &s_img}) room(*v, nch * BA_CHUNK);
        room(chunk_meta, nch * 4); room(chunk_slots, nch * BA_MAX_SLOTS); room(chunk_eptr, nch + 1);
        room(chunk_ent, o_en[n_batches] + BA_LIST_CAP);
        for (auto* v : {&ct_pid, &ct_first, &ct_m, &ct_mask}) room(*v, o_ct[n_batches]);
    }
    for (auto* v : {&chunk_obs, &slot_info, &slot_src, &s_pid, &s_img}) v->resize(nch * BA_CHUNK);
    chunk_meta.resize(nch * 4); chunk_slots.resize(nch * BA_MAX_SLOTS);
    chunk_eptr.resize(nch + 1);
    chunk_eptr[nch] = (int32_t)(o_en[n_batches] / 4);
    for (auto* v : {&ct_pid, &ct_first, &ct_m, &ct_mask}) v->resize(o_ct[n_batches]);
    slot_pair.resize(o_sl[n_batches]);
    // the entries, and one chunk's worth of zero padding so that a full-capacity copy of the last
    // chunk's list stays inside the array
    chunk_ent.resize((size_t)o_en[b0]);
    chunk_ent.resize((size_t)(o_en[n_batches] + BA_LIST_CAP), 0);
    uint32_t* ents = reinterpret_cast<uint32_t*>(chunk_ent.data());
    b_pos_slot.resize((size_t)n_batches * BA_MAX_SLOTS);
    parallel_for(n_batches - b0, [&](int64_t q0, int64_t q1) {
        for (int64_t b = b0 + q0; b < b0 + q1; ++b) {
            BatchOut& R = outs[b - b0];
            const int32_t ct0 = (int32_t)o_ct[b], e4 = (int32_t)(o_en[b] / 4);
            const size_t c0 = (size_t)o_ch[b] * BA_CHUNK;
            std::copy(R.chunk_obs.begin(), R.chunk_obs.end(), chunk_obs.begin() + c0);
            for (size_t q = 0; q < R.chunk_obs.size(); ++q) slot_src[c0 + q] = R.chunk_obs[q] >= 0 ? R.chunk_obs[q] : 0;
            std::copy(R.s_pid.begin(), R.s_pid.end(), s_pid.begin() + c0);
            std::copy(R.s_img.begin(), R.s_img.end(), s_img.begin() + c0);
            std::copy(R.slot_info.begin(), R.slot_info.end(), slot_info.begin() + c0);
            for (size_t c = 0; c < R.chunk_meta.size(); c += 4) {
                int32_t* d = chunk_meta.data() + o_ch[b] * 4 + c;
                d[0] = R.chunk_meta[c]; d[1] = R.chunk_meta[c + 1] + ct0; d[2] = R.chunk_meta[c + 2]; d[3] = R.chunk_meta[c + 3];
            }
            std::copy(R.ct_pid.begin(), R.ct_pid.end(), ct_pid.begin() + o_ct[b]);
            std::copy(R.ct_first.begin(), R.ct_first.end(), ct_first.begin() + o_ct[b]);
            std::copy(R.ct_m.begin(), R.ct_m.end(), ct_m.begin() + o_ct[b]);
            std::copy(R.ct_mask.begin(), R.ct_mask.end(), ct_mask.begin() + o_ct[b]);
            std::copy(R.slot_pair.begin(), R.slot_pair.end(), slot_pair.begin() + o_sl[b]);
            std::copy(R.chunk_slots.begin(), R.chunk_slots.end(), chunk_slots.begin() + o_ch[b] * BA_MAX_SLOTS);
            for (size_t c = 0; c < R.chunk_eptr.size(); ++c) chunk_eptr[o_ch[b] + c] = R.chunk_eptr[c] + e4;
            std::copy(R.ents.begin(), R.ents.end(), ents + o_en[b]);
            std::copy(R.pos_slot.begin(), R.pos_slot.end(), b_pos_slot.begin() + b * BA_MAX_SLOTS);
            R = BatchOut();                                    // release as we go
        }
    }, 1);
    b_chunk_ptr.resize(b0); b_slot_ptr.resize(b0);
    for (int b = b0; b <= n_batches; ++b) {
        b_chunk_ptr.push_back((int32_t)o_ch[b]);
        b_slot_ptr.push_back((int32_t)o_sl[b]);
    }
    b_imgs.resize((size_t)b0 * L); b_nimgs.resize(b0);
    for (int b = b0; b < n_batches; ++b) {
        for (int a = 0; a < L; ++a)
            b_imgs.push_back(a < (int)S.batches[b].imgs.size() ? S.batches[b].imgs[a] : -1);
        b_nimgs.push_back((int32_t)S.batches[b].imgs.size());
    }
    // Dispatch order of the Schur kernel's workgroups (one batch per CU at a time): most expensive
    // first, so that the last ones to start are short (longest-processing-time-first list
    // scheduling).  In plan order the busiest CU gets ~1.3x the mean load at config 2, since batch
    // sizes range from 118 to 205 chunks.  Cost estimate from the measured per-chunk phases:
    // ~5.3k cycles of operand formation per chunk, ~19 cycles of MFMA phase per list entry.
    {
        auto& b_order = P->v[BA_PA_B_ORDER];
        std::vector<int64_t> cost(n_batches);
        for (int b = 0; b < n_batches; ++b) cost[b] = 5300 * (o_ch[b + 1] - o_ch[b]) + 19 * (o_en[b + 1] - o_en[b]);
        b_order.resize(n_batches);
        std::iota(b_order.begin(), b_order.end(), 0);
        std::stable_sort(b_order.begin(), b_order.end(), [&](int32_t x, int32_t y) { return cost[x] > cost[y]; });
    }

    // ------------------------------------------------------------ global pairs
    int64_t n_slots = (int64_t)slot_pair.size();
    std::vector<int64_t> keys(n_slots);
    std::vector<uint8_t> swapped(n_slots, 0);
    for (int b = 0; b < n_batches; ++b)
        for (int s = b_slot_ptr[b]; s < b_slot_ptr[b + 1]; ++s) {
            int a = slot_pair[s] & 0xff, c = (slot_pair[s] >> 8) & 0xff;
            int64_t i1 = b_imgs[(int64_t)b * L + a], i2 = b_imgs[(int64_t)b * L + c];
            if (i1 > i2) { std::swap(i1, i2); swapped[s] = 1; }
            keys[s] = i1 * n_imgs + i2;
        }
    // slots by key (i1, i2), stable: counting sorts by i2, then by i1
    std::vector<int64_t> perm(n_slots);
    {
        std::vector<int64_t> tmp(n_slots), cnt(n_imgs + 1);
        std::fill(cnt.begin(), cnt.end(), 0);
        for (int64_t q = 0; q < n_slots; ++q) cnt[keys[q] % n_imgs + 1]++;
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        for (int64_t q = 0; q < n_slots; ++q) tmp[cnt[keys[q] % n_imgs]++] = q;
        std::fill(cnt.begin(), cnt.end(), 0);
        for (int64_t q = 0; q < n_slots; ++q) cnt[keys[q] / n_imgs + 1]++;
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        for (int64_t q : tmp) perm[cnt[keys[q] / n_imgs]++] = q;
    }
    auto& pair_i1 = P->v[BA_PA_PAIR_I1];
    auto& pair_i2 = P->v[BA_PA_PAIR_I2];
    auto& pair_ptr = P->v[BA_PA_PAIR_PTR];
    auto& pair_src = P->v[BA_PA_PAIR_SRC];
    pair_i1.clear(); pair_i2.clear(); pair_ptr.clear(); pair_src.clear();
    slot_gpair.assign(n_slots, -1);
    pair_ptr.push_back(0);
    for (int64_t q = 0; q < n_slots; ++q) {
        int64_t s = perm[q];
        if (q == 0 || keys[s] != keys[perm[q - 1]]) {
            if (q) pair_ptr.push_back((int32_t)q);
            pair_i1.push_back((int32_t)(keys[s] / n_imgs));
            pair_i2.push_back((int32_t)(keys[s] % n_imgs));
        }
        slot_gpair[s] = (int32_t)pair_i1.size() - 1;
        // the slot block is S[img(a), img(b)]; flag 1 = stored transposed w.r.t. (i1 <= i2)
        pair_src.push_back((int32_t)((s << 1) | swapped[s]));
    }
    pair_ptr.push_back((int32_t)n_slots);
    int n_pairs = (int)pair_i1.size();

    // image rows of the symmetric pair structure (for block SpMV): for image i, entries
    // (pair id, transposed flag) for every pair with i as row (i1 == i) or as column (i2 == i, i1 != i).
    auto& row_ptr = P->v[BA_PA_ROW_PTR];
    auto& row_ent = P->v[BA_PA_ROW_ENT];
    {
        std::vector<int32_t> cnt(n_imgs + 1, 0);
        for (int p = 0; p < n_pairs; ++p) {
            cnt[pair_i1[p] + 1]++;
            if (pair_i2[p] != pair_i1[p]) cnt[pair_i2[p] + 1]++;
        }
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        row_ptr.assign(cnt.begin(), cnt.end());
        row_ent.assign(cnt[n_imgs], 0);
        std::vector<int32_t> fill(cnt.begin(), cnt.end() - 1);
        for (int p = 0; p < n_pairs; ++p) {
            row_ent[fill[pair_i1[p]]++] = p << 1;
            if (pair_i2[p] != pair_i1[p]) row_ent[fill[pair_i2[p]]++] = (p << 1) | 1;
        }
    }
    // per-image partial sources: (batch * L + local image), in batch order
    auto& img_ptr = P->v[BA_PA_IMG_PTR];
    auto& img_src = P->v[BA_PA_IMG_SRC];
    {
        std::vector<int32_t> cnt(n_imgs + 1, 0);
        for (int b = 0; b < n_batches; ++b)
            for (int a = 0; a < b_nimgs[b]; ++a) cnt[b_imgs[(int64_t)b * L + a] + 1]++;
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        img_ptr.assign(cnt.begin(), cnt.end());
        img_src.assign(cnt[n_imgs], 0);
        std::vector<int32_t> fill(cnt.begin(), cnt.end() - 1);
        for (int b = 0; b < n_batches; ++b)
            for (int a = 0; a < b_nimgs[b]; ++a)
                img_src[fill[b_imgs[(int64_t)b * L + a]]++] = b * L + a;
    }

    int64_t max_slots_used = 0, max_chunks = 0;
    for (int b = 0; b < n_batches; ++b) {
        max_slots_used = std::max<int64_t>(max_slots_used, b_slot_ptr[b + 1] - b_slot_ptr[b]);
        max_chunks = std::max<int64_t>(max_chunks, b_chunk_ptr[b + 1] - b_chunk_ptr[b]);
    }
    P->scalars[BA_PS_N_CHUNKS] = nch;
    P->scalars[BA_PS_N_BATCHES] = n_batches;
    P->scalars[BA_PS_N_SLOTS] = n_slots;
    P->scalars[BA_PS_N_PAIRS] = n_pairs;
    P->scalars[BA_PS_N_CTRACKS] = (int64_t)ct_pid.size();
    P->scalars[BA_PS_L] = L;
    P->scalars[BA_PS_CHUNK] = BA_CHUNK;
    P->scalars[BA_PS_MAX_SLOTS_USED] = max_slots_used;
    P->scalars[BA_PS_MAX_CHUNKS_PER_BATCH] = max_chunks;
    P->scalars[BA_PS_N_PAIR_TERMS] = S.ncov;
    return true;
}

extern "C" const char* ba_plan_last_error(void) { return g_plan_err.c_str(); }
extern "C" int64_t ba_abi_sizeof(const char* name) {
    if (!name) return -1;
    const std::string n(name);
#define BA_SZ(T) if (n == #T) return (int64_t)sizeof(T)
    BA_SZ(ba_huber); BA_SZ(ba_layout); BA_SZ(ba_lin_args); BA_SZ(ba_pm_args); BA_SZ(ba_pcg_args);
    BA_SZ(ba_chol_args); BA_SZ(ba_sample_args); BA_SZ(ba_obs_set); BA_SZ(ba_gather_args); BA_SZ(ba_remove_args);
    BA_SZ(ba_tangent_args);
#undef BA_SZ
    return -1;
}

extern "C" void* ba_plan_create(const int32_t* cum_nkpts, int32_t n_imgs, const int32_t* pids, int64_t n_obs,
                                int32_t n_tracks, int32_t max_local_imgs, int32_t max_slots, int64_t max_batch_obs) {
    g_plan_err.clear();
    if (n_imgs <= 0 || n_obs < 0 || n_tracks < 0) { g_plan_err = "bad sizes"; return nullptr; }
    if (max_local_imgs < 1 || max_local_imgs > BA_MAX_LOCAL) { g_plan_err = "max_local_imgs out of range"; return nullptr; }
    if (max_slots < 1 || max_slots > BA_MAX_SLOTS) {
        g_plan_err = "max_slots must be in [1, " + std::to_string(BA_MAX_SLOTS) + "]";
        return nullptr;
    }
    if (n_obs >= (int64_t)1 << 30) { g_plan_err = "more than 2^30 observations"; return nullptr; }
    if ((int64_t)cum_nkpts[n_imgs - 1] != n_obs) { g_plan_err = "infos[0][-1] != number of observations"; return nullptr; }
    for (int i = 1; i < n_imgs; ++i)
        if (cum_nkpts[i] < cum_nkpts[i - 1]) { g_plan_err = "infos[0] must be non-decreasing"; return nullptr; }

    Plan* P = new Plan();
    P->n_imgs = n_imgs; P->n_obs = n_obs; P->n_tracks = n_tracks; P->L = max_local_imgs; P->max_slots = max_slots;
    P->max_batch_obs = max_batch_obs;
    PlanState& S = P->st;
    S.base.resize(n_imgs + 1);
    S.base[0] = 0;
    for (int i = 0; i < n_imgs; ++i) S.base[i + 1] = cum_nkpts[i];

    // Per-track observation lists in observation (= image) order: a counting sort over contiguous
    // observation ranges, one per thread.  Each thread counts its range's observations per track (one
    // byte per track: a track holds at most BA_CHUNK observations), the counts become per-thread
    // offsets inside each track's list, and each thread then writes its range in order, so every list
    // comes out in observation order without atomics or a sort.
    {
        unsigned hw = std::thread::hardware_concurrency();
        int64_t nth = std::max(1u, std::min(hw == 0 ? 1u : hw, 16u));
        nth = std::max<int64_t>(1, std::min<int64_t>(nth, n_obs / 65536));
        nth = std::max<int64_t>(1, std::min<int64_t>(nth, ((int64_t)256 << 20) / std::max(1, n_tracks)));
        const int64_t step = (n_obs + nth - 1) / nth;
        std::vector<std::vector<uint8_t>> cnt((size_t)nth);
        std::atomic<bool> bad_pid(false), too_long(false);
        auto over_ranges = [&](auto fn) {
            std::vector<std::thread> pool;
            for (int64_t w = 1; w < nth; ++w) pool.emplace_back(fn, w, std::min(n_obs, w * step), std::min(n_obs, (w + 1) * step));
            fn((int64_t)0, (int64_t)0, std::min(n_obs, step));
            for (auto& th : pool) th.join();
        };
        over_ranges([&](int64_t w, int64_t o0, int64_t o1) {
            std::vector<uint8_t>& c = cnt[w];
            c.assign(n_tracks, 0);
            bool bad = false, lng = false;
            for (int64_t o = o0; o < o1; ++o) {
                const int32_t t = pids[o];
                if (t < 0 || t >= n_tracks) { bad = true; continue; }
                if (c[t] == 255) lng = true; else c[t]++;
            }
            if (bad) bad_pid = true;
            if (lng) too_long = true;
        });
        if (bad_pid) { g_plan_err = "pid out of range"; delete P; return nullptr; }
        // per track: the threads' counts -> their first positions in the list (exclusive prefix)
        S.tptr.assign(n_tracks + 1, 0);
        parallel_for(n_tracks, [&](int64_t t0, int64_t t1) {
            bool lng = false;
            for (int64_t t = t0; t < t1; ++t) {
                int run = 0;
                for (int64_t w = 0; w < nth; ++w) {
                    const int x = cnt[w][t];
                    cnt[w][t] = (uint8_t)run;
                    run += x;
                }
                if (run > BA_CHUNK) lng = true;
                S.tptr[t + 1] = run;
            }
            if (lng) too_long = true;
        });
        if (too_long) {       // the first check tracks_ok makes, before any list is needed
            g_plan_err = "a track has more observations than one chunk holds (" + std::to_string(BA_CHUNK) + ")";
            delete P;
            return nullptr;
        }
        for (int t = 0; t < n_tracks; ++t) S.tptr[t + 1] += S.tptr[t];
        S.tob_img.reserve((size_t)(n_obs + n_obs / 8 + 4096));
        S.tob_pos.reserve((size_t)(n_obs + n_obs / 8 + 4096));
        S.tob_img.resize(n_obs);
        S.tob_pos.resize(n_obs);
        over_ranges([&](int64_t w, int64_t o0, int64_t o1) {
            if (o0 >= o1) return;
            std::vector<uint8_t>& c = cnt[w];
            // image of the range's first observation: the last image whose block starts at or before it
            int i = (int)(std::upper_bound(S.base.begin(), S.base.end() - 1, o0) - S.base.begin()) - 1;
            for (int64_t o = o0; o < o1; ++o) {
                while (o >= S.base[i + 1]) ++i;
                const int32_t t = pids[o];
                const int64_t k = S.tptr[t] + c[t]++;
                S.tob_img[k] = i;
                S.tob_pos[k] = (int32_t)(o - S.base[i]);
            }
        });
    }
    // room for appended tracks (ba_plan_append grows the per-track state in place)
    const size_t t_room = (size_t)n_tracks + n_tracks / 8 + 4096;
    for (auto* v : {&S.tmin, &S.tmax, &S.tdist}) v->reserve(t_room);
    S.tptr.reserve(t_room + 1);
    S.tmin.assign(n_tracks, INT32_MAX); S.tmax.assign(n_tracks, -1); S.tdist.assign(n_tracks, 0);
    track_extent(S, 0, n_tracks);
    if (!tracks_ok(S, 0, n_tracks, max_local_imgs)) { delete P; return nullptr; }
    // observed tracks ordered by (first image, last image, track id): two stable counting sorts
    {
        std::vector<int32_t> tmp;
        tmp.reserve(n_tracks);
        std::vector<int64_t> cnt(n_imgs + 1, 0);
        for (int t = 0; t < n_tracks; ++t) if (S.tptr[t + 1] > S.tptr[t]) cnt[S.tmax[t] + 1]++;
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        int64_t n_obs_tracks = cnt[n_imgs];
        tmp.resize(n_obs_tracks);
        for (int t = 0; t < n_tracks; ++t) if (S.tptr[t + 1] > S.tptr[t]) tmp[cnt[S.tmax[t]]++] = t;
        std::fill(cnt.begin(), cnt.end(), 0);
        for (int t : tmp) cnt[S.tmin[t] + 1]++;
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        S.order.reserve(t_room);
        S.order.resize(n_obs_tracks);
        for (int t : tmp) S.order[cnt[S.tmin[t]]++] = t;
    }
    S.oimg_ptr.reserve(t_room + 1);
    S.oimg.reserve((size_t)(n_obs + n_obs / 8 + 4096));
    S.oimg_ptr.assign(1, 0);
    order_images(S, 0);
    S.ncov = 0;
    for (int t = 0; t < n_tracks; ++t) S.ncov += (int64_t)S.tdist[t] * (S.tdist[t] + 1) / 2;
    if (!greedy(S, 0, n_imgs, max_local_imgs, max_slots, max_batch_obs) || !emit(P, 0)) { delete P; return nullptr; }
    return P;
}

// Plan of prev's structure with new tracks appended (tracks.py:84-102): n_imgs_new = prev's n_imgs + 1;
// image i keeps prev's observations and then gets add_cnt[i] new ones, whose track ids (add_pids, image by
// image) are n_tracks_prev .. n_tracks_new - 1.  Byte-identical to ba_plan_create on the merged structure:
// tracks keep their (first image, last image, id) order, so the batches that close before the first new
// track's place are the same and only the later ones are planned again; the earlier chunks keep their
// arrays with observation ids shifted by the new observations inserted before them (shift, per image).
// On success prev is consumed: the returned plan is prev's object, edited in place.  On failure (nullptr)
// prev is left exactly as it was and stays appendable: every limit the re-planning can hit is checked
// before prev is touched (per-track slot need) or before its arrays are written (MFMA entry-list
// capacity, which emit checks first), and the planning state edited before that point is restored.
extern "C" void* ba_plan_append(void* prev, const int32_t* add_cnt, int32_t n_imgs_new, const int32_t* add_pids,
                                int64_t n_add, int32_t n_tracks_new) {
    g_plan_err.clear();
    Plan* Q = (Plan*)prev;
    if (!Q || Q->st.tptr.empty()) { g_plan_err = "no plan state to append to"; return nullptr; }
    const int n_old = Q->n_imgs, T_old = Q->n_tracks;
    if (n_imgs_new != n_old + 1 || n_tracks_new < T_old || n_add < 0) { g_plan_err = "not an append"; return nullptr; }
    int64_t tot = 0;
    for (int i = 0; i < n_imgs_new; ++i) {
        if (add_cnt[i] < 0) { g_plan_err = "negative count"; return nullptr; }
        tot += add_cnt[i];
    }
    if (tot != n_add || Q->n_obs + n_add >= ((int64_t)1 << 30)) { g_plan_err = "bad appended counts"; return nullptr; }
    for (int64_t q = 0; q < n_add; ++q)
        if (add_pids[q] < T_old || add_pids[q] >= n_tracks_new) { g_plan_err = "appended pid out of range"; return nullptr; }
    // the new tracks' lists (image by image, so in observation order)
    const int T_new = n_tracks_new, T_add = T_new - T_old;
    std::vector<int64_t> nptr(T_add + 1, 0);
    for (int64_t q = 0; q < n_add; ++q) nptr[add_pids[q] - T_old + 1]++;
    for (int t = 0; t < T_add; ++t) nptr[t + 1] += nptr[t];
    for (int t = 0; t < T_add; ++t)
        if (nptr[t + 1] - nptr[t] > BA_CHUNK) {
            g_plan_err = "a track has more observations than one chunk holds (" + std::to_string(BA_CHUNK) + ")";
            return nullptr;
        }
    std::vector<int32_t> n_img(n_add), n_pos(n_add);
    {
        std::vector<int64_t> fill(nptr.begin(), nptr.end() - 1);
        int64_t q = 0;
        for (int i = 0; i < n_imgs_new; ++i) {
            const int64_t old_cnt = i < n_old ? Q->st.base[i + 1] - Q->st.base[i] : 0;
            for (int j = 0; j < add_cnt[i]; ++j, ++q) {
                const int64_t d = fill[add_pids[q] - T_old]++;
                n_img[d] = i;
                n_pos[d] = (int32_t)(old_cnt + j);
            }
        }
    }
    // the new tracks' extents and their limits, before touching prev
    std::vector<int32_t> dn(T_add, 0), mn(T_add, INT32_MAX), mx(T_add, -1);
    int32_t worst_d = 0;
    for (int t = 0; t < T_add; ++t) {
        int last = -1;
        for (int64_t k = nptr[t]; k < nptr[t + 1]; ++k) {
            const int i = n_img[k];
            if (i != last) { dn[t]++; last = i; }
            mn[t] = std::min(mn[t], i);
            mx[t] = std::max(mx[t], i);
        }
        worst_d = std::max(worst_d, dn[t]);
    }
    if (worst_d > Q->L) {
        g_plan_err = "a track spans more images (" + std::to_string(worst_d) + ") than max_local_imgs (" +
                     std::to_string(Q->L) + ")";
        return nullptr;
    }
    // greedy() fails only when one track alone needs more pair slots (all pairs of its images, diagonal
    // included) than max_slots; the old tracks passed that test when prev was planned
    if ((int64_t)worst_d * (worst_d + 1) / 2 > Q->max_slots) {
        g_plan_err = "a single track needs more pair slots than max_slots";
        return nullptr;
    }
    // new tracks in (first image, last image, id) order, merged into the old order
    std::vector<int32_t> nord;
    for (int t = 0; t < T_add; ++t) if (nptr[t + 1] > nptr[t]) nord.push_back(T_old + t);
    auto key_new = [&](int32_t t) { return std::make_tuple(mn[t - T_old], mx[t - T_old], t); };
    std::stable_sort(nord.begin(), nord.end(), [&](int32_t x, int32_t y) { return key_new(x) < key_new(y); });

    // ---- from here on prev's planning state is edited; the undo record below restores it on failure
    Plan* P = Q;
    PlanState& S = P->st;
    const int64_t n_obs_new = P->n_obs + n_add;
    std::vector<int64_t> base_old = S.base;
    const int64_t n_obs_old = P->n_obs, ncov_old = S.ncov;
    const std::vector<int32_t> shift_old = P->shift;
    int64_t stable_old[BA_PLAN_NARRAYS];
    std::copy(P->stable, P->stable + BA_PLAN_NARRAYS, stable_old);
    S.base.resize(n_imgs_new + 1);
    {
        int64_t acc = 0;
        for (int i = 0; i <= n_imgs_new; ++i) {
            const int64_t cnt_old = i < n_old ? base_old[i + 1] - base_old[i] : 0;
            S.base[i] = acc;
            if (i < n_imgs_new) acc += cnt_old + add_cnt[i];
        }
    }
    P->shift.assign(n_imgs_new, 0);
    for (int i = 0; i < n_old; ++i) P->shift[i] = (int32_t)(S.base[i] - base_old[i]);
    S.tptr.resize(T_new + 1);
    for (int t = 0; t < T_add; ++t) S.tptr[T_old + t + 1] = S.tptr[T_old] + nptr[t + 1];
    S.tob_img.insert(S.tob_img.end(), n_img.begin(), n_img.end());
    S.tob_pos.insert(S.tob_pos.end(), n_pos.begin(), n_pos.end());
    S.tmin.insert(S.tmin.end(), mn.begin(), mn.end());
    S.tmax.insert(S.tmax.end(), mx.begin(), mx.end());
    S.tdist.insert(S.tdist.end(), dn.begin(), dn.end());
    for (int t = 0; t < T_add; ++t) S.ncov += (int64_t)dn[t] * (dn[t] + 1) / 2;
    auto key = [&](int32_t t) { return std::make_tuple(S.tmin[t], S.tmax[t], t); };
    // first place of a new track in the merged order; the batches decided before it stay
    int64_t kstar = (int64_t)S.order.size();
    if (!nord.empty())
        kstar = std::lower_bound(S.order.begin(), S.order.end(), nord[0],
                                 [&](int32_t a, int32_t b) { return key(a) < key(b); }) - S.order.begin();
    int b_star = 0;
    {
        const int nb = (int)S.batches.size();
        while (b_star < nb && S.batches[b_star].k1 < kstar) ++b_star;
    }
    const int64_t k_re = b_star < (int)S.batches.size() ? S.batches[b_star].k0 : (int64_t)S.order.size();
    // undo record: the tails of the planning state that the re-planning from k_re / b_star rewrites
    const std::vector<int32_t> order_tail(S.order.begin() + kstar, S.order.end());
    const std::vector<int64_t> oimg_ptr_tail(S.oimg_ptr.begin() + k_re + 1, S.oimg_ptr.end());
    const std::vector<int32_t> oimg_tail(S.oimg.begin() + S.oimg_ptr[k_re], S.oimg.end());
    const std::vector<BatchDesc> batch_tail(S.batches.begin() + b_star, S.batches.end());
    const std::vector<int64_t> o_ch_old = S.o_ch, o_ct_old = S.o_ct, o_sl_old = S.o_sl, o_en_old = S.o_en;
    auto restore = [&]() {
        S.base = base_old;
        S.tptr.resize(T_old + 1);
        S.tob_img.resize(n_obs_old); S.tob_pos.resize(n_obs_old);
        S.tmin.resize(T_old); S.tmax.resize(T_old); S.tdist.resize(T_old);
        S.ncov = ncov_old;
        S.order.resize(kstar);
        S.order.insert(S.order.end(), order_tail.begin(), order_tail.end());
        S.oimg_ptr.resize(k_re + 1);
        S.oimg_ptr.insert(S.oimg_ptr.end(), oimg_ptr_tail.begin(), oimg_ptr_tail.end());
        S.oimg.resize(S.oimg_ptr[k_re]);
        S.oimg.insert(S.oimg.end(), oimg_tail.begin(), oimg_tail.end());
        S.batches.resize(b_star);
        S.batches.insert(S.batches.end(), batch_tail.begin(), batch_tail.end());
        S.o_ch = o_ch_old; S.o_ct = o_ct_old; S.o_sl = o_sl_old; S.o_en = o_en_old;
        P->n_imgs = n_old; P->n_obs = n_obs_old; P->n_tracks = T_old;
        P->shift = shift_old;
        std::copy(stable_old, stable_old + BA_PLAN_NARRAYS, P->stable);
    };
    {
        std::vector<int32_t> tail;
        tail.reserve(S.order.size() - kstar + nord.size());
        std::merge(S.order.begin() + kstar, S.order.end(), nord.begin(), nord.end(), std::back_inserter(tail),
                   [&](int32_t a, int32_t b) { return key(a) < key(b); });
        S.order.resize(kstar);
        S.order.insert(S.order.end(), tail.begin(), tail.end());
    }
    S.oimg_ptr.resize(k_re + 1);
    order_images(S, k_re);
    S.batches.resize(b_star);
    P->n_imgs = n_imgs_new; P->n_obs = n_obs_new; P->n_tracks = T_new;
    // what stays: the arrays of batches [0, b_star), observation ids shifted
    const int64_t c_keep = S.o_ch[b_star] * BA_CHUNK;
    for (int k = 0; k < BA_PLAN_NARRAYS; ++k) P->stable[k] = 0;
    P->stable[BA_PA_CHUNK_OBS] = P->stable[BA_PA_SLOT_INFO] = P->stable[BA_PA_SLOT_SRC] = c_keep;
    P->stable[BA_PA_S_PID] = P->stable[BA_PA_S_IMG] = c_keep;
    P->stable[BA_PA_CHUNK_META] = S.o_ch[b_star] * 4;
    P->stable[BA_PA_CHUNK_SLOTS] = S.o_ch[b_star] * BA_MAX_SLOTS;
    P->stable[BA_PA_CHUNK_EPTR] = S.o_ch[b_star];
    P->stable[BA_PA_CHUNK_ENT] = S.o_en[b_star];
    for (int k : {BA_PA_CT_PID, BA_PA_CT_FIRST, BA_PA_CT_M, BA_PA_CT_MASK}) P->stable[k] = S.o_ct[b_star];
    P->stable[BA_PA_SLOT_PAIR] = S.o_sl[b_star];
    P->stable[BA_PA_B_CHUNK_PTR] = P->stable[BA_PA_B_SLOT_PTR] = b_star + 1;
    P->stable[BA_PA_B_IMGS] = (int64_t)b_star * P->L;
    P->stable[BA_PA_B_NIMGS] = b_star;
    P->stable[BA_PA_B_POS_SLOT] = (int64_t)b_star * BA_MAX_SLOTS;
    // emit() writes prev's arrays only once every new batch's entry lists fit; nothing before that
    // point has touched them
    if (!greedy(S, k_re, n_imgs_new, P->L, P->max_slots, P->max_batch_obs) || !emit(P, b_star)) {
        restore();
        return nullptr;
    }
    {
        // the kept chunks' observation ids, in the merged structure's numbering (emit wrote only from
        // chunk o_ch[b_star] on, so the kept prefix still holds prev's ids)
        auto& co = P->v[BA_PA_CHUNK_OBS];
        auto& ss = P->v[BA_PA_SLOT_SRC];
        const auto& si = P->v[BA_PA_S_IMG];
        const int32_t* sh = P->shift.data();
        parallel_for(c_keep, [&](int64_t q0, int64_t q1) {
            for (int64_t q = q0; q < q1; ++q) {
                const int32_t d = sh[si[q]];
                ss[q] += d;
                if (co[q] >= 0) co[q] += d;
            }
        });
    }
    return P;
}

extern "C" int ba_plan_query(const void* plan, int64_t* scalars, int64_t* array_sizes) {
    const Plan* P = (const Plan*)plan;
    if (!P) return 1;
    for (int k = 0; k < BA_PLAN_NSCALARS; ++k) scalars[k] = P->scalars[k];
    for (int k = 0; k < BA_PLAN_NARRAYS; ++k) array_sizes[k] = (int64_t)P->v[k].size();
    return 0;
}

extern "C" int ba_plan_export(const void* plan, int32_t which, int32_t* dst) {
    const Plan* P = (const Plan*)plan;
    if (!P || which < 0 || which >= BA_PLAN_NARRAYS) return 1;
    if (!P->v[which].empty()) std::memcpy(dst, P->v[which].data(), P->v[which].size() * sizeof(int32_t));
    return 0;
}

extern "C" void ba_plan_destroy(void* plan) { delete (Plan*)plan; }

// the plan's array `which` in place (valid until the plan is destroyed or appended to)
extern "C" const int32_t* ba_plan_array(const void* plan, int32_t which) {
    const Plan* P = (const Plan*)plan;
    if (!P || which < 0 || which >= BA_PLAN_NARRAYS) return nullptr;
    return P->v[which].data();
}

// a plan made by ba_plan_append: per array, the leading elements equal to the parent's (after the shift of
// chunk_obs / slot_src); per image, the shift of the parent's observation ids (0 for a plan made by
// ba_plan_create, whose stable lengths are all 0)
extern "C" int ba_plan_stable(const void* plan, int64_t* stable, int32_t* shift) {
    const Plan* P = (const Plan*)plan;
    if (!P) return 1;
    for (int k = 0; k < BA_PLAN_NARRAYS; ++k) stable[k] = P->stable[k];
    if (shift)
        for (int i = 0; i < P->n_imgs; ++i) shift[i] = i < (int)P->shift.size() ? P->shift[i] : 0;
    return 0;
}

// ---------------------------------------------------------------------------- pair-major plan
namespace ba {
struct PmPlan {
    std::vector<int32_t> v[BA_PM_NARRAYS];
    int64_t scalars[BA_PM_NSCALARS] = {0};
};
}  // namespace ba

extern "C" void* ba_pm_plan_create(const int32_t* cum_nkpts, int32_t n_imgs, const int32_t* pids, int64_t n_obs,
                                   int32_t n_tracks) {
    g_plan_err.clear();
    if (n_imgs <= 0 || n_obs < 0 || n_tracks < 0) { g_plan_err = "bad sizes"; return nullptr; }
    if (n_obs >= (int64_t)1 << 30) { g_plan_err = "more than 2^30 observations"; return nullptr; }
    if ((int64_t)cum_nkpts[n_imgs - 1] != n_obs) { g_plan_err = "infos[0][-1] != number of observations"; return nullptr; }
    for (int i = 1; i < n_imgs; ++i)
        if (cum_nkpts[i] < cum_nkpts[i - 1]) { g_plan_err = "infos[0] must be non-decreasing"; return nullptr; }
    for (int64_t o = 0; o < n_obs; ++o)
        if (pids[o] < 0 || pids[o] >= n_tracks) { g_plan_err = "pid out of range"; return nullptr; }
    PmPlan* P = new PmPlan();
    auto& obs_img = P->v[BA_PM_OBS_IMG];
    obs_img.assign(n_obs, 0);
    auto obs0 = [&](int64_t i) -> int64_t { return i ? cum_nkpts[i - 1] : 0; };
    parallel_for(n_imgs, [&](int64_t i0, int64_t i1) {
        for (int64_t i = i0; i < i1; ++i)
            for (int64_t o = obs0(i); o < cum_nkpts[i]; ++o) obs_img[o] = (int32_t)i;
    }, 1);
    // runs: per image, the observations grouped by track id (stable), one run per distinct track
    auto& run_obs = P->v[BA_PM_RUN_OBS];
    run_obs.resize(n_obs);
    std::vector<int32_t> img_nruns(n_imgs, 0);
    parallel_for(n_imgs, [&](int64_t i0, int64_t i1) {
        for (int64_t i = i0; i < i1; ++i) {
            const int64_t b = obs0(i), e = cum_nkpts[i];
            std::iota(run_obs.begin() + b, run_obs.begin() + e, (int32_t)b);
            std::stable_sort(run_obs.begin() + b, run_obs.begin() + e,
                             [&](int32_t x, int32_t y) { return pids[x] < pids[y]; });
            int32_t n = 0;
            for (int64_t k = b; k < e; ++k)
                if (k == b || pids[run_obs[k]] != pids[run_obs[k - 1]]) ++n;
            img_nruns[i] = n;
        }
    }, 1);
    auto& img_run_ptr = P->v[BA_PM_IMG_RUN_PTR];
    img_run_ptr.assign(n_imgs + 1, 0);
    for (int i = 0; i < n_imgs; ++i) img_run_ptr[i + 1] = img_run_ptr[i] + img_nruns[i];
    const int64_t n_runs = img_run_ptr[n_imgs];
    auto& run_ptr = P->v[BA_PM_RUN_PTR];
    auto& run_trk = P->v[BA_PM_RUN_TRK];
    auto& run_img = P->v[BA_PM_RUN_IMG];
    run_ptr.assign(n_runs + 1, 0);
    run_trk.assign(n_runs, 0);
    run_img.assign(n_runs, 0);
    parallel_for(n_imgs, [&](int64_t i0, int64_t i1) {
        for (int64_t i = i0; i < i1; ++i) {
            int64_t r = img_run_ptr[i];
            const int64_t b = obs0(i), e = cum_nkpts[i];
            for (int64_t k = b; k < e; ++k)
                if (k == b || pids[run_obs[k]] != pids[run_obs[k - 1]]) {
                    run_ptr[r] = (int32_t)k;
                    run_trk[r] = pids[run_obs[k]];
                    run_img[r] = (int32_t)i;
                    ++r;
                }
        }
    }, 1);
    run_ptr[n_runs] = (int32_t)n_obs;
    // runs and observations of each track in image order (runs are visited image by image)
    auto& trk_run_ptr = P->v[BA_PM_TRK_RUN_PTR];
    auto& trk_run = P->v[BA_PM_TRK_RUN];
    auto& trk_obs_ptr = P->v[BA_PM_TRK_OBS_PTR];
    auto& trk_obs = P->v[BA_PM_TRK_OBS];
    trk_run_ptr.assign(n_tracks + 1, 0);
    trk_obs_ptr.assign(n_tracks + 1, 0);
    for (int64_t r = 0; r < n_runs; ++r) {
        trk_run_ptr[run_trk[r] + 1]++;
        trk_obs_ptr[run_trk[r] + 1] += run_ptr[r + 1] - run_ptr[r];
    }
    for (int t = 0; t < n_tracks; ++t) {
        trk_run_ptr[t + 1] += trk_run_ptr[t];
        trk_obs_ptr[t + 1] += trk_obs_ptr[t];
    }
    trk_run.assign(n_runs, 0);
    trk_obs.assign(n_obs, 0);
    {
        std::vector<int32_t> fr(trk_run_ptr.begin(), trk_run_ptr.end() - 1), fo(trk_obs_ptr.begin(), trk_obs_ptr.end() - 1);
        for (int64_t r = 0; r < n_runs; ++r) {
            const int t = run_trk[r];
            trk_run[fr[t]++] = (int32_t)r;
            for (int k = run_ptr[r]; k < run_ptr[r + 1]; ++k) trk_obs[fo[t]++] = run_obs[k];
        }
    }
    int64_t max_tr = 0;
    for (int t = 0; t < n_tracks; ++t) max_tr = std::max<int64_t>(max_tr, trk_run_ptr[t + 1] - trk_run_ptr[t]);
    // co-visible images after each image: for each run of image a, the later runs of its track
    std::vector<std::vector<int32_t>> nb(n_imgs);
    parallel_for(n_imgs, [&](int64_t i0, int64_t i1) {
        for (int64_t a = i0; a < i1; ++a) {
            auto& L = nb[a];
            for (int r = img_run_ptr[a]; r < img_run_ptr[a + 1]; ++r) {
                const int t = run_trk[r];
                for (int q = trk_run_ptr[t]; q < trk_run_ptr[t + 1]; ++q) {
                    const int b = run_img[trk_run[q]];
                    if (b > a) L.push_back(b);
                }
            }
            std::sort(L.begin(), L.end());
            L.erase(std::unique(L.begin(), L.end()), L.end());
        }
    }, 1);
    // pairs: (a, a) for every image with runs, then (a, b) for b in nb[a]
    std::vector<int64_t> pbase(n_imgs + 1, 0);
    for (int a = 0; a < n_imgs; ++a)
        pbase[a + 1] = pbase[a] + (img_nruns[a] > 0 ? 1 : 0) + (int64_t)nb[a].size();
    const int64_t n_pairs = pbase[n_imgs];
    if (n_pairs >= ((int64_t)1 << 30)) { g_plan_err = "too many image pairs"; delete P; return nullptr; }
    auto& pair_i1 = P->v[BA_PM_PAIR_I1];
    auto& pair_i2 = P->v[BA_PM_PAIR_I2];
    auto& diag_pair = P->v[BA_PM_DIAG_PAIR];
    pair_i1.assign(n_pairs, 0);
    pair_i2.assign(n_pairs, 0);
    diag_pair.assign(n_imgs, -1);
    for (int a = 0; a < n_imgs; ++a) {
        int64_t q = pbase[a];
        if (img_nruns[a] > 0) { diag_pair[a] = (int32_t)q; pair_i1[q] = a; pair_i2[q] = a; ++q; }
        for (int32_t b : nb[a]) { pair_i1[q] = a; pair_i2[q] = b; ++q; }
    }
    // terms of the off-diagonal pairs of row a, in run order of image a then track order
    std::vector<int64_t> tcnt(n_pairs + 1, 0);
    auto pair_of = [&](int a, int b) -> int64_t {
        const auto& L = nb[a];
        const int64_t k = std::lower_bound(L.begin(), L.end(), b) - L.begin();
        return pbase[a] + (img_nruns[a] > 0 ? 1 : 0) + k;
    };
    parallel_for(n_imgs, [&](int64_t i0, int64_t i1) {
        for (int64_t a = i0; a < i1; ++a)
            for (int r = img_run_ptr[a]; r < img_run_ptr[a + 1]; ++r) {
                const int t = run_trk[r];
                for (int q = trk_run_ptr[t]; q < trk_run_ptr[t + 1]; ++q) {
                    const int b = run_img[trk_run[q]];
                    if (b > a) tcnt[pair_of((int)a, b) + 1]++;
                }
            }
    }, 1);
    for (int64_t p = 0; p < n_pairs; ++p) tcnt[p + 1] += tcnt[p];
    const int64_t n_terms = tcnt[n_pairs];
    if (n_terms >= ((int64_t)1 << 30)) { g_plan_err = "too many pair terms"; delete P; return nullptr; }
    auto& term_ptr = P->v[BA_PM_TERM_PTR];
    auto& term = P->v[BA_PM_TERM];
    term_ptr.assign(n_pairs + 1, 0);
    for (int64_t p = 0; p <= n_pairs; ++p) term_ptr[p] = (int32_t)tcnt[p];
    term.assign(2 * n_terms, 0);
    parallel_for(n_imgs, [&](int64_t i0, int64_t i1) {
        std::vector<int64_t> fill;
        for (int64_t a = i0; a < i1; ++a) {
            const int64_t p0 = pbase[a], p1 = pbase[a + 1];
            fill.assign(tcnt.begin() + p0, tcnt.begin() + p1);
            for (int r = img_run_ptr[a]; r < img_run_ptr[a + 1]; ++r) {
                const int t = run_trk[r];
                for (int q = trk_run_ptr[t]; q < trk_run_ptr[t + 1]; ++q) {
                    const int rb = trk_run[q], b = run_img[rb];
                    if (b > a) {
                        const int64_t k = fill[pair_of((int)a, b) - p0]++;
                        term[2 * k] = r;
                        term[2 * k + 1] = rb;
                    }
                }
            }
        }
    }, 1);
    int64_t max_terms = 0;
    for (int64_t p = 0; p < n_pairs; ++p) max_terms = std::max<int64_t>(max_terms, tcnt[p + 1] - tcnt[p]);
    // the order k_pm_pairs takes the pairs in: by the co-visibility window of each pair's terms (the smallest
    // first image and the largest last image of their tracks), then pair id; pairs without terms last.
    // Pairs whose terms come from tracks of one neighbourhood then run close together and share their V
    // rows in the L2 (random co-visibility, config 3: 9.0 -> 7.4 ms against the (i1, i2) order).
    {
        std::vector<int32_t> tlo(n_tracks, 0), thi(n_tracks, 0), klo(n_pairs), khi(n_pairs);
        parallel_for(n_tracks, [&](int64_t t0, int64_t t1) {
            for (int64_t t = t0; t < t1; ++t)
                if (trk_run_ptr[t + 1] > trk_run_ptr[t]) {
                    tlo[t] = run_img[trk_run[trk_run_ptr[t]]];
                    thi[t] = run_img[trk_run[trk_run_ptr[t + 1] - 1]];
                }
        });
        parallel_for(n_pairs, [&](int64_t p0, int64_t p1) {
            for (int64_t p = p0; p < p1; ++p) {
                int32_t lo = n_imgs, hi = n_imgs;
                if (tcnt[p + 1] > tcnt[p]) { lo = INT32_MAX; hi = -1; }
                for (int64_t q = tcnt[p]; q < tcnt[p + 1]; ++q) {
                    const int t = run_trk[term[2 * q]];
                    lo = std::min(lo, tlo[t]);
                    hi = std::max(hi, thi[t]);
                }
                klo[p] = lo; khi[p] = hi;
            }
        });
        // two stable counting sorts over the keys 0 .. n_imgs: by the last image, then by the first
        std::vector<int32_t> tmp(n_pairs);
        std::vector<int64_t> cnt(n_imgs + 2);
        auto by = [&](const std::vector<int32_t>& key, const int32_t* in, int32_t* out) {
            std::fill(cnt.begin(), cnt.end(), 0);
            for (int64_t q = 0; q < n_pairs; ++q) cnt[key[in ? in[q] : q] + 1]++;
            for (int i = 0; i <= n_imgs; ++i) cnt[i + 1] += cnt[i];
            for (int64_t q = 0; q < n_pairs; ++q) {
                const int32_t p = in ? in[q] : (int32_t)q;
                out[cnt[key[p]]++] = p;
            }
        };
        auto& pair_sched = P->v[BA_PM_PAIR_SCHED];
        pair_sched.assign(n_pairs, 0);
        by(khi, nullptr, tmp.data());
        by(klo, tmp.data(), pair_sched.data());
    }
    // image rows of the symmetric pair structure, as in the batched plan
    auto& row_ptr = P->v[BA_PM_ROW_PTR];
    auto& row_ent = P->v[BA_PM_ROW_ENT];
    {
        std::vector<int32_t> cnt(n_imgs + 1, 0);
        for (int64_t p = 0; p < n_pairs; ++p) {
            cnt[pair_i1[p] + 1]++;
            if (pair_i2[p] != pair_i1[p]) cnt[pair_i2[p] + 1]++;
        }
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        row_ptr.assign(cnt.begin(), cnt.end());
        row_ent.assign(cnt[n_imgs], 0);
        std::vector<int32_t> fill(cnt.begin(), cnt.end() - 1);
        for (int64_t p = 0; p < n_pairs; ++p) {
            row_ent[fill[pair_i1[p]]++] = (int32_t)(p << 1);
            if (pair_i2[p] != pair_i1[p]) row_ent[fill[pair_i2[p]]++] = (int32_t)((p << 1) | 1);
        }
    }
    P->scalars[BA_PMS_N_RUNS] = n_runs;
    P->scalars[BA_PMS_N_PAIRS] = n_pairs;
    P->scalars[BA_PMS_N_TERMS] = n_terms;
    P->scalars[BA_PMS_MAX_TERMS] = max_terms;
    P->scalars[BA_PMS_MAX_TRACK_RUNS] = max_tr;
    return P;
}

extern "C" int ba_pm_plan_query(const void* plan, int64_t* scalars, int64_t* array_sizes) {
    const PmPlan* P = (const PmPlan*)plan;
    if (!P) return 1;
    for (int k = 0; k < BA_PM_NSCALARS; ++k) scalars[k] = P->scalars[k];
    for (int k = 0; k < BA_PM_NARRAYS; ++k) array_sizes[k] = (int64_t)P->v[k].size();
    return 0;
}

extern "C" int ba_pm_plan_export(const void* plan, int32_t which, int32_t* dst) {
    const PmPlan* P = (const PmPlan*)plan;
    if (!P || which < 0 || which >= BA_PM_NARRAYS) return 1;
    if (!P->v[which].empty()) std::memcpy(dst, P->v[which].data(), P->v[which].size() * sizeof(int32_t));
    return 0;
}

extern "C" void ba_pm_plan_destroy(void* plan) { delete (PmPlan*)plan; }
