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
#include <cstring>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "ba_plan.h"
#include "ba_hip.h"

namespace ba {

static std::string g_plan_err;

struct Plan {
    int32_t n_imgs = 0, n_tracks = 0, L = 0, max_slots = 0;
    int64_t n_obs = 0;
    std::vector<int32_t> v[BA_PLAN_NARRAYS];
    int64_t scalars[BA_PLAN_NSCALARS] = {0};
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

    // observation -> image, and per-track observation lists in observation (= image) order
    std::vector<int32_t> img(n_obs);
    parallel_for(n_imgs, [&](int64_t i0, int64_t i1) {
        for (int64_t i = i0; i < i1; ++i)
            for (int64_t o = i ? cum_nkpts[i - 1] : 0; o < cum_nkpts[i]; ++o) img[o] = (int32_t)i;
    }, 1);
    std::vector<int32_t> tcnt(n_tracks, 0);
    std::atomic<bool> bad_pid(false);
    parallel_for(n_obs, [&](int64_t o0, int64_t o1) {
        for (int64_t o = o0; o < o1; ++o) {
            const int32_t t = pids[o];
            if (t < 0 || t >= n_tracks) { bad_pid = true; continue; }
            __atomic_fetch_add(&tcnt[t], 1, __ATOMIC_RELAXED);
        }
    });
    if (bad_pid) { g_plan_err = "pid out of range"; delete P; return nullptr; }
    std::vector<int64_t> tptr(n_tracks + 1, 0);
    for (int t = 0; t < n_tracks; ++t) tptr[t + 1] = tptr[t] + tcnt[t];
    std::vector<int32_t> tobs(n_obs);
    {
        std::vector<int64_t> fill(tptr.begin(), tptr.end() - 1);
        parallel_for(n_obs, [&](int64_t o0, int64_t o1) {
            for (int64_t o = o0; o < o1; ++o) tobs[__atomic_fetch_add(&fill[pids[o]], 1, __ATOMIC_RELAXED)] = (int32_t)o;
        });
        parallel_for(n_tracks, [&](int64_t t0, int64_t t1) {        // each list back in observation order
            for (int64_t t = t0; t < t1; ++t) std::sort(tobs.begin() + tptr[t], tobs.begin() + tptr[t + 1]);
        });
    }
    // distinct images per track (observations of a track are in image order)
    std::vector<int32_t> tmin(n_tracks, INT32_MAX), tmax(n_tracks, -1), tdist(n_tracks, 0);
    std::atomic<int32_t> worst_m(0), worst_d(0);
    parallel_for(n_tracks, [&](int64_t t0, int64_t t1) {
        int32_t wm = 0, wd = 0;
        for (int64_t t = t0; t < t1; ++t) {
            int last = -1;
            for (int64_t k = tptr[t]; k < tptr[t + 1]; ++k) {
                const int i = img[tobs[k]];
                if (i != last) { tdist[t]++; last = i; }
                tmin[t] = std::min(tmin[t], i);
                tmax[t] = std::max(tmax[t], i);
            }
            wm = std::max<int32_t>(wm, (int32_t)(tptr[t + 1] - tptr[t]));
            wd = std::max(wd, tdist[t]);
        }
        int32_t c = worst_m.load();
        while (wm > c && !worst_m.compare_exchange_weak(c, wm)) {}
        c = worst_d.load();
        while (wd > c && !worst_d.compare_exchange_weak(c, wd)) {}
    });
    if (worst_m.load() > BA_CHUNK) {
        g_plan_err = "a track has more observations than one chunk holds (" + std::to_string(BA_CHUNK) + ")";
        delete P; return nullptr;
    }
    if (worst_d.load() > max_local_imgs) {
        g_plan_err = "a track spans more images (" + std::to_string(worst_d.load()) + ") than max_local_imgs (" +
                     std::to_string(max_local_imgs) + ")";
        delete P; return nullptr;
    }
    // observed tracks ordered by (first image, last image, track id): two stable counting sorts
    std::vector<int32_t> order;
    {
        std::vector<int32_t> tmp;
        tmp.reserve(n_tracks);
        std::vector<int64_t> cnt(n_imgs + 1, 0);
        for (int t = 0; t < n_tracks; ++t) if (tptr[t + 1] > tptr[t]) cnt[tmax[t] + 1]++;
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        int64_t n_obs_tracks = cnt[n_imgs];
        tmp.resize(n_obs_tracks);
        for (int t = 0; t < n_tracks; ++t) if (tptr[t + 1] > tptr[t]) tmp[cnt[tmax[t]]++] = t;
        std::fill(cnt.begin(), cnt.end(), 0);
        for (int t : tmp) cnt[tmin[t] + 1]++;
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        order.resize(n_obs_tracks);
        for (int t : tmp) order[cnt[tmin[t]]++] = t;
    }
    // distinct image list of each track, laid out in `order`
    std::vector<int64_t> oimg_ptr(order.size() + 1, 0);
    for (size_t k = 0; k < order.size(); ++k) oimg_ptr[k + 1] = oimg_ptr[k] + tdist[order[k]];
    std::vector<int32_t> oimg(oimg_ptr.back());
    parallel_for((int64_t)order.size(), [&](int64_t k0, int64_t k1) {
        for (int64_t k = k0; k < k1; ++k) {
            const int t = order[k];
            int64_t q = oimg_ptr[k];
            int last = -1;
            for (int64_t j = tptr[t]; j < tptr[t + 1]; ++j) {
                const int i = img[tobs[j]];
                if (i != last) { oimg[q++] = i; last = i; }
            }
        }
    });

    // ------------------------------------------------------------ greedy batching
    // Pass 1 (sequential): tracks are taken in order and a batch is closed when the next track
    // would exceed max_local_imgs images, max_slots pairs or max_batch_obs observations, so every
    // batch is a contiguous range of `order`.  Pass 2 (parallel over batches): chunks, MFMA entry
    // lists and wave placement of each batch.  Pass 3: concatenation in batch order.
    struct BatchDesc {
        int32_t k0, k1;                    // range of `order`
        std::vector<int32_t> imgs;         // local image -> global image
        std::vector<uint32_t> rows;        // rows[a] bit b: local pair (a, b), a <= b, is touched
    };
    std::vector<BatchDesc> batches;
    {
        std::vector<int32_t> cur_imgs;
        std::vector<uint32_t> rows(max_local_imgs, 0);
        std::vector<int32_t> limg_of(n_imgs, -1);
        int cur_nslots = 0, k_begin = 0, n_cur = 0;
        int64_t cur_obs = 0;
        auto close = [&](int k_end) {
            if (n_cur == 0) return;
            batches.push_back(BatchDesc{k_begin, k_end, cur_imgs, rows});
            for (int i : cur_imgs) limg_of[i] = -1;
            cur_imgs.clear();
            std::fill(rows.begin(), rows.end(), 0u);
            cur_nslots = 0; cur_obs = 0; n_cur = 0; k_begin = k_end;
        };
        for (int kk = 0; kk < (int)order.size(); ++kk) {
            const int t = order[kk];
            const int32_t* timgs = oimg.data() + oimg_ptr[kk];
            const int nti = (int)(oimg_ptr[kk + 1] - oimg_ptr[kk]);
            const int m = (int)(tptr[t + 1] - tptr[t]);
            for (int attempt = 0; attempt < 2; ++attempt) {
                // local ids of the track's images (images not yet local get provisional ids)
                const int n_loc = (int)cur_imgs.size();
                int prov = n_loc;
                uint32_t M = 0;
                for (int q = 0; q < nti; ++q) {
                    const int l = limg_of[timgs[q]];
                    M |= 1u << (l >= 0 ? l : prov++);
                }
                bool ok = prov <= max_local_imgs &&
                          (max_batch_obs <= 0 || cur_obs + m <= max_batch_obs || n_cur == 0);
                int add_slots = 0;
                if (ok) {
                    // local pairs (x <= y) within M that no earlier track of the batch touched
                    for (uint32_t r = M; r; r &= r - 1) {
                        const int x = __builtin_ctz(r);
                        add_slots += __builtin_popcount(M & ~((1u << x) - 1u) & ~rows[x]);
                    }
                    ok = cur_nslots + add_slots <= max_slots;
                }
                if (!ok) {
                    if (n_cur == 0) {
                        g_plan_err = "a single track needs more pair slots than max_slots";
                        delete P; return nullptr;
                    }
                    close(kk);
                    continue;
                }
                for (int q = 0; q < nti; ++q)
                    if (limg_of[timgs[q]] < 0) { limg_of[timgs[q]] = (int)cur_imgs.size(); cur_imgs.push_back(timgs[q]); }
                for (uint32_t r = M; r; r &= r - 1) {
                    const int x = __builtin_ctz(r);
                    rows[x] |= M & ~((1u << x) - 1u);
                }
                cur_nslots += add_slots;
                cur_obs += m;
                n_cur++;
                break;
            }
        }
        close((int)order.size());
    }

    // Pass 2: one batch's arrays, with chunk-track ids and entry offsets local to the batch
    struct BatchOut {
        std::vector<int32_t> chunk_obs, slot_info, chunk_meta, ct_pid, ct_first, ct_m, ct_mask, slot_pair,
            chunk_slots, chunk_eptr, pos_slot;
        std::vector<uint32_t> ents;
        bool overflow = false;
    };
    const int n_batches = (int)batches.size();
    std::vector<BatchOut> outs(n_batches);
    auto build_batch = [&](int batch, std::vector<int32_t>& limg_of) {
        const BatchDesc& bd = batches[batch];
        BatchOut& R = outs[batch];
        for (int a = 0; a < (int)bd.imgs.size(); ++a) limg_of[bd.imgs[a]] = a;
        // local pair slots in (b, a) order
        for (int b = 0; b < (int)bd.imgs.size(); ++b)
            for (int a = 0; a <= b; ++a)
                if ((bd.rows[a] >> b) & 1u) R.slot_pair.push_back(a | (b << 8));
        const int nsl = (int)R.slot_pair.size();
        std::vector<int16_t> lead;
        int k = bd.k0;
        while (k < bd.k1) {                                   // chunks: tracks packed whole, in order
            int used = 0, ntr = 0;
            const size_t base = R.chunk_obs.size();
            R.chunk_obs.resize(base + BA_CHUNK, -1);
            R.slot_info.resize(base + BA_CHUNK, -1);
            const int first_ct = (int)R.ct_pid.size();
            while (k < bd.k1) {
                const int t = order[k];
                const int m = (int)(tptr[t + 1] - tptr[t]);
                if (used + m > BA_CHUNK || ntr == BA_MAX_CT) break;
                uint32_t mask = 0;
                int last_img = -1, leader = -1;
                for (int j = 0; j < m; ++j) {
                    const int o = tobs[tptr[t] + j];
                    const int lim = limg_of[img[o]];
                    if (img[o] != last_img) { leader = used + j; last_img = img[o]; }
                    mask |= 1u << lim;
                    R.chunk_obs[base + used + j] = o;
                    R.slot_info[base + used + j] = lim | (ntr << 8) | (leader << 16);
                }
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
            lead.assign((size_t)ntr * BA_MAX_LOCAL, -1);
            for (int sidx = 0; sidx < used; ++sidx) {
                const int inf = R.slot_info[base + sidx];
                lead[(size_t)((inf >> 8) & 0xff) * BA_MAX_LOCAL + (inf & 0xff)] = (int16_t)(inf >> 16);
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
                    for (int tt = 0; tt < ntr; ++tt) {
                        const int la_ = lead[(size_t)tt * BA_MAX_LOCAL + a], lb_ = lead[(size_t)tt * BA_MAX_LOCAL + bq];
                        if (la_ >= 0 && lb_ >= 0) ent(la_ * BA_BLK, lb_ * BA_BLK);
                    }
                } else {
                    for (int sidx = 0; sidx < used; ++sidx)
                        if ((R.slot_info[base + sidx] & 0xff) == a) ent(sidx * BA_BLK + BA_JROW, sidx * BA_BLK + BA_JROW);
                    pad(e0 + off);
                    njg = (int)((R.ents.size() - e0 - off) / 4);
                    for (int sidx = 0; sidx < used; ++sidx) {
                        const int inf = R.slot_info[base + sidx];
                        if ((inf & 0xff) == a && (inf >> 16) == sidx) ent(sidx * BA_BLK, sidx * BA_BLK);
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
        // decreasing total work and each goes where the summed per-chunk maxima grow least.
        {
            const int nc = (int)(R.chunk_meta.size() / 4);
            std::vector<int32_t> wk((size_t)nc * nsl);                  // MFMAs of (chunk, slot)
            std::vector<int64_t> tot(nsl, 0);
            for (int c = 0; c < nc; ++c)
                for (int q = 0; q < nsl; ++q) {
                    wk[(size_t)c * nsl + q] = 3 * BA_TAB_NG(R.chunk_slots[(size_t)c * BA_MAX_SLOTS + q]);
                    tot[q] += wk[(size_t)c * nsl + q];
                }
            std::vector<int> sorder(nsl);
            std::iota(sorder.begin(), sorder.end(), 0);
            std::stable_sort(sorder.begin(), sorder.end(), [&](int x, int y) { return tot[x] > tot[y]; });
            constexpr int NS = 4;
            std::vector<int64_t> ls((size_t)nc * NS, 0), lw((size_t)nc * BA_WAVES, 0), ms(nc, 0), mw(nc, 0);
            int cnt[BA_WAVES] = {0};
            R.pos_slot.assign(BA_MAX_SLOTS, -1);
            for (int q : sorder) {
                int best = -1;
                int64_t best_cost = 0;
                for (int w = 0; w < BA_WAVES; ++w) {
                    if (cnt[w] >= BA_SLOTS_PER_WAVE) continue;
                    const int sd = w % NS;
                    int64_t cost = 0;
                    for (int c = 0; c < nc; ++c) {
                        const int64_t x = wk[(size_t)c * nsl + q];
                        cost += NS * std::max(ls[(size_t)c * NS + sd] + x, ms[c]) + std::max(lw[(size_t)c * BA_WAVES + w] + x, mw[c]);
                    }
                    if (best < 0 || cost < best_cost) { best = w; best_cost = cost; }
                }
                R.pos_slot[best + BA_WAVES * cnt[best]] = q;
                cnt[best]++;
                const int sd = best % NS;
                for (int c = 0; c < nc; ++c) {
                    const int64_t x = wk[(size_t)c * nsl + q];
                    ls[(size_t)c * NS + sd] += x;
                    lw[(size_t)c * BA_WAVES + best] += x;
                    ms[c] = std::max(ms[c], ls[(size_t)c * NS + sd]);
                    mw[c] = std::max(mw[c], lw[(size_t)c * BA_WAVES + best]);
                }
            }
        }
        for (int i : bd.imgs) limg_of[i] = -1;
    };
    {
        unsigned nth = std::thread::hardware_concurrency();
        nth = std::max(1u, std::min(nth == 0 ? 1u : nth, 16u));
        nth = (unsigned)std::min<int64_t>(nth, std::max(1, n_batches));
        std::atomic<int> next(0);
        auto work = [&]() {
            std::vector<int32_t> limg_of(n_imgs, -1);
            for (int b = next++; b < n_batches; b = next++) build_batch(b, limg_of);
        };
        std::vector<std::thread> pool;
        for (unsigned w = 1; w < nth; ++w) pool.emplace_back(work);
        work();
        for (auto& th : pool) th.join();
    }

    // Pass 3: concatenation in batch order
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
    bool list_overflow = false;
    // offsets of each batch in the concatenated arrays, then a parallel copy
    std::vector<int64_t> o_ch(n_batches + 1, 0), o_ct(n_batches + 1, 0), o_sl(n_batches + 1, 0), o_en(n_batches + 1, 0);
    for (int b = 0; b < n_batches; ++b) {
        o_ch[b + 1] = o_ch[b] + (int64_t)outs[b].chunk_meta.size() / 4;
        o_ct[b + 1] = o_ct[b] + (int64_t)outs[b].ct_pid.size();
        o_sl[b + 1] = o_sl[b] + (int64_t)outs[b].slot_pair.size();
        o_en[b + 1] = o_en[b] + (int64_t)outs[b].ents.size();
        list_overflow |= outs[b].overflow;
    }
    auto& slot_src = P->v[BA_PA_SLOT_SRC];
    auto& s_pid = P->v[BA_PA_S_PID];
    auto& s_img = P->v[BA_PA_S_IMG];
    chunk_obs.resize(o_ch[n_batches] * BA_CHUNK); slot_info.resize(o_ch[n_batches] * BA_CHUNK);
    slot_src.resize(o_ch[n_batches] * BA_CHUNK); s_pid.resize(o_ch[n_batches] * BA_CHUNK);
    s_img.resize(o_ch[n_batches] * BA_CHUNK);
    chunk_meta.resize(o_ch[n_batches] * 4); chunk_slots.resize(o_ch[n_batches] * BA_MAX_SLOTS);
    chunk_eptr.resize(o_ch[n_batches] + 1);
    chunk_eptr[o_ch[n_batches]] = (int32_t)(o_en[n_batches] / 4);
    for (auto* v : {&ct_pid, &ct_first, &ct_m, &ct_mask}) v->resize(o_ct[n_batches]);
    slot_pair.resize(o_sl[n_batches]);
    // the entries, and one chunk's worth of zero padding so that a full-capacity copy of the last
    // chunk's list stays inside the array
    chunk_ent.assign((size_t)(o_en[n_batches] + BA_LIST_CAP), 0);
    uint32_t* ents = reinterpret_cast<uint32_t*>(chunk_ent.data());
    b_pos_slot.resize((size_t)n_batches * BA_MAX_SLOTS);
    parallel_for(n_batches, [&](int64_t b0, int64_t b1) {
        for (int64_t b = b0; b < b1; ++b) {
            BatchOut& R = outs[b];
            const int32_t ct0 = (int32_t)o_ct[b], e4 = (int32_t)(o_en[b] / 4);
            std::copy(R.chunk_obs.begin(), R.chunk_obs.end(), chunk_obs.begin() + o_ch[b] * BA_CHUNK);
            for (size_t q = 0; q < R.chunk_obs.size(); ++q) {
                const int32_t o = R.chunk_obs[q];
                const size_t d = (size_t)o_ch[b] * BA_CHUNK + q;
                slot_src[d] = o >= 0 ? o : 0;
                s_pid[d] = o >= 0 ? pids[o] : 0;
                s_img[d] = o >= 0 ? img[o] : 0;
            }
            std::copy(R.slot_info.begin(), R.slot_info.end(), slot_info.begin() + o_ch[b] * BA_CHUNK);
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
    for (int b = 0; b <= n_batches; ++b) {
        b_chunk_ptr.push_back((int32_t)o_ch[b]);
        b_slot_ptr.push_back((int32_t)o_sl[b]);
    }
    for (int b = 0; b < n_batches; ++b) {
        for (int a = 0; a < max_local_imgs; ++a)
            b_imgs.push_back(a < (int)batches[b].imgs.size() ? batches[b].imgs[a] : -1);
        b_nimgs.push_back((int32_t)batches[b].imgs.size());
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
    if (list_overflow) {
        g_plan_err = "a chunk needs more than BA_LIST_CAP MFMA entries";
        delete P;
        return nullptr;
    }
    int64_t n_slots = (int64_t)slot_pair.size();
    std::vector<int64_t> keys(n_slots);
    std::vector<uint8_t> swapped(n_slots, 0);
    for (int b = 0; b < n_batches; ++b)
        for (int s = b_slot_ptr[b]; s < b_slot_ptr[b + 1]; ++s) {
            int a = slot_pair[s] & 0xff, c = (slot_pair[s] >> 8) & 0xff;
            int64_t i1 = b_imgs[(int64_t)b * max_local_imgs + a], i2 = b_imgs[(int64_t)b * max_local_imgs + c];
            if (i1 > i2) { std::swap(i1, i2); swapped[s] = 1; }
            keys[s] = i1 * n_imgs + i2;
        }
    std::vector<int64_t> perm(n_slots);
    std::iota(perm.begin(), perm.end(), 0);
    std::stable_sort(perm.begin(), perm.end(), [&](int64_t a, int64_t b) { return keys[a] < keys[b]; });
    auto& pair_i1 = P->v[BA_PA_PAIR_I1];
    auto& pair_i2 = P->v[BA_PA_PAIR_I2];
    auto& pair_ptr = P->v[BA_PA_PAIR_PTR];
    auto& pair_src = P->v[BA_PA_PAIR_SRC];
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
            for (int a = 0; a < b_nimgs[b]; ++a) cnt[b_imgs[(int64_t)b * max_local_imgs + a] + 1]++;
        for (int i = 0; i < n_imgs; ++i) cnt[i + 1] += cnt[i];
        img_ptr.assign(cnt.begin(), cnt.end());
        img_src.assign(cnt[n_imgs], 0);
        std::vector<int32_t> fill(cnt.begin(), cnt.end() - 1);
        for (int b = 0; b < n_batches; ++b)
            for (int a = 0; a < b_nimgs[b]; ++a)
                img_src[fill[b_imgs[(int64_t)b * max_local_imgs + a]]++] = b * max_local_imgs + a;
    }

    int64_t max_slots_used = 0, max_chunks = 0;
    for (int b = 0; b < n_batches; ++b) {
        max_slots_used = std::max<int64_t>(max_slots_used, b_slot_ptr[b + 1] - b_slot_ptr[b]);
        max_chunks = std::max<int64_t>(max_chunks, b_chunk_ptr[b + 1] - b_chunk_ptr[b]);
    }
    P->scalars[BA_PS_N_CHUNKS] = (int64_t)(chunk_meta.size() / 4);
    P->scalars[BA_PS_N_BATCHES] = n_batches;
    P->scalars[BA_PS_N_SLOTS] = n_slots;
    P->scalars[BA_PS_N_PAIRS] = n_pairs;
    P->scalars[BA_PS_N_CTRACKS] = (int64_t)ct_pid.size();
    P->scalars[BA_PS_L] = max_local_imgs;
    P->scalars[BA_PS_CHUNK] = BA_CHUNK;
    P->scalars[BA_PS_MAX_SLOTS_USED] = max_slots_used;
    P->scalars[BA_PS_MAX_CHUNKS_PER_BATCH] = max_chunks;
    int64_t ncov = 0;
    for (int t = 0; t < n_tracks; ++t) ncov += (int64_t)tdist[t] * (tdist[t] + 1) / 2;
    P->scalars[BA_PS_N_PAIR_TERMS] = ncov;
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
