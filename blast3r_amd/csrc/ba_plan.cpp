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
#include <cstdint>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "ba_plan.h"

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

extern "C" const char* ba_plan_last_error(void) { return g_plan_err.c_str(); }

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

    // observation -> image, and per-track observation lists sorted by (image, obs)
    std::vector<int32_t> img(n_obs);
    for (int i = 0, o = 0; i < n_imgs; ++i)
        for (; o < cum_nkpts[i]; ++o) img[o] = i;
    std::vector<int64_t> tptr(n_tracks + 1, 0);
    for (int64_t o = 0; o < n_obs; ++o) {
        int32_t t = pids[o];
        if (t < 0 || t >= n_tracks) { g_plan_err = "pid out of range"; delete P; return nullptr; }
        tptr[t + 1]++;
    }
    for (int t = 0; t < n_tracks; ++t) tptr[t + 1] += tptr[t];
    std::vector<int32_t> tobs(n_obs);
    {
        std::vector<int64_t> fill(tptr.begin(), tptr.end() - 1);
        for (int64_t o = 0; o < n_obs; ++o) tobs[fill[pids[o]]++] = (int32_t)o;   // image-major input: already sorted by image
    }
    // distinct images per track
    std::vector<int32_t> tmin(n_tracks, INT32_MAX), tmax(n_tracks, -1), tdist(n_tracks, 0);
    for (int t = 0; t < n_tracks; ++t) {
        int last = -1;
        for (int64_t k = tptr[t]; k < tptr[t + 1]; ++k) {
            int i = img[tobs[k]];
            if (i != last) { tdist[t]++; last = i; }
            tmin[t] = std::min(tmin[t], i);
            tmax[t] = std::max(tmax[t], i);
        }
        int64_t m = tptr[t + 1] - tptr[t];
        if (m > BA_CHUNK) { g_plan_err = "a track has more observations than one chunk holds (" + std::to_string(BA_CHUNK) + ")"; delete P; return nullptr; }
        if (tdist[t] > max_local_imgs) {
            g_plan_err = "a track spans more images (" + std::to_string(tdist[t]) + ") than max_local_imgs (" +
                         std::to_string(max_local_imgs) + ")";
            delete P; return nullptr;
        }
    }
    std::vector<int32_t> order;
    order.reserve(n_tracks);
    for (int t = 0; t < n_tracks; ++t) if (tptr[t + 1] > tptr[t]) order.push_back(t);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        if (tmin[a] != tmin[b]) return tmin[a] < tmin[b];
        if (tmax[a] != tmax[b]) return tmax[a] < tmax[b];
        return a < b;
    });

    // ------------------------------------------------------------ greedy batching
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
    auto& chunk_ent = P->v[BA_PA_CHUNK_ENT];      // 16-bit entries, two per word
    auto& chunk_eptr = P->v[BA_PA_CHUNK_EPTR];    // n_chunks
    auto& b_pos_slot = P->v[BA_PA_B_POS_SLOT];    // n_batches * BA_MAX_SLOTS
    std::vector<uint16_t> ents;                   // all chunks' entries (packed into chunk_ent at the end)
    bool list_overflow = false;

    std::vector<int32_t> cur_imgs;
    std::vector<uint8_t> cur_pairs((size_t)max_local_imgs * max_local_imgs, 0);
    int cur_nslots = 0;
    int64_t cur_obs = 0;
    std::vector<int32_t> cur_tracks;
    std::vector<int32_t> limg_of(n_imgs, -1);

    auto flush_batch = [&]() {
        if (cur_tracks.empty()) return;
        int batch = (int)b_nimgs.size();
        // local pair slots in (b, a) order
        int slot0 = (int)slot_pair.size();
        for (int b = 0; b < (int)cur_imgs.size(); ++b)
            for (int a = 0; a <= b; ++a)
                if (cur_pairs[a * max_local_imgs + b]) slot_pair.push_back(a | (b << 8));
        b_slot_ptr.push_back((int32_t)slot_pair.size());
        // chunks: pack tracks in order
        int ch_first_track = 0;
        size_t k = 0;
        while (k < cur_tracks.size()) {
            int used = 0;
            int ntr = 0;
            int chunk = (int)(chunk_meta.size() / 4);
            size_t base = chunk_obs.size();
            chunk_obs.resize(base + BA_CHUNK, -1);
            slot_info.resize(base + BA_CHUNK, -1);
            int first_ct = (int)ct_pid.size();
            while (k < cur_tracks.size()) {
                int t = cur_tracks[k];
                int m = (int)(tptr[t + 1] - tptr[t]);
                if (used + m > BA_CHUNK || ntr == BA_MAX_CT) break;
                uint32_t mask = 0;
                int last_img = -1, leader = -1;
                for (int j = 0; j < m; ++j) {
                    int o = tobs[tptr[t] + j];
                    int li = limg_of[img[o]];
                    if (img[o] != last_img) { leader = used + j; last_img = img[o]; }
                    mask |= 1u << li;
                    chunk_obs[base + used + j] = o;
                    slot_info[base + used + j] = li | (ntr << 8) | (leader << 16);
                }
                ct_pid.push_back(t);
                ct_first.push_back(used);
                ct_m.push_back(m);
                ct_mask.push_back((int32_t)mask);
                used += m;
                ntr++;
                k++;
            }
            chunk_meta.push_back(batch);
            chunk_meta.push_back(first_ct);
            chunk_meta.push_back(ntr);
            chunk_meta.push_back(used);
            (void)chunk; (void)ch_first_track;

            // MFMA entry lists of the chunk, slot by slot: an off-diagonal slot (a, b) pairs the
            // first observation of each covering track in a with the one in b (chunk-track order);
            // a diagonal slot (a, a) lists the J rows of every observation in a (slot order), then
            // the V rows of the first observation of each (track, image) run in a (slot order)
            {
                std::vector<int16_t> lead((size_t)ntr * BA_MAX_LOCAL, -1);
                for (int sidx = 0; sidx < used; ++sidx) {
                    const int inf = slot_info[base + sidx];
                    lead[(size_t)((inf >> 8) & 0xff) * BA_MAX_LOCAL + (inf & 0xff)] = (int16_t)(inf >> 16);
                }
                const size_t e0 = ents.size();
                chunk_eptr.push_back((int32_t)(e0 / 8));
                const int nsl = (int)slot_pair.size() - slot0;
                for (int q = 0; q < BA_MAX_SLOTS; ++q) {
                    if (q >= nsl) { chunk_slots.push_back(0); continue; }
                    const int a = slot_pair[slot0 + q] & 0xff, bq = (slot_pair[slot0 + q] >> 8) & 0xff;
                    const size_t off = ents.size() - e0;
                    auto ent = [&](int sa, int sb, int kind) {
                        ents.push_back((uint16_t)(sa | (sb << 7) | (kind << 14)));
                    };
                    if (a != bq) {
                        for (int tt = 0; tt < ntr; ++tt) {
                            const int la_ = lead[(size_t)tt * BA_MAX_LOCAL + a], lb_ = lead[(size_t)tt * BA_MAX_LOCAL + bq];
                            if (la_ >= 0 && lb_ >= 0) ent(la_, lb_, BA_ENT_V);
                        }
                    } else {
                        for (int sidx = 0; sidx < used; ++sidx)
                            if ((slot_info[base + sidx] & 0xff) == a) ent(sidx, sidx, BA_ENT_J);
                        for (int sidx = 0; sidx < used; ++sidx) {
                            const int inf = slot_info[base + sidx];
                            if ((inf & 0xff) == a && (inf >> 16) == sidx) ent(sidx, sidx, BA_ENT_V);
                        }
                    }
                    while ((ents.size() - e0 - off) % 4) ent(0, 0, BA_ENT_PAD);
                    const size_t len = ents.size() - e0 - off;
                    chunk_slots.push_back((int32_t)(off | (len << 16)));
                }
                if (ents.size() - e0 > BA_LIST_CAP) list_overflow = true;
                while ((ents.size() - e0) % 8) ents.push_back(0);
            }
        }
        b_chunk_ptr.push_back((int32_t)(chunk_meta.size() / 4));
        // place the batch's slots on the Schur kernel's waves (place wave + BA_WAVES * k, at most
        // BA_SLOTS_PER_WAVE per wave).  The MFMA phase of a chunk lasts as long as its busiest SIMD
        // (BA_WAVES / 4 waves share one MFMA pipe) and its busiest wave, so slots are taken by
        // decreasing total work and each goes where the summed per-chunk maxima grow least.
        {
            const int nsl = (int)slot_pair.size() - slot0;
            const int c0 = b_chunk_ptr[b_chunk_ptr.size() - 2], nc = b_chunk_ptr.back() - c0;
            std::vector<int32_t> wk((size_t)nc * nsl);                  // MFMAs of (chunk, slot)
            std::vector<int64_t> tot(nsl, 0);
            for (int c = 0; c < nc; ++c)
                for (int q = 0; q < nsl; ++q) {
                    const int len = chunk_slots[(size_t)(c0 + c) * BA_MAX_SLOTS + q] >> 16;
                    wk[(size_t)c * nsl + q] = 3 * (len / 4);
                    tot[q] += wk[(size_t)c * nsl + q];
                }
            std::vector<int> order(nsl);
            std::iota(order.begin(), order.end(), 0);
            std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return tot[x] > tot[y]; });
            constexpr int NS = 4, WPS = BA_WAVES / NS;
            std::vector<int64_t> ls((size_t)nc * NS, 0), lw((size_t)nc * BA_WAVES, 0), ms(nc, 0), mw(nc, 0);
            int cnt[BA_WAVES] = {0};
            const size_t pbase = b_pos_slot.size();
            b_pos_slot.resize(pbase + BA_MAX_SLOTS, -1);
            for (int q : order) {
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
                b_pos_slot[pbase + best + BA_WAVES * cnt[best]] = q;
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
            (void)WPS;
        }
        for (int a = 0; a < max_local_imgs; ++a)
            b_imgs.push_back(a < (int)cur_imgs.size() ? cur_imgs[a] : -1);
        b_nimgs.push_back((int32_t)cur_imgs.size());
        for (int i : cur_imgs) limg_of[i] = -1;
        cur_imgs.clear();
        std::fill(cur_pairs.begin(), cur_pairs.end(), 0);
        cur_nslots = 0;
        cur_obs = 0;
        cur_tracks.clear();
    };

    b_chunk_ptr.push_back(0);
    b_slot_ptr.push_back(0);
    std::vector<int32_t> timgs;
    for (int t : order) {
        timgs.clear();
        for (int64_t k = tptr[t]; k < tptr[t + 1]; ++k) {
            int i = img[tobs[k]];
            if (timgs.empty() || timgs.back() != i) timgs.push_back(i);
        }
        int m = (int)(tptr[t + 1] - tptr[t]);
        for (int attempt = 0; attempt < 2; ++attempt) {
            // new images and new pairs this track would add
            int new_imgs = 0;
            for (int i : timgs) if (limg_of[i] < 0) new_imgs++;
            bool ok = (int)cur_imgs.size() + new_imgs <= max_local_imgs &&
                      (max_batch_obs <= 0 || cur_obs + m <= max_batch_obs || cur_tracks.empty());
            int add_slots = 0;
            if (ok) {
                // count pairs not yet touched (images not yet local get provisional ids)
                int prov = (int)cur_imgs.size();
                std::vector<int> li(timgs.size());
                for (size_t q = 0; q < timgs.size(); ++q) li[q] = limg_of[timgs[q]] >= 0 ? limg_of[timgs[q]] : prov++;
                for (size_t p = 0; p < li.size(); ++p)
                    for (size_t q = p; q < li.size(); ++q) {
                        int a = std::min(li[p], li[q]), b = std::max(li[p], li[q]);
                        if (a >= (int)cur_imgs.size() || b >= (int)cur_imgs.size() || !cur_pairs[a * max_local_imgs + b]) add_slots++;
                    }
                ok = cur_nslots + add_slots <= max_slots;
            }
            if (!ok) {
                if (cur_tracks.empty()) {
                    g_plan_err = "a single track needs more pair slots than max_slots";
                    delete P; return nullptr;
                }
                flush_batch();
                continue;
            }
            for (int i : timgs) if (limg_of[i] < 0) { limg_of[i] = (int)cur_imgs.size(); cur_imgs.push_back(i); }
            for (size_t p = 0; p < timgs.size(); ++p)
                for (size_t q = p; q < timgs.size(); ++q) {
                    int a = std::min(limg_of[timgs[p]], limg_of[timgs[q]]);
                    int b = std::max(limg_of[timgs[p]], limg_of[timgs[q]]);
                    if (!cur_pairs[a * max_local_imgs + b]) { cur_pairs[a * max_local_imgs + b] = 1; cur_nslots++; }
                }
            cur_obs += m;
            cur_tracks.push_back(t);
            break;
        }
    }
    flush_batch();

    // ------------------------------------------------------------ global pairs
    int n_batches = (int)b_nimgs.size();
    if (list_overflow) {
        g_plan_err = "a chunk needs more than BA_LIST_CAP MFMA entries";
        delete P;
        return nullptr;
    }
    // two entries per word, and one chunk's worth of padding so that a full-capacity copy of the
    // last chunk's list stays inside the array
    ents.resize(ents.size() + BA_LIST_CAP, 0);
    if (ents.size() % 2) ents.push_back(0);
    chunk_ent.resize(ents.size() / 2);
    std::memcpy(chunk_ent.data(), ents.data(), ents.size() * sizeof(uint16_t));
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
