"""Structure plan (host C++ in libba_hip.so, no GPU needed) and a CPU emulation of the
fused Schur data flow driven by the plan's metadata.

The emulation takes per-observation blocks from the oracle (fp64), accumulates
them exactly the way k_schur / k_pair_reduce route them (batch slots, local
orientation, transposition flags, deterministic CSR order) and must reproduce the
oracle's dense Schur complement: this pins the plan metadata independently of the
GPU arithmetic.
"""
import numpy as np
import pytest
import torch

from blast3r_amd.plan import ARRAYS, BAPlan
from blast3r_amd.synthetic import make_problem
from oracle import kernels as ok
from oracle import solver as osol
from oracle import engine as oeng
from tests.helpers import rel_err, opts


def _plan(p, **kw):
    return BAPlan(p.infos, p.pids, p.n_tracks, device='cpu', **kw)


@pytest.mark.parametrize('cfg,nf,nt,kw', [(0, 6, 60, {}), (0, 32, 3000, {}), (1, 40, 4000, {}), (2, 60, 6000, {}),
                                          (2, 60, 6000, dict(max_batch_obs=500)), (0, 12, 500, dict(max_slots=40))])
def test_plan_invariants(cfg, nf, nt, kw):
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    pl = _plan(p, **kw)
    h, sc = pl.host, pl.scalars
    CH = 128
    obs = h['chunk_obs']
    assert obs.size == sc['n_chunks'] * CH
    # every observation exactly once
    seen = np.sort(obs[obs >= 0])
    assert np.array_equal(seen, np.arange(p.n_obs))
    pids = p.pids.numpy()
    img = pl.obs_img
    meta = h['chunk_meta'].reshape(-1, 4)
    slot_pair = h['slot_pair']
    for ck in range(sc['n_chunks']):
        b, f, n, used = meta[ck]
        imgs = h['b_imgs'][b * pl.L:(b + 1) * pl.L]
        info = h['slot_info'][ck * CH:(ck + 1) * CH]
        o = obs[ck * CH:(ck + 1) * CH]
        assert np.all(o[used:] == -1) and np.all(o[:used] >= 0)
        covered = set()
        for t in range(n):
            first, m, pid, mask = h['ct_first'][f + t], h['ct_m'][f + t], h['ct_pid'][f + t], h['ct_mask'][f + t]
            tob = o[first:first + m]
            assert np.all(pids[tob] == pid)
            assert m == np.sum(pids == pid)                 # whole track inside one chunk
            li = info[first:first + m] & 0xff
            assert np.all(imgs[li] == img[tob])
            assert mask == np.bitwise_or.reduce(1 << li)
            assert np.all((info[first:first + m] >> 8) & 0xff == t)
            lead = info[first:first + m] >> 16
            assert np.all(img[o[lead]] == img[tob])        # leader shares the image
            ls = sorted(set(li.tolist()))
            covered |= {(min(x, y), max(x, y)) for x in ls for y in ls}
        slots = {(s & 0xff, (s >> 8) & 0xff) for s in slot_pair[h['b_slot_ptr'][b]:h['b_slot_ptr'][b + 1]]}
        assert covered <= slots
        assert len(slots) <= 96
    # every slot appears exactly once among the pair sources, with the right orientation flag
    src = h['pair_src']
    assert np.array_equal(np.sort(src >> 1), np.arange(sc['n_slots']))
    for q in range(sc['n_pairs']):
        i1, i2 = h['pair_i1'][q], h['pair_i2'][q]
        assert i1 <= i2
        for e in src[h['pair_ptr'][q]:h['pair_ptr'][q + 1]]:
            s = e >> 1
            b = np.searchsorted(h['b_slot_ptr'], s, side='right') - 1
            a, c = slot_pair[s] & 0xff, (slot_pair[s] >> 8) & 0xff
            ga, gc = h['b_imgs'][b * pl.L + a], h['b_imgs'][b * pl.L + c]
            assert (min(ga, gc), max(ga, gc)) == (i1, i2)
            assert (e & 1) == int(ga > gc)


@pytest.mark.parametrize('cfg,nf,nt,kw', [(0, 6, 60, {}), (0, 32, 3000, {}), (2, 60, 6000, {}),
                                          (0, 12, 500, dict(max_slots=40))])
def test_plan_mfma_entry_lists(cfg, nf, nt, kw):
    """The per-chunk MFMA entry lists equal an independent reconstruction from slot_info.  An entry
    holds the LDS offsets (in doubles) of its A rows and B rows, A | B << 16, with observation slot s
    at s * 97 (V rows) and s * 97 + 48 (J rows) and a zero block at 128 * 97.  Per off-diagonal
    slot (a, b): one V entry per covering chunk track (chunk-track order) joining the first
    observations of its runs in a and b; per diagonal slot (a, a): one J entry per observation in a
    (slot order), padded to a multiple of 4 with zero-block entries, then one V entry per (track,
    image) run in a (slot order); each list padded to a multiple of 4; at most BA_LIST_CAP (1536)
    entries per chunk.  The slot table word is offset | groups << 12 | J groups << 21."""
    BLK, JROW, CAP, MS = 97, 48, 1536, 96
    ZERO = 128 * BLK
    PAD = ZERO | ZERO << 16
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    pl = _plan(p, **kw)
    h = pl.host
    ents = h['chunk_ent'].view(np.uint32)
    meta = h['chunk_meta'].reshape(-1, 4)
    n_chunks = len(meta)
    assert len(h['chunk_eptr']) == n_chunks + 1
    assert ents.size >= 4 * int(h['chunk_eptr'][-1]) + CAP
    total_real = 0
    for ck in range(n_chunks):
        batch, first_ct, n_ct, used = meta[ck]
        info = h['slot_info'][ck * 128:(ck + 1) * 128]
        lead = {}
        for sidx in range(used):
            li, t, ld = info[sidx] & 0xff, (info[sidx] >> 8) & 0xff, info[sidx] >> 16
            lead.setdefault((t, li), ld)
            assert lead[(t, li)] == ld
        s0, s1 = h['b_slot_ptr'][batch], h['b_slot_ptr'][batch + 1]
        base = 4 * int(h['chunk_eptr'][ck])
        tab = h['chunk_slots'][ck * MS:(ck + 1) * MS]
        end = 0
        for q in range(MS):
            off, ng, njg = int(tab[q]) & 0xfff, (int(tab[q]) >> 12) & 0x1ff, (int(tab[q]) >> 21) & 0x3f
            if q >= s1 - s0:
                assert tab[q] == 0
                continue
            pq = h['slot_pair'][s0 + q]
            a, b = pq & 0xff, (pq >> 8) & 0xff
            want, n_real, want_njg = [], 0, 0
            if a != b:
                for t in range(n_ct):
                    if (t, a) in lead and (t, b) in lead:
                        want.append(lead[(t, a)] * BLK | (lead[(t, b)] * BLK) << 16)
                n_real = len(want)
            else:
                js = [sidx * BLK + JROW for sidx in range(used) if info[sidx] & 0xff == a]
                want += [o | o << 16 for o in js]
                want += [PAD] * (-len(want) % 4)
                want_njg = len(want) // 4
                vs = [sidx * BLK for sidx in range(used) if info[sidx] & 0xff == a and info[sidx] >> 16 == sidx]
                want += [o | o << 16 for o in vs]
                n_real = len(js) + len(vs)
            total_real += n_real
            want += [PAD] * (-len(want) % 4)
            assert 4 * ng == len(want) and njg == want_njg
            assert off == end
            assert np.array_equal(ents[base + off:base + off + 4 * ng], np.array(want, dtype=np.uint32))
            end += 4 * ng
        assert end <= CAP
        # the kernel copies the chunk's list up to the next chunk's first entry
        assert end <= 4 * int(h['chunk_eptr'][ck + 1] - h['chunk_eptr'][ck])
    # every pair term and every observation once: sum over tracks of m(m+1)/2 plus n_obs
    assert total_real == pl.scalars['n_pair_terms'] + p.n_obs
    # kernel places: every batch slot at exactly one place, at most 6 places used per wave (16 waves)
    pos = h['b_pos_slot'].reshape(-1, MS)
    for b in range(len(pos)):
        ns = h['b_slot_ptr'][b + 1] - h['b_slot_ptr'][b]
        used = pos[b][pos[b] >= 0]
        assert np.array_equal(np.sort(used), np.arange(ns))
        per_wave = np.bincount(np.nonzero(pos[b] >= 0)[0] % 16, minlength=16)
        assert per_wave.max() <= 6


def test_plan_dispatch_order():
    """b_order is a permutation of the batches, most expensive first: greedy list scheduling of the
    batches (one per machine at a time, as the Schur kernel's workgroups on the CUs) in that order
    finishes no later than in plan order, by chunk count, on several machine counts."""
    import heapq
    p = make_problem(2, n_frames=400, n_tracks=120000)
    pl = _plan(p)
    h = pl.host
    nb = pl.scalars['n_batches']
    order = h['b_order']
    assert np.array_equal(np.sort(order), np.arange(nb))
    cost = np.diff(h['b_chunk_ptr']).astype(np.float64)
    assert cost[order[0]] >= np.percentile(cost, 90)

    def makespan(seq, m):
        heap = [0.0] * m
        for b in seq:
            heapq.heappush(heap, heapq.heappop(heap) + cost[b])
        return max(heap)

    for m in (nb // 8, nb // 4, nb // 3):
        assert makespan(order, m) <= makespan(np.arange(nb), m)


def test_plan_errors():
    p = make_problem(0, n_frames=8, n_tracks=50)
    with pytest.raises(RuntimeError, match='max_local_imgs'):
        BAPlan(p.infos, p.pids, p.n_tracks, device='cpu', max_local_imgs=2)
    bad = p.pids.clone()
    bad[0] = p.n_tracks + 3
    with pytest.raises(RuntimeError, match='pid out of range'):
        BAPlan(p.infos, bad, p.n_tracks, device='cpu')


def _batch_tracks(pl):
    """Per batch, its tracks in plan order (the chunks of a batch pack a contiguous run of the track order)."""
    h = pl.host
    meta = h['chunk_meta'].reshape(-1, 4)
    bcp = h['b_chunk_ptr']
    out = []
    for b in range(pl.scalars['n_batches']):
        c0, c1 = bcp[b], bcp[b + 1]
        out.append(h['ct_pid'][meta[c0, 1]:meta[c1 - 1, 1] + meta[c1 - 1, 2]])
    return out


@pytest.mark.parametrize('cfg,nf,nt,kw', [(2, 150, 120000, {}), (1, 120, 100000, {}),
                                          (2, 150, 120000, dict(max_batch_obs=3000)),
                                          (2, 150, 120000, dict(max_local_imgs=13, max_slots=80))])
def test_plan_batches_follow_the_greedy_rule(cfg, nf, nt, kw):
    """Each batch is the longest run of the track order, from where the previous one ended, within the
    limits (images, pair slots, observations): checked against the rule itself, at sizes where the planner
    cuts the order into segments planned in parallel and then joins them."""
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    pl = _plan(p, **kw)
    L, max_slots, mbo = kw.get('max_local_imgs', 16), kw.get('max_slots', 96), kw.get('max_batch_obs', 0)
    pids = p.pids.numpy()
    img = pl.obs_img
    srt = np.lexsort((img, pids))
    bounds = np.searchsorted(pids[srt], np.arange(p.n_tracks + 1))
    timgs = [np.unique(img[srt[bounds[t]:bounds[t + 1]]]) for t in range(p.n_tracks)]
    m = np.diff(bounds)
    batches = _batch_tracks(pl)
    assert sum(len(b) for b in batches) == int((m > 0).sum())
    assert pl.scalars['n_batches'] > 40
    for b, tr in enumerate(batches):
        imgs, pairs, nobs = set(), set(), 0
        for t in tr:
            imgs.update(timgs[t].tolist())
            ti = timgs[t]
            pairs.update(zip(*[a.ravel().tolist() for a in np.meshgrid(ti, ti)]))
            nobs += m[t]
        pairs = {(x, y) for x, y in pairs if x <= y}
        assert len(imgs) <= L and len(pairs) <= max_slots and (mbo <= 0 or nobs <= mbo or len(tr) == 1)
        if b + 1 < len(batches):            # the next track would break a limit
            t = batches[b + 1][0]
            ti = timgs[t]
            imgs2 = imgs | set(ti.tolist())
            pairs2 = pairs | {(x, y) for x in ti.tolist() for y in ti.tolist() if x <= y}
            assert len(imgs2) > L or len(pairs2) > max_slots or (mbo > 0 and nobs + m[t] > mbo)


def test_plan_errors_at_size():
    """The limits' errors at a size where the greedy runs in segments: a track whose pairs exceed
    max_slots (every segment meets one), and a track longer than a chunk."""
    p = make_problem(2, n_frames=150, n_tracks=120000)
    with pytest.raises(RuntimeError, match='a single track needs more pair slots than max_slots'):
        BAPlan(p.infos, p.pids, p.n_tracks, device='cpu', max_slots=60)
    pids = p.pids.clone()
    cnt = torch.diff(torch.cat([torch.zeros(1, dtype=torch.long), p.infos[0].long()]))
    # one track observed 4 times in each of the first 40 images: 160 observations
    long_track = torch.arange(40).repeat_interleave(4)
    keep_img = torch.repeat_interleave(torch.arange(len(cnt)), cnt)
    new_pids = torch.cat([torch.full((160,), p.n_tracks, dtype=pids.dtype), pids])
    new_img = torch.cat([long_track, keep_img])
    o = torch.argsort(new_img, stable=True)
    cnt2 = torch.bincount(new_img, minlength=len(cnt))
    infos = p.infos.clone()
    infos[0] = torch.cumsum(cnt2, 0).to(infos.dtype)
    with pytest.raises(RuntimeError, match='more observations than one chunk holds'):
        BAPlan(infos, new_pids[o].contiguous(), p.n_tracks + 1, device='cpu')


def _chol3(H, lam, jit=1e-12):
    """chol3x3 rules (.cu:560-634) on a (T,3,3) batch, returns lower factors."""
    A = H + (lam + jit) * torch.eye(3, dtype=H.dtype)
    return torch.linalg.cholesky(A)


@pytest.mark.parametrize('cfg,nf,nt', [(0, 6, 60), (0, 10, 300), (2, 30, 600)])
def test_schur_emulation_matches_oracle(cfg, nf, nt):
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    o = opts(p)
    loss, res, w = oeng.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                  p.pix2d_std, p.pix2d_dep, True, o['weight_z'], 1.0, o['clip_pix_err'],
                                  o['huber_delta'])
    Jc8, Jz, Jp = ok.jacobians_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids,
                                         p.pix2d_std, p.pix2d_dep, True, float64=True)
    prob = osol.Problem(p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks, p.C)
    ne, gvec, params = osol.build_normal_equations(prob, Jc8, Jz, Jp, res, w)
    S_ref = osol.dense_schur(ne)

    C = p.C
    d = 8 + C
    N = p.n_obs
    W = w.clamp(1e-6, 1e6)
    sW = torch.sqrt(W).double()
    Jc = torch.zeros((N, 3, d), dtype=torch.float64)
    Jc[:, :, :8] = Jc8
    Jc[:, 2, 8:] = Jz[:, 0]
    Jc = Jc * sW[:, :, None]
    Jpw = Jp * sW[:, :, None]
    H = torch.zeros((p.n_tracks, 3, 3), dtype=torch.float64)
    H.index_add_(0, p.pids.long(), Jpw.transpose(1, 2) @ Jpw)
    lam = 1e-12 * H.diagonal(dim1=-1, dim2=-2).abs().max()
    Lf = _chol3(H, lam)
    Hcp = Jc.transpose(1, 2) @ Jpw                                      # (N, d, 3)
    V = torch.linalg.solve_triangular(Lf[p.pids.long()], Hcp.transpose(1, 2), upper=False).transpose(1, 2)

    pl = _plan(p)
    h, sc = pl.host, pl.scalars
    partial = np.zeros((sc['n_slots'], d, d))
    obs = h['chunk_obs']
    meta = h['chunk_meta'].reshape(-1, 4)
    Vn, Jn = V.numpy(), Jc.numpy()
    for b in range(sc['n_batches']):
        s0, s1 = h['b_slot_ptr'][b], h['b_slot_ptr'][b + 1]
        for ck in range(h['b_chunk_ptr'][b], h['b_chunk_ptr'][b + 1]):
            _, f, n, used = meta[ck]
            info = h['slot_info'][ck * 128:(ck + 1) * 128]
            ob = obs[ck * 128:(ck + 1) * 128]
            for s in range(s0, s1):
                a, c = h['slot_pair'][s] & 0xff, (h['slot_pair'][s] >> 8) & 0xff
                for t in range(n):
                    mask = h['ct_mask'][f + t]
                    if not ((mask >> a) & 1 and (mask >> c) & 1):
                        continue
                    first, m = h['ct_first'][f + t], h['ct_m'][f + t]
                    li = info[first:first + m] & 0xff
                    Va = Vn[ob[first:first + m][li == a]].sum(0)
                    Vc = Vn[ob[first:first + m][li == c]].sum(0)
                    partial[s] -= Va @ Vc.T
                if a == c:
                    sel = ob[(np.arange(128) < used) & ((info & 0xff) == a)]
                    partial[s] += np.einsum('nri,nrj->ij', Jn[sel], Jn[sel])
    S_pairs = np.zeros((sc['n_pairs'], d, d))
    for q in range(sc['n_pairs']):
        for e in h['pair_src'][h['pair_ptr'][q]:h['pair_ptr'][q + 1]]:
            S_pairs[q] += partial[e >> 1].T if (e & 1) else partial[e >> 1]
    # image-level -> reference unknown order (mono focal, no rigs)
    nf_, nt_ = 2 * len(p.K), 6 * len(p.P_w2rig)
    cam, node = p.infos[2].long().numpy(), p.infos[1].long().numpy()
    n_c = nf_ + nt_ + C * p.n_imgs
    um = np.zeros((p.n_imgs, d), dtype=np.int64)
    for i in range(p.n_imgs):
        um[i, :2] = cam[i] * 2 + np.arange(2)
        um[i, 2:8] = nf_ + node[i] * 6 + np.arange(6)
        um[i, 8:] = nf_ + nt_ + i * C + np.arange(C)
    S = np.zeros((n_c, n_c))
    for q in range(sc['n_pairs']):
        i1, i2 = h['pair_i1'][q], h['pair_i2'][q]
        np.add.at(S, (um[i1][:, None], um[i2][None, :]), S_pairs[q])
        if i1 != i2:
            np.add.at(S, (um[i2][:, None], um[i1][None, :]), S_pairs[q].T)
    dg = np.diag(S_ref.numpy() - S)        # the damping is the only remaining difference
    Sd = torch.from_numpy(S) + torch.diag(torch.from_numpy(dg))
    assert rel_err(Sd, S_ref) < 1e-10
    # the difference is a per-leaf constant 1e-12 * max|diag(H_cc leaf)|
    for name, sl in (('foc', slice(0, nf_)), ('tau', slice(nf_, nf_ + nt_)), ('zcf', slice(nf_ + nt_, n_c))):
        leaf = ne.leaves[name]
        lam_leaf = float(leaf.diagonal(dim1=-1, dim2=-2).abs().max()) * 1e-12
        assert np.allclose(dg[sl], lam_leaf, rtol=1e-2, atol=0)   # rounding noise ~1e-16 * |S_ii|


def test_host_mask_for_device_observations_raises():
    """A mask tensor on another device than the observations raises RuntimeError before any launch
    (the kernels would read it at its address on their own device; the reference's indexing at
    ba_solver.py:98 raises for it too), except an all-False mask, which the reference turns into the
    zero matrix first (ba_solver.py:91-92).  A host tensor handed to a kernel argument raises."""
    from blast3r_amd import _lib
    from blast3r_amd.ba_solver import _flag
    dev = torch.device('cuda:0')
    with pytest.raises(RuntimeError, match='optim_P'):
        _flag(torch.tensor([True, False, True]), 'optim_P', 3, dev)
    assert _flag(torch.tensor([False, False, False]), 'optim_P', 3, dev) == (False, None, None)
    en, mask, idx = _flag(torch.tensor([True, False, True]), 'optim_P', 3, torch.device('cpu'))
    assert en and mask.dtype == torch.uint8 and idx.tolist() == [0, 2]
    with pytest.raises(ValueError):
        _flag(torch.tensor([1, 0, 1]), 'optim_P', 3, dev)
    with pytest.raises(RuntimeError, match='device tensor'):
        _lib.ptr(torch.zeros(4))
    assert _lib.ptr(None) is None


# ------------------------------------------------------------------ pair-major plan
def _pm_brute(cum, pids, n_tracks):
    """The pair-major structure restated with Python dicts: runs = (image, track) groups in image
    order then track order, observations in their original order inside a run."""
    n_imgs = len(cum)
    img = np.repeat(np.arange(n_imgs), np.diff(np.concatenate([[0], cum])))
    runs = {}
    for o in range(len(pids)):
        runs.setdefault((int(img[o]), int(pids[o])), []).append(o)
    keys = sorted(runs)
    rid = {k: r for r, k in enumerate(keys)}
    trk_runs = {t: [rid[k] for k in keys if k[1] == t] for t in range(n_tracks)}
    pairs = sorted({(i, i) for i, _ in keys} |
                   {(keys[a][0], keys[b][0]) for t in range(n_tracks) for a in trk_runs[t] for b in trk_runs[t]
                    if keys[a][0] < keys[b][0]})
    terms = {q: [(a, b) for t in range(n_tracks) for a in trk_runs[t] for b in trk_runs[t]
                 if (keys[a][0], keys[b][0]) == q] for q in pairs if q[0] != q[1]}
    return img, keys, runs, trk_runs, pairs, terms


@pytest.mark.parametrize('case', ['cfg0', 'dups', 'long', 'empty_imgs'])
def test_pm_plan_matches_brute_force(case):
    from blast3r_amd.plan import PMPlan
    rng = np.random.default_rng(7)
    if case == 'cfg0':
        p = make_problem(0, n_frames=8, n_tracks=60)
        cum, pids, T = p.infos[0].numpy(), p.pids.numpy(), p.n_tracks
        infos = p.infos
    else:
        n_imgs, T = (12, 40) if case != 'long' else (30, 10)
        counts = rng.integers(0, 25, n_imgs) if case == 'empty_imgs' else rng.integers(5, 25, n_imgs)
        if case == 'empty_imgs':
            counts[[0, 4, 11]] = 0
        cum = np.cumsum(counts).astype(np.int32)
        pids = rng.integers(0, T, int(cum[-1])).astype(np.int32)     # repeats inside an image: runs of >1
        infos = torch.stack([torch.from_numpy(cum), torch.arange(n_imgs, dtype=torch.int32),
                             torch.zeros(n_imgs, dtype=torch.int32)])
    pl = PMPlan(infos, torch.from_numpy(np.asarray(pids, dtype=np.int32)), T, device='cpu')
    h, sc = pl.host, pl.scalars
    img, keys, runs, trk_runs, pairs, terms = _pm_brute(np.asarray(cum), np.asarray(pids), T)
    n_runs = len(keys)
    assert sc['n_runs'] == n_runs and sc['n_pairs'] == len(pairs)
    assert np.array_equal(h['obs_img'], img)
    assert np.array_equal(h['run_trk'], [k[1] for k in keys]) and np.array_equal(h['run_img'], [k[0] for k in keys])
    for r, k in enumerate(keys):
        assert h['run_obs'][h['run_ptr'][r]:h['run_ptr'][r + 1]].tolist() == runs[k]
    assert h['run_ptr'][-1] == len(pids)
    for i in range(len(cum)):
        assert h['img_run_ptr'][i + 1] - h['img_run_ptr'][i] == sum(k[0] == i for k in keys)
    for t in range(T):
        assert h['trk_run'][h['trk_run_ptr'][t]:h['trk_run_ptr'][t + 1]].tolist() == trk_runs[t]
        assert h['trk_obs'][h['trk_obs_ptr'][t]:h['trk_obs_ptr'][t + 1]].tolist() == \
            [o for r in trk_runs[t] for o in runs[keys[r]]]
    assert sc['max_track_runs'] == max(len(v) for v in trk_runs.values())
    assert list(zip(h['pair_i1'].tolist(), h['pair_i2'].tolist())) == pairs
    for i in range(len(cum)):
        dp = h['diag_pair'][i]
        assert (dp == pairs.index((i, i))) if (i, i) in pairs else dp == -1
    n_terms = 0
    for q, pr in enumerate(pairs):
        tt = h['term'][2 * h['term_ptr'][q]:2 * h['term_ptr'][q + 1]].reshape(-1, 2)
        if pr[0] == pr[1]:
            assert len(tt) == 0
        else:
            assert [tuple(x) for x in tt.tolist()] == terms[pr]
            n_terms += len(tt)
    assert sc['n_terms'] == n_terms
    # rows: every pair once in the row of each of its images, the transposed flag on the second image
    for i in range(len(cum)):
        ent = h['row_ent'][h['row_ptr'][i]:h['row_ptr'][i + 1]]
        want = [(q << 1) | int(pr[0] != i) for q, pr in enumerate(pairs) if i in pr]
        assert ent.tolist() == want
    # schedule: pairs by (smallest first image, largest last image) over the tracks of their terms, then
    # pair id; pairs without terms (every diagonal pair) last, in pair order
    F = len(cum)
    t_imgs = {t: [keys[r][0] for r in rs] for t, rs in trk_runs.items() if rs}
    sched_key = []
    for q, pr in enumerate(pairs):
        tr = [keys[ra][1] for ra, _ in terms.get(pr, [])] if pr[0] != pr[1] else []
        lo = min((min(t_imgs[t]) for t in tr), default=F)
        hi = max((max(t_imgs[t]) for t in tr), default=F)
        sched_key.append((lo, hi, q))
    assert h['pair_sched'].tolist() == [q for _, _, q in sorted(sched_key)]


def test_pm_plan_errors():
    from blast3r_amd.plan import PMPlan
    p = make_problem(0, n_frames=8, n_tracks=50)
    bad = p.pids.clone()
    bad[0] = p.n_tracks + 3
    with pytest.raises(RuntimeError, match='pid out of range'):
        PMPlan(p.infos, bad, p.n_tracks, device='cpu')
    inf = p.infos.clone()
    inf[0, -1] += 1
    with pytest.raises(RuntimeError, match='number of observations'):
        PMPlan(inf, p.pids, p.n_tracks, device='cpu')


@pytest.mark.parametrize('cfg,nf,nt,wide', [(2, 60, 800, False), (1, 64, 800, False), (3, 512, 3000, True)])
def test_span_profile_median_track_span(cfg, nf, nt, wide):
    """SpanProfile (the path choice of path='auto' before any batched plan is built): the lower median over
    the observed tracks of last - first + 1 image, against a brute-force count; banded and retrieval
    neighbourhoods stay within two batches (32 images), random neighbours of a 512-frame collection do not."""
    from blast3r_amd.plan import SpanProfile, get_plan
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    cum = p.infos[0].numpy().astype(np.int64)
    img = np.repeat(np.arange(len(cum)), np.diff(np.concatenate([[0], cum])))
    pids = p.pids.numpy()
    spans = []
    for t in range(p.n_tracks):
        im = img[pids == t]
        if len(im):
            spans.append(int(im.max() - im.min() + 1))
    spans.sort()
    expect = spans[(len(spans) - 1) // 2]
    sp = SpanProfile(p.infos, p.pids, p.n_tracks)
    assert sp.median_span == expect
    assert (sp.median_span > 32) == wide
    # cached per structure like the plans, and not counted against the plan cache's size
    assert get_plan(p.infos, p.pids, p.n_tracks, kind='span') is get_plan(p.infos, p.pids, p.n_tracks, kind='span')


@pytest.mark.parametrize('cfg,nf,nt,kw', [(0, 6, 60, {}), (2, 30, 200, dict(track_len=(20, 30))),
                                          (4, 12, 150, dict(n_channels=16))])
def test_pm_schur_emulation_matches_oracle(cfg, nf, nt, kw):
    """The pair-major data flow (per-run V = sum of the run's J_c^T J_p times L^-T, per-image
    diagonal blocks from the J rows and the runs' V, per-pair blocks from the term lists) on the
    oracle's per-observation blocks reproduces the oracle's dense Schur complement."""
    from blast3r_amd.plan import PMPlan
    p = make_problem(cfg, n_frames=nf, n_tracks=nt, **kw)
    o = opts(p)
    loss, res, w = oeng.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                  p.pix2d_std, p.pix2d_dep, True, o['weight_z'], 1.0, o['clip_pix_err'],
                                  o['huber_delta'])
    Jc8, Jz, Jp = ok.jacobians_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids,
                                         p.pix2d_std, p.pix2d_dep, True, float64=True)
    fl = {k: False for k in ('optim_K', 'optim_P') if not p.options.get(k, True)}
    prob = osol.Problem(p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks, p.C)
    ne, gvec, params = osol.build_normal_equations(prob, Jc8, Jz, Jp, res, w, **fl)
    S_ref = osol.dense_schur(ne)
    C = p.C
    hasK, hasP = 'optim_K' not in fl, 'optim_P' not in fl
    cols = ([0, 1] if hasK else []) + (list(range(2, 8)) if hasP else [])
    d = len(cols) + C
    N = p.n_obs
    sW = torch.sqrt(w.clamp(1e-6, 1e6)).double()
    Jc = torch.zeros((N, 3, d), dtype=torch.float64)
    Jc[:, :, :len(cols)] = Jc8[:, :, cols]
    Jc[:, 2, len(cols):] = Jz[:, 0]
    Jc = Jc * sW[:, :, None]
    Jpw = Jp * sW[:, :, None]
    H = torch.zeros((p.n_tracks, 3, 3), dtype=torch.float64)
    H.index_add_(0, p.pids.long(), Jpw.transpose(1, 2) @ Jpw)
    lam = 1e-12 * H.diagonal(dim1=-1, dim2=-2).abs().max()
    Lf = _chol3(H, lam)
    pl = PMPlan(p.infos, p.pids, p.n_tracks, device='cpu')
    h, sc = pl.host, pl.scalars
    Jn = Jc.numpy()
    Hcp = (Jc.transpose(1, 2) @ Jpw).numpy()                                # (N, d, 3)
    Vr = np.zeros((sc['n_runs'], d, 3))
    for r in range(sc['n_runs']):
        ob = h['run_obs'][h['run_ptr'][r]:h['run_ptr'][r + 1]]
        Lt = Lf[h['run_trk'][r]].numpy()
        Vr[r] = np.linalg.solve(Lt, Hcp[ob].sum(0).T).T                      # (sum J_c^T J_p) L^-T
    S_pairs = np.zeros((sc['n_pairs'], d, d))
    for i in range(p.n_imgs):
        q = h['diag_pair'][i]
        if q < 0:
            continue
        r0, r1 = h['img_run_ptr'][i], h['img_run_ptr'][i + 1]
        ob = h['run_obs'][h['run_ptr'][r0]:h['run_ptr'][r1]]
        S_pairs[q] = np.einsum('nri,nrj->ij', Jn[ob], Jn[ob]) - np.einsum('rik,rjk->ij', Vr[r0:r1], Vr[r0:r1])
    for q in range(sc['n_pairs']):
        for a, b in h['term'][2 * h['term_ptr'][q]:2 * h['term_ptr'][q + 1]].reshape(-1, 2):
            S_pairs[q] -= Vr[a] @ Vr[b].T
    nf_, nt_ = 2 * len(p.K), 6 * len(p.P_w2rig)        # a switched-off leaf keeps its (zero) columns
    cam, node = p.infos[2].long().numpy(), p.infos[1].long().numpy()
    n_c = nf_ + nt_ + C * p.n_imgs
    um = np.zeros((p.n_imgs, d), dtype=np.int64)
    for i in range(p.n_imgs):
        c = 0
        if hasK:
            um[i, :2] = cam[i] * 2 + np.arange(2); c = 2
        if hasP:
            um[i, c:c + 6] = nf_ + node[i] * 6 + np.arange(6); c += 6
        um[i, c:] = nf_ + nt_ + i * C + np.arange(C)
    S = np.zeros((n_c, n_c))
    for q in range(sc['n_pairs']):
        i1, i2 = h['pair_i1'][q], h['pair_i2'][q]
        np.add.at(S, (um[i1][:, None], um[i2][None, :]), S_pairs[q])
        if i1 != i2:
            np.add.at(S, (um[i2][:, None], um[i1][None, :]), S_pairs[q].T)
    S_ref = S_ref.clone()
    assert S.shape == tuple(S_ref.shape)
    dg = np.diag(S_ref.numpy() - S).copy()
    assert rel_err(torch.from_numpy(S) + torch.diag(torch.from_numpy(dg)), S_ref) < 1e-10
    on = np.concatenate([np.full(nf_, hasK), np.full(nt_, hasP), np.ones(C * p.n_imgs, bool)])
    assert np.all(np.abs(dg[on]) <= 1e-9 * np.abs(np.diag(S_ref.numpy())).max())   # only the 1e-12 damping differs


def _online_steps(p, steps):
    """The structures an online pipeline builds with `old | new` (tracks.py:84-102) from problem p:
    S_k holds the tracks whose last image is <= k, numbered by (last image, id), and within an image the
    rows of earlier steps come first, so S_k = S_(k-1) | (the tracks ending at image k).  Yields
    (infos, pids, n_tracks, add_cnt, add_pids) for k = n_imgs - steps .. n_imgs - 1 (add_* None first)."""
    cum = p.infos[0].numpy().astype(np.int64)
    n_imgs = len(cum)
    obs_img = np.repeat(np.arange(n_imgs), np.diff(np.concatenate([[0], cum])))
    pids = p.pids.numpy().astype(np.int64)
    T = p.n_tracks
    tmax = np.full(T, -1)
    np.maximum.at(tmax, pids, obs_img)
    rank = np.empty(T, dtype=np.int64)
    rank[np.lexsort((np.arange(T), tmax))] = np.arange(T)
    prev = None
    for k in range(n_imgs - steps, n_imgs):
        sel = tmax[pids] <= k
        oi, pp, tm = obs_img[sel], rank[pids[sel]], tmax[pids[sel]]
        o = np.lexsort((np.arange(len(oi)), tm, oi))
        nppi = np.bincount(oi, minlength=k + 1)
        infos = torch.stack([torch.from_numpy(np.cumsum(nppi)), torch.arange(k + 1), torch.zeros(k + 1, dtype=torch.long)])
        pk = torch.from_numpy(pp[o].astype(np.int32))
        Tk = int((tmax <= k).sum())
        add = None
        if prev is not None:
            old_cnt = np.concatenate([prev[0], [0]])
            starts = np.concatenate([[0], np.cumsum(nppi)[:-1]])
            add_pids = np.concatenate([pp[o][starts[i] + old_cnt[i]: starts[i] + nppi[i]] for i in range(k + 1)])
            add = (nppi - old_cnt, add_pids)
        yield infos.to(torch.int32), pk, Tk, add
        prev = (nppi, Tk)


@pytest.mark.parametrize('cfg,nf,nt,steps,kw', [(2, 30, 1500, 6, {}), (0, 12, 400, 5, {}), (4, 20, 800, 5, {}),
                                                (2, 40, 2500, 4, dict(max_batch_obs=400)),
                                                (1, 40, 4000, 4, {}), (0, 6, 200, 5, dict(max_slots=40))])
def test_plan_append_equals_full_rebuild(cfg, nf, nt, steps, kw):
    """BAPlan.appended (ba_plan_append: `old | new` planned from the old structure's plan, only the batches
    from the first new track's place on planned again) equals a full BAPlan of the merged structure, every
    array and scalar, byte for byte, over a chain of appends; and reuses the old arrays' prefix."""
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    plan = None
    kept = []
    for infos, pk, Tk, add in _online_steps(p, steps):
        full = BAPlan(infos, pk, Tk, device='cpu', **kw)
        if plan is None:
            plan = full
            continue
        child = BAPlan.appended(plan, infos, pk, Tk, add[0], add[1])
        assert not plan.appendable and child.appendable
        assert child.scalars == full.scalars
        for name in full.sizes:
            assert child.sizes[name] == full.sizes[name], name
            assert torch.equal(child.dev[name], full.dev[name]), name
            assert np.array_equal(child.host[name], full.host[name]), name
        kept.append(child.stable_prefix['chunk_ent'] / max(1, full.sizes['chunk_ent']))
        plan = child
    print(f'cfg {cfg}: fraction of MFMA entries kept per append {np.round(kept, 3)}')


def test_plan_append_rejects_non_appends():
    """An appended id below the old track count, or an image count that is not one more, is refused and
    leaves the parent plan appendable (the caller then plans the structure in full)."""
    p = make_problem(2, n_frames=20, n_tracks=800)
    steps = list(_online_steps(p, 2))
    parent = BAPlan(*steps[0][:3], device='cpu')
    infos, pk, Tk, (add_cnt, add_pids) = steps[1]
    bad = add_pids.copy()
    bad[0] = 0
    with pytest.raises(RuntimeError, match='appended pid out of range'):
        BAPlan.appended(parent, infos, pk, Tk, add_cnt, bad)
    with pytest.raises(RuntimeError, match='not an append'):
        BAPlan.appended(parent, infos[:, :-1], pk, Tk, add_cnt[:-1], add_pids)
    assert parent.appendable
    child = BAPlan.appended(parent, infos, pk, Tk, add_cnt, add_pids)
    full = BAPlan(infos, pk, Tk, device='cpu')
    assert all(torch.equal(child.dev[n], full.dev[n]) for n in full.sizes)


@pytest.mark.parametrize('cfg,nf,nt,steps', [(2, 40, 2500, 6), (4, 24, 1200, 5), (0, 12, 400, 4)])
def test_plan_append_chain_equals_full_rebuild(cfg, nf, nt, steps):
    """BAPlan.appended_chain: several `old | new` in a row planned at once from the first structure's plan
    (as when the solver runs only every few merges) equals a full plan of the last structure, every array and
    scalar; the device copy keeps the shortest stable prefix of the chain, ids shifted by the summed shifts."""
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    seq = list(_online_steps(p, steps))
    parent = BAPlan(*seq[0][:3], device='cpu')
    links = [(add[0], add[1], Tk) for _, _, Tk, add in seq[1:]]
    infos, pk, Tk, _ = seq[-1]
    child = BAPlan.appended_chain(parent, infos, pk, Tk, links)
    full = BAPlan(infos, pk, Tk, device='cpu')
    assert child.scalars == full.scalars
    for name in full.sizes:
        assert torch.equal(child.dev[name], full.dev[name]), name
    assert child.stable_prefix['chunk_ent'] > 0 or cfg == 0


@pytest.mark.parametrize('plan_first', [True, False])
def test_lineage_plans_merges_from_a_dropped_parent(plan_first):
    """The solver-side path of `old | new` (tracks.py:84-102): note_append records each merge, every structure
    but the last is dropped as a pipeline does (`trk = trk | new`), and get_plan of the last one is made from the
    plan of the first (planned before the merges, or after the first merge while it is still alive) through the
    recorded lineage; it equals a full plan, and the consumed plan is let go."""
    import gc
    from blast3r_amd import plan as bp
    p = make_problem(4, n_frames=24, n_tracks=1200)
    seq = [(i, pk.clone(), T, a) for i, pk, T, a in _online_steps(p, 4)]
    infos0, prev_pids, prev_T, _ = seq[0]
    seq[0] = None
    if plan_first:
        bp.get_plan(infos0, prev_pids, prev_T, device=torch.device('cpu'))
    for j in range(1, len(seq)):
        infos, pk, Tk, add = seq[j]
        seq[j] = None
        bp.note_append(pk, prev_pids, prev_T, torch.from_numpy(add[0]), torch.from_numpy(add[1] - prev_T), Tk)
        if j == 1 and not plan_first:
            bp.get_plan(infos0, prev_pids, prev_T, device=torch.device('cpu'))
        prev_pids, prev_T = pk, Tk
        del pk
        gc.collect()
    rec = bp._lineage[id(prev_pids)]
    assert rec.depth == len(seq) - 1
    plan = bp.get_plan(infos, prev_pids, Tk, device=torch.device('cpu'))
    assert plan.stable_prefix is not None, 'the chain was planned in full'
    full = BAPlan(infos, prev_pids, Tk, device='cpu')
    assert plan.scalars == full.scalars
    for name in full.sizes:
        assert torch.equal(plan.dev[name], full.dev[name]), name
    r = rec
    while r is not None:
        assert not r.plans
        r = r.parent


def test_plan_append_from_two_threads_consumes_the_parent_once():
    """Two threads appending to one parent plan at once: one append consumes the parent's host plan and
    equals a full rebuild, the other is refused with a RuntimeError (it never touches the consumed plan)."""
    import threading
    p = make_problem(2, n_frames=30, n_tracks=1500)
    seq = list(_online_steps(p, 2))
    parent = BAPlan(*seq[0][:3], device='cpu')
    infos, pk, Tk, add = seq[1]
    out, errs = [], []
    gate = threading.Barrier(2)

    def run():
        gate.wait()
        try:
            out.append(BAPlan.appended(parent, infos, pk, Tk, add[0], add[1]))
        except RuntimeError as e:
            errs.append(str(e))
    ts = [threading.Thread(target=run) for _ in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert len(out) == 1 and len(errs) == 1 and 'already appended' in errs[0]
    full = BAPlan(infos, pk, Tk, device='cpu')
    for name in full.sizes:
        assert torch.equal(out[0].dev[name], full.dev[name]), name


def _append_one_track(infos, pids, T, imgs):
    """The structure `old | new` where new holds one track (id T) seen once in each of `imgs` (image ids of
    the merged structure, which has one image more than `infos`): merged infos and pids, add_cnt, add_pids."""
    cum = infos[0].numpy().astype(np.int64)
    n = len(cum)
    cnt_old = np.diff(np.concatenate([[0], cum]))
    add_cnt = np.zeros(n + 1, dtype=np.int32)
    add_cnt[list(imgs)] = 1
    rows, start = [], 0
    p = pids.numpy()
    for i in range(n + 1):
        c = int(cnt_old[i]) if i < n else 0
        rows.append(p[start:start + c])
        start += c
        rows.append(np.full(add_cnt[i], T, dtype=np.int32))
    nppi = np.concatenate([cnt_old, [0]]) + add_cnt
    new_infos = torch.stack([torch.from_numpy(np.cumsum(nppi)), torch.arange(n + 1), torch.zeros(n + 1, dtype=torch.long)])
    new_pids = torch.from_numpy(np.concatenate(rows).astype(np.int32))
    return new_infos.to(torch.int32), new_pids, T + 1, add_cnt, np.full(len(imgs), T, dtype=np.int32)


@pytest.mark.parametrize('cfg,span,kw', [(0, 10, dict(max_slots=40)), (2, 14, {})])
def test_failing_append_leaves_the_parent_plan_as_it_was(cfg, span, kw):
    """An append whose new track needs more pair slots than max_slots (10 images: 55 > 40; 14 images at the
    defaults: 105 > 96) is refused before the parent's host plan is touched: the parent stays appendable, its
    arrays equal a fresh plan of its structure, a valid append from it afterwards equals a full rebuild, and
    dropping every plan frees each host plan once."""
    import gc
    p = make_problem(cfg, n_frames=20, n_tracks=800)
    steps = list(_online_steps(p, 2))
    infos0, pk0, T0 = steps[0][:3]
    parent = BAPlan(infos0, pk0, T0, device='cpu', **kw)
    n0 = parent.n_imgs
    imgs = list(range(n0 + 1 - span, n0 + 1))
    infos_b, pids_b, T_b, add_cnt, add_pids = _append_one_track(infos0, pk0, T0, imgs)
    with pytest.raises(RuntimeError, match='pair slots'):
        BAPlan.appended(parent, infos_b, pids_b, T_b, add_cnt, add_pids)
    assert parent.appendable
    fresh = BAPlan(infos0, pk0, T0, device='cpu', **kw)
    assert parent.scalars == fresh.scalars
    for name in fresh.sizes:
        assert np.array_equal(parent._host_view(ARRAYS.index(name), fresh.sizes[name]), fresh.host[name]), name
    infos, pk, Tk, add = steps[1]
    child = BAPlan.appended(parent, infos, pk, Tk, add[0], add[1])
    full = BAPlan(infos, pk, Tk, device='cpu', **kw)
    assert child.scalars == full.scalars
    for name in full.sizes:
        assert torch.equal(child.dev[name], full.dev[name]), name
        assert np.array_equal(child.host[name], full.host[name]), name
    del parent, child, full, fresh
    gc.collect()


def test_host_arrays_read_during_an_append_of_the_plan():
    """A reader of a plan's host arrays (plan.host[...], as the solver's PCG and direct-solve set-up do)
    while another thread appends to that plan: every read equals the plan's own arrays, whether it runs
    before the append took the host plan (read from it under the append lock) or after (read from the
    device arrays, which an append leaves alone)."""
    import threading
    from blast3r_amd import plan as bp
    p = make_problem(2, n_frames=30, n_tracks=1500)
    seq = list(_online_steps(p, 2))
    parent = BAPlan(*seq[0][:3], device='cpu')
    ref = {name: parent.dev[name][:parent.sizes[name]].numpy().copy() for name in ARRAYS}
    infos, pk, Tk, add = seq[1]
    stop = threading.Event()
    bad, reads = [], [0]

    def reader():
        while not stop.is_set():
            h = bp._HostArrays(parent)
            for name in ARRAYS:
                if not np.array_equal(h[name], ref[name]):
                    bad.append(name)
            reads[0] += 1

    t = threading.Thread(target=reader)
    t.start()
    child = BAPlan.appended(parent, infos, pk, Tk, add[0], add[1])
    for _ in range(3):           # a few reads after the parent's host plan is gone
        n = reads[0]
        while reads[0] == n:
            pass
    stop.set()
    t.join()
    assert not bad, bad
    full = BAPlan(infos, pk, Tk, device='cpu')
    for name in full.sizes:
        assert torch.equal(child.dev[name], full.dev[name]), name
