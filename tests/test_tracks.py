"""ObservedTracks structure edits (tracks.py:19-127): oracle pins on the CPU, then the device
operations of blast3r_amd.data against the oracle, bit-exact (integer and copied fp32 data)."""
import pytest
import torch

import oracle.tracks as otr
from blast3r_amd.data import ObservedTracks

DEV = 'cuda'


def _random_set(seed, n_imgs, n_tracks, C=5, empty=(), max_per_img=40):
    """Image-major set; a track is seen at most once per image (as a real track)."""
    g = torch.Generator().manual_seed(seed)
    nppi, pids = [], []
    for i in range(n_imgs):
        m = 0 if i in empty else int(torch.randint(1, min(max_per_img, n_tracks) + 1, (1,), generator=g))
        pids.append(torch.randperm(n_tracks, generator=g)[:m].to(torch.int32))
        nppi.append(m)
    pids = torch.cat(pids) if pids else torch.zeros(0, dtype=torch.int32)
    n = len(pids)
    return (torch.tensor(nppi, dtype=torch.int32), pids, torch.rand((n, 2), generator=g) * 500,
            torch.rand((n, 2), generator=g) + 0.5, torch.randn((n, C), generator=g))


# ----------------------------------------------------------------------------- oracle pins (CPU)
def test_oracle_img_id_closed_form_and_empty_images():
    nppi = torch.tensor([3, 1, 4, 2], dtype=torch.int32)
    assert torch.equal(otr.img_id(nppi, 10), torch.repeat_interleave(torch.arange(4), nppi.long()))
    # an empty image: its delimiter coincides with the next one and counts once (known answer)
    assert otr.img_id(torch.tensor([2, 0, 3], dtype=torch.int32), 5).tolist() == [0, 0, 1, 1, 1]


def test_oracle_merge_is_side_by_side_in_dense_form():
    old = _random_set(1, 5, 30)
    new = _random_set(2, 6, 20)
    m = otr.merge(old, 30, new)
    assert m[0].tolist() == [int(a) + int(b) for a, b in zip(old[0].tolist() + [0], new[0].tolist())]
    dense = otr.to_dense(m, 50)
    ref = torch.cat([otr.to_dense(old, 30, n_imgs=6), otr.to_dense(new, 20)], dim=0)
    assert torch.equal(torch.nan_to_num(dense, nan=-1.0), torch.nan_to_num(ref, nan=-1.0))
    # rows of image j: the old rows first, then the new ones (pid >= 30)
    sl = otr.img_slices(m[0])
    for j in range(6):
        p = m[1][sl[j]]
        k = int(old[0][j]) if j < 5 else 0
        assert bool((p[:k] < 30).all()) and bool((p[k:] >= 30).all())


def test_oracle_remove_is_a_column_selection_of_the_dense_form():
    obs = _random_set(3, 7, 40, empty=(2,))
    bad = torch.tensor([5, 5, 17, 39, 99])                   # repeats and an id matching no row
    (nppi, pids, pix, std, dep), keep = otr.remove(obs, bad)
    present = torch.unique(obs[1])
    expect = present[~torch.isin(present, bad)]
    assert torch.equal(keep.long(), expect.long())
    d0 = otr.to_dense(obs, 40)
    d1 = otr.to_dense((nppi, pids, pix, std, dep), len(keep))
    assert torch.equal(torch.nan_to_num(d1, nan=-1.0), torch.nan_to_num(d0[keep.long()], nan=-1.0))
    assert int(nppi.sum()) == len(pids) and int(nppi[2]) == 0


def test_oracle_select_matches_one_image_views():
    obs = _random_set(4, 6, 25, empty=(1,))
    idx = torch.tensor([4, 1, 4, 0])
    s = otr.select(obs, idx)
    sl = otr.img_slices(obs[0])
    for k in range(1, 5):
        assert torch.equal(s[k], torch.cat([obs[k][sl[int(i)]] for i in idx]))
    assert s[0].tolist() == [int(obs[0][int(i)]) for i in idx]


# ----------------------------------------------------------------------------- device vs oracle
def _dev_tracks(obs, n_tracks):
    nppi, pids, pix, std, dep = obs
    return ObservedTracks(len(nppi), n_tracks, nppi.to(DEV), pids.to(DEV), pix.to(DEV), std.to(DEV), dep.to(DEV),
                          'log_multidepth')


def _same(t, obs):
    for got, ref in zip((t.nppi, t.pids, t.pix2d, t.pix2d_std, t.pix2d_dep), obs):
        assert got.dtype == ref.dtype and torch.equal(got.cpu(), ref), (got.dtype, ref.dtype)


@pytest.mark.gpu
@pytest.mark.parametrize('seed,n_old,T_old,T_new,empty', [(10, 5, 30, 20, ()), (11, 9, 200, 150, (0, 3)),
                                                          (12, 1, 8, 8, ())])
def test_merge_matches_oracle(seed, n_old, T_old, T_new, empty):
    old = _random_set(seed, n_old, T_old, empty=empty)
    new = _random_set(seed + 100, n_old + 1, T_new, empty=empty)
    got = _dev_tracks(old, T_old) | _dev_tracks(new, T_new)
    assert got.n_imgs == n_old + 1 and got.n_tracks == T_old + T_new
    _same(got, otr.merge(old, T_old, new))
    assert (None | got) is got


@pytest.mark.gpu
def test_merge_with_no_old_tracks_returns_new():
    new = _dev_tracks(_random_set(13, 4, 10), 10)
    old = _dev_tracks((torch.zeros(3, dtype=torch.int32), torch.zeros(0, dtype=torch.int32), torch.zeros((0, 2)),
                       torch.zeros((0, 2)), torch.zeros((0, 5))), 0)
    assert (old | new) is new


@pytest.mark.gpu
@pytest.mark.parametrize('bad_kind', ['int64', 'int32', 'tuple', 'all_but_one'])
def test_remove_matches_oracle(bad_kind):
    obs = _random_set(20, 8, 60, empty=(5,))
    if bad_kind == 'all_but_one':
        bad = torch.arange(1, 60)
    else:
        bad = torch.tensor([3, 3, 59, 0, 1000, -4])
    ref, keep_r = otr.remove(obs, bad)
    arg = {'int64': bad, 'int32': bad.to(torch.int32), 'tuple': tuple(bad.tolist()),
           'all_but_one': bad.to(DEV)}[bad_kind]
    t, keep = _dev_tracks(obs, 60).remove(arg)
    assert t.n_tracks == len(keep_r)
    assert keep.dtype == keep_r.dtype and torch.equal(keep.cpu(), keep_r)
    _same(t, ref)


@pytest.mark.gpu
def test_remove_nothing_and_everything():
    obs = _random_set(21, 4, 12)
    t0 = _dev_tracks(obs, 12)
    same, keep = t0.remove(())
    assert same is t0 and keep.shape == (0,)
    t, keep = t0.remove(torch.arange(12))
    assert t.n_tracks == 0 and t.n_kpts == 0 and keep.numel() == 0 and t.nppi.tolist() == [0, 0, 0, 0]


@pytest.mark.gpu
def test_select_to_dense_img_id_match_oracle():
    obs = _random_set(30, 7, 50, empty=(2, 3))
    t = _dev_tracks(obs, 50)
    idx = torch.tensor([6, 2, 0, 6, 4])
    s = t[idx.to(DEV)]
    _same(s, otr.select(obs, idx))
    v = t[4]                                                    # one-image view
    sl = otr.img_slices(obs[0])[4]
    assert v.n_imgs == 1 and torch.equal(v.pids.cpu(), obs[1][sl])
    for n_imgs in (None, 9):
        d = t.to_dense(n_imgs)
        r = otr.to_dense(obs, 50, n_imgs)
        assert d.shape == r.shape and torch.equal(torch.nan_to_num(d.cpu(), nan=-7.0), torch.nan_to_num(r, nan=-7.0))
    iid = t.img_id
    assert iid.dtype == torch.int64 and torch.equal(iid.cpu(), otr.img_id(obs[0], len(obs[1])).to(torch.int64))


@pytest.mark.gpu
def test_merge_at_pipeline_size():
    """Merge at config-2 scale (8M rows kept, one new image) against the per-image slices."""
    g = torch.Generator(device=DEV).manual_seed(5)
    n_imgs, T = 1024, 1_000_000
    nppi = torch.randint(7000, 8600, (n_imgs,), device=DEV, dtype=torch.int32)
    n = int(nppi.sum())
    old = ObservedTracks(n_imgs, T, nppi, torch.randint(0, T, (n,), device=DEV, dtype=torch.int32, generator=g),
                         torch.rand((n, 2), device=DEV, generator=g), torch.rand((n, 2), device=DEV, generator=g),
                         torch.rand((n, 5), device=DEV, generator=g), 'log_multidepth')
    nppi_n = torch.zeros(n_imgs + 1, dtype=torch.int32, device=DEV)
    nppi_n[-12:] = 500
    m = int(nppi_n.sum())
    new = ObservedTracks(n_imgs + 1, 1000, nppi_n, torch.randint(0, 1000, (m,), device=DEV, dtype=torch.int32,
                                                                generator=g),
                         torch.rand((m, 2), device=DEV, generator=g), torch.rand((m, 2), device=DEV, generator=g),
                         torch.rand((m, 5), device=DEV, generator=g), 'log_multidepth')
    got = old | new
    for j in (0, 511, n_imgs - 12, n_imgs - 1, n_imgs):
        so = old.img_slices[j] if j < n_imgs else slice(0, 0)
        sn = new.img_slices[j]
        sg = got.img_slices[j]
        assert torch.equal(got.pids[sg], torch.cat([old.pids[so], new.pids[sn] + T]))
        assert torch.equal(got.pix2d_dep[sg], torch.cat([old.pix2d_dep[so], new.pix2d_dep[sn]]))
    assert torch.equal(got.nppi[:-1], nppi + nppi_n[:-1])


@pytest.mark.gpu
def test_merge_then_plan_is_an_append_equal_to_a_full_plan():
    """`old | new` records its lineage; the solver's plan for the merged structure is then made from the old
    structure's cached plan by ba_plan_append (only the batches from the first new track on planned again),
    and equals a full plan of the merged structure on every device array, bit for bit; an LM step on the
    merged structure gives the same result on either plan."""
    import numpy as np
    from blast3r_amd import engine, plan as bplan
    from blast3r_amd.plan import BAPlan, get_plan
    from blast3r_amd.synthetic import make_problem
    p = make_problem(2, n_frames=40, n_tracks=2500)
    n = p.n_imgs
    cum = p.infos[0].numpy().astype(np.int64)
    obs_img = np.repeat(np.arange(n), np.diff(np.concatenate([[0], cum])))
    pids = p.pids.numpy().astype(np.int64)
    T = p.n_tracks
    tmax = np.full(T, -1)
    np.maximum.at(tmax, pids, obs_img)
    rank = np.empty(T, dtype=np.int64)
    rank[np.lexsort((np.arange(T), tmax))] = np.arange(T)
    T_old = int((tmax < n - 1).sum())
    # old: the tracks ending before the last image, over images 0 .. n-2; new: the others, over all images
    def part(sel, n_imgs, shift, n_tracks):
        oi = obs_img[sel]
        o = np.lexsort((np.arange(len(oi)), oi))
        idx = torch.from_numpy(np.nonzero(sel)[0][o])
        nppi = torch.from_numpy(np.bincount(oi, minlength=n_imgs).astype(np.int32))
        return ObservedTracks(n_imgs, n_tracks, nppi.to(DEV),
                              torch.from_numpy((rank[pids[idx.numpy()]] - shift).astype(np.int32)).to(DEV),
                              p.pix2d[idx].to(DEV), p.pix2d_std[idx].to(DEV), p.pix2d_dep[idx].to(DEV), 'log_multidepth')
    old = part(tmax[pids] < n - 1, n - 1, 0, T_old)
    new = part(tmax[pids] == n - 1, n, T_old, T - T_old)
    merged = old | new
    assert merged.n_tracks == T

    def infos_of(trk, k):
        return torch.stack([torch.cumsum(trk.nppi.long(), 0), p.infos[1, :k].to(DEV).long(),
                            p.infos[2, :k].to(DEV).long()]).to(torch.int32)
    inf_old, inf_new = infos_of(old, n - 1), infos_of(merged, n)
    get_plan(inf_old, old.pids, old.n_tracks, device=torch.device(DEV))
    plan_new = get_plan(inf_new, merged.pids, merged.n_tracks, device=torch.device(DEV))
    assert plan_new.stable_prefix is not None, 'the merged structure was planned in full'
    full = BAPlan(inf_new, merged.pids, merged.n_tracks, device=DEV)
    for name in full.sizes:
        assert torch.equal(plan_new.dev[name], full.dev[name]), name
    assert plan_new.scalars == full.scalars
    kept = plan_new.stable_prefix['chunk_ent'] / full.sizes['chunk_ent']
    print(f'appended plan: {kept:.3f} of the MFMA entries kept', flush=True)

    pts3d = torch.empty_like(p.pts3d)
    pts3d[torch.from_numpy(rank)] = p.pts3d
    o = p.options
    inp = dict(rigs=inf_new, pids=merged.pids, pix2d=merged.pix2d, pix2d_std=merged.pix2d_std,
               pix2d_dep=merged.pix2d_dep, K=p.K.to(DEV), P_rig2cam=p.P_rig2cam.to(DEV), P_w2rig=p.P_w2rig.to(DEV),
               z_coefs=p.z_coefs.to(DEV), pts3d=pts3d.to(DEV))
    kw = dict(dtype=torch.float64,
              weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, optim_K=o['optim_K'],
              optim_P=o['optim_P'])
    up_a, st_a = engine.lm_step(**inp, **kw)
    bplan._cache.clear()
    up_f, st_f = engine.lm_step(**inp, **kw)
    assert float(st_a.new_loss) == float(st_f.new_loss)
    for k in up_a:
        assert torch.equal(up_a[k], up_f[k]), k


@pytest.mark.gpu
def test_chain_of_merges_is_planned_from_the_last_planned_structure():
    """Three `old | new` in a row with no plan in between (the solver runs every few frames): the plan of the
    last structure is made from the first one's cached plan through the recorded lineage, and equals a full
    plan on every device array."""
    import numpy as np
    from blast3r_amd.plan import BAPlan, get_plan
    from blast3r_amd.synthetic import make_problem
    p = make_problem(4, n_frames=24, n_tracks=1200)
    n = p.n_imgs
    cum = p.infos[0].numpy().astype(np.int64)
    obs_img = np.repeat(np.arange(n), np.diff(np.concatenate([[0], cum])))
    pids = p.pids.numpy().astype(np.int64)
    T = p.n_tracks
    tmax = np.full(T, -1)
    np.maximum.at(tmax, pids, obs_img)
    rank = np.empty(T, dtype=np.int64)
    rank[np.lexsort((np.arange(T), tmax))] = np.arange(T)

    def part(sel, n_imgs, shift, n_tracks):
        oi = obs_img[sel]
        o = np.lexsort((np.arange(len(oi)), oi))
        idx = torch.from_numpy(np.nonzero(sel)[0][o])
        nppi = torch.from_numpy(np.bincount(oi, minlength=n_imgs).astype(np.int32))
        return ObservedTracks(n_imgs, n_tracks, nppi.to(DEV),
                              torch.from_numpy((rank[pids[idx.numpy()]] - shift).astype(np.int32)).to(DEV),
                              p.pix2d[idx].to(DEV), p.pix2d_std[idx].to(DEV), p.pix2d_dep[idx].to(DEV), 'log_multidepth')

    def infos_of(trk, k):
        return torch.stack([torch.cumsum(trk.nppi.long(), 0), p.infos[1, :k].to(DEV).long(),
                            p.infos[2, :k].to(DEV).long()]).to(torch.int32)
    k0 = n - 4
    T0 = int((tmax <= k0).sum())
    cur = part(tmax[pids] <= k0, k0 + 1, 0, T0)
    get_plan(infos_of(cur, k0 + 1), cur.pids, cur.n_tracks, device=torch.device(DEV))
    for k in range(k0 + 1, n):
        Tk = int((tmax <= k).sum())
        cur = cur | part(tmax[pids] == k, k + 1, cur.n_tracks, Tk - cur.n_tracks)
    inf = infos_of(cur, n)
    plan = get_plan(inf, cur.pids, cur.n_tracks, device=torch.device(DEV))
    assert plan.stable_prefix is not None, 'the chain was planned in full'
    full = BAPlan(inf, cur.pids, cur.n_tracks, device=DEV)
    assert plan.scalars == full.scalars
    for name in full.sizes:
        assert torch.equal(plan.dev[name], full.dev[name]), name
