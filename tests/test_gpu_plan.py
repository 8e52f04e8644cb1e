"""GPU: the pair-major structure plan built on the device (ba_pm_dplan_create) against the host planner
(ba_pm_plan_create), array for array, on the benchmark structures and on hand-made edge cases."""
import time

import numpy as np
import pytest
import torch

from blast3r_amd.plan import PM_ARRAYS, PMPlan
from blast3r_amd.synthetic import make_problem

pytestmark = pytest.mark.gpu
DEV = 'cuda:0'


def _both(infos, pids, n_tracks):
    host = PMPlan(infos, pids, n_tracks, device='cpu')
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dv = PMPlan(infos.to(DEV), pids.to(DEV), n_tracks, device=DEV)
    torch.cuda.synchronize()
    return host, dv, time.perf_counter() - t0


def _assert_equal(host, dv):
    assert dv.scalars == host.scalars, (dv.scalars, host.scalars)
    for name in PM_ARRAYS:
        a, b = dv.host[name], host.host[name]
        assert a.shape == b.shape and np.array_equal(a, b), name
        assert torch.equal(dv.dev[name][:dv.sizes[name]].cpu(), torch.from_numpy(b)), name


@pytest.mark.parametrize('cfg,nf,nt,kw', [(0, 6, 60, {}), (0, 32, 2000, {}), (1, 32, 400, {}), (2, 24, 800, {}),
                                          (3, 24, 600, {}), (4, 12, 300, {}), (2, 40, 300, dict(track_len=(20, 30)))])
def test_device_pairmajor_plan_equals_the_host_plan(cfg, nf, nt, kw):
    """Runs, the tracks' runs and observations, the image pairs with their terms and the image rows: the
    device planner's arrays and scalars equal the host planner's on every configuration."""
    p = make_problem(cfg, n_frames=nf, n_tracks=nt, **kw)
    host, dv, _ = _both(p.infos, p.pids, p.n_tracks)
    _assert_equal(host, dv)


def test_device_pairmajor_plan_edge_structures():
    """Images without observations (first, middle, last), a track with no observation, several observations
    of one track in one image (runs longer than one observation, rows not sorted by track id), and a
    single image: the device planner equals the host planner."""
    rng = np.random.default_rng(5)
    nppi = np.array([0, 7, 0, 0, 12, 5, 9, 0])
    n = int(nppi.sum())
    T = 9                                      # track 8 is never observed
    pids = rng.integers(0, 8, n).astype(np.int32)
    pids[1:4] = pids[0]                        # one track three times in image 1
    infos = torch.stack([torch.from_numpy(np.cumsum(nppi)), torch.arange(len(nppi)), torch.zeros(len(nppi), dtype=torch.long)])
    host, dv, _ = _both(infos.to(torch.int32), torch.from_numpy(pids), T)
    _assert_equal(host, dv)
    assert host.scalars['n_runs'] < n
    one = torch.tensor([[4], [0], [0]], dtype=torch.int32)
    host, dv, _ = _both(one, torch.tensor([2, 0, 2, 1], dtype=torch.int32), 3)
    _assert_equal(host, dv)
    assert dv.scalars['n_terms'] == 0 and dv.scalars['n_pairs'] == 1


def test_device_pairmajor_plan_rejects_bad_structures():
    """A pid outside [0, n_tracks) and a decreasing infos[0] are refused with the host planner's messages."""
    p = make_problem(0, n_frames=6, n_tracks=60)
    bad = p.pids.clone()
    bad[3] = p.n_tracks
    with pytest.raises(RuntimeError, match='pid out of range'):
        PMPlan(p.infos.to(DEV), bad.to(DEV), p.n_tracks, device=DEV)
    inf = p.infos.clone()
    inf[0, 2] = inf[0, 1] - 1
    with pytest.raises(RuntimeError, match='non-decreasing'):
        PMPlan(inf.to(DEV), p.pids.to(DEV), p.n_tracks, device=DEV)


@pytest.mark.parametrize('cfg', [3, 2])
def test_device_pairmajor_plan_full_size(cfg):
    """Full benchmark sizes (config 3: 22.5 M observations, 85 M pair terms; config 2: 8.0 M observations):
    the device plan equals the host plan, array for array; both build times are printed."""
    p = make_problem(cfg)
    print(f'[full cfg{cfg}] {p.n_obs} observations', flush=True)
    t0 = time.perf_counter()
    host = PMPlan(p.infos, p.pids, p.n_tracks, device='cpu')
    th = time.perf_counter() - t0
    ip, pp = p.infos.to(DEV), p.pids.to(DEV)
    PMPlan(ip, pp, p.n_tracks, device=DEV)           # first call: allocator and code objects
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dv = PMPlan(ip, pp, p.n_tracks, device=DEV)
    torch.cuda.synchronize()
    td = time.perf_counter() - t0
    print(f'[full cfg{cfg}] host planner {th * 1e3:.0f} ms, device planner {td * 1e3:.1f} ms: {dv.scalars}', flush=True)
    _assert_equal(host, dv)
