"""Dense tangent prior (engine.py:15-200): oracle pins on the CPU, then the device kernel
(ba_tangent_prior through blast3r_amd.tangent) against the oracle.

Tolerances: on the fp64 path the loss and the Gauss-Newton terms agree to 1e-6 relative (the
planar confidence and the pointmap tangents are fp32 in both, computed with exp and sqrt
implementations that may differ in the last bit); the fp32 loss agrees to 1e-4 relative
(neighbouring points are differenced, which amplifies last-bit differences of the depth by the
ratio |X| / |t|, about 100 at stride 4) and the fp32 Gauss-Newton terms to 1e-3 (the reference
sums them in fp32, the kernel in fp64).
"""
import math

import pytest
import torch

import oracle.tangent as ot


def _scene(seed, n_imgs=2, H=22, W=26, C=4, n_cams=1, stride_ch=None, dtype=torch.float32):
    """Log-depth channels around a tilted plane, a reference pointmap from the plane itself (nearly
    planar, so that the planar confidence is far from 0), per-camera K."""
    g = torch.Generator().manual_seed(seed)
    yy, xx = torch.meshgrid(torch.arange(H, dtype=torch.float64), torch.arange(W, dtype=torch.float64),
                            indexing='ij')
    maps, refs = [], []
    K = torch.zeros((n_cams, 3, 3))
    for c in range(n_cams):
        f = 25 + 10 * float(torch.rand(1, generator=g))
        K[c] = torch.tensor([[f, 0, W / 2 + 0.3], [0, f * 1.05, H / 2 - 0.2], [0, 0, 1]])
    for i in range(n_imgs):
        plane = 2.0 + 0.03 * xx + (0.01 + 0.005 * i) * yy
        ch = [torch.log(plane) + 0.02 * torch.sin(0.3 * xx + i) * torch.cos(0.2 * yy)]
        for k in range(1, C):
            a, b, p = (torch.rand(3, generator=g) * torch.tensor([0.3, 0.3, 6.0])).tolist()
            ch.append(0.2 * torch.sin(a * xx + b * yy + p) + 0.05 * torch.randn((H, W), generator=g, dtype=torch.float64))
        m = torch.stack(ch, -1).float()
        if stride_ch:                                                  # a channel slice of a wider map
            wide = torch.randn((H, W, stride_ch))
            wide[..., :C] = m
            m = wide[..., :C]
        maps.append(m)
        d0 = plane + 1e-4 * torch.randn((H, W), generator=g, dtype=torch.float64)
        Kc = K[i % n_cams].double()
        ray = torch.stack([(xx + 0.5 - Kc[0, 2]) / Kc[0, 0], (yy + 0.5 - Kc[1, 2]) / Kc[1, 1], torch.ones_like(xx)], -1)
        refs.append((ray * d0[..., None]).float())
    cam_ids = torch.arange(n_imgs, dtype=torch.int32) % n_cams
    z = torch.zeros((n_imgs, C))
    z[:, 0] = 1.0
    z[:, 1:] = 0.3 * torch.randn((n_imgs, C - 1), generator=g)
    return cam_ids, K, z, maps, refs


# ----------------------------------------------------------------------------- oracle pins (CPU)
def test_oracle_planar_confidence_known_answers():
    D = torch.ones((3, 3))
    D[1, 1] = 2.0
    c = ot.planar_confidence(D.clone(), alpha=0.01)
    assert math.isclose(float(c[1, 1]), math.exp(-0.08), rel_tol=1e-6)      # lx = ly = 2, min 1
    assert math.isclose(float(c[0, 0]), math.exp(-0.02), rel_tol=1e-6)      # one neighbour each way
    assert float(c[0, 1]) == 1.0                                              # lx = 0, ly = 2 - 2 = 0
    # an affine map with exact values: zero Laplacian inside, border columns/rows far from planar
    yy, xx = torch.meshgrid(torch.arange(6.0), torch.arange(7.0), indexing='ij')
    A = 2 + 0.25 * xx + 0.5 * yy
    c = ot.planar_confidence(A.clone())
    assert torch.equal(c[1:-1, 1:-1], torch.ones(4, 5))
    assert float(c[0].max()) == 0.0 and float(c[:, -1].max()) == 0.0


def _weighted_residuals(a, L, Ks, X0, normalize, eps, weight, scale0):
    """sqrt(scale * w) * r for both directions of one image, as a function of a (fp64)."""
    D = torch.exp((L * a).sum(-1).clamp(max=80))
    Ki = torch.linalg.inv(Ks)
    Hs, Ws = D.shape
    u = torch.arange(Ws, dtype=torch.float64) + 0.5
    v = torch.arange(Hs, dtype=torch.float64) + 0.5
    uv = torch.stack(torch.meshgrid(u, v, indexing='xy'), -1)
    ray = uv @ Ki[:, :2].T + Ki[:, 2]
    X = ray * D[..., None]
    if scale0 is not None:
        X0 = (scale0.float() * X0).double()          # the reference scales the fp32 pointmap in fp32
    Cw = ot.planar_confidence(X0[:, :, 2].float().clone()).double()    # fp32, as in the reference
    out = []
    for dim in (0, 1):
        n = X.shape[dim] - 1
        t = X.narrow(dim, 1, n) - X.narrow(dim, 0, n)
        X0f = X0.float()                                  # the pointmap's tangents stay fp32
        t0 = X0f.narrow(dim, 1, n) - X0f.narrow(dim, 0, n)
        is0 = 1.0 / t0.norm(dim=-1, keepdim=True).clamp(min=eps)
        th = t * ((1.0 / t.norm(dim=-1, keepdim=True).clamp(min=eps)) if normalize else is0.double())
        r = th - (t0 * is0).double()
        w = (Cw.narrow(dim, 1, n) * Cw.narrow(dim, 0, n)).clamp(min=0).sqrt()        # loss weight of w r^2
        out.append((torch.sqrt(w * weight / r.numel())[..., None] * r).reshape(-1))
    return torch.cat(out)


@pytest.mark.parametrize('normalize', [True, False])
def test_oracle_gauss_newton_terms_match_autograd(normalize):
    """g = J^T rho and H = J^T J of the weighted residuals rho(a) differentiated by autograd, a the
    image's z-coefficients (the rescaling of X0 without normalisation is a constant, as the
    reference detaches it)."""
    cam_ids, K, z, maps, refs = _scene(1, n_imgs=2, C=4)
    s, o = 3, 1
    _, g, H = ot.tangent_prior_terms(cam_ids, K, z, maps, refs, weight_tan=0.7, tan_stride=s, dtype=torch.float64,
                                     normalize_tangents=normalize)
    for i in range(2):
        Ks = K[int(cam_ids[i])].double().clone()
        Ks[:2, 2] -= o
        Ks[:2] /= s
        L = maps[i][o::s, o::s].double()
        X0 = refs[i][o::s, o::s].double()             # exact copy of the fp32 pointmap
        scale0 = None
        if not normalize:
            with torch.no_grad():
                D = torch.exp((L * z[i].double()).sum(-1).clamp(max=80))
                keep = X0[..., 2] > 1e-6
                scale0 = torch.median(D[keep] / X0[..., 2][keep])
        f = lambda a: _weighted_residuals(a, L, Ks, X0, normalize, 1e-4, 0.7, scale0)
        a = z[i].double()
        J = torch.autograd.functional.jacobian(f, a)
        rho = f(a)
        assert float(rho.abs().max()) > 0 and int((J.abs().sum(1) > 0).sum()) > rho.numel() // 4
        assert float((g[i] - J.T @ rho).norm() / (J.T @ rho).norm()) < 1e-5
        assert float((H[i] - J.T @ J).norm() / (J.T @ J).norm()) < 1e-5


def test_oracle_zero_when_depth_matches_reference():
    cam_ids, K, z, maps, refs = _scene(2, n_imgs=1, C=3)
    s, o = 4, 2
    Ks = K[0].clone()
    Ks[:2, 2] -= o
    Ks[:2] /= s
    L = maps[0][o::s, o::s]
    X = ot._rays(L.shape[0], L.shape[1], Ks, torch.float32) * torch.exp(torch.einsum('c,hwc->hw', z[0], L))[..., None]
    ref = refs[0].clone()
    ref[o::s, o::s] = X                                                # X0 == X at the sampled points
    loss, _, _ = ot.tangent_prior_terms(cam_ids, K, z, maps, [ref], weight_tan=1.0, tan_stride=s, compute_gn=False)
    assert float(loss) == 0.0
    loss2, _, _ = ot.tangent_prior_terms(cam_ids, K, z, maps, refs, weight_tan=1.0, tan_stride=s, compute_gn=False)
    assert float(loss2) > 0.0


def test_oracle_skips_and_optim_Z0():
    cam_ids, K, z, maps, refs = _scene(3, n_imgs=2, C=4)
    # one channel: every image skipped (min(W', C) < 2)
    l1, g1, H1 = ot.tangent_prior_terms(cam_ids, K, z[:, :1], [m[..., :1] for m in maps], refs, weight_tan=1.0,
                                        dtype=torch.float64)
    assert float(l1) == 0.0 and float(g1.abs().max()) == 0.0 and float(H1.abs().max()) == 0.0
    # a subsampled width of 1 (W = 3, stride 4): skipped as well
    l2, _, _ = ot.tangent_prior_terms(cam_ids, K, z, [m[:, :3] for m in maps], [r[:, :3] for r in refs],
                                      weight_tan=1.0, dtype=torch.float64)
    assert float(l2) == 0.0
    _, g, H = ot.tangent_prior_terms(cam_ids, K, z, maps, refs, weight_tan=1.0, dtype=torch.float64, optim_Z0=False)
    _, g_on, H_on = ot.tangent_prior_terms(cam_ids, K, z, maps, refs, weight_tan=1.0, dtype=torch.float64)
    assert float(g[:, 0].abs().max()) == 0.0 and float(H[:, 0].abs().max()) == 0.0 and float(H[:, :, 0].abs().max()) == 0
    assert torch.equal(g[:, 1:], g_on[:, 1:]) and torch.equal(H[:, 1:, 1:], H_on[:, 1:, 1:])


# ----------------------------------------------------------------------------- device vs oracle
DEV = 'cuda'


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    n = float(b.norm())
    return float((a - b).norm()) / n if n > 0 else float((a - b).norm())


def _oracle_reduced(p, z_prior, optim_Z, dampen):
    """The oracle's reduced system (S, rhs) and z offset for problem p with the prior z_prior."""
    from oracle import kernels as ok
    from oracle import solver as osol
    from oracle import engine as oeng
    inp, o = p.lm_inputs(), p.options
    _, res, w = oeng.objective(inp['rigs'], inp['K'], inp['P_rig2cam'], inp['P_w2rig'], inp['z_coefs'], inp['pts3d'],
                               inp['pids'], inp['pix2d'], inp['pix2d_std'], inp['pix2d_dep'], True, o['weight_z'],
                               1.0, 100.0, o['huber_delta'])
    Jc, Jz, Jp = ok.jacobians_with_rigs(inp['rigs'], inp['K'], inp['P_rig2cam'], inp['P_w2rig'], inp['z_coefs'],
                                        inp['pts3d'], inp['pids'], inp['pix2d_std'], inp['pix2d_dep'], True,
                                        float64=True)
    prob = osol.Problem(inp['rigs'], inp['pids'], len(inp['K']), len(inp['P_w2rig']), len(inp['pts3d']),
                        inp['z_coefs'].shape[1])
    ne, g, _ = osol.build_normal_equations(prob, Jc, Jz, Jp, res, w, optim_Z=optim_Z, dampen=dampen,
                                           z_prior=z_prior)
    return osol.dense_schur(ne), osol.reduced_rhs(ne, g), ne.leaf_offsets['zcf']


def test_oracle_prior_enters_the_normal_equations_before_damping():
    """What bs:141-173 fixes, on the oracle's reduced system (dampen 1e-3 so that the damping's
    dependence on the prior shows): with optim_Z the prior adds H_z to each image's z block, g_z to
    the z rhs and nothing elsewhere, and the z leaf's damping is recomputed from the diagonal that
    includes H_z; with optim_Z=False the z block is exactly H_z + dampen max(diag H_z) I, decoupled
    from every other unknown, and the z rhs is g_z."""
    from blast3r_amd.synthetic import make_problem
    p = make_problem(0, n_frames=4, n_tracks=60)
    n_imgs, C = p.z_coefs.shape
    g = torch.Generator().manual_seed(5)
    A = torch.randn((n_imgs, C, C), generator=g, dtype=torch.float64)
    H_z = A @ A.transpose(1, 2) + 0.1 * torch.eye(C, dtype=torch.float64)
    g_z = torch.randn((n_imgs, C), generator=g, dtype=torch.float64)
    dampen = 1e-3
    S0, r0, oz = _oracle_reduced(p, None, True, dampen)
    S1, r1, oz1 = _oracle_reduced(p, (H_z, g_z), True, dampen)
    assert oz == oz1
    nz = n_imgs * C
    z = slice(oz, oz + nz)
    dS = S1 - S0
    Hb = torch.block_diag(*H_z)
    off = dS.clone()
    off[z, z] = 0
    assert float(off.abs().max()) == 0.0                              # nothing outside the z block moves
    lam_diff = torch.diagonal(dS[z, z] - Hb)                           # (lam1 - lam0) on every z unknown
    assert float((lam_diff - lam_diff[0]).abs().max()) <= 1e-12 * float(Hb.abs().max())
    assert float((dS[z, z] - Hb - torch.diag(lam_diff)).abs().max()) <= 1e-12 * float(Hb.abs().max())
    assert float(lam_diff[0]) > 0                                      # the damping grew with the diagonal
    dr = r1 - r0
    assert oz + nz == len(dr) and float(dr[:oz].abs().max()) == 0.0     # z comes last in the reduced system
    assert float((dr[z] - g_z.reshape(-1)).abs().max()) <= 1e-12 * float(g_z.abs().max())
    # optim_Z=False: the z block under the prior alone
    S2, r2, oz2 = _oracle_reduced(p, (H_z, g_z), False, dampen)
    lam = dampen * float(torch.diagonal(H_z, dim1=1, dim2=2).max())
    assert float((S2[z, z] - Hb - lam * torch.eye(nz, dtype=torch.float64)).abs().max()) <= 1e-12 * float(Hb.abs().max())
    assert float(S2[z, :oz].abs().max()) == 0.0 and float(S2[:oz, z].abs().max()) == 0.0
    assert torch.equal(r2[z], g_z.reshape(-1))


@pytest.mark.gpu
@pytest.mark.parametrize('normalize', [True, False])
@pytest.mark.parametrize('dtype', [torch.float64, torch.float32])
@pytest.mark.parametrize('C,stride,n_cams,wide', [(5, 4, 1, None), (9, 3, 3, 12), (14, 4, 2, None), (3, 1, 1, None),
                                                  (17, 4, 1, None), (23, 3, 2, 30)])
def test_device_tangent_prior_matches_oracle(normalize, dtype, C, stride, n_cams, wide):
    """C <= 16: one workgroup per tile holds all of H; C = 17 and 23: H split over row groups."""
    cam_ids, K, z, maps, refs = _scene(7 + C, n_imgs=3, H=40, W=52, C=C, n_cams=n_cams, stride_ch=wide)
    kw = dict(weight_tan=0.8, tan_stride=stride, normalize_tangents=normalize, dtype=dtype)
    from blast3r_amd.tangent import dense_tangent_prior_terms
    rigs = torch.stack([torch.zeros(3, dtype=torch.int32), torch.arange(3, dtype=torch.int32), cam_ids]).to(DEV)
    conf = [torch.ones(1)] * 3
    for gn in (True, False):
        lr, gr, Hr = ot.tangent_prior_terms(cam_ids, K, z, maps, refs, compute_gn=gn, optim_Z0=False, **kw)
        lg, gg, Hg = dense_tangent_prior_terms(rigs, K.to(DEV), z.to(DEV), [m.to(DEV) for m in maps], conf,
                                               [r.to(DEV) for r in refs], compute_gn=gn, optim_Z0=False, **kw)
        assert lg.dtype == dtype and lg.shape == ()
        assert abs(float(lg) - float(lr)) <= 1e-4 * abs(float(lr)), (float(lg), float(lr))
        if gn:
            tol = 1e-6 if dtype == torch.float64 else 1e-3
            assert gg.dtype == dtype and Hg.dtype == dtype
            assert _rel(gg, gr) < tol and _rel(Hg, Hr) < tol, (_rel(gg, gr), _rel(Hg, Hr))
            assert float(gg[:, 0].abs().max()) == 0.0 and float(Hg[:, 0].abs().max()) == 0.0
            assert torch.equal(Hg, Hg.transpose(1, 2))
        else:
            assert gg is None and Hg is None


@pytest.mark.gpu
def test_device_tangent_prior_per_image_sizes_and_stacked_maps():
    """Maps of different sizes per image (address table + per-image sizes) and one stacked tensor."""
    from blast3r_amd.tangent import dense_tangent_prior_terms
    cam_ids, K, z, maps, refs = _scene(21, n_imgs=2, H=40, W=52, C=5)
    maps2 = [maps[0], maps[1][:31, :45].contiguous()]
    refs2 = [refs[0], refs[1][:31, :45].contiguous()]
    rigs = torch.stack([torch.zeros(2, dtype=torch.int32), torch.arange(2, dtype=torch.int32), cam_ids]).to(DEV)
    for mm, rr in ((maps2, refs2), (torch.stack(maps), torch.stack(refs))):
        ml = list(mm) if isinstance(mm, list) else list(mm.unbind(0))
        rl = list(rr) if isinstance(rr, list) else list(rr.unbind(0))
        lr, gr, Hr = ot.tangent_prior_terms(cam_ids, K, z, ml, rl, weight_tan=1.0, dtype=torch.float64)
        dm = [m.to(DEV) for m in mm] if isinstance(mm, list) else mm.to(DEV)
        dr = [r.to(DEV) for r in rr] if isinstance(rr, list) else rr.to(DEV)
        lg, gg, Hg = dense_tangent_prior_terms(rigs, K.to(DEV), z.to(DEV), dm, [1, 1], dr,
                                               weight_tan=1.0, dtype=torch.float64)
        assert abs(float(lg) - float(lr)) <= 1e-6 * abs(float(lr))
        assert _rel(gg, gr) < 1e-6 and _rel(Hg, Hr) < 1e-6


@pytest.mark.gpu
def test_device_planar_confidence_matches_oracle():
    from blast3r_amd.tangent import confident_in_planar_regions
    g = torch.Generator().manual_seed(3)
    yy, xx = torch.meshgrid(torch.arange(33.0), torch.arange(47.0), indexing='ij')
    for D in (2 + 0.25 * xx + 0.5 * yy, 3 + 0.01 * torch.randn((33, 47), generator=g), torch.rand((1, 9)) + 1):
        ref = ot.planar_confidence(D.clone())
        got = confident_in_planar_regions(D.to(DEV)).cpu()
        assert float((got - ref).abs().max()) <= 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize('optim_Z,n_channels', [(True, None), (False, None), (True, 16)])
def test_lm_step_with_tangent_prior_parity(optim_Z, n_channels):
    """lm_step with weight_tan > 0 (prior loss in every objective, GN terms added to the z blocks)
    against the oracle with the same prior, checked as test_lm_step_parity checks a step: the step
    delta against the oracle's PCG iterate after the same number of updates (1e-4), the oracle's
    line search on the device's delta (same scales, loss and parameters within 1e-5); the
    start-of-step loss (Huber mean + prior) to 1e-4.  optim_Z=False: the z-coefficients move under the
    prior alone (their zero Jacobian block becomes H_z, bs:163-164); 16 channels: C = 17, d = 25."""
    from blast3r_amd.synthetic import make_problem
    from blast3r_amd import engine as gpu_engine
    import oracle.engine as oeng
    from helpers import rel_err
    p = make_problem(0, n_frames=6, n_tracks=150, n_channels=n_channels)
    o = p.options
    n_imgs, C = p.z_coefs.shape
    H, W = 96, 128
    g = torch.Generator().manual_seed(9)
    yy, xx = torch.meshgrid(torch.arange(H, dtype=torch.float64), torch.arange(W, dtype=torch.float64), indexing='ij')
    maps, refs = [], []
    for i in range(n_imgs):
        plane = 3.0 + 0.004 * xx + 0.003 * (i + 1) * yy
        ch = [torch.log(plane) + 0.01 * torch.sin(0.05 * xx + i)]
        for k in range(1, C):
            ch.append(0.1 * torch.sin(0.03 * (k + 1) * xx + 0.02 * yy + k))
        maps.append(torch.stack(ch, -1).float())
        Kc = p.K[int(p.infos[2, i])].double()
        ray = torch.stack([(xx + 0.5 - Kc[0, 2]) / Kc[0, 0], (yy + 0.5 - Kc[1, 2]) / Kc[1, 1], torch.ones_like(xx)], -1)
        refs.append((ray * plane[..., None]).float())
    kw = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, weight_tan=0.5, tan_stride=4)
    conf = [torch.ones(1)] * n_imgs
    import oracle.tangent as T_
    from tests.step_checks import check_line_search, check_step_delta, device_system, oracle_system
    tan_kw = dict(weight_tan=0.5, tan_stride=4, optim_Z0=True, normalize_tangents=True)
    prior = lambda zc, gn, dt: T_.tangent_prior_terms(p.infos[2], p.K, zc, maps, refs, dtype=dt, compute_gn=gn,
                                                      **tan_kw)
    extra = lambda zc: prior(zc, False, torch.float32)[0]
    _, g_z, H_z = prior(p.z_coefs, True, torch.float64)
    gp = p.to(DEV)
    info = {}
    up_g, st_g, _ = gpu_engine._lm_step(**gp.lm_inputs(), log_depth_maps=[m.to(DEV) for m in maps], conf=conf,
                                        pts3d_ref=[r.to(DEV) for r in refs], dtype=torch.float64, info=info,
                                        optim_Z=optim_Z, **kw)
    inp = p.lm_inputs()
    hp = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, clip_pix_err=100)
    sysd = oracle_system(inp, hp, dict(optim_Z=optim_Z), z_prior=(H_z, g_z), extra_loss=extra)
    assert abs(float(st_g.init_loss) - float(sysd['loss'])) <= 1e-4 * abs(float(sysd['loss']))
    check_step_delta(sysd, info['delta'], info['pcg_istate'].cpu(), seed=9,
                     reduced=device_system(info['solver']))
    check_line_search(inp, hp, sysd, info['delta'], info, st_g, up_g, extra_loss=extra)
