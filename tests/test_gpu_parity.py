"""GPU parity: libba_hip.so against the CPU oracle on identical seeded inputs.

Tolerances (norm-wise relative, ||gpu - oracle|| / ||oracle||):
  * fp32 residuals / Huber errors / weights: 1e-5 (the reference computes them in fp32)
  * fp64 Jacobian blocks: 1e-9 (same fp64 formula from the same fp32 inputs)
  * reduced-system blocks S, rhs, point blocks: 1e-5 (fp64, differences come from the
    fp32 residual/weight rounding of logf/powf on either side)
  * PCG step and LM step: 1e-4 on delta and on sqrt(W) J delta (the north-star step tolerance)
    against the oracle's iterate after the same number of CG updates, widened only where the
    system's conditioning makes CG amplify rounding: to 5x the move of the oracle's own iterate
    under 1e-15 perturbations of b; the line search then run by the oracle on the device's step:
    the same scales, loss and updated parameters within 1e-5
"""
import numpy as np
import pytest
import torch

from blast3r_amd import cujac
from blast3r_amd.ba_solver import GaussNewtonSolver
from blast3r_amd import engine as gpu_engine
from blast3r_amd.synthetic import make_problem
from oracle import kernels as ok
from oracle import solver as osol
from oracle import engine as oeng
from tests.helpers import rel_err, tiny_problem, opts
from tests.step_checks import check_line_search as _check_line_search
from tests.step_checks import check_step_delta as _check_step_delta
from tests.step_checks import device_system, oracle_system as _oracle_system

pytestmark = pytest.mark.gpu
DEV = 'cuda:0'


def _gpu(p):
    return p.to(DEV)


def _oracle_res(p, pnorm=1.0, **kw):
    o = opts(p)
    o.update(kw)
    return ok.residuals_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                  p.pix2d_std, p.pix2d_dep, True, o['weight_z'], pnorm, o['clip_pix_err'],
                                  o['huber_delta'])


@pytest.mark.parametrize('cfg,nf,nt', [(0, 6, 60), (0, 32, 2000), (2, 40, 3000), (4, 30, 2000)])
def test_residuals_parity(cfg, nf, nt):
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    ref = _oracle_res(p)
    assert out.shape == ref.shape == (p.n_obs, 9)
    assert out.stride() == (1, p.n_obs)                    # transposed SoA view (.cu:1100)
    for sl in (slice(0, 3), slice(3, 6), slice(6, 9)):
        assert rel_err(out[:, sl], ref[:, sl]) < 1e-5
    # pnorm = -1 -> 3 outputs only
    out3 = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                             g.pix2d, g.pix2d_std, g.pix2d_dep, True)
    assert out3.shape == (p.n_obs, 3)
    assert rel_err(out3, ref[:, :3]) < 1e-5


@pytest.mark.parametrize('pnorm', [1.0, 2.0, 0.5, 1.5])
def test_residuals_huber_exponents(pnorm):
    """The Huber error and IRLS weight for the exponents with closed forms (p = 1: r and 1/r; p = 2: r^2 and
    1) and for general ones (powf), with residuals beyond delta and beyond the clip value present, against
    the oracle's torch pow (.cu:240-258)."""
    p = make_problem(0, n_frames=12, n_tracks=800)
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], pnorm,
                                            o['clip_pix_err'], o['huber_delta'])
    ref = _oracle_res(p, pnorm=pnorm)
    r = ref[:, :2].abs()
    assert bool((r > o['huber_delta']).any()) and bool((r < o['huber_delta']).any())
    assert bool((r >= o['clip_pix_err']).any())
    for sl in (slice(0, 3), slice(3, 6), slice(6, 9)):
        assert rel_err(out[:, sl], ref[:, sl]) < 1e-5


@pytest.mark.parametrize('case', ['wide_C', 'empty_images', 'many_small_images'])
def test_residuals_block_image_ranges(case):
    """k_residuals takes each block's image range from two searches and stages the cameras and
    z-coefficients of its first four images in LDS: blocks whose range holds empty images, more than
    four images (the rest read from memory) or more z-coefficients than the staging holds (C = 41) give
    the oracle's residuals, errors and weights."""
    if case == 'wide_C':
        p = make_problem(0, n_frames=12, n_tracks=600, n_channels=40)
    elif case == 'many_small_images':
        p = make_problem(1, n_frames=64, n_tracks=120)
    else:
        p = make_problem(0, n_frames=16, n_tracks=800)
        cum = p.infos[0].long()
        img = torch.repeat_interleave(torch.arange(p.n_imgs), torch.diff(torch.cat([cum.new_zeros(1), cum])))
        keep = (img != 0) & (img != 3) & (img != 4) & (img != p.n_imgs - 1)
        p.pids, p.pix2d, p.pix2d_std, p.pix2d_dep = (t[keep] for t in (p.pids, p.pix2d, p.pix2d_std, p.pix2d_dep))
        infos = p.infos.clone()
        infos[0] = torch.cumsum(torch.bincount(img[keep], minlength=p.n_imgs), 0).to(infos.dtype)
        p.infos = infos
    print(f'residual block ranges: {case}, {p.n_imgs} images, {p.pids.numel()} obs, C={p.pix2d_dep.shape[1]}',
          flush=True)
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    ref = _oracle_res(p)
    assert out.shape == ref.shape
    for sl in (slice(0, 3), slice(3, 6), slice(6, 9)):
        assert rel_err(out[:, sl], ref[:, sl]) < 1e-5


def test_residuals_invalid_depth_rows_are_zero():
    p = tiny_problem()
    P = p.P_w2rig.clone()
    P[0, 2, 3] -= 100.0           # push every point of image 0 behind the camera
    p.P_w2rig = P
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta']).cpu()
    n0 = int(p.infos[0, 0])
    assert n0 > 0 and torch.all(out[:n0] == 0)
    assert torch.any(out[n0:] != 0)


def test_depth_threshold_at_1e3f():
    """z <= 1e-3 (.cu:212, :408) compares against the double literal: a point at z = 1e-3f keeps its
    residual and Jacobian rows on the device, the next float below drops them, as in the oracle."""
    import numpy as np
    for z, kept in ((float(np.float32(1e-3)), True), (float(np.nextafter(np.float32(1e-3), np.float32(0))), False)):
        eye = torch.eye(4).view(1, 4, 4)
        d = dict(infos=torch.tensor([[1], [0], [0]], dtype=torch.int32),
                 K=torch.tensor([[[500.0, 0, 256.0], [0, 500.0, 192.0], [0, 0, 1]]]), P_rig2c=eye.expand(1, 4, 4),
                 P_w2rig=eye.clone(), z_coefs=torch.tensor([[1.0, 0.0, 0.0]]), pts3d=torch.tensor([[0.0, 0.0, z]]),
                 pids=torch.tensor([0], dtype=torch.int32), pix2d=torch.tensor([[259.0, 191.0]]),
                 pix2d_std=torch.tensor([[1.0, 2.0]]), pix2d_dep=torch.tensor([[0.0, 1.0, 0.0]]))
        g = {k: v.to(DEV) for k, v in d.items()}
        args = ('infos', 'K', 'P_rig2c', 'P_w2rig', 'z_coefs', 'pts3d', 'pids', 'pix2d', 'pix2d_std', 'pix2d_dep')
        out = cujac.compute_residuals_with_rigs(*[g[k] for k in args], True, 1.0, 1.0, 100.0, 2.0).cpu()
        ref = ok.residuals_with_rigs(*[d[k] for k in args], True, 1.0, 1.0, 100.0, 2.0)
        assert bool(torch.count_nonzero(out) > 0) == kept, z
        assert rel_err(out, ref) <= 1e-6
        jargs = ('infos', 'K', 'P_rig2c', 'P_w2rig', 'z_coefs', 'pts3d', 'pids', 'pix2d_std', 'pix2d_dep')
        for f64 in (True, False):
            Jg = cujac.compute_jacobians_with_rigs(*[g[k] for k in jargs], True, float64=f64)
            assert bool(torch.count_nonzero(Jg[2]) > 0) == kept, (z, f64)


@pytest.mark.parametrize('float64', [True, False])
def test_jacobians_parity(float64):
    p = make_problem(0, n_frames=10, n_tracks=500)
    g = _gpu(p)
    Jg = cujac.compute_jacobians_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                           g.pix2d_std, g.pix2d_dep, True, float64=float64)
    Jr = ok.jacobians_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d_std,
                                p.pix2d_dep, True, float64=float64)
    tol = 1e-9 if float64 else 1e-5
    for a, b in zip(Jg, Jr):
        assert a.dtype == b.dtype and a.shape == b.shape
        assert rel_err(a, b) < tol


def test_lin_depth_mode_residuals_and_jacobians():
    """depth_mode='lin' (r2 = fbar log(g / z), .cu:238; its Jacobian rows .cu:497-499): residuals, Huber
    errors and weights (fp32, 1e-5) and the Jacobian blocks in fp64 (1e-9) and fp32 (1e-5) against the
    oracle, on linear depth channels with no ones channel."""
    p = make_problem(0, n_frames=10, n_tracks=500, depth_mode='lin')
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d,
                                            g.pix2d_std, g.pix2d_dep, False, o['weight_z'], 1.0, o['clip_pix_err'],
                                            o['huber_delta'])
    ref = ok.residuals_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                 p.pix2d_std, p.pix2d_dep, False, o['weight_z'], 1.0, o['clip_pix_err'],
                                 o['huber_delta'])
    assert bool(ref[:, 2].abs().gt(0).any())
    for k in range(3):
        assert rel_err(out[:, 3 * k:3 * k + 3].cpu(), ref[:, 3 * k:3 * k + 3]) < 1e-5, k
    for f64, tol in ((True, 1e-9), (False, 1e-5)):
        Jg = cujac.compute_jacobians_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                               g.pix2d_std, g.pix2d_dep, False, float64=f64)
        Jr = ok.jacobians_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d_std,
                                    p.pix2d_dep, False, float64=f64)
        for a, b in zip(Jg, Jr):
            assert a.dtype == b.dtype and a.shape == b.shape
            assert rel_err(a.cpu(), b) < tol, f64


@pytest.mark.parametrize('cfg,nf,nt,path', [(0, 8, 200, 'auto'), (2, 24, 800, 'auto'), (2, 24, 800, 'pairmajor'),
                                            (4, 12, 300, 'auto'), (3, 24, 600, 'pairmajor')])
def test_reduced_system_parity_lin(cfg, nf, nt, path):
    """The fused linearize + Schur pass in depth_mode='lin' (both paths) against the oracle's damped
    reduced system, rhs and point blocks (1e-5)."""
    print(f'lin reduced system cfg {cfg} {path}', flush=True)
    _check_reduced_system(make_problem(cfg, n_frames=nf, n_tracks=nt, depth_mode='lin'), path)


@pytest.mark.parametrize('cfg,nf,nt,path', [(0, 8, 300, 'auto'), (2, 30, 1500, 'auto'), (3, 24, 600, 'auto')])
def test_lm_step_parity_lin(cfg, nf, nt, path):
    """lm_step(depth_mode='lin') against the oracle with the bars of test_lm_step_parity."""
    print(f'lin lm_step parity cfg {cfg}', flush=True)
    _check_lm_step(make_problem(cfg, n_frames=nf, n_tracks=nt, depth_mode='lin'), cfg + 40, dict(path=path))


def test_compat_ops():
    torch.manual_seed(0)
    # chol3x3_solve
    A = torch.randn(100, 3, 5, dtype=torch.float64)
    H = A @ A.transpose(1, 2)
    b = torch.randn(100, 3, dtype=torch.float64)
    for dt in (torch.float64, torch.float32):
        x = cujac.chol3x3_solve(H.to(DEV, dt), b.to(DEV, dt)).cpu()
        assert rel_err(x, ok.chol3x3_solve(H.to(dt), b.to(dt))) < (1e-12 if dt == torch.float64 else 1e-4)
    # blockcoo_matvec, both orientations and index dtypes
    blocks = torch.randn(50, 3, 6, dtype=torch.float64)
    rows = torch.randint(0, 7, (50,))
    cols = torch.randint(0, 9, (50,))
    for idt in (torch.int32, torch.int64):
        for tr in (False, True):
            x = torch.randn(7 * 3 if tr else 9 * 6, dtype=torch.float64)
            y = cujac.blockcoo_matvec(blocks.to(DEV), rows.to(DEV, idt), cols.to(DEV, idt), x.to(DEV), 7, 9, tr)
            yr = ok.blockcoo_matvec(blocks, rows, cols, x, 7, 9, tr)
            assert rel_err(y, yr) < 1e-12
    # fused_einsum_bki_bkj including the (5, 6, 1) case missing from the reference dispatch
    for (I, J, K) in [(5, 6, 1), (3, 6, 3), (9, 9, 1), (2, 6, 3), (17, 17, 1)]:
        L = torch.randn(40, K, I, dtype=torch.float64)
        R = torch.randn(40, K, J, dtype=torch.float64)
        assert rel_err(cujac.fused_einsum_bki_bkj(L.to(DEV), R.to(DEV)), ok.fused_einsum_bki_bkj(L, R)) < 1e-12
    # exp_se3 against torch.matrix_exp of the hat matrix (fp32)
    xi = torch.randn(64, 6) * torch.tensor([0.3, 0.3, 0.3, 1.0, 1.0, 1.0])
    xi[:4, :3] *= 1e-6
    assert rel_err(cujac.exp_se3(xi.to(DEV)), ok.exp_se3(xi)) < 1e-6

@pytest.mark.parametrize('bh,bw', [(3, 6), (3, 5), (6, 6), (17, 2)])
def test_blockcoo_matvec_sorted_segments(bh, bw):
    """ba_blockcoo_matvec (.cu:1171-1219 semantics) on 20k blocks in random order with repeats over 300 x 40
    block positions: equal to the oracle's dense product in both orientations and index dtypes (fp64 1e-12,
    fp32 1e-5); bit-identical over repeated calls (each output sums its blocks in ascending block order);
    output blocks that no block touches are exactly zero; an empty block list gives a zero vector; block
    indices outside the matrix are ignored (the reference would read or write out of bounds)."""
    g = torch.Generator().manual_seed(bh * 100 + bw)
    HB1, WB1, n = 300, 40, 20000
    rows = torch.randint(0, HB1 - 7, (n,), generator=g)          # the last 7 block rows stay empty
    cols = torch.randint(0, WB1, (n,), generator=g)
    blocks = torch.randn(n, bh, bw, generator=g, dtype=torch.float64)
    for dt, tol in ((torch.float64, 1e-12), (torch.float32, 1e-5)):
        for idt in (torch.int32, torch.int64):
            for tr in (False, True):
                x = torch.randn(HB1 * bh if tr else WB1 * bw, generator=g, dtype=torch.float64)
                args = (blocks.to(DEV, dt), rows.to(DEV, idt), cols.to(DEV, idt), x.to(DEV, dt), HB1, WB1, tr)
                y = cujac.blockcoo_matvec(*args)
                yr = ok.blockcoo_matvec(blocks, rows, cols, x, HB1, WB1, tr)
                assert rel_err(y.double(), yr) < tol, (dt, idt, tr)
                assert torch.equal(cujac.blockcoo_matvec(*args), y)
                if not tr:
                    assert not y.view(HB1, bh)[HB1 - 7:].any()
    # empty block list
    x = torch.randn(WB1 * bw, dtype=torch.float64)
    y0 = cujac.blockcoo_matvec(blocks[:0].to(DEV), rows[:0].to(DEV), cols[:0].to(DEV), x.to(DEV), HB1, WB1, False)
    assert y0.shape == (HB1 * bh,) and not y0.any()
    # out-of-range block indices are skipped, the rest is summed as usual
    bad_r, bad_c = rows.clone(), cols.clone()
    bad_r[:50] = HB1 + 3
    bad_r[50:100] = -1
    bad_c[100:150] = WB1
    keep = torch.ones(n, dtype=torch.bool)
    keep[:150] = False
    for tr in (False, True):
        x = torch.randn(HB1 * bh if tr else WB1 * bw, generator=g, dtype=torch.float64)
        y = cujac.blockcoo_matvec(blocks.to(DEV), bad_r.to(DEV), bad_c.to(DEV), x.to(DEV), HB1, WB1, tr)
        yr = ok.blockcoo_matvec(blocks[keep], rows[keep], cols[keep], x, HB1, WB1, tr)
        assert rel_err(y, yr) < 1e-12, tr



def _is_log(p):
    return p.options.get('depth_mode', 'log') == 'log'


def _oracle_ne(p, dtype=torch.float64, **flags):
    o = opts(p)
    loss, res, w = oeng.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                  p.pix2d_std, p.pix2d_dep, _is_log(p), o['weight_z'], 1.0, o['clip_pix_err'],
                                  o['huber_delta'])
    Jc, Jz, Jp = ok.jacobians_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids,
                                        p.pix2d_std, p.pix2d_dep, _is_log(p), float64=dtype == torch.float64)
    if not flags.get('optim_Z0', True):
        Jz[:, 0, 0] = 0
    prob = osol.Problem(p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks, p.C)
    f = {k: v for k, v in flags.items() if k in ('optim_K', 'optim_P', 'optim_Z', 'optim_X', 'no_grad_f_from_rz')}
    ne, gvec, params = osol.build_normal_equations(prob, Jc, Jz, Jp, res, w, **f)
    return ne, gvec, params, (Jc, Jz, Jp), res, w


def _cfg_flags(p):
    """The configuration's own optimisation flags (config 4 keeps K and P fixed)."""
    return {k: p.options[k] for k in ('optim_K', 'optim_P') if not p.options.get(k, True)}


def _gpu_solver(p, path='auto', solver='pcg', dtype=torch.float64, **flags):
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, _is_log(p), o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    gs = GaussNewtonSolver(len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks, DEV, dtype=dtype,
                           no_grad_f_from_rz=flags.get('no_grad_f_from_rz', False), path=path, solver=solver)
    hp = dict(weight_z=o['weight_z'], pnorm=1.0, max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    fl = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in flags.items()
          if k in ('optim_K', 'optim_P', 'optim_Z', 'optim_X', 'optim_Z0')}
    J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                             g.pix2d_dep, _is_log(p), pix2d=g.pix2d, hp=hp, **fl)
    delta = gs.solve_delta(J, res, w)
    return gs, delta, g


# pair-major path cases: every configuration, image-level width 16 and 17 (config 4 with 15 and 16
# depth channels, focal and pose fixed) and 25 (config 2 with 16 depth channels), tracks spanning 20
# to 30 images
PM_CASES = [(0, 6, 60, {}), (1, 32, 400, {}), (2, 24, 800, {}), (3, 24, 600, {}), (4, 12, 300, {}),
            (4, 12, 200, dict(n_channels=16)), (2, 16, 300, dict(n_channels=16)),
            (2, 40, 300, dict(track_len=(20, 30))), (4, 12, 200, dict(n_channels=15))]
PM_IDS = ['cfg0', 'cfg1', 'cfg2', 'cfg3', 'cfg4', 'd17', 'd25', 'long', 'd16']


@pytest.mark.parametrize('cfg,nf,nt', [(0, 6, 60), (0, 8, 200), (1, 32, 400), (2, 20, 400), (3, 24, 600), (4, 12, 300)])
def test_reduced_system_parity(cfg, nf, nt):
    """S = H_cc - H_cp H_pp^-1 H_pc (damped, reference unknown order) and rhs against the oracle."""
    _check_reduced_system(make_problem(cfg, n_frames=nf, n_tracks=nt), 'auto')


@pytest.mark.parametrize('cfg,nf,nt,kw', PM_CASES, ids=PM_IDS)
def test_reduced_system_parity_pairmajor(cfg, nf, nt, kw):
    """The pair-major linearize + Schur path against the oracle, as the batched path."""
    print(f'pair-major reduced system cfg {cfg} {kw}', flush=True)
    _check_reduced_system(make_problem(cfg, n_frames=nf, n_tracks=nt, **kw), 'pairmajor')


@pytest.mark.parametrize('cfg,path', [(0, 'auto'), (2, 'auto'), (0, 'pairmajor'), (2, 'pairmajor')])
def test_reduced_system_with_empty_images_and_a_bare_track(cfg, path):
    """Images with no observations (the first, two inner ones and the last: no image pair, no diagonal block)
    and a track with none (its point block only the damping): S, rhs and the point blocks against the oracle
    on both fused paths, a finite PCG step, and the direct solve (the empty images' blocks hold only their
    damping) with every pivot positive and the device's system solved to 1e-10."""
    p = make_problem(cfg, n_frames=16, n_tracks=800)
    cum = p.infos[0].long()
    img = torch.repeat_interleave(torch.arange(p.n_imgs), torch.diff(torch.cat([cum.new_zeros(1), cum])))
    keep = (img != 0) & (img != 3) & (img != 4) & (img != p.n_imgs - 1) & (p.pids.long() != 7)
    p.pids, p.pix2d, p.pix2d_std, p.pix2d_dep = (t[keep] for t in (p.pids, p.pix2d, p.pix2d_std, p.pix2d_dep))
    infos = p.infos.clone()
    infos[0] = torch.cumsum(torch.bincount(img[keep], minlength=p.n_imgs), 0).to(infos.dtype)
    p.infos = infos
    assert int((torch.bincount(p.pids.long(), minlength=p.n_tracks) == 0).sum()) >= 1
    print(f'empty images cfg {cfg} {path}: {p.n_obs} obs', flush=True)
    _check_reduced_system(p, path)
    _, delta, _ = _gpu_solver(p, path=path, **_cfg_flags(p))
    assert bool(torch.isfinite(delta).all())
    # the direct solve on the same system: the empty images' blocks hold only their damping
    from tests.step_checks import device_system
    gs, delta, _ = _gpu_solver(p, path=path, solver='cholesky', **_cfg_flags(p))
    assert gs.last['direct'] is not None and gs.last['direct']['first_bad_pivot'] is None
    S_dev, rhs_dev, _ = device_system(gs)
    x = gs.last['x'][:S_dev.shape[0]].cpu()
    assert float((S_dev @ x - rhs_dev).norm() / rhs_dev.norm()) <= 1e-10
    assert bool(torch.isfinite(delta).all())


def _check_reduced_system(p, path):
    ne, gvec, params, _, _, _ = _oracle_ne(p, **_cfg_flags(p))
    S_ref = osol.dense_schur(ne)
    rhs_ref = osol.reduced_rhs(ne, gvec)
    gs, delta, _ = _gpu_solver(p, path=path, **_cfg_flags(p))
    if path == 'pairmajor':
        assert gs.last['path'] == 'pairmajor'
    S, rhs = gs.reduced_system_dense()
    assert S.shape == S_ref.shape
    assert rel_err(S, S_ref) < 1e-5
    assert rel_err(rhs, rhs_ref) < 1e-5
    assert rel_err(S, S.T) < 1e-12                     # symmetric by construction
    # point blocks and their damping
    T = p.n_tracks
    H = gs.point_blocks()[0].cpu()
    Hr = ne.leaves['pts'] - float(gs.last['lam_p'].cpu()) * torch.eye(3, dtype=torch.float64)
    iu = [(0, 0), (0, 1), (0, 2), (1, 1), (1, 2), (2, 2)]
    Hr6 = torch.stack([Hr[:, i, j] for i, j in iu], 1)
    assert rel_err(H, Hr6) < 1e-5


def _with_repeats(p, frac=0.15, seed=3):
    """p with about frac of its observations repeated in their own image (the copy right after the
    original, so pids stay ascending inside each image), its pixel moved by (0.7, -0.4): runs of two
    observations of one track in one image, which both fused paths sum into one V per run."""
    import dataclasses
    rng = np.random.default_rng(seed)
    n = p.n_obs
    rep = rng.random(n) < frac
    idx = torch.from_numpy(np.repeat(np.arange(n), np.where(rep, 2, 1)))
    second = torch.zeros(len(idx), dtype=torch.bool)
    second[1:] = idx[1:] == idx[:-1]
    cum = p.infos[0].long()
    start = torch.cat([cum.new_zeros(1), cum[:-1]])
    img = torch.repeat_interleave(torch.arange(p.n_imgs), cum - start)
    cnt = torch.bincount(img[idx], minlength=p.n_imgs)
    infos = p.infos.clone()
    infos[0] = torch.cumsum(cnt, 0).to(torch.int32)
    pix = p.pix2d[idx].clone()
    pix[second] += torch.tensor([0.7, -0.4])
    return dataclasses.replace(p, infos=infos.contiguous(), pids=p.pids[idx].contiguous(), pix2d=pix.contiguous(),
                               pix2d_std=p.pix2d_std[idx].contiguous(), pix2d_dep=p.pix2d_dep[idx].contiguous())


@pytest.mark.parametrize('cfg,nf,nt,path', [(0, 8, 200, 'batched'), (0, 8, 200, 'pairmajor'), (2, 24, 800, 'batched'),
                                            (2, 24, 800, 'pairmajor'), (3, 24, 600, 'pairmajor')])
def test_repeated_observations_in_one_image(cfg, nf, nt, path):
    """A track observed twice in one image (about 15% of the observations repeated): S, rhs and the point
    blocks, then the PCG step with its back-substitution, against the oracle on both fused paths (the
    batched pass sums the run's V into its first slot, the pair-major runs sum their observations in
    k_pm_runs and k_pm_backsub reads one V per run)."""
    print(f'repeated observations cfg {cfg} ({nf} frames, {nt} tracks), {path}', flush=True)
    p = _with_repeats(make_problem(cfg, n_frames=nf, n_tracks=nt))
    cum = p.infos[0].long()
    img = torch.repeat_interleave(torch.arange(p.n_imgs), torch.diff(torch.cat([cum.new_zeros(1), cum])))
    key = img * p.n_tracks + p.pids.long()
    assert (torch.diff(key) == 0).sum() > 0.1 * p.n_obs     # the repeats are there, next to each other
    _check_reduced_system(p, path)
    _check_pcg_step(p, path, cfg)


def test_auto_path_on_far_apart_track_images_builds_no_batched_plan():
    """path='auto' where tracks lie on far-apart images (config 3's random neighbours in a 96-frame
    collection, median span 77 images): the pair-major pass, decided from the structure's track spans
    without building the batched plan, with the reduced system against the oracle."""
    from blast3r_amd import plan as P
    p = make_problem(3, n_frames=96, n_tracks=1200)
    _check_reduced_system(p, 'auto')
    gs, _, g = _gpu_solver(p, 'auto')
    assert gs.last['path'] == 'pairmajor'
    kinds = [ent[6].kind for ent in P._cache.get(id(g.pids), []) if ent[0]() is g.pids]
    assert 'span' in kinds and 'pairmajor' in kinds and 'batched' not in kinds, kinds


@pytest.mark.parametrize('cfg,nf,nt', [(0, 6, 60), (0, 12, 600), (1, 32, 400), (2, 24, 800), (3, 24, 600),
                                        (4, 12, 300)])
def test_pcg_step_parity(cfg, nf, nt):
    _check_pcg_step(make_problem(cfg, n_frames=nf, n_tracks=nt), 'auto', cfg)


@pytest.mark.parametrize('cfg,nf,nt,kw', PM_CASES, ids=PM_IDS)
def test_pcg_step_parity_pairmajor(cfg, nf, nt, kw):
    print(f'pair-major PCG step cfg {cfg} {kw}', flush=True)
    _check_pcg_step(make_problem(cfg, n_frames=nf, n_tracks=nt, **kw), 'pairmajor', cfg)


def _check_pcg_step(p, path, cfg):
    """delta from the device PCG against the oracle restatement of _pcg.

    The device's iterate (after k updates: the converged one, else the best so far) is compared
    with the oracle's iterate after the same k updates.  On an ill-conditioned system CG amplifies
    rounding: perturbing b by 1e-15 relative moves the oracle's own k-th iterate by ~1e-3 on
    configs 1 and 4 (condition numbers ~1e11).  So the bar is max(1e-4, 5x the largest such move
    over four perturbed oracle runs: three of b, one applying S as a dense matrix) on delta and on
    J.delta; on well-conditioned cases (configs 0, 2, 3) that is the plain 1e-4.  The stopping
    decisions are checked separately: the same converged flag, a converged count within 5% of the
    oracle's (at least 2: config 4's moves between 151 and 156 under those perturbations; twice the
    largest move of the oracle's own count under those perturbations where that is larger), the
    stopping test met on the oracle's S (to 2x: the device stops on its own rounding of S), and a
    run stopped at maxiter reaching the oracle's reduced residual.
    """
    fl = _cfg_flags(p)
    ne, gvec, params, (Jc, Jz, Jp), res, w = _oracle_ne(p, **fl)
    d_ref, it_ref, conv_ref = osol.solve_reduced_pcg(ne, gvec)
    gs, delta, _ = _gpu_solver(p, path=path, **fl)
    assert gs.last['path'] == path or path == 'auto'
    ist = gs.last['istate'].cpu()
    assert int(ist[3]) == int(conv_ref)
    from oracle.dense import dense_jacobian
    Jd = dense_jacobian(Jc, Jz, Jp, p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks)
    sW = w.clamp(1e-6, 1e6).reshape(-1).double().sqrt()
    Jdelta = lambda d: sW[:, None] * Jd @ d.cpu().double()
    n_c = ne.sizes['n_c']
    S = osol.dense_schur(ne)
    rhs = osol.reduced_rhs(ne, gvec)
    diagA = osol.A_diag(ne).clamp(min=1e-12)
    M = lambda v: v / diagA
    red = lambda dc: float((rhs - S @ dc).norm() / rhs.norm())
    if conv_ref:
        # the oracle's own count under the same rounding perturbations as below (a 1e-15 relative
        # change of b moves it from 249 to 275 on the width-16 case, condition number ~1e19)
        gen = torch.Generator().manual_seed(1000 + cfg)
        spread = 0
        for A_mv, b in [(lambda v: S @ v, rhs)] + [
                (lambda v: osol.S_matvec(ne, v), rhs * (1 + 1e-15 * torch.randn(rhs.shape, generator=gen,
                                                                                 dtype=rhs.dtype)))
                for _ in range(3)]:
            _, it_alt, conv_alt = osol.pcg(A_mv, b, M_mv=M, tol=1e-6, maxiter=300)
            spread = max(spread, abs(it_alt - it_ref) if conv_alt else 300)
        assert abs(int(ist[2]) - it_ref) <= max(2, 0.05 * it_ref, 2 * spread), (int(ist[2]), it_ref, spread)
        assert red(delta[:n_c].cpu().double()) <= 2e-6
    else:
        assert red(delta[:n_c].cpu().double()) <= 1.5 * red(d_ref[:n_c])
    # the oracle's iterate after the device's k updates, and its sensitivity to rounding there
    k = int(ist[2]) if conv_ref else int(ist[4])
    assert k >= 1
    full = lambda dc: torch.cat([dc, osol._D_solve(ne, gvec[n_c:] - osol._C_matvec(ne, dc))])

    def kth(A_mv, b):
        hist = []
        osol.pcg(A_mv, b, M_mv=M, tol=0.0, maxiter=k, history=hist)
        return full(hist[k - 1])

    ref_k = kth(lambda v: osol.S_matvec(ne, v), rhs)
    gen = torch.Generator().manual_seed(cfg)
    alts = [kth(lambda v: S @ v, rhs)]
    for _ in range(3):
        e = 1 + 1e-15 * torch.randn(rhs.shape, generator=gen, dtype=rhs.dtype)
        alts.append(kth(lambda v: osol.S_matvec(ne, v), rhs * e))
    tol_d = max([1e-4] + [5 * rel_err(d, ref_k) for d in alts])
    tol_j = max([1e-4] + [5 * rel_err(Jdelta(d), Jdelta(ref_k)) for d in alts])
    assert rel_err(delta, ref_k.to(torch.float32)) < tol_d, (rel_err(delta, ref_k.to(torch.float32)), tol_d)
    # gauge-invariant check: the predicted residual change J.delta
    assert rel_err(Jdelta(delta), Jdelta(ref_k)) < tol_j


def _device_pcg_dense(A, b, tol, maxiter, d):
    """ba_pcg_solve on a dense system laid out as n / d images of d parameters, every image pair a
    block, identity unknown map, no damping; returns (x, istate)."""
    import ctypes
    import numpy as np
    from blast3r_amd._lib import BaPcgArgs, check, lib, stream_ptr
    n = len(b)
    assert n % d == 0
    m = n // d
    pairs = [(i1, i2) for i1 in range(m) for i2 in range(i1, m)]
    S_pairs = np.stack([A[i1 * d:(i1 + 1) * d, i2 * d:(i2 + 1) * d] for i1, i2 in pairs])
    rows = [[] for _ in range(m)]
    for q, (i1, i2) in enumerate(pairs):
        rows[i1].append(q << 1)
        if i2 != i1:
            rows[i2].append((q << 1) | 1)
    row_ptr = np.cumsum([0] + [len(r) for r in rows])
    t = lambda a, dt: torch.as_tensor(np.ascontiguousarray(a), dtype=dt, device=DEV)
    i32, f64 = torch.int32, torch.float64
    keep = dict(umap=t(np.arange(n), i32), inv_ptr=t(np.arange(n + 1), i32), inv_src=t(np.arange(n), i32),
                leaf=t(np.zeros(n), i32), row_ptr=t(row_ptr, i32), row_ent=t(np.concatenate(rows), i32),
                pair_i1=t([q[0] for q in pairs], i32), pair_i2=t([q[1] for q in pairs], i32),
                S_pairs=t(S_pairs, f64), e_img=t(b, f64), dg_img=t(np.diag(A), f64))
    n_ent = int(row_ptr[-1])
    for name, size in dict(rhs=n, diagA=n, damp=n, x=n, xbest=n, r=n, z=n, p=2 * n, y_img=n, img_part=m,
                           partials=int(lib().ba_pcg_partials_size(n)), state=16, S_rows=n_ent * d * d).items():
        keep[name] = torch.zeros(size, dtype=f64, device=DEV)
    keep['istate'] = torch.zeros(8, dtype=i32, device=DEV)
    keep['row_u'] = torch.zeros(n_ent * 16, dtype=i32, device=DEV)
    keep['long_u'] = torch.zeros(1, dtype=i32, device=DEV)
    keep['long_ptr'] = torch.zeros((n + 255) // 256 + 1, dtype=i32, device=DEV)
    keep['long_idx'] = torch.full((n,), -1, dtype=i32, device=DEV)
    pa = BaPcgArgs()
    pa.n_u, pa.n_imgs, pa.d = n, m, d
    pa.dampen, pa.adaptive, pa.maxiter, pa.tol = 0.0, 0, int(maxiter), float(tol)
    pa.n_row_ent, pa.n_long = n_ent, 0
    for name, v in keep.items():
        setattr(pa, name, v.data_ptr())
    check(lib().ba_pcg_solve(ctypes.byref(pa), stream_ptr(DEV)))
    torch.cuda.synchronize()
    return keep['x'].cpu(), keep['istate'].cpu()


@pytest.mark.parametrize('case,d,rtol', [('converges', 15, 1e-6), ('maxiter_hit', 15, 1e-12), ('ill_conditioned', 10, None),
                                         ('indefinite', 6, 1e-12), ('zero_rhs', 15, 0.0)])
def test_device_pcg_against_reference_vectors(case, d, rtol):
    """ba_pcg_solve's iterate sequence, stopping rule and best-so-far choice against the reference
    _pcg's own outputs (tests/golden/pcg_golden.npz).  Tolerances: the converging case follows a
    45-step fp64 recurrence whose rounding depends on the order of the dot-product sums: its last
    step drops the residual from about 4x to between 0.45x and 1.24x the threshold depending on that
    order alone, so it stops at iteration 45 or 46 (either way x agrees with the reference's to
    5e-8; bar 1e-6); the short cases match to rounding (1e-12); at condition number 1e9 a different
    summation order already changes the best iterate (a reordered fp64 restatement picks iteration
    15 where the reference picks 24), so only the outcome (not converged) is compared there."""
    import os
    import numpy as np
    print(f'device pcg golden case {case}', flush=True)
    z = np.load(os.path.join(os.path.dirname(__file__), 'golden', 'pcg_golden.npz'))
    A, b = z[f'{case}/A'], z[f'{case}/b']
    x, ist = _device_pcg_dense(A, b, float(z[f'{case}/tol']), int(z[f'{case}/maxiter']), d)
    conv = bool(z[f'{case}/converged'])
    assert bool(ist[3]) == conv
    if rtol is None:
        return
    slack = 1 if case == 'converges' else 0
    assert abs(int(ist[2] if conv else ist[4]) - int(z[f'{case}/iters'])) <= slack
    xr = torch.from_numpy(z[f'{case}/x'])
    if float(xr.norm()) == 0:
        assert float(x.norm()) == 0.0
    else:
        assert rel_err(x, xr) <= rtol


def test_pcg_graph_replay_matches_eager():
    """The PCG replayed from its captured HIP graph equals the eager launches bit for bit on every
    replay, with the program's own eager work and synchronisations between the replays."""
    p = make_problem(0, n_frames=12, n_tracks=600)
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    hp = dict(weight_z=o['weight_z'], pnorm=1.0, max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])

    def solve(use_graph):
        gs = GaussNewtonSolver(len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks, DEV, dtype=torch.float64, use_graph=use_graph)
        J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                                 g.pix2d_dep, True, pix2d=g.pix2d, hp=hp)
        d = gs.solve_delta(J, res, w)
        return d.clone(), gs.last['istate'].clone()

    d_e, ist_e = solve(False)
    torch.cuda.synchronize()
    for rep in range(3):
        d_g, ist_g = solve(True)
        torch.cuda.synchronize()
        y = torch.randn(4096, device=DEV)
        assert float((y * y).sum()) > 0                     # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(ist_g, ist_e), rep
        assert torch.equal(d_g, d_e), rep


def test_solver_flags_parity():
    """optim_K / optim_P off (depth stitching), optim_X off, tensor masks, optim_Z0 off.  The tensor
    optim_X case checks the per-track semantics this build gives a track mask (the observations of a
    disabled track drop out, the enabled tracks are compacted in order); the reference indexes the
    mask by the observation's image id instead (ba_solver.py:83, :98), which for a track mask is an
    indexing slip, not a rule a caller could rely on."""
    p4 = make_problem(4, n_frames=10, n_tracks=300)
    p0 = make_problem(0, n_frames=10, n_tracks=300)
    cases = [(p4, dict(optim_K=False, optim_P=False)),
             (p0, dict(optim_X=False)),
             (p0, dict(optim_Z0=False)),
             (p0, dict(no_grad_f_from_rz=True)),
             (p0, dict(optim_K=False)),
             (p0, dict(optim_P=torch.tensor([True] * 5 + [False] * 5))),
             (p0, dict(optim_Z=torch.tensor([False] * 3 + [True] * 7))),
             (p0, dict(optim_X=torch.arange(p0.n_tracks) % 3 != 0))]
    for p, flags in cases:
        ne, gvec, params, _, _, _ = _oracle_ne(p, **flags)
        d_ref, _, _ = osol.solve_reduced_pcg(ne, gvec)
        gs, delta, _ = _gpu_solver(p, **flags)
        assert delta.shape == d_ref.shape, flags
        assert rel_err(delta, d_ref.to(torch.float32)) < 1e-4, flags


def test_two_masks_of_equal_size_on_one_plan():
    """Two solve_delta calls on one structure plan with different pose masks holding the same number
    of True entries (the unknown maps are cached per plan, keyed by the mask's content): each step
    matches the oracle's for its own mask."""
    p = make_problem(0, n_frames=10, n_tracks=300)
    T_, F_ = [True] * 5, [False] * 5
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    hp = dict(weight_z=o['weight_z'], pnorm=1.0, max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    plans = set()
    for mask in (torch.tensor(T_ + F_), torch.tensor(F_ + T_), torch.tensor(T_ + F_)):
        ne, gvec, params, _, _, _ = _oracle_ne(p, optim_P=mask)
        d_ref, _, _ = osol.solve_reduced_pcg(ne, gvec)
        gs = GaussNewtonSolver(len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks, DEV, dtype=torch.float64)
        J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                                 g.pix2d_dep, True, pix2d=g.pix2d, hp=hp, optim_P=mask.to(DEV))
        delta = gs.solve_delta(J, res, w)
        plans.add(id(gs.last['plan']))
        assert rel_err(delta, d_ref.to(torch.float32)) < 1e-4, mask
    assert len(plans) == 1


@pytest.mark.parametrize('cfg,nf,nt,kw,path', [(0, 8, 300, {}, 'pairmajor'), (0, 8, 300, {}, 'batched'),
                                                (2, 24, 800, {}, 'pairmajor'), (2, 24, 800, {}, 'batched'),
                                                (3, 24, 600, {}, 'pairmajor'), (4, 12, 300, {}, 'pairmajor'),
                                                (4, 12, 300, {}, 'batched'), (2, 16, 300, dict(n_channels=16), 'pairmajor')],
                         ids=['cfg0-pm', 'cfg0-batched', 'cfg2-pm', 'cfg2-batched', 'cfg3-pm', 'cfg4-pm', 'cfg4-batched',
                              'd25-pm'])
def test_reduced_system_fp32(cfg, nf, nt, kw, path):
    """dtype=torch.float32, the reference's GaussNewtonSolver default (bs:22: fp32 Jacobian, fp32 normal
    equations and Schur algebra, bs:37, :128): the pass in fp32 on either path (fp32 sums, point factors and
    16x16x4 fp32 MFMA tiles) gives S, the rhs and the point blocks within 5x (at least 1e-5) of the distance
    of the oracle's own fp32 algebra from the fp64 result, i.e. no less accurate than the reference's
    fp32 path."""
    print(f'fp32 reduced system cfg {cfg} {kw} {path}', flush=True)
    p = make_problem(cfg, n_frames=nf, n_tracks=nt, **kw)
    flags = _cfg_flags(p)
    ne64, g64, _, _, _, _ = _oracle_ne(p, **flags)
    ne32, g32, _, _, _, _ = _oracle_ne(p, dtype=torch.float32, **flags)
    S64, rhs64 = osol.dense_schur(ne64), osol.reduced_rhs(ne64, g64)
    S32, rhs32 = osol.dense_schur(ne32).double(), osol.reduced_rhs(ne32, g32).double()
    gs, delta, _ = _gpu_solver(p, path=path, dtype=torch.float32, **flags)
    assert gs.last['path'] == path and gs.last['S_pairs'].dtype == torch.float32
    assert delta.dtype == torch.float32 and bool(torch.isfinite(delta).all())
    S, rhs = gs.reduced_system_dense()
    for name, dev, ref, orc in (('S', S.cpu(), S64, S32), ('rhs', rhs.cpu(), rhs64, rhs32)):
        e_dev, e_or = rel_err(dev, ref), rel_err(orc, ref)
        print(f'  {name}: device fp32 {e_dev:.2e}, oracle fp32 {e_or:.2e} from fp64', flush=True)
        assert e_dev <= max(1e-5, 5 * e_or), (name, e_dev, e_or)
    iu = [(0, 0), (0, 1), (0, 2), (1, 1), (1, 2), (2, 2)]
    H = gs.point_blocks()[0].cpu()
    H64 = torch.stack([ne64.leaves['pts'][:, i, j] for i, j in iu], 1)
    H32 = torch.stack([ne32.leaves['pts'][:, i, j] for i, j in iu], 1).double()
    assert rel_err(H, H64) <= max(1e-5, 5 * rel_err(H32, H64))


@pytest.mark.parametrize('cfg,nf,nt', [(0, 8, 300), (2, 30, 1500), (3, 24, 600), (4, 20, 800)])
def test_lm_step_default_dtype_is_the_fp32_solver(cfg, nf, nt):
    """lm_step called without dtype runs the reference's fp32 solver (GaussNewtonSolver's default,
    bs:22, which lm_step uses unless told otherwise, en:284): the step is checked against the oracle's
    lm_step with its own default (fp32 throughout):
      * the same initial loss (1e-5);
      * the device's fp32 PCG against the oracle's fp32 _pcg (bs:1197-1238) on the device's own reduced
        system, after the device's number of updates, to 1e-4 widened only by 5x the move of that iterate
        when S is applied transposed or b moves by one fp32 ulp;
      * sqrt(W) J delta, the residual change the step predicts, within 5x (at least 1e-4) of the distance
        of the oracle's fp32 step from the exact (fp64, direct) solution of the same system;
      * the oracle's line search (en:305-333) run on the device's step: the same scales and accepted
        one, loss and parameters within 1e-5."""
    from tests.step_checks import weighted_jdelta
    print(f'lm_step default dtype (fp32) cfg {cfg}', flush=True)
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    o = p.options
    kw = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, optim_K=o['optim_K'],
              optim_P=o['optim_P'])
    hp = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, clip_pix_err=100)
    info = {}
    up_g, st_g, _ = gpu_engine._lm_step(**_gpu(p).lm_inputs(), **kw, info=info)
    gs = info['solver']
    assert gs.dtype == torch.float32 and gs.last['S_pairs'].dtype == torch.float32
    print(f"  path {gs.last['path']}", flush=True)
    inp = p.lm_inputs()
    _, st_o, info_o = oeng.lm_step(**inp, **kw)
    assert info_o['delta'].dtype == torch.float32 and info_o['ne'].leaves['foc'].dtype == torch.float32
    sysd = _oracle_system(inp, hp, dict(optim_K=o['optim_K'], optim_P=o['optim_P']))
    assert abs(float(st_g.init_loss) - float(sysd['loss'])) <= 1e-5 * abs(float(sysd['loss']))
    # the device's fp32 PCG against the oracle's fp32 _pcg on the device's own system
    S_dev, rhs_dev, dA_dev = device_system(gs)
    S32, b32, d32 = S_dev.float(), rhs_dev.float(), dA_dev.clamp(min=1e-12).float()
    ist = info['pcg_istate'].cpu()
    k = int(ist[2]) if int(ist[3]) else int(ist[4])
    assert k >= 1

    def kth(A_mv, b):
        hist = []
        osol.pcg(A_mv, b, M_mv=lambda v: v / d32, tol=0.0, maxiter=k, history=hist)
        return hist[k - 1]
    gen = torch.Generator().manual_seed(cfg)
    same = kth(lambda v: S32 @ v, b32)
    alts = [kth(lambda v: S32.T @ v, b32),
            kth(lambda v: S32 @ v, b32 * (1 + 2.0 ** -23 * torch.randn(b32.shape, generator=gen)))]
    n_c = b32.shape[0]
    tol_d = max([1e-4] + [5 * rel_err(a, same) for a in alts])
    e_d = rel_err(info['delta'][:n_c].cpu(), same)
    # sqrt(W) J delta against the exact solution, beside the oracle's own fp32 step
    jd_true = weighted_jdelta(sysd, osol.solve_reduced_direct(sysd['ne'], sysd['g']))
    e_dev = rel_err(weighted_jdelta(sysd, info['delta']), jd_true)
    e_or = rel_err(weighted_jdelta(sysd, info_o['delta']), jd_true)
    print(f'  k={k}: device PCG vs oracle fp32 _pcg {e_d:.2e} (bar {tol_d:.2e}); sqrt(W) J delta from the exact '
          f'step: device {e_dev:.2e}, oracle fp32 {e_or:.2e}', flush=True)
    assert e_d <= tol_d, (e_d, tol_d)
    assert e_dev <= max(1e-4, 5 * e_or), (e_dev, e_or)
    _check_line_search(inp, hp, sysd, info['delta'], info, st_g, up_g)


def test_fp32_solver_limits():
    """The direct (fp64) Cholesky refuses dtype=torch.float32 with an error instead of running in another
    precision; other dtypes are refused too; both passes take fp32."""
    with pytest.raises(ValueError, match='float64'):
        GaussNewtonSolver(1, 4, 4, 10, DEV, dtype=torch.float32, solver='cholesky')
    for path in ('batched', 'pairmajor', 'auto'):
        assert GaussNewtonSolver(1, 4, 4, 10, DEV, dtype=torch.float32, path=path).real32
    with pytest.raises(ValueError, match='dtype'):
        GaussNewtonSolver(1, 4, 4, 10, DEV, dtype=torch.float16)
    assert GaussNewtonSolver(1, 4, 4, 10, DEV).dtype == torch.float32


def _cpu_inputs(d):
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


@pytest.mark.parametrize('cfg,nf,nt', [(0, 8, 300), (1, 32, 400), (2, 30, 1500), (3, 24, 600), (4, 20, 800)])
def test_lm_step_parity(cfg, nf, nt):
    """Full lm_step against the oracle, with no widening beyond the rounding-sensitivity bound:
    the step delta it solved against the oracle's PCG iterate after the same number of updates
    (1e-4 on delta and on sqrt(W) J delta), then the oracle's line search on that same delta: the same
    scales tried and accepted, loss and updated parameters within 1e-5."""
    print(f'lm_step parity cfg {cfg} ({nf} frames, {nt} tracks)', flush=True)
    _check_lm_step(make_problem(cfg, n_frames=nf, n_tracks=nt), cfg, {})


@pytest.mark.parametrize('cfg,nf,nt,kw', [PM_CASES[i] for i in (2, 3, 5, 6, 7)],
                         ids=[PM_IDS[i] for i in (2, 3, 5, 6, 7)])
def test_lm_step_parity_pairmajor(cfg, nf, nt, kw):
    """lm_step on the pair-major path (forced), same bars as the batched path."""
    print(f'pair-major lm_step parity cfg {cfg} {kw}', flush=True)
    _check_lm_step(make_problem(cfg, n_frames=nf, n_tracks=nt, **kw), cfg, dict(path='pairmajor'))


@pytest.mark.parametrize('cfg,nf,nt', [(0, 8, 300), (2, 70, 3000), (4, 20, 800)])
def test_lm_step_direct_solve_parity(cfg, nf, nt):
    """lm_step with solver='cholesky' (the reference's _solve_dense_S, ba_solver.py:208-226, in place of its
    default _solve_CG; banded by cyclic reduction on configs 2 and 4): the step delta against the oracle's
    direct solve on sqrt(W) J delta to 1e-6 (widened only by 5x the oracle's own move when its fp32 inputs
    are rounded differently), then the oracle's line search on that same delta: the same scales tried and
    accepted, loss and updated parameters within 1e-5."""
    from tests.step_checks import rounded_differently, weighted_jdelta
    print(f'lm_step (direct solve) parity cfg {cfg} ({nf} frames, {nt} tracks)', flush=True)
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    o = p.options
    kw = dict(dtype=torch.float64,
              weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, optim_K=o['optim_K'],
              optim_P=o['optim_P'], solver='cholesky')
    hp = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, clip_pix_err=100)
    g = _gpu(p)
    info = {}
    up_g, st_g, _ = gpu_engine._lm_step(**g.lm_inputs(), **kw, info=info)
    direct = info['solver'].last['direct']
    assert direct is not None and direct['first_bad_pivot'] is None
    if cfg in (2, 4):
        assert direct['layout'] == 'banded' and direct['superblocks'] >= 1
    inp = p.lm_inputs()
    sysd = _oracle_system(inp, hp, dict(optim_K=o['optim_K'], optim_P=o['optim_P']))
    assert abs(float(st_g.init_loss) - float(sysd['loss'])) <= 1e-5 * abs(float(sysd['loss']))
    ref = osol.solve_reduced_direct(sysd['ne'], sysd['g'])
    jd_ref = weighted_jdelta(sysd, ref)
    gen = torch.Generator().manual_seed(cfg)
    moves = [rel_err(weighted_jdelta(sysd, osol.solve_reduced_direct(alt['ne'], alt['g'])), jd_ref)
             for alt in (rounded_differently(sysd, gen) for _ in range(2))]
    bar = max([1e-6] + [5 * m for m in moves])
    e_j = rel_err(weighted_jdelta(sysd, info['delta']), jd_ref)
    print(f'  {direct}: sqrt(W) J delta {e_j:.2e} (bar {bar:.1e})', flush=True)
    assert e_j <= bar, (e_j, bar)
    _check_line_search(inp, hp, sysd, info['delta'], info, st_g, up_g)


def _check_lm_step(p, cfg, solver_kw):
    o = p.options
    kw = dict(dtype=torch.float64,
              weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, optim_K=o['optim_K'],
              optim_P=o['optim_P'], depth_mode=o['depth_mode'], **solver_kw)
    hp = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, clip_pix_err=100,
              is_depth_log=_is_log(p))
    g = _gpu(p)
    info = {}
    up_g, st_g, _ = gpu_engine._lm_step(**g.lm_inputs(), **kw, info=info)
    if solver_kw.get('path') == 'pairmajor':
        assert info['solver'].last['path'] == 'pairmajor'
    inp = p.lm_inputs()
    sysd = _oracle_system(inp, hp, dict(optim_K=o['optim_K'], optim_P=o['optim_P']))
    assert abs(float(st_g.init_loss) - float(sysd['loss'])) <= 1e-5 * abs(float(sysd['loss']))
    _check_step_delta(sysd, info['delta'], info['pcg_istate'].cpu(), seed=cfg,
                      reduced=device_system(info['solver']))
    _check_line_search(inp, hp, sysd, info['delta'], info, st_g, up_g)


def _ba_inputs(p, dev):
    from blast3r_amd.data import from_problem
    rig, trk, X = from_problem(p)
    return rig.to(dev), trk.to(dev), X.to(dev)


def test_bundle_adjustment_reuses_trial_objective_exactly():
    """bundle_adjustment starts each step from the objective its accepted trial already evaluated
    (instead of evaluating it again, en:281); the parameters it returns equal, bit for bit, those of
    a chain of lm_step calls that each evaluate their own start."""
    p = make_problem(0, n_frames=8, n_tracks=200)
    o = p.options
    rig, trk, X = _ba_inputs(p, DEV)
    kw = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'])
    rig_out, X_out = gpu_engine.bundle_adjustment(rig, trk, X, z_coefs=p.z_coefs.to(DEV), max_iters=4, pnorm=1.0,
                                                  verbose=False, **kw)
    var = dict(K=rig.K, P_rig2cam=rig.P_rig2cam, P_w2rig=rig.P_w2rig, z_coefs=p.z_coefs.to(DEV), pts3d=X)
    infos = rig.infos(trk)
    n_acc = 0
    for _ in range(4):
        up, st = gpu_engine.lm_step(infos, trk.pids, trk.pix2d, trk.pix2d_std, trk.pix2d_dep, **var, pnorm=1.0,
                                    depth_mode='log', dampen=1e-12, adaptive_dampen=True, dtype=torch.float64, **kw)
        if st.new_loss >= st.init_loss:
            break
        var.update(up)
        n_acc += 1
    assert n_acc >= 2
    for k, got in (('K', rig_out.K), ('P_w2rig', rig_out.P_w2rig), ('z_coefs', rig_out.z_coefs), ('pts3d', X_out)):
        assert torch.equal(got, var[k]), k


@pytest.mark.parametrize('cfg,nf,nt', [(0, 8, 300), (2, 20, 600), (3, 20, 500)])
def test_bundle_adjustment_parity(cfg, nf, nt, monkeypatch):
    _check_bundle_adjustment(make_problem(cfg, n_frames=nf, n_tracks=nt), cfg, [3, None], monkeypatch)


@pytest.mark.parametrize('case', ['d25', 'long'])
def test_bundle_adjustment_parity_wide_and_long(case, monkeypatch):
    """Two phases with n_zcfs [1, 17] on 17 depth channels (image-level width 9, batched path, then
    25, pair-major path), and two phases on tracks spanning 20 to 30 images (pair-major path), with
    the same step-by-step checks."""
    if case == 'd25':
        p = make_problem(2, n_frames=16, n_tracks=300, n_channels=16)
        _check_bundle_adjustment(p, 20, [1, 17], monkeypatch, paths={'batched', 'pairmajor'})
    else:
        p = make_problem(2, n_frames=40, n_tracks=300, track_len=(20, 30))
        _check_bundle_adjustment(p, 21, [3, None], monkeypatch, paths={'pairmajor'})


def _check_bundle_adjustment(p, cfg, n_zcfs, monkeypatch, paths=None):
    """Two phases (pnorm 1 then 0.5; n_zcfs 3 -> first coefficient frozen, 4 columns) on a circle
    (config 0), forward motion (config 2) and random neighbours with a camera per frame (config 3),
    replayed step by step against the oracle: every lm_step bundle_adjustment takes is checked where
    it starts (the device's own parameters, narrowed depth channels and z-coefficients, optim_Z0):
    initial loss, step delta (1e-4, rounding-sensitivity bound only) and the oracle's line search on
    that delta (same scales, loss and parameters within 1e-5); the phase loop then stops where the
    oracle's loss test says (en:496-497) and the z-coefficients keep their frozen column."""
    print(f'bundle_adjustment parity case {cfg} n_zcfs {n_zcfs}', flush=True)
    o = p.options
    kw = dict(max_iters=[2, 2], pnorm=[1.0, 0.5], n_zcfs=n_zcfs, weight_z=o['weight_z'],
              huber_delta=o['huber_delta'])
    n_last = n_zcfs[-1] or n_zcfs[0] + 1
    steps = []
    real = gpu_engine._lm_step

    def spy(rigs, pids, pix2d, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs, pts3d, **k):
        inp = _cpu_inputs(dict(rigs=rigs, pids=pids, pix2d=pix2d, pix2d_std=pix2d_std, pix2d_dep=pix2d_dep, K=K,
                               P_rig2cam=P_rig2cam, P_w2rig=P_w2rig, z_coefs=z_coefs, pts3d=pts3d))
        info = {}
        out = real(rigs, pids, pix2d, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs, pts3d, info=info, **k)
        info['reduced'] = device_system(info['solver'])       # before the next step reuses the plan
        steps.append((inp, dict(k), info, out))
        return out

    monkeypatch.setattr(gpu_engine, '_lm_step', spy)
    rig, trk, X = _ba_inputs(p, DEV)
    rig_out, X_out = gpu_engine.bundle_adjustment(rig, trk, X, z_coefs=p.z_coefs.to(DEV), verbose=False, **kw)
    assert torch.equal(trk.pix2d_dep, p.pix2d_dep.to(DEV))            # restored after the phases
    assert rig_out.z_coefs.shape == (p.z_coefs.shape[0], n_last)
    if n_zcfs[-1] is None:                                              # the last phase keeps column 0 frozen
        assert torch.equal(rig_out.z_coefs[:, 0].cpu(), p.z_coefs[:, 0])
    assert len(steps) >= 3
    if paths is not None:
        assert {info['solver'].last['path'] for _, _, info, _ in steps} == paths
    accepted = 0
    for n, (inp, k, info, (up_g, st_g, _)) in enumerate(steps):
        hp = dict(weight_z=k['weight_z'], huber_delta=k.get('huber_delta', o['huber_delta']), pnorm=k['pnorm'],
                  clip_pix_err=k.get('clip_pix_err', 100))
        flags = {f: k[f] for f in ('optim_K', 'optim_P', 'optim_Z', 'optim_X', 'optim_Z0')}
        flags['no_grad_f_from_rz'] = k.get('no_grad_f_from_rz', False)
        sysd = _oracle_system(inp, hp, flags)
        assert abs(float(st_g.init_loss) - float(sysd['loss'])) <= 1e-5 * abs(float(sysd['loss'])), n
        _check_step_delta(sysd, info['delta'], info['pcg_istate'].cpu(), seed=100 * cfg + n,
                          reduced=info['reduced'])
        ls = _check_line_search(inp, hp, sysd, info['delta'], info, st_g, up_g)
        stop = not bool(ls['new_loss'] < ls['init_loss'])               # en:496
        assert stop == bool(st_g.new_loss >= st_g.init_loss), n
        accepted += not stop
    assert accepted >= 2
    # the returned parameters are the last accepted step's
    last = [s for s in steps if not bool(s[3][1].new_loss >= s[3][1].init_loss)][-1][3][0]
    for key, got in (('K', rig_out.K), ('P_w2rig', rig_out.P_w2rig), ('z_coefs', rig_out.z_coefs), ('pts3d', X_out)):
        assert torch.equal(got, last[key]), key


@pytest.mark.parametrize('cfg,nf,nt,q', [(0, 8, 300, 5), (2, 20, 600, 12), (3, 20, 500, 7)])
def test_frozen_single_image_bundle_adjustment(cfg, nf, nt, q, monkeypatch):
    """The online pipeline's per-frame BA (pipeline.py:219-224): bundle_adjustment of frame q alone
    (rigs[q], one camera and node), over the tracks seen in it restricted to that frame (tracks[q]), with
    the points frozen (optim_X=False) and the focal frozen for a shared camera (optim_K=not mono_cam), in
    one phase (max_n_phases=1): every lm_step it takes is replayed against the oracle (initial loss, step
    delta, the oracle's line search on that delta), and the result written back through rigs[q][:] lands
    in frame q's rows only."""
    print(f'frozen single-image BA cfg {cfg} frame {q}', flush=True)
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    o = p.options
    rig, trk, X = _ba_inputs(p, DEV)
    # the pipeline's new tracks: those seen in frame q, renumbered (tracks.py:116-127), then frame q alone
    seen = torch.zeros(p.n_tracks, dtype=torch.bool)
    seen[trk[q].pids.long().cpu()] = True
    new_trk, keep = trk.remove(torch.nonzero(~seen).squeeze(1).to(DEV))
    X_new = X[keep.long()]
    q_trk = new_trk[q]
    assert q_trk.n_kpts == new_trk.n_tracks
    mono = rig.n_cams == 1
    before = {k: getattr(rig, k).clone() for k in ('K', 'P_w2rig', 'z_coefs')}
    steps = []
    real = gpu_engine._lm_step

    def spy(rigs, pids, pix2d, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs, pts3d, **k):
        inp = _cpu_inputs(dict(rigs=rigs, pids=pids, pix2d=pix2d, pix2d_std=pix2d_std, pix2d_dep=pix2d_dep, K=K,
                               P_rig2cam=P_rig2cam, P_w2rig=P_w2rig, z_coefs=z_coefs, pts3d=pts3d))
        info = {}
        out = real(rigs, pids, pix2d, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs, pts3d, info=info, **k)
        info['reduced'] = device_system(info['solver'])
        steps.append((inp, dict(k), info, out))
        return out

    monkeypatch.setattr(gpu_engine, '_lm_step', spy)
    q_rig = rig[q]
    out_rig, _ = gpu_engine.bundle_adjustment(q_rig, q_trk, X_new, optim_X=False, optim_K=not mono, max_iters=4,
                                              max_n_phases=1, pnorm=1.0, weight_z=o['weight_z'],
                                              huber_delta=o['huber_delta'], verbose=False)
    q_rig[:] = out_rig
    assert len(steps) >= 1
    accepted = 0
    for n, (inp, k, info, (up_g, st_g, _)) in enumerate(steps):
        assert inp['rigs'].shape == (3, 1) and not k['optim_X']
        hp = dict(weight_z=k['weight_z'], huber_delta=k.get('huber_delta', o['huber_delta']), pnorm=k['pnorm'],
                  clip_pix_err=k.get('clip_pix_err', 100))
        flags = {f: k[f] for f in ('optim_K', 'optim_P', 'optim_Z', 'optim_X', 'optim_Z0')}
        flags['no_grad_f_from_rz'] = k.get('no_grad_f_from_rz', False)
        sysd = _oracle_system(inp, hp, flags)
        assert abs(float(st_g.init_loss) - float(sysd['loss'])) <= 1e-5 * abs(float(sysd['loss'])), n
        _check_step_delta(sysd, info['delta'], info['pcg_istate'].cpu(), seed=300 + 10 * cfg + n,
                          reduced=info['reduced'])
        ls = _check_line_search(inp, hp, sysd, info['delta'], info, st_g, up_g)
        stop = not bool(ls['new_loss'] < ls['init_loss'])
        assert stop == bool(st_g.new_loss >= st_g.init_loss), n
        accepted += not stop
    assert accepted >= 1
    # written back into frame q's rows of the full rig data only
    node, cam = int(rig.nod_ids[q]), int(rig.cam_ids[q])
    others = torch.arange(p.n_imgs) != q
    assert torch.equal(rig.z_coefs[others.to(DEV)], before['z_coefs'][others.to(DEV)])
    assert not torch.equal(rig.P_w2rig[node], before['P_w2rig'][node])
    assert torch.equal(rig.P_w2rig[torch.arange(len(rig.P_w2rig)) != node], before['P_w2rig'][torch.arange(len(rig.P_w2rig)) != node])
    assert torch.equal(rig.K[cam], before['K'][cam]) if mono else True


def test_objective_reproj_exact():
    p = make_problem(0, n_frames=12, n_tracks=1000)
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    r = gpu_engine.reproj_score(out[:, :3])
    ref = oeng.reproj_score(out[:, :3].cpu())
    assert abs(float(r) - float(ref)) <= 1e-6 * abs(float(ref))
    loss, _ = gpu_engine._objective(out.T, p.n_obs, True)
    assert abs(float(loss) - float(out[:, 3:6].cpu().double().mean())) <= 1e-6 * float(loss)


def test_nonfinite_flags_match_torch_isfinite():
    """ba_nonfinite_flags (the batched isfinite assertions of lm_step, en:340-344) against
    torch.isfinite on spans of every alignment and size, with NaN / +-inf at the edges and inside."""
    import ctypes
    from blast3r_amd._lib import check, lib, stream_ptr
    base = torch.randn(3_000_011, device=DEV)
    cases = []
    for off, n in [(0, 0), (0, 1), (1, 1), (2, 3), (3, 5), (1, 17), (0, 64), (5, 1000), (7, 1_000_003),
                   (0, 3_000_000), (2, 2_999_999)]:
        for where in (None, 'first', 'last', 'mid'):
            if where is not None and n == 0:
                continue
            cases.append((off, n, where))
    vals = [float('nan'), float('inf'), float('-inf')]
    for start in range(0, len(cases), 16):
        part = cases[start:start + 16]
        views = []
        for j, (off, n, where) in enumerate(part):
            t = base[off:off + n].clone() if n else base[:0]
            if n and where is not None:
                i = {'first': 0, 'last': n - 1, 'mid': n // 2}[where]
                t[i] = vals[j % 3]
            # the same values at the case's offset inside a fresh buffer (alignment as in the case)
            buf = torch.randn(off + n + 4, device=DEV)
            buf[off:off + n] = t
            views.append(buf[off:off + n])
        m = len(views)
        ptrs = (ctypes.c_void_p * m)(*[v.data_ptr() for v in views])
        counts = (ctypes.c_int64 * m)(*[v.numel() for v in views])
        flags = torch.full((m,), 7, dtype=torch.int32, device=DEV)
        check(lib().ba_nonfinite_flags(ptrs, counts, m, flags.data_ptr(), stream_ptr(DEV)))
        want = torch.tensor([0 if v.isfinite().all() else 1 for v in views], dtype=torch.int32)
        assert torch.equal(flags.cpu(), want), part


def test_lm_step_rejects_nonfinite_inputs():
    """lm_step asserts isfinite on its inputs (en:340-344): the check is launched at the start of the
    step and read with the first line-search trial, before any decision is taken."""
    p = make_problem(0, n_frames=6, n_tracks=60)
    o = p.options
    kw = dict(dtype=torch.float64, weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0)
    g = _gpu(p)
    gpu_engine.lm_step(**g.lm_inputs(), **kw)                  # finite inputs pass
    for name, idx, v in [('pix2d_dep', (3, 1), float('nan')), ('K', (0, 0, 0), float('inf')),
                         ('pts3d', (-1, 2), float('-inf')), ('pix2d_std', (0, 0), float('nan'))]:
        inp = g.lm_inputs()
        bad = inp[name].clone()
        bad[idx] = v
        inp[name] = bad
        with pytest.raises(AssertionError):
            gpu_engine.lm_step(**inp, **kw)


def test_schur_work_queue_is_deterministic():
    """The camera-pair kernel's batch queue (one workgroup per CU taking batches in the planner's
    cost order) writes every batch's partial blocks to fixed places: the reduced system (S blocks,
    rhs, diag) is bit-identical to one workgroup per batch in plan order, on a plan with more
    batches than CUs (so workgroups take several batches), over repeated runs."""
    import ctypes
    from blast3r_amd._lib import check, lib
    p = make_problem(2, n_frames=100, n_tracks=20000)
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    hp = dict(weight_z=o['weight_z'], pnorm=1.0, max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    gs = GaussNewtonSolver(len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks, DEV, dtype=torch.float64,
                           plan_options=dict(max_batch_obs=400))
    J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                             g.pix2d_dep, True, pix2d=g.pix2d, hp=hp)
    ctx = gs.prepare(J, res, w)
    a, st = ctx['args'], ctx['stream']
    assert ctx['plan'].scalars['n_batches'] > torch.cuda.get_device_properties(0).multi_processor_count
    assert a.work_ctr and a.b_order

    def run():
        check(lib().ba_linearize_schur(ctypes.byref(a), st))
        torch.cuda.synchronize()
        return [ctx[k].clone() for k in ('S_pairs', 'e_img', 'dg_img')]

    ref = None
    for mode in ('queue', 'per_batch', 'plan_order', 'queue'):
        a.work_ctr = ptr_of(ctx, 'work_ctr') if mode == 'queue' else None
        a.b_order = ctx['plan'].dev['b_order'].data_ptr() if mode != 'plan_order' else None
        got = run()
        if ref is None:
            ref = got
            continue
        for x, y in zip(got, ref):
            assert torch.equal(x, y), mode


def ptr_of(ctx, name):
    return ctx['plan'].workspace(name, (1,), torch.int32).data_ptr()


def test_stream_triad():
    """ba_stream_triad (the benchmark's achievable-bandwidth probe) computes a = b + s c exactly
    (one fp64 multiply-add per element, as torch's b + s * c rounds it) for even and odd sizes,
    and rejects arrays that are not 16-byte aligned."""
    from blast3r_amd._lib import lib, stream_ptr
    for n in (1, 2, 7, 1000, 262145):
        b = torch.randn(n + 2, dtype=torch.float64, device=DEV)
        c = torch.randn(n + 2, dtype=torch.float64, device=DEV)
        a = torch.full((n + 2,), 7.0, dtype=torch.float64, device=DEV)
        assert lib().ba_stream_triad(a.data_ptr(), b.data_ptr(), c.data_ptr(), 0.25, n, stream_ptr(DEV)) == 0
        torch.cuda.synchronize()
        ref = torch.addcmul(b[:n], c[:n], torch.tensor(0.25, dtype=torch.float64, device=DEV))
        assert torch.allclose(a[:n], ref, rtol=1e-15, atol=0), n
        assert torch.all(a[n:] == 7.0)                        # nothing written past n
    x = torch.zeros(8, dtype=torch.float64, device=DEV)
    assert lib().ba_stream_triad(x.data_ptr() + 8, x.data_ptr(), x.data_ptr(), 1.0, 4, stream_ptr(DEV)) != 0


def test_backsubstitute_image_level_delta_matches_unknown_map():
    """ba_backsubstitute gives the same point steps, bit for bit, whether it reads delta_c at image
    level (dc_img) or through the unknown map (dc, umap), and with a masked parameter group."""
    import ctypes
    from blast3r_amd._lib import check, lib, ptr
    p = make_problem(2, n_frames=20, n_tracks=600)
    g = _gpu(p)
    o = opts(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    hp = dict(weight_z=o['weight_z'], pnorm=1.0, max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    for flags in ({}, dict(optim_P=False)):
        gs = GaussNewtonSolver(len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks, DEV, dtype=torch.float64)
        J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                                 g.pix2d_dep, True, pix2d=g.pix2d, hp=hp, **flags)
        gs.solve_delta(J, res, w)
        x, um, d = gs.last['x'], gs.last['unknowns'], gs.last['lay']['d']
        ctx = gs.prepare(J, res, w)                    # the same workspace, records of this linearisation
        a, st = ctx['args'], ctx['stream']
        check(lib().ba_linearize_stage(ctypes.byref(a), 0, st))
        umap = um['umap'].view(p.n_imgs, d).long()
        dc_img = torch.where(umap >= 0, x[umap.clamp(min=0)], torch.zeros((), dtype=x.dtype, device=DEV))
        outs = []
        for use_img in (True, False):
            dX = torch.zeros((p.n_tracks, 3), dtype=torch.float32, device=DEV)
            a.dc, a.umap, a.dX, a.dX64 = ptr(x), ptr(um['umap']), ptr(dX), None
            a.dc_img = ptr(dc_img) if use_img else None
            check(lib().ba_backsubstitute(ctypes.byref(a), st))
            torch.cuda.synchronize()
            outs.append(dX)
        assert torch.equal(outs[0], outs[1]), flags
        assert outs[0].abs().sum() > 0


_FULL_SIZE = {1: (256, 200_000), 2: (1024, 1_000_000), 3: (4096, 3_000_000), 4: (1024, 1_000_000)}


@pytest.mark.parametrize('cfg,path,dtype', [(2, 'auto', torch.float64), (2, 'pairmajor', torch.float64),
                                            (3, 'auto', torch.float64), (1, 'auto', torch.float64),
                                            (4, 'auto', torch.float64), (2, 'auto', torch.float32),
                                            (3, 'auto', torch.float32)],
                         ids=['cfg2', 'cfg2-pm', 'cfg3', 'cfg1', 'cfg4', 'cfg2-fp32', 'cfg3-fp32'])
def test_reduced_system_full_size_against_oracle(cfg, path, dtype):
    """Full benchmark sizes (config 1: 256 frames, 200 k tracks on 24-frame neighbourhoods, 1.3 M
    observations, pair-major; config 2: 1024 frames, 1 M tracks, 8.0 M observations, on the batched and
    the pair-major path; config 3: 4096 frames with a camera each, 3 M tracks on random neighbours,
    22.5 M observations, pair-major; config 4: config 2's scene with 9 depth channels, focal and poses
    fixed, 8.0 M observations, batched): the reduced rhs, the point blocks and S v for seeded v against
    the oracle's normal equations at the same size and with the configuration's own flags (the oracle's
    pass takes seconds on the host's threads), to the 1e-5 bar; also with dtype=torch.float32 (the
    reference's default solver precision: the pass in fp32 throughout, batched at config 2 and pair-major
    at config 3), against the same fp64 normal equations and bar."""
    import os
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    p = make_problem(cfg)
    assert (p.n_imgs, p.n_tracks) == _FULL_SIZE[cfg]
    print(f'[full cfg{cfg} {path}] {p.n_obs} observations', flush=True)
    flags = _cfg_flags(p)
    gs, _, _ = _gpu_solver(p, path=path, dtype=dtype, **flags)
    last = gs.last
    batched = (cfg, path) in ((2, 'auto'), (4, 'auto'))
    assert last['path'] == ('batched' if batched else 'pairmajor') and last['S_pairs'].dtype == dtype
    um, d, plan = last['unknowns'], last['lay']['d'], last['plan']
    rhs = last['rhs'].double().cpu()
    H = gs.point_blocks()[0].cpu()
    n_pairs = plan.scalars['n_pairs']
    B = last['S_pairs'][:n_pairs].view(n_pairs, d, d).double()
    i1 = plan.dev['pair_i1'][:n_pairs].long()
    i2 = plan.dev['pair_i2'][:n_pairs].long()
    umap = um['umap'].long().view(p.n_imgs, d)
    valid = umap >= 0
    n_u = int(um['n_u'])

    def s_matvec(v):                                  # S_u v = P^T S_img P v + damp v
        v = v.to(DEV)
        v_img = torch.where(valid, v[umap.clamp(min=0)], torch.zeros((), dtype=v.dtype, device=DEV))
        y_img = torch.zeros_like(v_img)
        y_img.index_add_(0, i1, torch.bmm(B, v_img[i2].unsqueeze(2)).squeeze(2))
        off = i1 != i2
        Bt = B[off].transpose(1, 2).contiguous()
        y_img.index_add_(0, i2[off], torch.bmm(Bt, v_img[i1[off]].unsqueeze(2)).squeeze(2))
        y = torch.zeros(n_u, dtype=v.dtype, device=DEV)
        y.index_add_(0, umap[valid], y_img[valid])
        return (y + last['damp'].double() * v).cpu()

    ne, gvec, _, _, _, _ = _oracle_ne(p, **flags)
    print(f'[full cfg{cfg}] oracle normal equations built', flush=True)
    assert rel_err(rhs, osol.reduced_rhs(ne, gvec)) < 1e-5
    Hr = ne.leaves['pts'] - float(last['lam_p'].cpu()) * torch.eye(3, dtype=torch.float64)
    iu = [(0, 0), (0, 1), (0, 2), (1, 1), (1, 2), (2, 2)]
    assert rel_err(H, torch.stack([Hr[:, i, j] for i, j in iu], 1)) < 1e-5
    gen = torch.Generator().manual_seed(7)
    for k in range(3):
        v = torch.randn(n_u, dtype=torch.float64, generator=gen)
        assert rel_err(s_matvec(v), osol.S_matvec(ne, v)) < 1e-5, k
    # S v is symmetric: u.(S v) = v.(S u)
    u = torch.randn(n_u, dtype=torch.float64, generator=gen)
    a, b = torch.dot(u, s_matvec(v)), torch.dot(v, s_matvec(u))
    assert abs(a - b) <= 1e-10 * (abs(a) + abs(b))


def test_lm_step_full_config2_line_search():
    """One lm_step at the benchmark's full config-2 size (1024 frames, 1 M tracks, 8.0 M observations):
    its initial loss equals the oracle objective at the inputs (1e-5), and the oracle's line search
    (en:305-333) run on the device's own step delta tries the same scales, accepts the same one and
    reaches the same loss (1e-5) and parameters (1e-5 on their change); every parameter stays finite."""
    import os
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    p = make_problem(2)
    o = p.options
    kw = dict(dtype=torch.float64,
              weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, optim_K=o['optim_K'],
              optim_P=o['optim_P'])
    hp = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, clip_pix_err=100)
    print(f'[full cfg2 lm_step] {p.n_obs} observations', flush=True)
    info = {}
    up_g, st_g, _ = gpu_engine._lm_step(**_gpu(p).lm_inputs(), **kw, info=info)
    up = {k: v.cpu() for k, v in up_g.items()}
    for k in ('K', 'z_coefs', 'pts3d', 'P_w2rig'):
        assert torch.isfinite(up[k]).all(), k
    inp = p.lm_inputs()
    l0 = oeng.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d, p.pix2d_std,
                        p.pix2d_dep, True, o['weight_z'], 1.0, o['clip_pix_err'], o['huber_delta'])[0]
    assert abs(float(st_g.init_loss) - float(l0)) <= 1e-5 * abs(float(l0))
    # every group optimised, no mask: the unknowns are [foc | tau | zcf | pts] without compaction
    params = [osol._Param(n) for n in (len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks)]
    sysd = dict(loss=l0, params=params)
    ls = _check_line_search(inp, hp, sysd, info['delta'], info, st_g, up_g)
    print(f'[full cfg2 lm_step] loss {float(l0):.6g} -> {float(ls["new_loss"]):.6g} at scale {ls["scale"]}',
          flush=True)


@pytest.mark.parametrize('cfg,nf,nt', [(0, 8, 300), (2, 30, 1500)])
def test_reduced_solve_cholesky_fallback_runs_pcg_and_points_again(cfg, nf, nt):
    """When the direct solve reports a pivot that is not positive (forced here from the host: the status
    read says so), solve_delta runs the device PCG on the same system and the point back-substitution
    again, so the step equals solver='pcg''s bit for bit; the status is read once, after the first
    back-substitution was enqueued."""
    print(f'cholesky fallback cfg {cfg} ({nf} frames, {nt} tracks)', flush=True)
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    o = p.options
    flags = _cfg_flags(p)
    g = _gpu(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    hp = dict(weight_z=o['weight_z'], pnorm=1.0, max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    deltas, reads = [], []
    for solver in ('cholesky', 'pcg'):
        gs = GaussNewtonSolver(len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks, DEV, dtype=torch.float64, solver=solver)
        if solver == 'cholesky':
            real = gs._direct_status

            def forced(info, real=real):
                reads.append(real(info))
                gs.last['direct']['first_bad_pivot'] = 0
                return False
            gs._direct_status = forced
        J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                                 g.pix2d_dep, True, pix2d=g.pix2d, hp=hp, **flags)
        deltas.append(gs.solve_delta(J, res, w))
        if solver == 'cholesky':
            assert reads == [True] and gs.last['direct']['first_bad_pivot'] == 0
    assert torch.equal(deltas[0], deltas[1])


@pytest.mark.parametrize('cfg,nf,nt,maxiter', [(0, None, None, 300), (2, 30, 1500, 300), (0, 16, 600, 60),
                                                (0, 8, 300, 20)])
def test_pcg_chunked_graphs_equal_the_whole_sequence(cfg, nf, nt, maxiter):
    """The PCG replayed from chunk graphs, where the host stops launching chunks once the loop has stopped
    (ba_pcg_solve_range, the flag read from pinned memory), gives the bits of the whole launch sequence
    (ba_pcg_solve, use_graph off): delta and the loop's outcome equal, also on a second solve that replays the
    captured graphs; where the loop converges early (full config 0) fewer iterations are launched, at most two
    chunks past the stop."""
    from blast3r_amd.ba_solver import PCG_CHUNK
    print(f'pcg chunks cfg {cfg} ({nf} frames, {nt} tracks), maxiter {maxiter}', flush=True)
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    o = p.options
    flags = _cfg_flags(p)
    g = _gpu(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    hp = dict(weight_z=o['weight_z'], pnorm=1.0, max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    runs = {}
    for use_graph in (True, False):
        gs = GaussNewtonSolver(len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks, DEV, dtype=torch.float64, use_graph=use_graph,
                               pcg_maxiter=maxiter)
        J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                                 g.pix2d_dep, True, pix2d=g.pix2d, hp=hp, **flags)
        d1 = gs.solve_delta(J, res, w)
        d2 = gs.solve_delta(J, res, w)
        runs[use_graph] = (d1, d2, gs.last['istate'].cpu(), gs.last['pcg_launched'])
    (c1, c2, c_ist, launched), (w1, w2, w_ist, _) = runs[True], runs[False]
    k, conv = int(w_ist[2]), int(w_ist[3])
    print(f'  stopped after {k} iterations (converged {conv}), launched {launched} of {maxiter}', flush=True)
    assert torch.equal(c1, w1) and torch.equal(c2, w1) and torch.equal(w2, w1)
    assert torch.equal(c_ist, w_ist)
    assert k <= launched <= maxiter
    if conv and k + 2 * PCG_CHUNK < maxiter and maxiter > PCG_CHUNK:
        assert launched <= k + 2 * PCG_CHUNK
    if cfg == 0 and nf is None:
        assert conv == 1 and launched < maxiter


_CHOL_CASES = [(0, 8, 300), (1, 32, 400), (2, 30, 1500), (3, 24, 600), (4, 20, 800), (2, 70, 3000)]


@pytest.mark.parametrize('cfg,nf,nt,layout', [c + (l,) for l in ('dense', 'auto') for c in _CHOL_CASES] +
                         [c + ('banded_sequential',) for c in _CHOL_CASES if c[0] in (0, 2, 4)] +
                         [(2, 150, 4000, 'auto')])
def test_reduced_solve_cholesky_parity(cfg, nf, nt, layout):
    """solver='cholesky' (ba_reduced_solve, L L^T of the damped reduced system on the device) against
    the oracle's direct solve of the reference's explicit Schur system (solve_reduced_direct,
    ba_solver.py:208-226): the device's own system is solved to a relative residual of 1e-10, and the
    full step agrees with the oracle's on sqrt(W) J delta to 1e-6, widened only by 5x the oracle's own
    move when its fp32 inputs are rounded differently.  layout 'auto' takes the banded factor wherever
    the structure allows it (configs 0, 2 and 4 here: every image pair within w images), by block cyclic
    reduction over super-blocks (checked to have run, on several levels at 70 and 150 frames), the dense
    one elsewhere; 'dense' forces the dense one, 'banded_sequential' the one-workgroup banded walk."""
    from tests.step_checks import oracle_system, rounded_differently, weighted_jdelta, device_system
    print(f'cholesky parity cfg {cfg} ({nf} frames, {nt} tracks), layout {layout}', flush=True)
    p = make_problem(cfg, n_frames=nf, n_tracks=nt)
    o = p.options
    flags = _cfg_flags(p)
    g = _gpu(p)
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids,
                                            g.pix2d, g.pix2d_std, g.pix2d_dep, True, o['weight_z'], 1.0,
                                            o['clip_pix_err'], o['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    gs = GaussNewtonSolver(len(p.K), len(p.P_w2rig), p.n_imgs, p.n_tracks, DEV, dtype=torch.float64, solver='cholesky',
                           cholesky_layout=layout)
    hp = dict(weight_z=o['weight_z'], pnorm=1.0, max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                             g.pix2d_dep, True, pix2d=g.pix2d, hp=hp, **flags)
    delta = gs.solve_delta(J, res, w)
    assert gs.last['direct'] is not None and gs.last['direct']['first_bad_pivot'] is None
    if layout == 'auto' and cfg == 2:
        assert gs.last['direct']['layout'] == 'banded' and gs.last['direct']['superblocks'] >= (5 if nf >= 70 else 1)
    if layout == 'banded_sequential':
        assert gs.last['direct']['layout'] == 'banded_sequential' and gs.last['direct']['superblocks'] == 0
    ist = gs.last['istate'].cpu()
    assert int(ist[2]) == 0 and int(ist[3]) == 1
    S_dev, rhs_dev, _ = device_system(gs)
    n_c = S_dev.shape[0]
    x = gs.last['x'][:n_c].cpu()
    res_rel = float((S_dev @ x - rhs_dev).norm() / rhs_dev.norm())
    hpo = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=1.0, clip_pix_err=o['clip_pix_err'])
    sysd = oracle_system(p.lm_inputs(), hpo, flags)
    ref = osol.solve_reduced_direct(sysd['ne'], sysd['g'])
    jd_ref = weighted_jdelta(sysd, ref)
    gen = torch.Generator().manual_seed(cfg)
    moves = []
    for _ in range(2):
        alt = rounded_differently(sysd, gen)
        moves.append(rel_err(weighted_jdelta(sysd, osol.solve_reduced_direct(alt['ne'], alt['g'])), jd_ref))
    bar = max([1e-6] + [5 * m for m in moves])
    e_j = rel_err(weighted_jdelta(sysd, delta), jd_ref)
    print(f'  n_u {n_c} {gs.last["direct"]}: device residual {res_rel:.1e}; sqrt(W) J delta {e_j:.2e} (bar {bar:.1e}); '
          f'delta {rel_err(delta, ref.to(torch.float32)):.2e}', flush=True)
    assert res_rel <= 1e-10
    assert e_j <= bar, (e_j, bar)
