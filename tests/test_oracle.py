"""CPU pins of the oracle: each restated function is checked against something other than its
own formula (closed forms, special cases, torch.func autodiff, dense linear algebra, the
reference's own `_pcg` vectors), chosen so that a dropped term, a sign or index error or a
transposed operand fails.  Tolerances are stated per assertion.
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle.dense as od
import oracle.engine as oe
import oracle.kernels as ok
import oracle.solver as osol
from helpers import rel_err, tiny_problem

HERE = os.path.dirname(os.path.abspath(__file__))


# ----------------------------------------------------------------------------- residuals (A3)
def _one_obs(X, pix=(259.0, 191.0), std=(1.0, 2.0), dep=None, zc=None, f=500.0):
    K = torch.tensor([[[f, 0, 256.0], [0, f, 192.0], [0, 0, 1]]])
    eye = torch.eye(4).view(1, 4, 4)
    dep = torch.tensor([dep if dep is not None else [0.0, 1.0, 0.0]])
    zc = torch.tensor([zc if zc is not None else [1.0, 0.0, 0.0]])
    return dict(infos=torch.tensor([[1], [0], [0]], dtype=torch.int32), K=K, P_rig2c=eye.expand(1, 4, 4),
                P_w2rig=eye.clone(), z_coefs=zc, pts3d=torch.tensor([X]), pids=torch.tensor([0], dtype=torch.int32),
                pix2d=torch.tensor([pix]), pix2d_std=torch.tensor([std]), pix2d_dep=dep)


def _res(d, **kw):
    a = dict(is_depth_log=True, weight_z=1.0, pnorm=1.0, max_pix_err=100.0, huber_delta=2.0, w_pts_null=1e-16)
    a.update(kw)
    return ok.residuals_with_rigs(d['infos'], d['K'], d['P_rig2c'], d['P_w2rig'], d['z_coefs'], d['pts3d'], d['pids'],
                                  d['pix2d'], d['pix2d_std'], d['pix2d_dep'], **a)[0]


def test_residual_on_axis_point_and_huber_pnorm1():
    """Identity pose, point on the optical axis projects to (cx, cy); pnorm = 1 is textbook Huber/IRLS:
    err = r^2 / (2 delta) (|r| <= delta) or |r| - delta / 2, w = 1 / max(|r|, delta)."""
    z = 5.0
    d = _one_obs([0.0, 0.0, z], dep=[math.log(z) + 0.01, 1.0, 0.0], zc=[1.0, 0.003, 0.0])
    out = _res(d)
    r0, r1 = (256.0 - 259.0) / 1.0, (192.0 - 191.0) / 2.0
    r2 = 500.0 * 0.013                                          # fbar (g - ln z), g = ln z + 0.013
    assert torch.allclose(out[:3], torch.tensor([r0, r1, r2]), rtol=1e-5, atol=1e-4)
    delta = 2.0
    huber = lambda r: r * r / (2 * delta) if abs(r) <= delta else abs(r) - delta / 2
    assert torch.allclose(out[3:6], torch.tensor([huber(r0), huber(r1), huber(r2)]), rtol=1e-5)
    assert torch.allclose(out[6:9], torch.tensor([1 / max(abs(r), delta) for r in (r0, r1, r2)]), rtol=1e-6)


def test_residual_clip_weight_z_and_invalid_depth():
    """|r| clipped at M: err = wz (M - delta/2), w = w_null (no wz); weight_z scales row 2 only;
    a point behind the camera (z <= 1e-3) gives all-zero rows."""
    d = _one_obs([0.0, 0.0, 5.0], pix=(256.0 + 150.0, 192.0), dep=[math.log(5.0) + 0.5, 1.0, 0.0])
    out = _res(d, weight_z=0.25)
    assert out[0].item() == pytest.approx(-150.0, rel=1e-6)
    assert out[3].item() == pytest.approx(100.0 - 1.0, rel=1e-6)          # clipped, pnorm 1
    assert out[6].item() == pytest.approx(1e-16, rel=1e-6)                # w_null
    r2 = 500.0 * 0.5
    assert out[2].item() == pytest.approx(r2, rel=1e-5)
    assert out[5].item() == pytest.approx(0.25 * (100.0 - 1.0), rel=1e-5)  # clipped and scaled by weight_z
    assert out[8].item() == pytest.approx(1e-16, rel=1e-6)
    behind = _res(_one_obs([0.0, 0.0, -2.0]))
    assert torch.count_nonzero(behind) == 0


def test_depth_threshold_is_a_double_comparison():
    """.cu:212 and :408 test `z <= 1e-3` with a float (or double) z against the double literal
    1e-3.  float32(1e-3) = 0.0010000000475 lies above it, so a point at exactly z = 1e-3f keeps its
    residual and Jacobian rows; the next float below (0.00099999993) drops them.  An fp32
    comparison (z > 1e-3f) would drop the first one too."""
    z_keep = float(np.float32(1e-3))
    z_drop = float(np.nextafter(np.float32(1e-3), np.float32(0)))
    assert z_keep > 1e-3 > z_drop
    for z, kept in ((z_keep, True), (z_drop, False)):
        d = _one_obs([0.0, 0.0, z])
        assert float(d['pts3d'][0, 2]) == z
        out = _res(d)
        assert bool(torch.count_nonzero(out) > 0) == kept, z
        assert out[0].item() == (pytest.approx(-3.0, rel=1e-6) if kept else 0.0)     # (cx - u) / std
        for f64 in (True, False):
            Jc, Jz, Jp = ok.jacobians_with_rigs(d['infos'], d['K'], d['P_rig2c'], d['P_w2rig'], d['z_coefs'],
                                                d['pts3d'], d['pids'], d['pix2d_std'], d['pix2d_dep'], True,
                                                float64=f64)
            assert bool(torch.count_nonzero(Jp) > 0) == kept, (z, f64)


def test_residual_pnorm2_and_lin_mode():
    """pnorm = 2: a = p delta^(p-2) / 2 = 1 and b = 0, so err = r^2 on both sides of delta and w = 1;
    lin depth mode r2 = fbar ln(g / z)."""
    z = 4.0
    d = _one_obs([0.0, 0.0, z], dep=[2.0 * z, 1.0, 0.0], zc=[1.0, 0.0, 0.0])
    out = _res(d, pnorm=2.0, is_depth_log=False)
    r2 = 500.0 * math.log(2.0)
    assert out[2].item() == pytest.approx(r2, rel=1e-5)
    assert out[3].item() == pytest.approx(out[0].item() ** 2, rel=1e-5)
    assert out[4].item() == pytest.approx(out[1].item() ** 2, rel=1e-5)
    assert torch.allclose(out[6:8], torch.ones(2))
    nores = _res(d, pnorm=-1.0)                                   # pnorm -1: residual rows only
    assert nores.shape == (3,)


# ----------------------------------------------------------------------------- Jacobians (A4)
def _jac_inputs(p):
    return (p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d_std, p.pix2d_dep)


def test_jacobians_match_autodiff():
    """Camera pose (left perturbation), points, z-coefficients and the r0/r1 focal columns equal
    torch.func derivatives of an independent fp64 residual; the r2 focal column equals
    d r2 / d f rounded to fp32 where g > 0 (the reference's J_k_f quirk)."""
    p = tiny_problem(0, n_frames=6, n_tracks=50)
    Jc, Jz, Jp = ok.jacobians_with_rigs(*_jac_inputs(p), True, float64=True)
    af, at, az, ax = od.autodiff_jacobians(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                           p.pix2d_std, p.pix2d_dep, True)
    assert rel_err(Jp, ax) < 1e-12
    assert rel_err(Jc[:, :, 2:], at) < 1e-12
    assert rel_err(Jz[:, 0], az[:, 2]) < 1e-12 and torch.count_nonzero(az[:, :2]) == 0
    assert rel_err(Jc[:, :2, :2], af[:, :2]) < 1e-12
    g_pos = (p.z_coefs[ok.obs_to_img(p.infos, len(p.pids))] * p.pix2d_dep).sum(1) > 0
    assert bool(g_pos.all())
    assert rel_err(Jc[:, 2, :2], af[:, 2]) < 1e-7                      # fp32-rounded column


def test_jacobians_match_autodiff_lin_mode():
    """depth_mode='lin' (.cu:481-501): r2 = fbar ln(g / z) has true derivatives fbar dep_c / g in the
    z-coefficients and (1/2) ln(g / z) in each focal (held in fp32 by the reference, the same quirk as
    in log mode), so every block equals torch.func derivatives of the independent fp64 residual."""
    from blast3r_amd.synthetic import make_problem
    p = make_problem(0, n_frames=6, n_tracks=50, depth_mode='lin')
    Jc, Jz, Jp = ok.jacobians_with_rigs(*_jac_inputs(p), False, float64=True)
    af, at, az, ax = od.autodiff_jacobians(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                           p.pix2d_std, p.pix2d_dep, False)
    g_pos = (p.z_coefs[ok.obs_to_img(p.infos, len(p.pids))] * p.pix2d_dep).sum(1) > 0
    assert bool(g_pos.all())
    assert rel_err(Jp, ax) < 1e-12
    assert rel_err(Jc[:, :, 2:], at) < 1e-12
    assert rel_err(Jz[:, 0], az[:, 2]) < 1e-12 and torch.count_nonzero(az[:, :2]) == 0
    assert rel_err(Jc[:, :2, :2], af[:, :2]) < 1e-12
    assert rel_err(Jc[:, 2, :2], af[:, 2]) < 1e-6                      # fp32-rounded column


def test_jacobian_focal_gate_for_negative_guidance():
    """J_k_f = 0 when g <= 0 even though the true derivative is not (reference quirk, .cu:481-489)."""
    p = tiny_problem(0, n_frames=5, n_tracks=30)
    dep = p.pix2d_dep.clone()
    dep[:, 0] -= 10.0                                               # log-depth channel shifted below 0
    Jc, _, _ = ok.jacobians_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d_std,
                                      dep, True, float64=True)
    af, _, _, _ = od.autodiff_jacobians(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                        p.pix2d_std, dep, True)
    assert torch.count_nonzero(Jc[:, 2, :2]) == 0
    assert torch.count_nonzero(af[:, 2]) > 0


# ----------------------------------------------------------------------------- small operators (A8, A6, A9, A14)
def test_chol3x3_solve_matches_linalg_and_jitter_rules():
    g = torch.Generator().manual_seed(3)
    M = torch.randn(200, 3, 3, generator=g, dtype=torch.float64)
    A = M @ M.transpose(1, 2) + 0.1 * torch.eye(3, dtype=torch.float64)
    b = torch.randn(200, 3, generator=g, dtype=torch.float64)
    x = ok.chol3x3_solve(A, b)
    ref = torch.linalg.solve(A + 1e-12 * torch.eye(3, dtype=torch.float64), b.unsqueeze(-1)).squeeze(-1)
    assert rel_err(x, ref) < 1e-10
    # off-diagonals are averaged: an asymmetric block solves like its symmetric part
    Aa = A.clone()
    Aa[:, 0, 1] += 0.05
    Aa[:, 1, 0] -= 0.05
    assert rel_err(ok.chol3x3_solve(Aa, b), x) < 1e-10
    # singular (rank-1) blocks: non-positive pivots get the jitter, the result stays finite
    v = torch.randn(10, 3, 1, generator=g, dtype=torch.float64)
    S = v @ v.transpose(1, 2)
    assert torch.isfinite(ok.chol3x3_solve(S, b[:10])).all()


def test_blockcoo_matvec_against_dense_assembly():
    g = torch.Generator().manual_seed(4)
    nb, bh, bw, HB1, WB1 = 70, 3, 6, 9, 11
    blocks = torch.randn(nb, bh, bw, generator=g, dtype=torch.float64)
    rows = torch.randint(0, HB1, (nb,), generator=g)
    cols = torch.randint(0, WB1, (nb,), generator=g)          # duplicates included
    D = torch.zeros(HB1 * bh, WB1 * bw, dtype=torch.float64)
    for k in range(nb):
        D[rows[k] * bh:(rows[k] + 1) * bh, cols[k] * bw:(cols[k] + 1) * bw] += blocks[k]
    x = torch.randn(WB1 * bw, generator=g, dtype=torch.float64)
    y = ok.blockcoo_matvec(blocks, rows, cols, x.view(WB1, bw), HB1, WB1).reshape(-1)
    assert rel_err(y, D @ x) < 1e-12
    xt = torch.randn(HB1 * bh, generator=g, dtype=torch.float64)
    yt = ok.blockcoo_matvec(blocks, rows, cols, xt.view(HB1, bh), HB1, WB1, transpose_blocks=True).reshape(-1)
    assert rel_err(yt, D.T @ xt) < 1e-12


def test_fused_einsum_is_batched_transpose_product():
    g = torch.Generator().manual_seed(5)
    L = torch.randn(20, 3, 5, generator=g, dtype=torch.float64)
    R = torch.randn(20, 3, 7, generator=g, dtype=torch.float64)
    out = ok.fused_einsum_bki_bkj(L, R)
    ref = torch.stack([L[b].T @ R[b] for b in range(20)])
    assert rel_err(out, ref) < 1e-14


def test_exp_se3_closed_forms():
    """Rotation about z by theta (Rodrigues) and a pure translation."""
    th = 0.7
    xi = torch.tensor([[0.0, 0.0, th, 0.0, 0.0, 0.0], [0.0, 0.0, 0.0, 1.0, -2.0, 0.5]])
    T = ok.exp_se3(xi)
    Rz = torch.tensor([[math.cos(th), -math.sin(th), 0.0], [math.sin(th), math.cos(th), 0.0], [0.0, 0.0, 1.0]])
    assert torch.allclose(T[0, :3, :3], Rz, atol=1e-6) and torch.allclose(T[0, :3, 3], torch.zeros(3), atol=1e-7)
    assert torch.allclose(T[1, :3, :3], torch.eye(3)) and torch.allclose(T[1, :3, 3], xi[1, 3:], atol=1e-7)
    assert torch.allclose(T[:, 3], torch.tensor([0.0, 0.0, 0.0, 1.0]).expand(2, 4))


def test_update_K_and_reproj_score():
    K = torch.tensor([[[300.0, 0, 1], [0, 120.0, 2], [0, 0, 1]]])
    Kn = oe.update_K(K, torch.tensor([[50.0, 40.0]]))
    assert Kn[0, 0, 0].item() == 250.0 and Kn[0, 1, 1].item() == 100.0      # clip at 100 (engine.py:352-353)
    Kc = oe.update_K(K, torch.tensor([[0.0, 30.0]]))
    assert Kc[0, 1, 1].item() == 100.0
    r = torch.zeros(10, 3)
    r[:, 0] = torch.arange(10.0)                                           # norms 0..9
    assert oe.reproj_score(r).item() == pytest.approx(sum(range(8)) / 8)   # lowest 80% = 8 values


# ----------------------------------------------------------------------------- normal equations and Schur (A5-A12)
def _system(p, **flags):
    o = p.options
    _, res, w = oe.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d, p.pix2d_std,
                             p.pix2d_dep, True, o['weight_z'], 1.0, o['clip_pix_err'], o['huber_delta'])
    Jc, Jz, Jp = ok.jacobians_with_rigs(*_jac_inputs(p), True, float64=True)
    prob = osol.Problem(p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks, p.C)
    ne, g, params = osol.build_normal_equations(prob, Jc, Jz, Jp, res, w, **flags)
    Jd = od.dense_jacobian(Jc, Jz, Jp, p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks)
    sizes = (2 * len(p.K), 6 * len(p.P_w2rig), p.C * p.n_imgs, 3 * p.n_tracks)
    Hd, gd = od.dense_normal_equations(Jd, res, w, sizes)
    return ne, g, Hd, gd, Jd


def test_normal_equations_match_dense_products():
    p = tiny_problem(0, n_frames=5, n_tracks=40)
    ne, g, Hd, gd, _ = _system(p)
    n_c = ne.sizes['n_c']
    # 1e-7: the reference forms W*r in fp32 and scales J by an fp32 sqrt(W) (ba_solver.py:128-132);
    # the dense products here use W in fp64, so the two differ by fp32 rounding only
    assert rel_err(g, gd) < 1e-7
    assert rel_err(osol.dense_A(ne), Hd[:n_c, :n_c]) < 1e-7
    Hpp = torch.block_diag(*ne.leaves['pts'])
    assert rel_err(Hpp, Hd[n_c:, n_c:]) < 1e-7
    # cross blocks through the operators: B y = H_cp y
    y = torch.randn(Hd.shape[0] - n_c, dtype=torch.float64)
    assert rel_err(osol._B_matvec(ne, y), Hd[:n_c, n_c:] @ y) < 1e-7


def test_track_mask_drops_the_disabled_tracks_columns():
    """A tensor optim_X (per track) gives the normal equations of the dense Jacobian with the
    disabled tracks' point columns deleted and the enabled ones kept in order (the per-track
    reading of enable(), ba_solver.py:72-108, for a track mask)."""
    p = tiny_problem(0, n_frames=5, n_tracks=40)
    mask = torch.arange(p.n_tracks) % 3 != 0
    o = p.options
    _, res, w = oe.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d, p.pix2d_std,
                             p.pix2d_dep, True, o['weight_z'], 1.0, o['clip_pix_err'], o['huber_delta'])
    Jc, Jz, Jp = ok.jacobians_with_rigs(*_jac_inputs(p), True, float64=True)
    prob = osol.Problem(p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks, p.C)
    ne, g, params = osol.build_normal_equations(prob, Jc, Jz, Jp, res, w, optim_X=mask)
    Jd = od.dense_jacobian(Jc, Jz, Jp, p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks)
    n_c = 2 * len(p.K) + 6 * len(p.P_w2rig) + p.C * p.n_imgs
    en = torch.nonzero(mask).squeeze(-1)
    keep = torch.cat([torch.arange(n_c), (n_c + 3 * en[:, None] + torch.arange(3)).reshape(-1)])
    sizes = (2 * len(p.K), 6 * len(p.P_w2rig), p.C * p.n_imgs, 3 * len(en))
    Hd, gd = od.dense_normal_equations(Jd[:, keep], res, w, sizes)
    assert ne.sizes['n_c'] == n_c and g.shape == gd.shape
    assert rel_err(g, gd) < 1e-7
    assert rel_err(osol.dense_A(ne), Hd[:n_c, :n_c]) < 1e-7
    assert rel_err(torch.block_diag(*ne.leaves['pts']), Hd[n_c:, n_c:]) < 1e-7
    y = torch.randn(3 * len(en), dtype=torch.float64)
    assert rel_err(osol._B_matvec(ne, y), Hd[:n_c, n_c:] @ y) < 1e-7


def test_schur_identity_symmetry_psd_and_gauge():
    """Reduced solve + back-substitution equals the dense solve of the damped system; S is symmetric
    PSD; the seven similarity directions lie in its (near-)nullspace (damping 1e-12 max diag)."""
    p = tiny_problem(0, n_frames=5, n_tracks=40)
    ne, g, Hd, gd, Jd = _system(p)
    n_c = ne.sizes['n_c']
    d_red = osol.solve_reduced_direct(ne, g)
    d_full = torch.linalg.solve(Hd, gd)
    assert rel_err(Jd @ d_red, Jd @ d_full) < 1e-6                  # equal up to the (damped) gauge span
    S = osol.dense_schur(ne)
    assert rel_err(S, S.T) < 1e-12
    ev = torch.linalg.eigvalsh(0.5 * (S + S.T))
    assert ev.min().item() > -1e-9 * ev.max().item()
    B = od.similarity_gauge_basis(p.P_w2rig, p.pts3d, p.n_imgs, len(p.K), p.C)
    assert rel_err(Jd @ B, torch.zeros(Jd.shape[0], 7, dtype=torch.float64)) < 1e-6 * Jd.norm() * B.norm()
    Sv = S @ B[:n_c]
    assert float(Sv.norm()) < 1e-6 * float(S.norm()) * float(B[:n_c].norm())


def test_converged_pcg_equals_direct_solve():
    p = tiny_problem(0, n_frames=5, n_tracks=40)
    ne, g, _, _, Jd = _system(p)
    d_pcg, it, conv = osol.solve_reduced_pcg(ne, g, tol=1e-13, maxiter=5000)
    d_dir = osol.solve_reduced_direct(ne, g)
    assert rel_err(Jd @ d_pcg, Jd @ d_dir) < 1e-6


# ----------------------------------------------------------------------------- PCG control flow (A10)
@pytest.mark.parametrize('case', ['converges', 'maxiter_hit', 'ill_conditioned', 'indefinite', 'zero_rhs'])
def test_pcg_against_reference_vectors(case):
    """Iterate sequence, stopping rule and best-so-far choice against the reference `_pcg`
    (vectors from tests/golden/make_pcg_golden.py)."""
    z = np.load(os.path.join(HERE, 'golden', 'pcg_golden.npz'))
    A = torch.from_numpy(z[f'{case}/A'])
    b = torch.from_numpy(z[f'{case}/b'])
    d = A.diagonal().clamp(min=1e-12)
    x, k, conv = osol.pcg(lambda v: A @ v, b, M_mv=lambda v: v / d, tol=float(z[f'{case}/tol']),
                          maxiter=int(z[f'{case}/maxiter']))
    assert int(k) == int(z[f'{case}/iters']) and bool(conv) == bool(z[f'{case}/converged'])
    xr = torch.from_numpy(z[f'{case}/x'])
    assert rel_err(x, xr) < 1e-12 if xr.norm() > 0 else float(x.norm()) == 0.0


# ----------------------------------------------------------------------------- the LM step (A14)
def test_oracle_lm_step_decreases_loss_and_follows_schedule():
    p = tiny_problem(0, n_frames=6, n_tracks=80)
    o = p.options
    up, st, info = oe.lm_step(**p.lm_inputs(), weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=o['pnorm'])
    assert float(st.new_loss) < float(st.init_loss)
    assert info['scale'] in [1.0, 0.5, 0.25, 0.125, 1 / 64, 1 / 512, 1 / 4096, 0.0]


def _residuals_fp64(p, K, P_w2rig, z_coefs, pts3d):
    """Every observation's three residuals in fp64 from the independent model equations
    (oracle/dense.py residual_fp64, pinned against the oracle's fp32 residual) at the given parameters."""
    from torch.func import vmap
    d = torch.float64
    n = len(p.pids)
    img = ok.obs_to_img(p.infos, n)
    node, cam = p.infos[1].long()[img], p.infos[2].long()[img]
    Kc = K.to(d)[cam]
    fxy = torch.stack([Kc[:, 0, 0], Kc[:, 1, 1]], 1)
    f = lambda a, b, c, e, *rest: od.residual_fp64(a, b, c, e, *rest, is_depth_log=True)
    return vmap(f)(fxy, torch.zeros((n, 6), dtype=d), z_coefs.to(d)[img], pts3d.to(d)[p.pids.long()],
                   Kc[:, 0, 2], Kc[:, 1, 2], P_w2rig.to(d)[node], p.P_rig2cam.to(d)[cam], p.pix2d.to(d),
                   p.pix2d_std.to(d), p.pix2d_dep.to(d))


def _first_order_errors(p, update, group, seed=7):
    """||r(update(x, t delta)) - r(x) + t J delta|| / ||t J delta|| for t = 1e-3 and 1e-4, with delta nonzero
    in one parameter group only and J the autodiff derivatives of residual_fp64 under the model's own
    parametrisation (f += df, P <- exp(xi^) P, z += dz, X += dX).  A correct update x <- x (+) (-t delta)
    (en:310-313) gives errors of order t, shrinking tenfold from t = 1e-3 to 1e-4."""
    d = torch.float64
    K, P, Z, X = p.K.to(d), p.P_w2rig.to(d), p.z_coefs.to(d), p.pts3d.to(d)
    g = torch.Generator().manual_seed(seed)
    dK, dP = torch.zeros((len(K), 2), dtype=d), torch.zeros((len(P), 6), dtype=d)
    dZ, dX = torch.zeros_like(Z), torch.zeros_like(X)
    if group == 'K':
        dK = 20.0 * torch.randn(dK.shape, generator=g, dtype=d)
    elif group == 'P':
        dP = torch.randn(dP.shape, generator=g, dtype=d) * torch.tensor([0.05] * 3 + [0.2] * 3, dtype=d)
    elif group == 'Z':
        dZ = 0.2 * torch.randn(dZ.shape, generator=g, dtype=d)
    else:
        dX = 0.2 * torch.randn(dX.shape, generator=g, dtype=d)
    Jf, Jxi, Jz, Jx = od.autodiff_jacobians(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids,
                                            p.pix2d, p.pix2d_std, p.pix2d_dep)
    img = ok.obs_to_img(p.infos, len(p.pids))
    node, cam = p.infos[1].long()[img], p.infos[2].long()[img]
    Jd = (torch.einsum('nrc,nc->nr', Jf, dK[cam]) + torch.einsum('nrc,nc->nr', Jxi, dP[node]) +
          torch.einsum('nrc,nc->nr', Jz, dZ[img]) + torch.einsum('nrc,nc->nr', Jx, dX[p.pids.long()]))
    r0 = _residuals_fp64(p, K, P, Z, X)
    errs = []
    for t in (1e-3, 1e-4):
        up = update(K, P, Z, X, dK, dP, dZ, dX, t)
        rt = _residuals_fp64(p, up['K'], up['P_w2rig'], up['z_coefs'], up['pts3d'])
        errs.append(float((rt - r0 + t * Jd).norm() / (t * Jd).norm()))
    return errs


def _passes_first_order(errs):
    # the residuals are linear in the focal and the z-coefficients: there the error is rounding alone
    return errs[0] < 2e-2 and (errs[1] < errs[0] / 5 or max(errs) < 1e-9)


@pytest.mark.parametrize('group', ['K', 'P', 'Z', 'X'])
def test_oracle_update_rule_is_the_first_order_step(group):
    """The oracle's parameter update (apply_update, en:310-313 with update_K en:347-354 and exp_se3
    cujac/__init__.py:56-58), used by its lm_step and by the GPU step checks, moves the residuals by
    -t J delta to first order in every parameter group: the focal decrement, the left pose update
    exp(-t dP^) P, the z-coefficient and point decrements.  The same check rejects the update with the
    sign of any group's step flipped, and the pose update applied on the right (P exp(-t dP^)), which
    the loss-decrease and schedule checks of the LM step do not see."""
    p = tiny_problem(0, n_frames=6, n_tracks=80)
    errs = _first_order_errors(p, oe.apply_update, group)
    assert _passes_first_order(errs), (group, errs)

    def flipped(K, P, Z, X, dK, dP, dZ, dX, t):
        s = {g: (-1.0 if g == group else 1.0) for g in 'KPZX'}
        return oe.apply_update(K, P, Z, X, dK * s['K'], dP * s['P'], dZ * s['Z'], dX * s['X'], t)

    def right_pose(K, P, Z, X, dK, dP, dZ, dX, t):
        up = oe.apply_update(K, P, Z, X, dK, dP * 0, dZ, dX, t)
        up['P_w2rig'] = P @ ok.exp_se3(-(dP * t))
        return up

    bad = {'flipped sign': flipped}
    if group == 'P':
        bad['right-multiplied pose'] = right_pose
    for name, fn in bad.items():
        e = _first_order_errors(p, fn, group)
        assert not _passes_first_order(e), (group, name, e)


# Known answers for the acceptance rule of en:305-333, worked out by hand from the reference text:
# trials are evaluated at scales 1, 1/2, 1/4, 1/8, 1/64, 1/512, 1/4096 (delta *= a / last_a over
# [0.5, 0.25, 0.125, 1/64, 1/512, 1/4096, 0]); a trial is taken when loss + 1e-4 < init_loss (fp32)
# and reproj >= 0.01; a NaN loss is replaced by init_loss and `+= 1e-4` then lands on init_loss
# itself (en:317-319), so init_loss grows by 1e-4 for the rest of the step.
_F = lambda x: float(torch.tensor(x, dtype=torch.float32))
_ALL_SCALES = [1.0, 0.5, 0.25, 0.125, 1 / 64, 1 / 512, 1 / 4096]
_LS_CASES = {
    # name: ([(loss, reproj) per trial], accepted scale, trials, init_loss after, new_loss, accepted)
    'first_trial': ([(0.9, 1.0)], 1.0, 1, 1.0, _F(_F(0.9) + _F(1e-4)), True),
    'margin_rejects': ([(0.99995, 1.0), (0.9998, 1.0)], 0.5, 2, 1.0, _F(_F(0.9998) + _F(1e-4)), True),
    'reproj_collapse': ([(0.5, 0.001), (0.6, 0.02)], 0.5, 2, 1.0, _F(_F(0.6) + _F(1e-4)), True),
    # NaN, then 0.99995: 0.99995 + 1e-4 = 1.00005 < 1.0001 (the aliased init_loss) is taken;
    # without the aliasing it would be rejected and the third trial (0.9) taken at scale 1/4
    'nan_aliases_init': ([(float('nan'), 1.0), (0.99995, 1.0), (0.9, 1.0)], 0.5, 2, _F(_F(1.0) + _F(1e-4)),
                         _F(_F(0.99995) + _F(1e-4)), True),
    'two_nans': ([(float('nan'), 1.0), (float('nan'), 1.0), (1.00005, 1.0)], 0.25, 3,
                 _F(_F(_F(1.0) + _F(1e-4)) + _F(1e-4)), _F(_F(1.00005) + _F(1e-4)), True),
    'none_decreases': ([(1.5, 1.0)] * 7, 1 / 4096, 7, 1.0, _F(_F(1.5) + _F(1e-4)), False),
}


@pytest.mark.parametrize('name', sorted(_LS_CASES))
@pytest.mark.parametrize('impl', ['oracle', 'device_engine_host_logic'])
def test_line_search_acceptance_known_answers(name, impl):
    """Both line searches (the oracle restatement and the device engine's host-side decision loop, fed
    CPU tensors here) against the hand-worked outcomes above: the scales tried, the accepted scale,
    the init_loss after NaN aliasing and the returned new_loss."""
    from blast3r_amd import engine as de
    seq, scale, n_trials, init_after, new_loss, accepted = _LS_CASES[name]
    calls = []

    def trial(s):
        loss, reproj = seq[len(calls)]
        calls.append(s)
        return torch.tensor(loss, dtype=torch.float32), torch.tensor(reproj, dtype=torch.float32), len(calls)

    init = torch.tensor(1.0, dtype=torch.float32)
    fn = oe.line_search if impl == 'oracle' else de.line_search
    out = fn(trial, init, 1e-4, 0.01)
    assert calls == _ALL_SCALES[:n_trials]
    assert out['scale'] == scale and out['scales'] == calls
    assert out['accepted'] == accepted and out['payload'] == n_trials
    assert float(out['init_loss']) == init_after
    assert float(out['new_loss']) == new_loss
    assert float(init) == 1.0                                   # the caller's tensor is left alone



def test_oracle_bundle_adjustment_phases():
    """en:405-503: a phase with n_zcfs=3 in log mode keeps the first coefficient frozen
    (optim_Z0 = False, n_zcfs + 1 = 4 columns, en:455-458) and the loss falls across accepted steps;
    a second phase (n_zcfs=None) keeps the narrowed depth channels and z-coefficients."""
    from blast3r_amd.data import from_problem
    p = tiny_problem(0, n_frames=6, n_tracks=80)
    o = p.options
    rig, trk, X = from_problem(p)
    z0 = p.z_coefs.clone()
    var, steps = oe.bundle_adjustment(rig, trk, X, z_coefs=z0, max_iters=[2, 1], pnorm=[1.0, 0.5], n_zcfs=[3, None],
                                      weight_z=o['weight_z'], huber_delta=o['huber_delta'])
    assert var['z_coefs'].shape == (p.z_coefs.shape[0], 4)
    assert steps[0] >= 1 and len(steps) == 2
    assert torch.equal(var['z_coefs'][:, 0], p.z_coefs[:, 0])              # frozen column, exactly
    assert torch.equal(trk.pix2d_dep, p.pix2d_dep)                         # input not modified
    l0, _, _ = oe.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs[:, :4].contiguous(), X, p.pids, p.pix2d,
                            p.pix2d_std, p.pix2d_dep[:, :4].contiguous(), True, o['weight_z'], 1.0, 100,
                            o['huber_delta'])
    l1, _, _ = oe.objective(p.infos, var['K'], p.P_rig2cam, var['P_w2rig'], var['z_coefs'], var['pts3d'], p.pids,
                            p.pix2d, p.pix2d_std, p.pix2d_dep[:, :4].contiguous(), True, o['weight_z'], 1.0, 100,
                            o['huber_delta'])
    assert float(l1) < float(l0)

# ----------------------------------------------------------------------------- the C ABI library
def _header_functions():
    import re
    names = []
    for fn in sorted(os.listdir(os.path.join(HERE, '..', 'include'))):
        if fn.endswith('.h'):
            text = open(os.path.join(HERE, '..', 'include', fn)).read()
            text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
            names += re.findall(r'^[A-Za-z_][\w\s\*]*?\b(ba_\w+)\s*\(', text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    """libba_hip.so loads without a GPU and exports every function include/*.h declares; the
    Python binding knows the signature of each (no compute call is made here)."""
    import ctypes
    from blast3r_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from blast3r_amd.build import build
        build()
    so = ctypes.CDLL(_lib.LIB_PATH)
    names = _header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing
    unbound = [n for n in names if n not in _lib._SIGS]
    assert not unbound, unbound
    # every argument struct the header declares has a ctypes mirror of the library's size
    hdr = open(os.path.join(os.path.dirname(_lib.LIB_PATH), '..', 'include', 'ba_hip.h')).read()
    import re
    structs = set(re.findall(r'}\s*(ba_\w+)\s*;', hdr))
    assert structs == set(_lib.ABI_STRUCTS), structs ^ set(_lib.ABI_STRUCTS)
    L = _lib.lib()
    for n, cls in _lib.ABI_STRUCTS.items():
        assert L.ba_abi_sizeof(n.encode()) == ctypes.sizeof(cls), n
    assert L.ba_abi_sizeof(b'no_such_struct') == -1


def test_entry_points_reject_null_pointers_without_a_gpu():
    """The fused-pass, back-substitution and PCG entry points name a NULL pointer they would
    dereference and return an error before any device call (so they run here, without a GPU)."""
    import ctypes
    from blast3r_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from blast3r_amd.build import build
        build()
    L = _lib.lib()
    a = _lib.BaLinArgs()
    a.lay.d, a.lay.C, a.lay.off_tau, a.lay.off_zcf, a.lay.hasK, a.lay.hasP, a.lay.hasZ = 13, 5, 2, 8, 1, 1, 1
    a.L, a.n_chunks, a.n_batches, a.n_pairs, a.n_ctracks, a.n_imgs = 16, 1, 1, 1, 1, 1
    for stage in (0, 1, 2):
        assert L.ba_linearize_stage(ctypes.byref(a), stage, None) != 0
        assert b'null pointer' in L.ba_last_error(), stage
    assert L.ba_backsubstitute(ctypes.byref(a), None) != 0
    assert b'null pointer' in L.ba_last_error()
    assert L.ba_linearize_stage(ctypes.byref(a), 7, None) != 0
    pa = _lib.BaPcgArgs()
    pa.n_u, pa.n_imgs, pa.d, pa.maxiter = 4, 1, 4, 10
    n = (ctypes.c_int32 * 8)()
    pa.long_ptr, pa.long_idx, pa.img_part = ctypes.addressof(n), ctypes.addressof(n), ctypes.addressof(n)
    assert L.ba_pcg_solve(ctypes.byref(pa), None) != 0
    assert b'null pointer' in L.ba_last_error()


def test_boundary_helpers_known_answers():
    """The device engine's host helpers against outcomes worked out by hand from the reference text:
    iter_on (en:364-383: phases = the longest list, one-value lists repeat, scalars repeat, a list of
    another length fails), used_depth_channels (en:386-402: n channels per phase, + the frozen main
    channel in log mode unless n is 2 or all; None reads all), update_K (en:347-354: focal minus the
    step, clipped at 100, NaN kept) and RigsData.z_coefs_from_scale (rigs.py:69-94: new rows from the
    scale, [s, 0..] lin / [1, log s, 0..] log, existing rows kept)."""
    from blast3r_amd import engine as de
    from blast3r_amd.data import RigsData
    assert list(de.iter_on(1.0, [1, 2], [3])) == [(1.0, 1, 3), (1.0, 2, 3)]
    assert list(de.iter_on(0.5)) == [(0.5,)]
    assert list(de.iter_on([None, 3], 'x')) == [(None, 'x'), (3, 'x')]
    for bad in (([1, 2], [1, 2, 3]), ([],)):
        with pytest.raises(AssertionError):
            list(de.iter_on(*bad))
    uc = de.used_depth_channels
    assert uc(None, 5, 'log') == 5 and uc([1, None], 5, 'log') == 5
    assert uc(3, 5, 'log') == 4 and uc(3, 5, 'lin') == 3 and uc(2, 5, 'log') == 2 and uc(5, 5, 'log') == 5
    assert uc([1, 17], 17, 'log_multidepth') == 17 and uc([1, 4], 17, 'log') == 5 and uc(9, 5, 'lin') == 5
    K = torch.tensor([[[500., 0, 256], [0, 510, 192], [0, 0, 1]], [[120., 0, 1], [0, 99, 2], [0, 0, 1]]])
    K2 = de.update_K(K, torch.tensor([[10., -5.], [30., float('nan')]]))
    assert K2[0, 0, 0] == 490 and K2[0, 1, 1] == 515 and K2[1, 0, 0] == 100 and torch.isnan(K2[1, 1, 1])
    assert torch.equal(K2[:, :, 2], K[:, :, 2]) and K[1, 1, 1] == 99            # the input is left alone
    scale = torch.tensor([2.0, 0.5, 4.0])
    trk = type('T', (), {'n_imgs': 3, 'pix2d_dep': torch.zeros((7, 4))})()
    for mode, row in (('lin', [4.0, 0, 0, 0]), ('log', [1.0, math.log(4.0), 0, 0])):
        r = RigsData(1, torch.zeros(3, dtype=torch.int32), K[:1], K[:1], scale, None, mode, 3,
                     torch.arange(3, dtype=torch.int32), K[:1])
        z = r.z_coefs_from_scale(trk)
        assert z.shape == (3, 4) and torch.allclose(z[2], torch.tensor(row))
        r.z_coefs = z[:2] * 0 + 7                                    # two rows exist: only the third is made
        z = r.z_coefs_from_scale(trk)
        assert torch.equal(z[:2], torch.full((2, 4), 7.0)) and torch.allclose(z[2], torch.tensor(row))
    bad = RigsData(1, torch.zeros(3, dtype=torch.int32), K[:1], K[:1], scale, None, 'cube', 3,
                   torch.arange(3, dtype=torch.int32), K[:1])
    with pytest.raises(ValueError):
        bad.z_coefs_from_scale(trk)
