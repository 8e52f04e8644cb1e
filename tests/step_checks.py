"""Step-level parity checks shared by the GPU tests of lm_step and bundle_adjustment.

A device LM step is compared with the oracle in two parts, neither widened by the tolerance-induced
spread of the reference's PCG:
  * the step delta: the device's reduced system against the oracle's (1e-5), the oracle's PCG and
    back-substitution on the device's system against the device's delta after the same number of CG
    updates (1e-4), and sqrt(W) J delta against the oracle's own pipeline (1e-4); each 1e-4 widened
    only by the rounding-sensitivity bound of CG;
  * the oracle's line search (en:305-333) run on the device's own delta: the same scales tried and
    accepted, the loss and the updated parameters within 1e-5.
"""
import torch

from oracle import engine as oeng
from oracle import kernels as ok
from oracle import solver as osol
from tests.helpers import rel_err


def oracle_system(inp, hp, flags, z_prior=None, extra_loss=None):
    """The oracle's objective and damped normal equations at one LM step's inputs (CPU tensors).
    z_prior (H_z, g_z) is added to the z-coefficient blocks (bs:141-173); extra_loss(z_coefs), when
    given, is added to the objective (the tangent prior's loss, en:270-277)."""
    lg = hp.get('is_depth_log', True)
    loss, res, w = oeng.objective(inp['rigs'], inp['K'], inp['P_rig2cam'], inp['P_w2rig'], inp['z_coefs'],
                                  inp['pts3d'], inp['pids'], inp['pix2d'], inp['pix2d_std'], inp['pix2d_dep'], lg,
                                  hp['weight_z'], hp['pnorm'], hp['clip_pix_err'], hp['huber_delta'])
    Jc, Jz, Jp = ok.jacobians_with_rigs(inp['rigs'], inp['K'], inp['P_rig2cam'], inp['P_w2rig'], inp['z_coefs'],
                                        inp['pts3d'], inp['pids'], inp['pix2d_std'], inp['pix2d_dep'], lg,
                                        float64=True)
    if not flags.get('optim_Z0', True):
        Jz[:, 0, 0] = 0
    prob = osol.Problem(inp['rigs'], inp['pids'], len(inp['K']), len(inp['P_w2rig']), len(inp['pts3d']),
                        inp['z_coefs'].shape[1])
    f = {k: v for k, v in flags.items() if k in ('optim_K', 'optim_P', 'optim_Z', 'optim_X', 'no_grad_f_from_rz')}
    ne, gvec, params = osol.build_normal_equations(prob, Jc, Jz, Jp, res, w, z_prior=z_prior, **f)
    if extra_loss is not None:
        loss = loss + extra_loss(inp['z_coefs'])
    return dict(loss=loss, res=res, w=w, J=(Jc, Jz, Jp), prob=prob, ne=ne, g=gvec, params=params, flags=f,
                z_prior=z_prior, inp=inp, hp=hp, all_flags=flags)


def weighted_jdelta(sysd, delta):
    """sqrt(W) J delta per residual (fp64), from the per-observation blocks: the change of the weighted
    residuals a step predicts, which the similarity gauge leaves unchanged."""
    Jc, Jz, Jp = sysd['J']
    pr = sysd['prob']
    C = Jz.shape[2]
    dK, dP, dZ, dX = (t.double() for t in osol.unpack_delta(delta.cpu().double(), sysd['params'], C))
    cam = torch.cat([dK[pr.cam], dP[pr.node]], 1)                        # (N, 8) = [fx fy | w v]
    y = torch.einsum('nrc,nc->nr', Jc, cam) + torch.einsum('nrc,nc->nr', Jp, dX[pr.pid])
    y[:, 2] += (Jz[:, 0, :] * dZ[pr.img]).sum(1)
    sW = sysd['w'].clamp(1e-6, 1e6).double().sqrt()
    return (sW * y).reshape(-1)


def _ulp_flips(t, gen):
    """t with about half of its fp32 entries moved by one ulp, up or down at random."""
    flip = torch.rand(t.shape, generator=gen) < 0.5
    up = torch.rand(t.shape, generator=gen) < 0.5
    inf = torch.full_like(t, float('inf'))
    return torch.where(flip, torch.nextafter(t, torch.where(up, inf, -inf)), t)


def rounded_differently(sysd, gen):
    """The oracle's system rebuilt from inputs moved by one ulp (pixel positions, depth samples and
    points): what a different rounding of one fp32 operation does to the system.  The residuals
    carry cancellations the reference computes in fp32 (r2 = fbar (sum z_c dep_c - ln z), with fbar ~
    500; r0 = (proj - u) / std with u ~ 256), so one ulp of g, ln z or proj moves a residual by far
    more than one ulp of itself; moving the inputs reproduces that."""
    inp = dict(sysd['inp'])
    for k in ('pix2d', 'pix2d_dep', 'pts3d'):
        inp[k] = _ulp_flips(inp[k], gen)
    return oracle_system(inp, sysd['hp'], sysd['all_flags'], z_prior=sysd['z_prior'])


def device_system(solver):
    """(S with damping, rhs, diag(H_cc)) of the solver's last solve_delta, on the host.  Read it right
    after the step: the structure plan's workspaces are reused by the next solve on the same plan."""
    S, rhs = solver.reduced_system_dense()
    return S.cpu(), rhs.cpu(), solver.last['diagA'].cpu()


def check_step_delta(sysd, delta, istate, seed, reduced):
    """The device step delta (fp32) of one LM step against the reference's algorithm, in three parts:
      * the device's reduced system (S with damping, rhs) equals the oracle's to 1e-5, widened only by
        5x its own move when the oracle's fp32 inputs are rounded differently (rounded_differently;
        near the optimum the reduced rhs is a small difference of large terms);
      * the oracle's _pcg (bs:1197-1238) run on the device's own reduced system for the device's
        number of updates (its converged count, else its best iterate's), followed by the oracle's
        back-substitution (bs:203), gives the device's delta to 1e-4, widened only by the
        rounding-sensitivity bound: 5x the largest move of that iterate under another summation order
        (S applied transposed) and a 1e-15 relative perturbation of b;
      * sqrt(W) J delta, the residual change the step predicts (blind to the similarity gauge, where
        only the 1e-12 damping fixes the step), against the oracle's own pipeline on its own system to
        1e-4, widened by 5x the move of the oracle's iterate when its fp32 inputs are rounded
        differently (the device evaluates logf, powf, the sums and divisions with its own roundings), b
        is perturbed by 1e-15, or S is applied densely.
    Comparing the raw delta across the two systems would measure rounding, not the implementation:
    on these damped systems S has condition numbers up to ~1e16, and CG amplifies 1e-7 differences
    in S by that much along the weakly determined directions."""
    ne, gvec = sysd['ne'], sysd['g']
    n_c = ne.sizes['n_c']
    conv = bool(int(istate[3]))
    k = int(istate[2]) if conv else int(istate[4])
    assert k >= 1
    gen = torch.Generator().manual_seed(seed)

    def kth(A_mv, b, diagA):
        hist = []
        osol.pcg(A_mv, b, M_mv=lambda v: v / diagA, tol=0.0, maxiter=k, history=hist)
        return hist[k - 1]

    backsub = lambda ne_, g_, dc: torch.cat([dc, osol._D_solve(ne_, g_[n_c:] - osol._C_matvec(ne_, dc))])
    # (1) the device's reduced system against the oracle's; near the optimum the reduced rhs
    # g_c - H_cp H_pp^-1 g_p is a small difference of large terms, so its bar also takes 5x its own
    # move when the fp32 inputs are rounded differently
    S_dev, rhs_dev, dA_dev = reduced
    dA_dev = dA_dev.clamp(min=1e-12)
    S_or = osol.dense_schur(ne)
    rhs_or = osol.reduced_rhs(ne, gvec)
    flipped = [rounded_differently(sysd, gen) for _ in range(2)]
    e_S, e_r = rel_err(S_dev, S_or), rel_err(rhs_dev, rhs_or)
    tol_S = max([1e-5] + [5 * rel_err(osol.dense_schur(f['ne']), S_or) for f in flipped])
    tol_r = max([1e-5] + [5 * rel_err(osol.reduced_rhs(f['ne'], f['g']), rhs_or) for f in flipped])
    assert e_S < tol_S and e_r < tol_r, (e_S, tol_S, e_r, tol_r)
    # (2) the reference's PCG and back-substitution on the device's own system
    same = kth(lambda v: S_dev @ v, rhs_dev, dA_dev)
    alts = [kth(lambda v: S_dev.T @ v, rhs_dev, dA_dev),
            kth(lambda v: S_dev @ v, rhs_dev * (1 + 1e-15 * torch.randn(n_c, generator=gen, dtype=torch.float64)),
                dA_dev)]
    ref_same = backsub(ne, gvec, same)
    tol_d = max([1e-4] + [5 * rel_err(backsub(ne, gvec, a), ref_same) for a in alts])
    e_d = rel_err(delta, ref_same.to(torch.float32))
    # (3) sqrt(W) J delta against the oracle's pipeline on its own system
    dA_or = osol.A_diag(ne).clamp(min=1e-12)
    ref_k = backsub(ne, gvec, kth(lambda v: osol.S_matvec(ne, v), rhs_or, dA_or))
    jalts = [backsub(ne, gvec, kth(lambda v: S_or @ v, rhs_or, dA_or)),
             backsub(ne, gvec, kth(lambda v: osol.S_matvec(ne, v),
                                   rhs_or * (1 + 1e-15 * torch.randn(n_c, generator=gen, dtype=torch.float64)),
                                   dA_or))]
    for f in flipped:
        ne2, g2 = f['ne'], f['g']
        jalts.append(backsub(ne2, g2, kth(lambda v: osol.S_matvec(ne2, v), osol.reduced_rhs(ne2, g2),
                                          osol.A_diag(ne2).clamp(min=1e-12))))
    jd_ref = weighted_jdelta(sysd, ref_k)
    tol_j = max([1e-4] + [5 * rel_err(weighted_jdelta(sysd, d), jd_ref) for d in jalts])
    e_j = rel_err(weighted_jdelta(sysd, delta), jd_ref)
    print(f'  step: k={k}; S {e_S:.1e} (bar {tol_S:.0e}), rhs {e_r:.1e} (bar {tol_r:.0e}); delta vs PCG on the device system {e_d:.2e} (bar {tol_d:.2e}); '
          f'sqrt(W) J delta {e_j:.2e} (bar {tol_j:.2e}); raw delta vs the oracle system '
          f'{rel_err(delta, ref_k.to(torch.float32)):.2e}', flush=True)
    assert e_d < tol_d, (e_d, tol_d, k)
    assert e_j < tol_j, (e_j, tol_j, k)
    return dict(k=k, err_S=e_S, err_rhs=e_r, err_delta=e_d, tol_delta=tol_d, err_jdelta=e_j, tol_jdelta=tol_j)


def check_line_search(inp, hp, sysd, delta, dev_info, st_g, up_g, min_reproj=0.01, min_loss_delta=1e-4,
                      extra_loss=None):
    """The oracle's trial loop (en:305-333) run on the device's own step: the same scales tried, the
    same accepted one, the new loss within 1e-5 and the updated parameters' change within 1e-5 (plus
    the fp32 rounding of the parameters themselves)."""
    C = inp['z_coefs'].shape[1]
    dK, dP, dZ, dX = osol.unpack_delta(delta.cpu(), sysd['params'], C)
    K, P, Z, X = inp['K'], inp['P_w2rig'], inp['z_coefs'], inp['pts3d']

    def trial(scale):
        up = oeng.apply_update(K, P, Z, X, dK, dP, dZ, dX, scale)
        loss, res, _ = oeng.objective(inp['rigs'], up['K'], inp['P_rig2cam'], up['P_w2rig'], up['z_coefs'],
                                      up['pts3d'], inp['pids'], inp['pix2d'], inp['pix2d_std'], inp['pix2d_dep'],
                                      hp.get('is_depth_log', True), hp['weight_z'], hp['pnorm'], hp['clip_pix_err'],
                                      hp['huber_delta'])
        if extra_loss is not None:
            loss = loss + extra_loss(up['z_coefs'])
        return loss, oeng.reproj_score(res), up

    ls = oeng.line_search(trial, sysd['loss'], min_loss_delta, min_reproj)
    assert dev_info['scales'] == ls['scales'], (dev_info['scales'], ls['scales'])
    assert abs(float(st_g.init_loss) - float(ls['init_loss'])) <= 1e-5 * abs(float(ls['init_loss']))
    assert abs(float(st_g.new_loss) - float(ls['new_loss'])) <= 1e-5 * abs(float(ls['new_loss']))
    # the updated parameters are fp32: their change is compared to 1e-5 of its size plus 4 ulps of the
    # parameters' own size (the rounding of the fp32 update both sides make, visible for small steps)
    for k, x0 in (('K', K), ('P_w2rig', P), ('z_coefs', Z), ('pts3d', X)):
        ref = (ls['payload'][k] - x0).double()
        got = (up_g[k].cpu() - x0).double()
        err = float((got - ref).norm())
        bar = 1e-5 * float(ref.norm()) + 2.0 ** -21 * float(x0.double().norm())
        assert err <= bar, (k, err, bar, float(ref.norm()))
    return ls
