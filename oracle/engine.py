"""Oracle restatement of the reference LM step (test infrastructure only).

Follows ``lm_step`` (src/blast3r/inference/engine.py:206-334, abbreviated ``en``)
on CPU with the oracle kernels and solver: objective = mean Huber error
(en:263-278), linearisation + Schur solve (en:284-303), update of K, P, z, X
(en:310-313, en:347-354, cujac/__init__.py:56-58) and the step-halving line
search over a in [0.5, 0.25, 0.125, 1/64, 1/512, 1/4096, 0] with the
min_loss_delta and reproj_score tests (en:308-333, en:357-361).
``bundle_adjustment`` restates the phase loop of en:405-503 (per-phase options,
z-coefficient add/remove, stop on no decrease).  The tangent prior (en:15-179)
is restated separately in ``oracle.tangent``.
"""
from collections import namedtuple

import torch

from . import kernels as K_
from . import tangent as T_
from .solver import Problem, build_normal_equations, solve_reduced_pcg, solve_reduced_direct, unpack_delta

BA_Status = namedtuple('BA_Status', 'init_loss, init_residuals, new_loss, new_residuals')

STEP_SCHEDULE = [0.5, 0.25, 0.125, 1 / 64, 1 / 512, 1 / 4096, 0]      # en:309


def update_K(K0, delta_focal, min_f=100):
    """en:347-354."""
    dfx, dfy = delta_focal.T
    K = K0.clone()
    K[:, 0, 0] -= dfx
    K[:, 1, 1] -= dfy
    K[:, 0, 0].clip_(min=min_f)
    K[:, 1, 1].clip_(min=min_f)
    return K


def apply_update(K, P_w2rig, z_coefs, pts3d, dK, dP, dZ, dX, scale=1.0):
    """en:310-313: the parameters after a step of `scale` times delta: f -= dK (clipped, en:347-354),
    P <- exp(-dP^) P (cujac/__init__.py:56-58, a left update), z -= dZ, X -= dX."""
    return dict(K=update_K(K, dK * scale), P_w2rig=K_.exp_se3(-(dP * scale)) @ P_w2rig,
                z_coefs=z_coefs - dZ * scale, pts3d=pts3d - dX * scale)


def reproj_score(res):
    """Mean of the lowest 80% of ||r[:, :2]|| (en:357-361)."""
    e = res[:, :2].norm(dim=-1).sort().values
    n80 = len(e) * 80 // 100
    return e[:n80].mean()


def line_search(trial, init_loss, min_loss_delta=1e-4, min_reproj=0.01):
    """The trial loop of en:305-333.  trial(scale) returns (loss, reproj_score, payload) for the update
    at `scale` times the step (en:310-313 with delta scaled in place by a / last_a, en:330).

    Written with the reference's in-place tensor operations: after a NaN loss `new_loss = init_loss`
    makes both names one tensor and `new_loss += min_loss_delta` (en:317-319) adds min_loss_delta to
    init_loss itself, which every later comparison and the returned status see.  The caller's tensor
    is cloned first, so only this step's init_loss changes, as in the reference where it is a fresh
    result of objective().  Returns dict(scale, scales, init_loss, new_loss, payload, accepted)."""
    init_loss = init_loss.clone()
    last_a = 1
    scale = 1.0
    scales = []
    accepted = False
    for a in STEP_SCHEDULE:
        scales.append(scale)
        new_loss, reproj, payload = trial(scale)
        new_loss = new_loss.clone()
        if new_loss.isnan():                                                    # en:316-318
            new_loss = init_loss
        new_loss += min_loss_delta                                              # en:319
        new_reproj = float(reproj)                                              # en:324
        degenerate = new_reproj < min_reproj
        if new_loss < init_loss and not degenerate:                             # en:328
            accepted = True
            break
        scale = scale * (a / last_a)     # delta *= a / last_a (en:330) applied to every slice
        last_a = a
    return dict(scale=scales[-1], scales=scales, init_loss=init_loss, new_loss=new_loss, payload=payload,
                accepted=accepted)


def objective(rigs, K, P_rig2cam, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std, pix2d_dep,
              is_depth_log, weight_z, pnorm, clip_pix_err, huber_delta):
    """en:263-278 without the tangent prior."""
    out = K_.residuals_with_rigs(rigs, K, P_rig2cam, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std,
                                 pix2d_dep, is_depth_log, weight_z, pnorm, clip_pix_err, huber_delta)
    res, err, w = out.reshape(-1, 3, 3).unbind(dim=1)
    return err.mean(), res, w


def linearize_and_solve(rigs, pids, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs, pts3d,
                        residuals, w_pts, is_depth_log=True, optim_K=True, optim_Z=True, optim_P=True,
                        optim_X=True, optim_Z0=True, optim_Z_1st_cam=True, no_grad_f_from_rz=False,
                        dampen=1e-12, adaptive_dampen=True, dtype=torch.float64, solver='pcg',
                        pcg_tol=1e-6, pcg_maxiter=300, z_prior=None):
    """compute_jacobians + solve_delta + unpack (bs:34-40, bs:110-248). Returns (dK, dP, dZ, dX, info)."""
    J_cam, J_zcf, J_pts = K_.jacobians_with_rigs(rigs, K, P_rig2cam, P_w2rig, z_coefs, pts3d, pids, pix2d_std,
                                                 pix2d_dep, is_depth_log, float64=(dtype == torch.float64))
    if not optim_Z_1st_cam:                                                           # bs:38
        J_zcf[0, 0, 0] = 0
    if not optim_Z0:                                                                  # bs:39
        J_zcf[:, 0, 0:1] = 0
    prob = Problem(rigs, pids, len(K), len(P_w2rig), len(pts3d), z_coefs.shape[1])
    ne, g, params = build_normal_equations(prob, J_cam, J_zcf, J_pts, residuals, w_pts, optim_K=optim_K,
                                           optim_P=optim_P, optim_Z=optim_Z, optim_X=optim_X,
                                           no_grad_f_from_rz=no_grad_f_from_rz, dampen=dampen,
                                           adaptive_dampen=adaptive_dampen, z_prior=z_prior)
    info = dict(ne=ne, g=g, params=params)
    if solver == 'pcg':
        delta, niter, conv = solve_reduced_pcg(ne, g, tol=pcg_tol, maxiter=pcg_maxiter)
        info.update(niter=niter, converged=conv)
    else:
        delta = solve_reduced_direct(ne, g)
    delta = delta.to(torch.float32)                                                   # bs:182
    info['delta'] = delta
    return unpack_delta(delta, params, z_coefs.shape[1]) + (info,)


def lm_step(rigs, pids, pix2d, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs, pts3d, depth_mode='log',
            pnorm=1, clip_pix_err=100, huber_delta=0.5, min_reproj=0.01, dampen=1e-12, min_loss_delta=1e-4,
            weight_z=1, optim_K=True, optim_Z=True, optim_P=True, optim_X=True, optim_Z0=True,
            no_grad_f_from_rz=False, adaptive_dampen=True, dtype=torch.float32, solver='pcg', verbose=False,
            pcg_tol=1e-6, pcg_maxiter=300, log_depth_maps=None, conf=None, pts3d_ref=None, weight_tan=0.0,
            tan_stride=4, normalize_tangents=True):
    """en:206-334 on CPU. Returns (update dict, BA_Status, info).  dtype defaults to torch.float32, the
    reference's GaussNewtonSolver default that lm_step uses when the caller passes none (bs:22, en:284);
    bundle_adjustment passes torch.float64 (en:490)."""
    assert depth_mode in ('lin', 'log')
    is_depth_log = depth_mode == 'log'
    K_tan = K.detach()
    tan_kw = dict(weight_tan=float(weight_tan), tan_stride=int(tan_stride), optim_Z0=optim_Z0,
                  normalize_tangents=bool(normalize_tangents))

    def obj(K, P_w2rig, pts3d, z_coefs):
        loss, res, w = objective(rigs, K, P_rig2cam, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std, pix2d_dep,
                                 is_depth_log, weight_z, pnorm, clip_pix_err, huber_delta)
        if weight_tan > 0:                                                        # en:270-277
            loss = loss + T_.tangent_prior_terms(rigs[2], K_tan, z_coefs, log_depth_maps, pts3d_ref, dtype=loss.dtype,
                                                 compute_gn=False, **tan_kw)[0]
        return loss, res, w

    init_loss, init_residuals, w_pts = obj(K, P_w2rig, pts3d, z_coefs)
    z_prior = None
    if weight_tan > 0:                                                            # en:288-298
        _, g_z, H_z = T_.tangent_prior_terms(rigs[2], K_tan, z_coefs, log_depth_maps, pts3d_ref, dtype=dtype,
                                             compute_gn=True, **tan_kw)
        z_prior = (H_z, g_z)
    dK, dP, dZ, dX, info = linearize_and_solve(rigs, pids, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs,
                                               pts3d, init_residuals, w_pts, is_depth_log=is_depth_log,
                                               optim_K=optim_K, optim_Z=optim_Z, optim_P=optim_P, optim_X=optim_X,
                                               optim_Z0=optim_Z0, no_grad_f_from_rz=no_grad_f_from_rz,
                                               dampen=dampen, adaptive_dampen=adaptive_dampen, dtype=dtype,
                                               solver=solver, pcg_tol=pcg_tol, pcg_maxiter=pcg_maxiter,
                                               z_prior=z_prior)
    def trial(scale):
        update = apply_update(K, P_w2rig, z_coefs, pts3d, dK, dP, dZ, dX, scale)
        new_loss, new_residuals, _ = obj(**update)
        return new_loss, reproj_score(new_residuals), (update, new_residuals)

    ls = line_search(trial, init_loss, min_loss_delta, min_reproj)
    update, new_residuals = ls['payload']
    init_loss, new_loss = ls['init_loss'], ls['new_loss']
    trials, scale = len(ls['scales']), ls['scale']
    info['trials'] = trials
    info['scale'] = scale
    return update, BA_Status(init_loss, init_residuals, new_loss, new_residuals), info


def iter_on(*iterators):
    """en:364-383: per-phase values; scalars repeat, lists give one value per phase."""
    iterable = lambda it: isinstance(it, (tuple, list))
    n = max([len(it) for it in iterators if iterable(it)] + [1])
    its = []
    for it in iterators:
        if iterable(it):
            assert len(it) in (1, n)
            its.append(it[0] if len(it) == 1 else it)
        else:
            its.append(it)
    for k in range(n):
        yield tuple(it[k] if iterable(it) else it for it in its)


def bundle_adjustment(rigs_data, track_data, pts3d, z_coefs=None, max_iters=1000, pnorm=0.5, optim_P=True,
                      optim_Z=True, optim_Z0=True, optim_K=True, optim_X=True, weight_z=0.1, n_zcfs=None,
                      no_Jfz=False, max_n_phases=-1, **lm_kwargs):
    """en:405-503 on CPU with the oracle lm_step (no tangent prior).

    rigs_data needs K, P_rig2cam, P_w2rig, z_coefs, depth_mode, infos(tracks), z_coefs_from_scale(tracks);
    track_data needs pids, pix2d, pix2d_std, pix2d_dep.  Returns (dict of the optimised K, P_w2rig,
    z_coefs, pts3d, number of accepted steps per phase)."""
    trk, rig = track_data, rigs_data
    if z_coefs is None:
        z_coefs = rig.z_coefs_from_scale(trk)
    dep0 = trk.pix2d_dep
    var = dict(K=rig.K, P_w2rig=rig.P_w2rig, z_coefs=z_coefs, pts3d=pts3d)
    steps = []
    phase = 0
    dep = dep0             # the reference narrows track_data.pix2d_dep in place; it persists across phases
    for pnorm, max_iters, optim_K, optim_P, optim_Z, optim_X, weight_z, n_zcfs in \
            iter_on(pnorm, max_iters, optim_K, optim_P, optim_Z, optim_X, weight_z, n_zcfs):
        phase += 1
        if phase > (max_n_phases % 1000):                                       # en:447
            break
        if n_zcfs is not None:                                                  # en:451-471
            optim_Z0 = True
            if rig.depth_mode[:3] == 'log':
                optim_Z0 = (n_zcfs == 2) or (n_zcfs == dep0.shape[1])
                n_zcfs += not optim_Z0
            dep = dep0[:, :n_zcfs].contiguous()
            zc = var['z_coefs']
            if n_zcfs < zc.shape[1]:
                var['z_coefs'] = zc[:, :n_zcfs].contiguous()
            elif n_zcfs > zc.shape[1]:
                var['z_coefs'] = torch.cat((zc, zc.new_zeros((len(zc), n_zcfs - zc.shape[1]))), dim=1).contiguous()
        infos = rig.infos(trk)
        k = 0
        while k < max_iters:                                                    # en:476-497
            up, st, _ = lm_step(infos, trk.pids, trk.pix2d, trk.pix2d_std, dep, var['K'], rig.P_rig2cam,
                                var['P_w2rig'], var['z_coefs'], var['pts3d'], depth_mode=rig.depth_mode,
                                pnorm=pnorm, weight_z=weight_z, optim_K=optim_K, optim_Z=optim_Z, optim_P=optim_P,
                                optim_X=optim_X, optim_Z0=optim_Z0, no_grad_f_from_rz=no_Jfz, dtype=torch.float64,
                                **lm_kwargs)
            if st.new_loss >= st.init_loss:
                break
            var.update(up)
            k += 1
        steps.append(k)
    return var, steps
