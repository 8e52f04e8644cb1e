"""MI355X LM driver: drop-in for src/blast3r/inference/engine.py (``en``) on the BA path.

``lm_step`` and ``bundle_adjustment`` keep the reference signatures, defaults,
return values and control flow (en:206-334, en:405-503).  The numerical work
runs in libba_hip.so: residuals (ba_residuals), the fused linearize + Schur +
PCG + back-substitution step (GaussNewtonSolver), the parameter update
(ba_apply_update) and the line-search objective with an exact radix-select
reproj_score (ba_objective), and the dense tangent prior (ba_tangent_prior, en:15-200) when
weight_tan > 0.
"""
from collections import namedtuple

import ctypes

import torch

from . import cujac
from ._lib import check, lib, ptr, stream_ptr
from .ba_solver import GaussNewtonSolver, _param_state
from .tangent import confident_in_planar_regions, dense_tangent_prior_terms as _dense_tangent_prior_terms

BA_Status = namedtuple('BA_Status', 'init_loss, init_residuals, new_loss, new_residuals')

STEP_SCHEDULE = [0.5, 0.25, 0.125, 1 / 64, 1 / 512, 1 / 4096, 0]     # en:309


def shape_of(tensor, is_contiguous=True, check_finite=True):
    """The shape of an lm_step input once it has passed the input checks of en:340-344: fp32 or int32,
    contiguous unless is_contiguous is False, and finite (check_finite=False leaves that check to one
    batched device check of all inputs, _nonfinite_flag)."""
    assert tensor.dtype in (torch.float32, torch.int32) and (not is_contiguous or tensor.is_contiguous())
    if check_finite:
        _assert_finite(tensor)
    return tensor.shape


def _nonfinite_flag(*tensors):
    """The isfinite check of every tensor (en:343) for the device fp32 inputs, launched without a
    host read: returns a 0-d device bool (True when a value is non-finite), or None when no input is
    on the device.  Host inputs are asserted at once; int32 tensors are finite by type."""
    floats = [t for t in tensors if t.dtype != torch.int32]
    dev = [t for t in floats if t.is_cuda]
    for t in floats:
        if not t.is_cuda:
            assert t.isfinite().all()
    if not dev:
        return None
    views = [t if t.is_contiguous() else t.contiguous() for t in dev]
    flags = torch.empty(len(views), dtype=torch.int32, device=views[0].device)
    for k in range(0, len(views), 16):
        part = views[k:k + 16]
        n = len(part)
        ptrs = (ctypes.c_void_p * n)(*[t.data_ptr() for t in part])
        counts = (ctypes.c_int64 * n)(*[t.numel() for t in part])
        check(lib().ba_nonfinite_flags(ptrs, counts, n, ptr(flags[k:k + n]), stream_ptr(part[0].device)))
    return flags.any()


def _assert_finite(*tensors):
    """``assert t.isfinite().all()`` for every tensor (en:343), one launch and one host read for all
    device fp32 inputs (ba_nonfinite_flags)."""
    f = _nonfinite_flag(*tensors)
    if f is not None:
        assert not bool(f.cpu()), 'non-finite input'


def update_K(K0, delta_focal, min_f=100):
    """Intrinsics after a focal step (en:347-354): (fx, fy) <- max((fx, fy) - delta_focal, min_f), the
    rest of K0 unchanged (a NaN focal stays NaN)."""
    K = K0.clone()
    diag = torch.arange(2, device=K0.device)
    K[:, diag, diag] = torch.clamp(K0[:, diag, diag] - delta_focal, min=min_f)
    return K


def reproj_score(res):
    """Mean of the lowest 80% of ||r[:, :2]|| (en:357-361); device radix select, no sort."""
    n = res.shape[0]
    buf = res[:, :2].T.contiguous() if not (res.stride(0) == 1) else None
    base = buf if buf is not None else res.T   # (k, n) with unit stride along n
    return _objective(base, n, has_err=False)[1]


def _objective(res_kn, n, has_err):
    """(loss, reproj) as 0-d device tensors from a (>=3 or 2, n) SoA buffer with unit inner stride."""
    dev = res_kn.device
    if res_kn.stride(1) != 1 or (res_kn.shape[0] > 1 and res_kn.stride(0) != n):
        res_kn = res_kn.contiguous()
    ws = torch.empty(int(lib().ba_objective_workspace_bytes(n)), dtype=torch.uint8, device=dev)
    out = torch.empty(2, dtype=torch.float32, device=dev)
    check(lib().ba_objective(ptr(res_kn), n, int(has_err), ptr(ws), ptr(out), stream_ptr(dev)))
    return out[0], out[1]


def iter_on(*params):
    """The per-phase values of bundle_adjustment's phase-wise arguments (en:364-383): as many phases as
    the longest list or tuple (at least one); a list or tuple gives its k-th value in phase k, or its
    only value in every phase; anything else is the same in every phase.  A list of another length
    fails the assertion the reference makes, when the first phase is asked for."""
    is_seq = lambda v: isinstance(v, (tuple, list))
    n_phases = max([1] + [len(v) for v in params if is_seq(v)])
    for v in params:
        if is_seq(v):
            assert len(v) in (1, n_phases), f'missing {n_phases - len(v)} values for parameter={v}'
    per_phase = [(lambda k, v=v: v[0]) if is_seq(v) and len(v) == 1 else
                 (lambda k, v=v: v[k]) if is_seq(v) else (lambda k, v=v: v) for v in params]
    for k in range(n_phases):
        yield tuple(f(k) for f in per_phase)


def used_depth_channels(n_zcfs, n_channels, depth_mode):
    """The leading depth channels bundle_adjustment reads for the phases' n_zcfs (en:386-402): a phase
    of n coefficients reads n channels, plus the frozen main channel in a log mode unless n is 2 or
    every channel; a phase with n_zcfs None reads all of them.  At most n_channels."""
    phases = list(n_zcfs) if isinstance(n_zcfs, (list, tuple)) else [n_zcfs]
    if any(n is None for n in phases):
        return n_channels
    frozen_main = depth_mode.startswith('log')
    reads = [n + int(frozen_main and n not in (2, n_channels)) for n in phases]
    return min(max(reads, default=0), n_channels)


def line_search(trial, init_loss, min_loss_delta, min_reproj, nonfinite=None):
    """The step-halving loop of lm_step (en:308-333), on 0-d loss tensors.

    trial(scale) evaluates the update at `scale` times the step and returns (loss, reproj_score,
    payload); the scales tried are 1, then the running product of a / last_a over the schedule
    (en:330 scales every slice of delta in place).  A trial is accepted when loss + min_loss_delta <
    init_loss and reproj_score >= min_reproj.  A NaN loss takes the reference's aliasing
    (en:317-319: `new_loss = init_loss; new_loss += min_loss_delta` adds min_loss_delta to init_loss
    itself): init_loss grows by min_loss_delta for the rest of the step and is returned so.  All
    comparisons use the fp32 sums formed on the loss's device, read with one copy per trial.
    nonfinite, when given, is lm_step's input check (a 0-d device bool): it travels with the first
    trial's values, and the step raises there, before any decision, as the reference raises at its
    start (en:343).
    Returns a dict: scale, scales (every scale tried), init_loss, new_loss (with min_loss_delta),
    trial_loss (the last trial's objective as evaluated), payload, accepted."""
    scale = 1.0
    last_a = 1
    scales = []
    accepted = False
    for a in STEP_SCHEDULE:
        scales.append(scale)
        trial_loss, reproj_t, payload = trial(scale)
        # one read for every decision: the sums + min_loss_delta are formed on the device, as the
        # reference forms them, so the comparison sees the same fp32 values
        plus = trial_loss + min_loss_delta
        init_plus = init_loss + min_loss_delta
        items = [trial_loss, init_loss, reproj_t, plus, init_plus]
        if nonfinite is not None:
            items.append(nonfinite)
        vals = torch.stack([t.reshape(()).to(torch.float32) for t in items]).cpu()
        if nonfinite is not None:
            assert not bool(vals[5]), 'non-finite input'
            nonfinite = None
        if torch.isnan(vals[0]):
            print('Warning: loss is NaN')
            init_loss = new_loss = init_plus     # en:317-319: new_loss aliases init_loss, += adds to both
            lhs, rhs = float(vals[4]), float(vals[4])
        else:
            new_loss = plus
            lhs, rhs = float(vals[3]), float(vals[1])
        new_reproj = float(vals[2])
        degenerate = new_reproj < min_reproj
        if degenerate:
            print(f'Rejecting step: reprojection residual collapsed to {new_reproj:.2e}')
        if lhs < rhs and not degenerate:
            accepted = True
            break
        scale = scale * (a / last_a)       # delta *= a/last_a (en:330): every slice scaled together
        last_a = a
    else:
        print('Warning: loss is not decreasing')
    return dict(scale=scales[-1], scales=scales, init_loss=init_loss, new_loss=new_loss, trial_loss=trial_loss,
                payload=payload, accepted=accepted)


def lm_step(rigs, pids, pix2d, pix2d_std, pix2d_dep,
            K, P_rig2cam, P_w2rig, z_coefs, pts3d,
            depth_mode='log',
            pnorm=1,
            clip_pix_err=100,
            huber_delta=0.5,
            min_reproj=0.01,
            dampen=1e-12,
            min_loss_delta=1e-4,
            weight_z=1,
            log_depth_maps=None, conf=None, pts3d_ref=None, weight_tan=0.0, tan_stride=4,
            normalize_tangents=True,
            optim_K=True, optim_Z=True, optim_P=True, optim_X=True, optim_Z0=True, verbose_steps=False,
            **ba_options):
    """Levenberg-Marquardt step (en:206-334) on MI355X.  Returns (update, BA_Status)."""
    update, status, _ = _lm_step(rigs, pids, pix2d, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs, pts3d,
                                 depth_mode=depth_mode, pnorm=pnorm, clip_pix_err=clip_pix_err,
                                 huber_delta=huber_delta, min_reproj=min_reproj, dampen=dampen,
                                 min_loss_delta=min_loss_delta, weight_z=weight_z, log_depth_maps=log_depth_maps,
                                 conf=conf, pts3d_ref=pts3d_ref, weight_tan=weight_tan, tan_stride=tan_stride,
                                 normalize_tangents=normalize_tangents, optim_K=optim_K, optim_Z=optim_Z,
                                 optim_P=optim_P, optim_X=optim_X, optim_Z0=optim_Z0, **ba_options)
    return update, status


def _lm_step(rigs, pids, pix2d, pix2d_std, pix2d_dep, K, P_rig2cam, P_w2rig, z_coefs, pts3d,
             depth_mode='log', pnorm=1, clip_pix_err=100, huber_delta=0.5, min_reproj=0.01, dampen=1e-12,
             min_loss_delta=1e-4, weight_z=1, log_depth_maps=None, conf=None, pts3d_ref=None, weight_tan=0.0,
             tan_stride=4, normalize_tangents=True, optim_K=True, optim_Z=True, optim_P=True, optim_X=True,
             optim_Z0=True, init_eval=None, info=None, **ba_options):
    """lm_step, plus the objective of the last evaluated trial (loss before min_loss_delta, residuals,
    w_pts) as a third result.  init_eval, when given, is that triple for (K, P_w2rig, z_coefs, pts3d)
    under the same hyper-parameters: the evaluation at the start of the step (en:281) is then taken
    from it instead of being recomputed (same inputs, same kernels, so the same values).  info, when
    a dict, receives the accepted step scale, the scales tried, the fp32 step delta, the PCG's
    istate and the solver (for inspection; nothing else reads it)."""
    assert depth_mode in ('lin', 'log')
    is_depth_log = depth_mode == 'log'
    if weight_tan > 0:
        assert is_depth_log, 'tangent prior currently only implemented for depth_mode="log"'
    n_imgs = rigs.shape[1]
    # en:219-233; the isfinite part of every shape_of runs once for all inputs below
    chk = dict(check_finite=False)
    assert shape_of(rigs, **chk) == (3, n_imgs)
    n_cams = len(K)
    assert shape_of(K, **chk) == (n_cams, 3, 3)
    assert shape_of(P_rig2cam, is_contiguous=False, **chk) == (n_cams, 4, 4)
    n_nodes = len(P_w2rig)
    assert shape_of(P_w2rig, **chk) == (n_nodes, 4, 4)
    n_zcf = z_coefs.shape[1]
    assert shape_of(z_coefs, **chk) == (n_imgs, n_zcf)
    n_tracks = len(pts3d)
    assert shape_of(pts3d, **chk) == (n_tracks, 3)
    n_obs = len(pids)
    assert shape_of(pids, **chk) == (n_obs,)
    assert shape_of(pix2d, **chk) == (n_obs, 2)
    assert shape_of(pix2d_std, **chk) == (n_obs, 2)
    assert shape_of(pix2d_dep, **chk) == (n_obs, n_zcf), \
        f'expected pix2d_dep of shape {(n_obs, n_zcf)}, got {shape_of(pix2d_dep, **chk)}'
    # the isfinite assertions (en:343): launched here, read with the first line-search trial (one host
    # round trip fewer; nothing the step does before that depends on the answer)
    nonfinite = _nonfinite_flag(K, P_rig2cam, P_w2rig, z_coefs, pts3d, pix2d, pix2d_std, pix2d_dep)
    assert 0 <= weight_z <= 10
    assert n_obs >= n_tracks, 'there must be more 2d kpts than tracks'
    assert huber_delta >= 0.1

    w_null = 1e-16
    K_tan = K.detach()          # the prior treats the intrinsics as constant within the step (en:250-252)
    tan_kw = dict(weight_tan=float(weight_tan), tan_stride=int(tan_stride), optim_Z0=optim_Z0,
                  normalize_tangents=bool(normalize_tangents))

    def objective(K, P_w2rig, pts3d, z_coefs):
        out = cujac.compute_residuals_with_rigs(rigs, K, P_rig2cam, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std,
                                                pix2d_dep, is_depth_log, weight_z, pnorm, clip_pix_err, huber_delta,
                                                w_null)
        buf = out.T                                               # (9, n) buffer
        residuals_, err_, w_pts_ = out.view(-1, 3, 3).unbind(dim=1)
        loss, reproj = _objective(buf, n_obs, has_err=pnorm > 0)
        if weight_tan > 0:                                        # en:270-277
            tan_loss, _, _ = _dense_tangent_prior_terms(rigs, K_tan, z_coefs, log_depth_maps, conf, pts3d_ref,
                                                        dtype=loss.dtype, compute_gn=False, **tan_kw)
            loss = loss + tan_loss
        return loss, residuals_, w_pts_, reproj

    if init_eval is not None:
        init_loss, init_residuals, w_pts = init_eval
    else:
        init_loss, init_residuals, w_pts, _ = objective(K, P_w2rig, pts3d, z_coefs)

    hp = dict(weight_z=weight_z, pnorm=pnorm, max_pix_err=clip_pix_err, huber_delta=huber_delta, w_pts_null=w_null)
    jac = GaussNewtonSolver(n_cams, n_nodes, n_imgs, n_tracks, pts3d.device, dampen=dampen, **ba_options)
    J = jac.compute_jacobians(rigs, K, P_rig2cam, P_w2rig, z_coefs, pts3d, pids, pix2d_std, pix2d_dep,
                              optim_K=optim_K, optim_Z=optim_Z, optim_Z0=optim_Z0, optim_P=optim_P, optim_X=optim_X,
                              is_depth_log=is_depth_log, pix2d=pix2d, hp=hp)
    init_residuals._ba_state = _param_state(J)
    z_prior = None
    if weight_tan > 0:                                            # en:288-298: GN terms on z_coefs only
        _, g_z, H_z = _dense_tangent_prior_terms(rigs, K_tan, z_coefs, log_depth_maps, conf, pts3d_ref,
                                                 dtype=jac.dtype, compute_gn=True, **tan_kw)
        z_prior = (H_z, g_z)
    delta = jac.solve_delta(J, init_residuals, w_pts, z_prior=z_prior)
    delta_K, delta_P, delta_zcf, delta_pts = jac.unpack_delta_inplace(delta)

    dKc = delta_K.contiguous()
    dPc = delta_P.contiguous()
    dZc = delta_zcf.contiguous()
    dXc = delta_pts.contiguous()
    dev = pts3d.device

    def trial(scale):
        Kn = torch.empty_like(K)
        Pn = torch.empty_like(P_w2rig)
        Zn = torch.empty_like(z_coefs)
        Xn = torch.empty_like(pts3d)
        check(lib().ba_apply_update(ptr(K), ptr(P_w2rig), ptr(z_coefs), ptr(pts3d), ptr(dKc), ptr(dPc), ptr(dZc),
                                    ptr(dXc), float(scale), 100.0, n_cams, n_nodes, n_imgs, n_zcf, n_tracks,
                                    ptr(Kn), ptr(Pn), ptr(Zn), ptr(Xn), stream_ptr(dev)))
        update = dict(K=Kn, P_w2rig=Pn, z_coefs=Zn, pts3d=Xn)
        new_loss, new_residuals, new_w, new_reproj = objective(**update)
        return new_loss, new_reproj, (update, new_residuals, new_w)

    ls = line_search(trial, init_loss, min_loss_delta, min_reproj, nonfinite=nonfinite)
    update, new_residuals, new_w = ls['payload']
    if info is not None:
        ist = jac.last.get('istate')
        info.update(scale=ls['scale'], scales=ls['scales'], trials=len(ls['scales']), delta=delta,
                    pcg_istate=None if ist is None else ist.clone(), solver=jac)
    # the objective of the last trial, before min_loss_delta (what the next step starts from)
    last_eval = (ls['trial_loss'], new_residuals, new_w)
    init_loss, new_loss = ls['init_loss'], ls['new_loss']
    return update, BA_Status(init_loss, init_residuals, new_loss, new_residuals), last_eval


def bundle_adjustment(rigs_data, track_data, pts3d=None, z_coefs=None,
                      max_iters=1000,
                      pnorm=0.5,
                      optim_P=True,
                      optim_Z=True,
                      optim_Z0=True,
                      optim_K=True,
                      optim_X=True,
                      weight_z=0.1,
                      dense_depth=None,
                      dense_conf=None,
                      dense_pts3d_ref=None,
                      tangent_reg=0.0,
                      tan_stride=4,
                      normalize_tangents=True,
                      n_zcfs=None,
                      no_Jfz=False,
                      max_n_phases=-1,
                      device='cuda',
                      verbose=True,
                      **other_lm_kwargs):
    """Main bundle-adjustment loop (en:405-503)."""
    trk = track_data.to(device)
    rig = rigs_data.to(device)
    todev = lambda x: None if x is None else (x.to(device) if isinstance(x, torch.Tensor) else [t.to(device) for t in x])
    dense_depth, dense_conf, dense_pts3d_ref = todev(dense_depth), todev(dense_conf), todev(dense_pts3d_ref)
    if z_coefs is None:
        z_coefs = rig.z_coefs_from_scale(trk)
    original_pix2d_dep = trk.pix2d_dep
    assert pts3d is not None, 'the 3D points must be initialized before bundle adjustment'
    pts3d = pts3d.to(device)
    variables = dict(K=rig.K, P_rig2cam=rig.P_rig2cam, P_w2rig=rig.P_w2rig, z_coefs=z_coefs, pts3d=pts3d)
    phase_num = 0
    for pnorm, max_iters, optim_K, optim_P, optim_Z, optim_X, weight_z, n_zcfs, tangent_reg in \
            iter_on(pnorm, max_iters, optim_K, optim_P, optim_Z, optim_X, weight_z, n_zcfs, tangent_reg):
        phase_num += 1
        if phase_num > (max_n_phases % 1000):
            break
        dense_depth_use = dense_depth
        if n_zcfs is not None:
            z_coefs = variables['z_coefs']
            optim_Z0 = True
            if rig.depth_mode[:3] == 'log':
                optim_Z0 = (n_zcfs == 2) or (n_zcfs == original_pix2d_dep.shape[1])
                n_zcfs += not optim_Z0
            trk.pix2d_dep = original_pix2d_dep[:, :n_zcfs].contiguous()
            if dense_depth is not None:                       # en:460-464
                assert len(dense_depth) == rig.n_imgs, 'log_depth_maps must be n_imgs x (H, W, C)'
                assert all(d.shape[-1] >= n_zcfs for d in dense_depth), \
                    'not enough dense depth channels for the requested n_zcfs'
                dense_depth_use = [d[..., :n_zcfs] for d in dense_depth]
            if n_zcfs < z_coefs.shape[1]:
                assert n_zcfs >= 1
                variables['z_coefs'] = z_coefs[:, :n_zcfs].contiguous()
            elif n_zcfs > z_coefs.shape[1]:
                assert trk.pix2d_dep.shape[1] == n_zcfs, 'not enough multi-depthmaps in the original data'
                variables['z_coefs'] = torch.cat((z_coefs, z_coefs.new_zeros((len(z_coefs), n_zcfs - z_coefs.shape[1]))),
                                                 dim=1).contiguous()
        if verbose:
            print(f"Starting phase {phase_num}, with {variables['z_coefs'].shape[1]} z-coefs.")
        it = 0
        carry = None          # objective at `variables`, from the trial that produced them
        infos = rig.infos(trk)
        while it < max_iters:
            update, status, last_eval = _lm_step(infos, trk.pids, trk.pix2d, trk.pix2d_std, trk.pix2d_dep,
                                                 **variables, log_depth_maps=dense_depth_use, conf=dense_conf,
                                                 pts3d_ref=dense_pts3d_ref, weight_tan=tangent_reg,
                                                 tan_stride=tan_stride,
                                                 normalize_tangents=normalize_tangents,
                                                 optim_K=optim_K, optim_Z=optim_Z, optim_P=optim_P,
                                                 optim_X=optim_X, optim_Z0=optim_Z0, pnorm=pnorm,
                                                 weight_z=weight_z, no_grad_f_from_rz=no_Jfz,
                                                 depth_mode=rig.depth_mode, dampen=1e-12, adaptive_dampen=True,
                                                 dtype=torch.float64, init_eval=carry, **other_lm_kwargs)
            if verbose:
                reproj_before = float(reproj_score(status.init_residuals))
                reproj_after = float(reproj_score(status.new_residuals))
                avg_focal = float((update['K'][:, 0, 0].mean() + update['K'][:, 1, 1].mean()) / 2)
                print(f"Loss at iter={it}: {float(status.init_loss):.3f} --> {float(status.new_loss):.3f}, "
                      f"reproj_score: {reproj_before:.3f} --> reproj_after={reproj_after:.3f}, avg_focal={avg_focal:.2f}")
            if status.new_loss >= status.init_loss:
                break
            variables.update(update)
            # the next step starts where this trial ended: reuse its objective (en:281 would recompute
            # it from the same parameters).  The tangent prior term depends on the step's K, so with
            # the prior on the start-of-step objective is evaluated afresh.
            carry = last_eval if not tangent_reg > 0 else None
            it += 1
    trk.pix2d_dep = original_pix2d_dep
    pts3d = variables.pop('pts3d')
    return rigs_data.update(**variables), pts3d
