"""MI355X ``GaussNewtonSolver``: drop-in for src/blast3r/inference/ba_solver.py:20-248 (``bs``).

Same constructor, same ``compute_jacobians`` / ``solve_delta`` /
``unpack_delta_inplace`` signatures, same unknown order
[foc (n_cams x 2) | tau (n_nodes x 6) | zcf (n_imgs x C) | pts (n_tracks x 3)]
(bs:119, bs:229), same fp32 delta (bs:182).  What changes is how the step is
computed: ``compute_jacobians`` returns a light handle instead of materialised
fp64 Jacobian blocks, and ``solve_delta`` runs the fused HIP path

    ba_linearize_schur   J, J^T W r, H_pp, camera-pair blocks of S, rhs (fp64, on chip)
    ba_pcg_solve         the reference's Jacobi-PCG (bs:184-206, :1197-1238) on the explicit S
    ba_backsubstitute    delta_p = H_pp^-1 (g_p - H_pc delta_c)

with no host synchronisation between them.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import PCG_BLOCK, PCG_LONG_LIST, BaLinArgs, BaPcgArgs, check, lib, ptr, stream_ptr
from .plan import MAX_LOCAL, get_plan

N_FOC = 2   # focal columns (bs:11)
N_TAU = 6   # pose columns (bs:12)


class Param:
    """bs:15-18."""
    def __init__(self, n):
        self.n = self.true_n = n
        self.true_idxs = None


class Linearization:
    """What ``compute_jacobians`` hands to ``solve_delta``: the inputs of the fused kernels.

    ``shape`` is the shape the reference's J would have (bs:119), so callers that
    assert on it keep working.
    """
    def __init__(self, solver, **kw):
        self.__dict__.update(kw)
        self.solver = solver

    @property
    def shape(self):
        s = self.solver
        return (3 * s.n_kpts, s.cams.n * N_FOC + s.nodes.n * N_TAU + s.imgs.n * s.n_zcf + s.tracks.n * 3)

    def with_z_by_prior(self):
        """This linearisation with the z-coefficient columns of every image in the reduced system and
        their Jacobian entries zero: the switched-off z block (a ZerosMat) that a tangent prior turns
        into its H_z (bs:163-164), so that z moves under the prior alone."""
        kw = dict(self.__dict__)
        solver = kw.pop('solver')
        en = dict(kw['en'])
        en['Z'] = (True, torch.zeros(solver.imgs.true_n, dtype=torch.uint8, device=self.pids.device), None)
        kw['en'] = en
        return Linearization(solver, **kw)


def _flag(status, name, count, device):
    """Normalise an optim_* flag: returns (enabled_group, uint8 mask or None, kept indices or None).

    A mask tensor must live on the solver's device: the kernels read it there.  The reference
    indexes the mask with the device's per-observation ids (bs:98), which raises RuntimeError for a
    host mask unless every entry is False (then it returns the zero matrix first, bs:91-92)."""
    if status is True:
        return True, None, None
    if status is False:
        return False, None, None
    if isinstance(status, torch.Tensor):
        if status.dtype != torch.bool or status.shape != (count,):
            raise ValueError(f'bad {name}={status}')
        idxs = status.nonzero().squeeze(-1)
        if len(idxs) == 0:
            return False, None, None     # all columns removed -> zero matrix (bs:91-92)
        if status.device != device:
            raise RuntimeError(f'{name}: indices should be either on cpu or on the same device as the indexed '
                               f'tensor (mask on {status.device}, observations on {device})')
        return True, status.to(torch.uint8).contiguous(), idxs
    raise ValueError(f'bad {name}={status}')


PCG_CHUNK = 25          # PCG iterations per graph when the host stops launching after the loop stops


class GaussNewtonSolver:
    """Bundle-adjustment Gauss-Newton step on MI355X (bs:20-248)."""

    def __init__(self, n_cams, n_nodes, n_imgs, n_tracks, device, no_grad_f_from_rz=False, dampen=1e-12,
                 adaptive_dampen=True, dtype=torch.float32, solver='pcg', pcg_tol=1e-6, pcg_maxiter=300,
                 plan_options=None, use_graph=True, cholesky_layout='auto', path='auto'):
        self.cams = Param(n_cams)
        self.nodes = Param(n_nodes)
        self.imgs = Param(n_imgs)
        self.tracks = Param(n_tracks)
        self.device = torch.device(device)
        # dtype is the precision of the linearisation's products and sums, the reduced system, the PCG and
        # the back-substitution, as in the reference (bs:22, :37, :128): torch.float64 (bundle_adjustment's
        # choice, en:490) or torch.float32 (its default), on either path: every kernel has a fp32 variant
        # (the Jacobian core is evaluated in fp64 and rounded to fp32)
        if dtype not in (torch.float32, torch.float64):
            raise ValueError(f'dtype must be torch.float32 or torch.float64, not {dtype}')
        self.dtype = dtype
        self.real32 = dtype == torch.float32
        self.dampen = dampen
        self.adaptive_dampen = adaptive_dampen
        self.no_grad_f_from_rz = no_grad_f_from_rz
        if solver not in ('pcg', 'cholesky'):
            raise ValueError(f'unknown reduced solver {solver!r} (supported: "pcg", "cholesky")')
        if solver == 'cholesky' and self.real32:
            raise ValueError("solver='cholesky' factors the reduced system in fp64: pass dtype=torch.float64")
        self.solver = solver
        # solver='cholesky': 'banded' when every image pair lies within w images and few unknowns are shared
        # by several images: block cyclic reduction over super-blocks of 128 unknowns when w d <= 128 and
        # at most 15 are shared, else one workgroup walking the images when its window of w + 1 images
        # fits LDS ((w + 1) d <= 160) and at most 8 are shared; 'banded_sequential' forces the
        # one-workgroup walk; 'dense' any structure ('auto' picks banded where it applies)
        if cholesky_layout not in ('auto', 'dense', 'banded', 'banded_sequential'):
            raise ValueError(f'unknown cholesky_layout {cholesky_layout!r}')
        self.cholesky_layout = cholesky_layout
        self.pcg_tol = pcg_tol
        self.pcg_maxiter = pcg_maxiter
        self.plan_options = dict(plan_options or {})
        # linearize + Schur: 'batched' (chunk batches, d <= 15, tracks within 13 images and 128
        # observations, fastest on banded structures), 'pairmajor' (any track length, d <= 31, any
        # co-visibility), 'auto' (batched where it applies and pays, else pair-major); an explicit
        # 'batched' outside its limits raises instead of switching paths
        if path not in ('auto', 'batched', 'pairmajor'):
            raise ValueError(f'unknown path {path!r}')
        self.path = path
        self.use_graph = bool(use_graph)        # replay the PCG launches from a captured graph
        self.last = {}

    # ------------------------------------------------------------------ bs:34-40
    def compute_jacobians(self, rigs, K, P_rig2cam, P_w2rig, z_coefs, pts3d, pids, pix2d_std, pix2d_dep, is_depth_log,
                          optim_Z_1st_cam=True, optim_Z0=True, optim_K=True, optim_Z=True, optim_P=True, optim_X=True,
                          pix2d=None, hp=None):
        assert rigs.shape == (3, self.imgs.n)
        self.n_kpts = int(pids.shape[0])
        self.n_zcf = int(z_coefs.shape[1])
        assert pix2d_dep.shape == (self.n_kpts, self.n_zcf)
        en = {}
        dev = pids.device
        en['K'] = _flag(optim_K, 'optim_K', self.cams.n, dev)
        en['P'] = _flag(optim_P, 'optim_P', self.nodes.n, dev)
        en['Z'] = _flag(optim_Z, 'optim_Z', self.imgs.n, dev)
        en['X'] = _flag(optim_X, 'optim_X', self.tracks.n, dev)
        for key, par in (('K', self.cams), ('P', self.nodes), ('Z', self.imgs), ('X', self.tracks)):
            if en[key][2] is not None:              # column compaction (bs:86-104)
                par.n = len(en[key][2])
                par.true_idxs = en[key][2]
        return Linearization(self, rigs=rigs, K=K, P_rig2cam=P_rig2cam, P_w2rig=P_w2rig, z_coefs=z_coefs,
                             pts3d=pts3d, pids=pids, pix2d_std=pix2d_std, pix2d_dep=pix2d_dep, pix2d=pix2d,
                             is_depth_log=bool(is_depth_log), optim_Z_1st_cam=bool(optim_Z_1st_cam),
                             optim_Z0=bool(optim_Z0), en=en, hp=hp)

    # ------------------------------------------------------------------ unknown maps
    def _unknown_maps(self, J, lay, plan):
        """Image-level parameter -> unknown index (-1 inactive), its inverse CSR and leaf ids.

        Unknowns follow the reference order [foc | tau | zcf] over the compacted
        entities; groups whose optim flag is False keep their (decoupled) unknowns,
        like the reference's ZerosMat leaves (bs:510-517).
        """
        d, C = lay['d'], self.n_zcf
        n_imgs = self.imgs.true_n
        # masks are keyed by content: a new mask tensor may reuse a freed one's address and version
        host_idx = {k: (None if J.en[k][2] is None else J.en[k][2].cpu().numpy().astype(np.int64))
                    for k in ('K', 'P', 'Z')}
        ident = lambda a: None if a is None else (len(a), a.tobytes())
        key = (d, C, lay['hasK'], lay['hasP'], lay['hasZ'], self.cams.n, self.nodes.n, self.imgs.n, n_imgs,
               ident(host_idx['K']), ident(host_idx['P']), ident(host_idx['Z']))
        cache = plan.__dict__.setdefault('_umaps', {})
        if key in cache:
            return cache[key]
        if len(cache) > 8:
            cache.clear()
        cam_ids, node_ids = plan.cam_ids, plan.node_ids

        def compact(key, par):
            m = np.arange(par.true_n)
            if host_idx[key] is not None:
                keep = np.full(par.true_n, -1, dtype=np.int64)
                idx = host_idx[key]
                keep[idx] = np.arange(len(idx))
                m = keep
            return m

        cam_map, node_map, img_map = compact('K', self.cams), compact('P', self.nodes), compact('Z', self.imgs)
        nf, nt, nz = self.cams.n * N_FOC, self.nodes.n * N_TAU, self.imgs.n * C
        umap = np.full((n_imgs, max(d, 1)), -1, dtype=np.int64)
        col = 0
        if lay['hasK']:
            c = cam_map[cam_ids]
            for k in range(2):
                umap[:, col + k] = np.where(c >= 0, c * 2 + k, -1)
            col += 2
        if lay['hasP']:
            n = node_map[node_ids]
            for k in range(6):
                umap[:, col + k] = np.where(n >= 0, nf + n * 6 + k, -1)
            col += 6
        if lay['hasZ']:
            im = img_map[np.arange(n_imgs)]
            for k in range(C):
                umap[:, col + k] = np.where(im >= 0, nf + nt + im * C + k, -1)
            col += C
        n_u = nf + nt + nz
        flat = umap.reshape(-1)
        valid = np.nonzero(flat >= 0)[0]
        order = np.argsort(flat[valid], kind='stable')
        src = valid[order]
        counts = np.bincount(flat[valid], minlength=n_u) if n_u else np.zeros(0, np.int64)
        inv_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        leaf = np.zeros(n_u, dtype=np.int32)
        leaf[nf:nf + nt] = 1
        leaf[nf + nt:] = 2
        # a group switched off entirely is a zero leaf damped by dampen * I (non-adaptive)
        if not lay['hasK']:
            leaf[:nf] += 3
        if not lay['hasP']:
            leaf[nf:nf + nt] += 3
        if not lay['hasZ']:
            leaf[nf + nt:] += 3
        dev = self.device
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.int32)).to(dev)
        long_u = np.nonzero(counts > PCG_LONG_LIST)[0]
        nblk = (n_u + PCG_BLOCK - 1) // PCG_BLOCK
        long_ptr = np.searchsorted(long_u, np.arange(nblk + 1) * PCG_BLOCK).astype(np.int32)
        long_idx = np.full(max(n_u, 1), -1, dtype=np.int32)
        long_idx[long_u] = np.arange(len(long_u)) - long_ptr[long_u // PCG_BLOCK]
        src1 = np.full(max(n_u, 1), -1, dtype=np.int64)         # lists resolved ahead (one load fewer)
        one = np.nonzero(counts == 1)[0]
        src1[one] = src[inv_ptr[one]]
        long_rng = np.stack([inv_ptr[long_u], inv_ptr[long_u + 1]], 1).reshape(-1) if len(long_u) else np.zeros(2)
        kind = np.where(counts == 0, 0, np.where(counts == 1, 1, 2)) if n_u else np.zeros(1)
        shared_u = np.nonzero(counts >= 2)[0] if n_u else np.zeros(0)
        out = dict(n_u=n_u, umap=t(umap), inv_ptr=t(inv_ptr), inv_src=t(src if len(src) else np.zeros(1)),
                   kind=t(kind), shared_u=t(shared_u if len(shared_u) else np.zeros(1)), n_shared=len(shared_u),
                   leaf=t(leaf if n_u else np.zeros(1)), long_u=t(long_u if len(long_u) else np.zeros(1)),
                   n_long=len(long_u), long_ptr=t(long_ptr), long_idx=t(long_idx), src1=t(src1),
                   long_rng=t(long_rng))
        cache[key] = out
        return out

    # ------------------------------------------------------------------ bs:110-182
    def solve_delta(self, J, residuals, w_pts, clamp_w=(1e-6, 1e6), z_prior=None):
        """Solve (J^T W J + damping) delta = J^T W r by Schur reduction; returns fp32 delta."""
        if z_prior is not None and z_prior[0] is not None and z_prior[1] is not None and not J.en['Z'][0]:
            J = J.with_z_by_prior()
        ctx = self.prepare(J, residuals, w_pts, clamp_w)
        st = ctx['stream']
        if ctx['lay']['d'] > 0:
            if ctx['path'] == 'pairmajor':
                check(lib().ba_pm_linearize_schur(ctx['args'], st))
            else:
                check(lib().ba_linearize_schur(ctx['args'], st))
        else:
            ctx['S_pairs'].zero_(); ctx['e_img'].zero_(); ctx['dg_img'].zero_()
        if z_prior is not None:
            self._add_z_prior(z_prior, ctx['lay'], ctx['plan'], ctx['S_pairs'], ctx['e_img'], ctx['dg_img'])
        return self.reduce_and_backsubstitute(J, ctx)

    def prepare(self, J, residuals, w_pts, clamp_w=(1e-6, 1e6)):
        """Plan, workspaces and the ba_lin_args of one linearisation (no kernel launched)."""
        assert isinstance(J, Linearization)
        assert J.shape == (3 * self.n_kpts, self.cams.n * N_FOC + self.nodes.n * N_TAU + self.imgs.n * self.n_zcf +
                           self.tracks.n * 3)
        assert residuals.shape == (self.n_kpts, 3)
        assert w_pts.shape in ((self.n_kpts, 1), (self.n_kpts, 3))
        dev = self.device
        C = self.n_zcf
        en = J.en
        hasK, hasP, hasZ = en['K'][0], en['P'][0], en['Z'][0]
        d = 2 * hasK + 6 * hasP + C * hasZ
        lay = dict(d=d, hasK=hasK, hasP=hasP, hasZ=hasZ)
        plan = None
        if self.path == 'batched' and d > 15:
            raise ValueError(f"path='batched' takes at most 15 reduced parameters per image (here {d}); "
                             "use path='pairmajor' or 'auto'")
        if self.path == 'pairmajor' or d > 15:
            return self._prepare_pm(J, residuals, w_pts, clamp_w, lay)
        L_img = int(self.plan_options.get('max_local_imgs', MAX_LOCAL))
        if self.path == 'auto' and get_plan(J.rigs, J.pids, self.tracks.true_n, kind='span').median_span > 2 * L_img:
            # tracks on far-apart images (random co-visibility): batches would hardly share image pairs, which
            # the rule below finds only after building the batched plan (seconds at 20M observations)
            return self._prepare_pm(J, residuals, w_pts, clamp_w, lay)
        try:
            plan = get_plan(J.rigs, J.pids, self.tracks.true_n, device=dev, **self.plan_options)
        except RuntimeError as e:
            # the batched planner's limits (a track longer than a chunk or spanning more images than a
            # batch holds): the pair-major path has none
            if self.path == 'batched' or 'track' not in str(e):
                raise
            return self._prepare_pm(J, residuals, w_pts, clamp_w, lay)
        sc = plan.scalars
        if self.path == 'auto' and sc['n_chunks'] >= 256 and sc['n_batches'] * 2 > sc['n_chunks']:
            # batches that hardly share image pairs (random co-visibility): every chunk would write its
            # own partial blocks; the pair-major path writes each pair block once
            return self._prepare_pm(J, residuals, w_pts, clamp_w, lay)
        T = self.tracks.true_n
        s_pix, s_std, s_dep = plan.slot_data(J.pix2d if J.pix2d is not None else J.pix2d_std, J.pix2d_std,
                                             J.pix2d_dep)
        ws = plan.workspace
        n_imgs = self.imgs.true_n
        n_ct = sc['n_ctracks']
        R = self.dtype                         # the working precision of every array below but ct_pt
        Hpp = ws('Hpp', (max(n_ct, 1), 6), R)  # chunk-track order
        gp = ws('gp', (max(n_ct, 1), 3), R)
        ct_pt = ws('ct_pt', (max(n_ct, 1), 4), torch.float32)
        pfac = ws('pfac', (max(n_ct, 1), 12), R)
        work_ctr = ws('work_ctr', (1,), torch.int32)
        # linearisation records: the Jacobian core, 20 fp64 fields per slot; the fp32 solver's rounded to
        # fp32, 24 fields (22 used)
        if self.real32:
            core = ws('core', (max(sc['n_chunks'], 1), 24, sc['chunk']), torch.float32)
        else:
            core = ws('core', (max(sc['n_chunks'], 1), 20, sc['chunk']), torch.float64)
        chunk_max = ws('chunk_max', (sc['n_chunks'] + 1,), R)
        lam_p = ws('lam_p', (1,), R)
        dd = max(d, 1)
        partials = ws('partials', (max(sc['n_slots'], 1), dd, dd), R)
        img_partials = ws('img_partials', (max(sc['n_batches'], 1), plan.L, 2, dd), R)
        # outputs live in the plan's workspace: fixed addresses across LM steps (graph replay)
        S_pairs = ws('S_pairs', (max(sc['n_pairs'], 1), dd, dd), R)
        e_img = ws('e_img', (n_imgs, dd), R)
        dg_img = ws('dg_img', (n_imgs, dd), R)

        a = BaLinArgs()
        pd = plan.dev
        a.real32 = int(self.real32)
        a.infos = ptr(J.rigs.contiguous())
        a.n_imgs = n_imgs
        for name in ('chunk_obs', 'chunk_meta', 'slot_info', 'ct_pid', 'ct_first', 'ct_m', 'ct_mask', 'b_chunk_ptr',
                     'b_imgs', 'b_nimgs', 'b_slot_ptr', 'slot_pair', 'pair_ptr', 'pair_src', 'img_ptr', 'img_src',
                     'chunk_slots', 'chunk_ent', 'chunk_eptr', 'b_pos_slot', 'b_order'):
            setattr(a, name, ptr(pd[name]))
        a.L = plan.L
        a.s_pix, a.s_std, a.s_dep = ptr(s_pix), ptr(s_std), ptr(s_dep)
        a.s_pid, a.s_img = ptr(pd['s_pid']), ptr(pd['s_img'])
        a.K, a.P_rig2cam, a.P_rig2cam_stride = ptr(J.K), ptr(J.P_rig2cam), J.P_rig2cam.stride(0)
        a.P_w2rig, a.z_coefs, a.pts3d = ptr(J.P_w2rig), ptr(J.z_coefs), ptr(J.pts3d)
        a.enK, a.enP, a.enZ, a.enX = (ptr(en[k][1]) for k in ('K', 'P', 'Z', 'X'))
        hp = J.hp or {}
        a.hp.weight_z = float(hp.get('weight_z', 1.0))
        a.hp.pnorm = float(hp.get('pnorm', 1.0))
        a.hp.max_pix_err = float(hp.get('max_pix_err', 100.0))
        a.hp.huber_delta = float(hp.get('huber_delta', 0.5))
        a.hp.w_pts_null = float(hp.get('w_pts_null', 1e-16))
        a.hp.is_depth_log = int(J.is_depth_log)
        L_ = a.lay
        L_.d, L_.C = d, C
        L_.off_tau, L_.off_zcf = 2 * hasK, 2 * hasK + 6 * hasP
        L_.hasK, L_.hasP, L_.hasZ = int(hasK), int(hasP), int(hasZ)
        L_.no_grad_f_from_rz = int(bool(self.no_grad_f_from_rz))
        L_.optim_Z0, L_.optim_Z_1st_cam = int(J.optim_Z0), int(J.optim_Z_1st_cam)
        L_.wmin, L_.wmax = float(clamp_w[0]), float(clamp_w[1])
        L_.dampen = float(self.dampen)
        L_.adaptive = int(bool(self.adaptive_dampen))
        L_.x_off = int(not en['X'][0])
        a.Hpp, a.gp, a.chunk_max, a.lam_p = ptr(Hpp), ptr(gp), ptr(chunk_max), ptr(lam_p)
        a.ct_pt, a.n_ctracks, a.core, a.pfac = ptr(ct_pt), n_ct, ptr(core), ptr(pfac)
        a.work_ctr = ptr(work_ctr)
        a.partials, a.img_partials = ptr(partials), ptr(img_partials)
        a.n_chunks, a.n_batches, a.n_pairs = sc['n_chunks'], sc['n_batches'], sc['n_pairs']
        a.S_pairs, a.e_img, a.dg_img = ptr(S_pairs), ptr(e_img), ptr(dg_img)
        # residuals / weights: recompute in-kernel when they are this step's own objective output,
        # otherwise read the caller's tensors (bs:123-128 semantics)
        W = w_pts.expand(-1, 3)
        own = getattr(residuals, '_ba_state', None)
        if own is None or own != _param_state(J) or J.pix2d is None:
            a.r_in, a.w_in = ptr(residuals), ptr(W)
            a.r_s0, a.r_s1 = residuals.stride(0), residuals.stride(1)
            a.w_s0, a.w_s1 = W.stride(0), W.stride(1)
        return dict(args=a, stream=stream_ptr(dev), lay=lay, plan=plan, S_pairs=S_pairs, e_img=e_img, dg_img=dg_img,
                    Hpp=Hpp, gp=gp, lam_p=lam_p, keep=(s_pix, s_std, s_dep, W, residuals), path='batched')

    def _layout_args(self, L_, J, lay, clamp_w):
        C = self.n_zcf
        en = J.en
        L_.d, L_.C = lay['d'], C
        L_.off_tau, L_.off_zcf = 2 * lay['hasK'], 2 * lay['hasK'] + 6 * lay['hasP']
        L_.hasK, L_.hasP, L_.hasZ = int(lay['hasK']), int(lay['hasP']), int(lay['hasZ'])
        L_.no_grad_f_from_rz = int(bool(self.no_grad_f_from_rz))
        L_.optim_Z0, L_.optim_Z_1st_cam = int(J.optim_Z0), int(J.optim_Z_1st_cam)
        L_.wmin, L_.wmax = float(clamp_w[0]), float(clamp_w[1])
        L_.dampen = float(self.dampen)
        L_.adaptive = int(bool(self.adaptive_dampen))
        L_.x_off = int(not en['X'][0])

    @staticmethod
    def _huber_args(h, J):
        hp = J.hp or {}
        h.weight_z = float(hp.get('weight_z', 1.0))
        h.pnorm = float(hp.get('pnorm', 1.0))
        h.max_pix_err = float(hp.get('max_pix_err', 100.0))
        h.huber_delta = float(hp.get('huber_delta', 0.5))
        h.w_pts_null = float(hp.get('w_pts_null', 1e-16))
        h.is_depth_log = int(J.is_depth_log)

    def _prepare_pm(self, J, residuals, w_pts, clamp_w, lay):
        """Plan, workspaces and the ba_pm_args of one pair-major linearisation (no kernel launched)."""
        dev = self.device
        d = lay['d']
        if d > 31:
            raise ValueError(f'{d} image-level parameters: the pair-major path supports at most 31')
        plan = get_plan(J.rigs, J.pids, self.tracks.true_n, kind='pairmajor', device=dev)
        sc, pd, ws = plan.scalars, plan.dev, plan.workspace
        T = self.tracks.true_n
        n_imgs = self.imgs.true_n
        n_obs = int(J.pids.shape[0])
        dp = 16 if d <= 15 else 32
        dd = max(d, 1)
        a = _lib.BaPmArgs()
        a.infos = ptr(J.rigs.contiguous())
        a.n_imgs, a.n_tracks = n_imgs, T
        for name in ('run_ptr', 'run_obs', 'run_trk', 'run_img', 'img_run_ptr', 'trk_run_ptr', 'trk_run',
                     'trk_obs_ptr', 'trk_obs', 'obs_img', 'pair_i1', 'pair_i2', 'diag_pair', 'term_ptr', 'term',
                     'pair_sched'):
            setattr(a, name, ptr(pd[name]))
        a.n_obs, a.n_runs, a.n_pairs = n_obs, sc['n_runs'], sc['n_pairs']
        pix = J.pix2d if J.pix2d is not None else J.pix2d_std
        a.pids, a.pix2d, a.pix2d_std, a.pix2d_dep = ptr(J.pids), ptr(pix), ptr(J.pix2d_std), ptr(J.pix2d_dep)
        a.K, a.P_rig2cam, a.P_rig2cam_stride = ptr(J.K), ptr(J.P_rig2cam), J.P_rig2cam.stride(0)
        a.P_w2rig, a.z_coefs, a.pts3d = ptr(J.P_w2rig), ptr(J.z_coefs), ptr(J.pts3d)
        en = J.en
        a.enK, a.enP, a.enZ, a.enX = (ptr(en[k][1]) for k in ('K', 'P', 'Z', 'X'))
        self._huber_args(a.hp, J)
        self._layout_args(a.lay, J, lay, clamp_w)
        R = self.dtype                         # the working precision of every array below but wobs
        a.real32 = int(self.real32)
        Hpp = ws('Hpp', (max(T, 1), 6), R)
        gp = ws('gp', (max(T, 1), 3), R)
        lam_p = ws('lam_p', (1,), R)
        S_pairs = ws('S_pairs', (max(sc['n_pairs'], 1), dd, dd), R)
        e_img = ws('e_img', (n_imgs, dd), R)
        dg_img = ws('dg_img', (n_imgs, dd), R)
        a.pobs = ptr(ws('pobs', (max(n_obs, 1), 9), R))
        a.wobs = ptr(ws('wobs', (max(n_obs, 1), 4), torch.float32))
        nsl = lambda n: int(lib().ba_pm_slot_doubles(n, n_imgs, d))
        a.jslots = ptr(ws('jslots', (max(nsl(n_obs), 1),), R))
        a.vslots = ptr(ws('vslots', (max(nsl(sc['n_runs']), 1),), R))
        a.Hpp, a.gp, a.lam_p = ptr(Hpp), ptr(gp), ptr(lam_p)
        a.tmax = ptr(ws('tmax', ((T + 255) // 256 + 1,), R))
        a.pfac = ptr(ws('pfac', (max(T, 1), 16), R))     # the pair-major factor record, point included
        a.V = ptr(ws('V', (max(sc['n_runs'], 1), 3, dp), R))
        a.S_pairs, a.e_img, a.dg_img = ptr(S_pairs), ptr(e_img), ptr(dg_img)
        W = w_pts.expand(-1, 3)
        own = getattr(residuals, '_ba_state', None)
        if own is None or own != _param_state(J) or J.pix2d is None:
            a.r_in, a.w_in = ptr(residuals), ptr(W)
            a.r_s0, a.r_s1 = residuals.stride(0), residuals.stride(1)
            a.w_s0, a.w_s1 = W.stride(0), W.stride(1)
        return dict(args=a, stream=stream_ptr(dev), lay=lay, plan=plan, S_pairs=S_pairs, e_img=e_img, dg_img=dg_img,
                    Hpp=Hpp, gp=gp, lam_p=lam_p, keep=(W, residuals), path='pairmajor')

    def reduce_and_backsubstitute(self, J, ctx):
        """Device PCG on the reduced system and point back-substitution; returns fp32 delta."""
        a, st, lay, plan = ctx['args'], ctx['stream'], ctx['lay'], ctx['plan']
        S_pairs, e_img, dg_img = ctx['S_pairs'], ctx['e_img'], ctx['dg_img']
        Hpp, gp, lam_p = ctx['Hpp'], ctx['gp'], ctx['lam_p']
        dev, d, sc, pd, ws = self.device, lay['d'], plan.scalars, plan.dev, plan.workspace
        en = J.en
        T = self.tracks.true_n
        n_imgs = self.imgs.true_n
        um = self._unknown_maps(J, lay, plan)
        n_u = um['n_u']
        R = S_pairs.dtype                      # the working precision
        if n_u > 0 and d > 0:
            x = ws('pcg_x', (n_u,), R)
            istate = ws('pcg_istate', (8,), torch.int32)
        else:
            x = torch.zeros(max(n_u, 1), dtype=R, device=dev)
            istate = torch.zeros(8, dtype=torch.int32, device=dev)
        if n_u > 0 and d > 0:
            pa = BaPcgArgs()
            pa.n_u, pa.n_imgs, pa.d = n_u, n_imgs, d
            pa.umap, pa.inv_ptr, pa.inv_src, pa.leaf = ptr(um['umap']), ptr(um['inv_ptr']), ptr(um['inv_src']), ptr(
                um['leaf'])
            pa.row_ptr, pa.row_ent = ptr(pd['row_ptr']), ptr(pd['row_ent'])
            pa.pair_i1, pa.pair_i2 = ptr(pd['pair_i1']), ptr(pd['pair_i2'])
            pa.S_pairs, pa.e_img, pa.dg_img = ptr(S_pairs), ptr(e_img), ptr(dg_img)
            pa.dampen, pa.adaptive = float(self.dampen), int(bool(self.adaptive_dampen))
            pa.maxiter, pa.tol = int(self.pcg_maxiter), float(self.pcg_tol)
            pa.real32 = int(R == torch.float32)
            vec = lambda name: ws('pcg_' + name, (n_u,), R)
            rhs, diagA, damp = vec('rhs'), vec('diagA'), vec('damp')
            xbest, r, z = vec('xbest'), vec('r'), vec('z')
            p = ws('pcg_p2', (2 * n_u,), R)
            y_img = ws('pcg_y', (n_imgs * d,), R)
            part = ws('pcg_part', (int(lib().ba_pcg_partials_size(n_u)),), R)
            state = ws('pcg_state', (16,), R)
            pa.rhs, pa.diagA, pa.damp, pa.x, pa.xbest = ptr(rhs), ptr(diagA), ptr(damp), ptr(x), ptr(xbest)
            pa.r, pa.z, pa.p, pa.y_img = ptr(r), ptr(z), ptr(p), ptr(y_img)
            pa.img_part = ptr(ws('pcg_img_part', (n_imgs,), R))
            pa.partials, pa.state, pa.istate = ptr(part), ptr(state), ptr(istate)
            pa.long_u, pa.n_long = ptr(um['long_u']), um['n_long']
            pa.long_ptr, pa.long_idx = ptr(um['long_ptr']), ptr(um['long_idx'])
            pa.src1, pa.long_rng = ptr(um['src1']), ptr(um['long_rng'])
            self.last['direct'] = None
            direct_info = self._run_direct(pa, plan, st, n_imgs, um) if self.solver == 'cholesky' else None
            if direct_info is None:
                self._pcg_rows(pa, plan, d, n_imgs)
                self._run_pcg(pa, plan, st)
            self.last.update(rhs=rhs, diagA=diagA, damp=damp)
        else:
            direct_info = None
        pm = ctx['path'] == 'pairmajor'
        has_X = en['X'][0] and (sc['n_runs'] > 0 if pm else sc['n_chunks'] > 0)

        def backsubstitute():
            # back-substitution for the points
            dX = torch.zeros((max(T, 1), 3), dtype=torch.float32, device=dev)
            if has_X:
                if 'umap_pad' not in um:               # -1 -> the appended zero, once per structure
                    um['umap_pad'] = torch.where(um['umap'] >= 0, um['umap'], x.numel()).long().view(-1)
                dc_img = torch.nn.functional.pad(x, (0, 1))[um['umap_pad']]
                a.dc_img = ptr(dc_img)                 # delta_c at image level (one load fewer per obs)
                a.dX = ptr(dX)
                a.dX64 = None
                if pm:
                    check(lib().ba_pm_backsubstitute(a, st))
                else:
                    a.dc = ptr(x)
                    a.umap = ptr(um['umap'])
                    check(lib().ba_backsubstitute(a, st))
                ctx['keep_dc'] = dc_img
            return dX

        dX = backsubstitute()
        if direct_info is not None and not self._direct_status(direct_info):
            # a pivot was not positive: the device PCG solves the same system, then the points again
            self._pcg_rows(pa, plan, d, n_imgs)
            self._run_pcg(pa, plan, st)
            dX = backsubstitute()
        self.last.update(S_pairs=S_pairs, e_img=e_img, dg_img=dg_img, unknowns=um, lay=lay, plan=plan, x=x,
                         istate=istate, Hpp=Hpp, gp=gp, lam_p=lam_p, path=ctx['path'])
        dc = x[:n_u].to(torch.float32)
        dXa = dX[:T]
        if en['X'][2] is not None:
            dXa = dXa[en['X'][2]]
        return torch.cat([dc, dXa.reshape(-1)])

    @staticmethod
    def _pcg_rows(pa, plan, d, n_imgs):
        """The PCG's image-row copies of the pair blocks (workspace fields of ba_pcg_args), in the working
        precision pa.real32 names."""
        ws = plan.workspace
        rp = plan.host['row_ptr']
        n_ent = int(rp[-1]) if len(rp) else 0
        # rows at a fixed capacity (the SpMV then needs no row_ptr load) when that pads by <= 25%
        longest = int(np.diff(rp).max()) if len(rp) > 1 else 0
        cap = -(-longest // 8) * 8
        row_cap = cap if 0 < cap and n_imgs * cap <= 1.25 * n_ent else 0
        n_blk = n_imgs * row_cap if row_cap else n_ent
        S_rows = ws('pcg_S_rows', (max(n_blk, 1), d, d), torch.float32 if pa.real32 else torch.float64)
        pa.S_rows, pa.n_row_ent, pa.row_cap = ptr(S_rows), n_ent, row_cap
        gw = 16 if d <= 16 else 32                     # row_u entries per block (the SpMV's lanes per group)
        pa.row_u = ptr(ws('pcg_row_u', (max(n_blk, 1) * gw,), torch.int32))

    def _run_direct(self, pa, plan, st, n_imgs, um):
        """Enqueues ba_reduced_solve (L L^T of the damped reduced system, banded or dense) and returns
        its status word on the device, read by _direct_status once the back-substitution is enqueued too
        (so the host's read does not stall the queue between the two)."""
        L = lib()
        ws = plan.workspace
        d = pa.d
        n_p = plan.scalars['n_pairs']
        pidx = plan.workspace_cache.get('pair_idx')
        if pidx is None:                       # pair id of every image pair (i <= j), once per structure
            i1 = plan.dev['pair_i1'][:n_p].long()
            i2 = plan.dev['pair_i2'][:n_p].long()
            pidx = torch.full((n_imgs * n_imgs,), -1, dtype=torch.int32, device=self.device)
            pidx[i1 * n_imgs + i2] = torch.arange(n_p, dtype=torch.int32, device=self.device)
            plan.workspace_cache['pair_idx'] = pidx
            h1, h2 = plan.host['pair_i1'][:n_p], plan.host['pair_i2'][:n_p]
            plan.workspace_cache['band_w'] = int((h2 - h1).max()) if n_p else 0
        w = max(1, min(plan.workspace_cache['band_w'], max(n_imgs - 1, 0)))
        ns = um['n_shared']
        if 'bcol' not in um:                   # band columns: image-level columns local in some image
            kind = um['kind'].cpu().numpy()
            umh = um['umap'].cpu().numpy()
            loc = (umh >= 0) & (kind[np.clip(umh, 0, None)] == 1)
            bcol = np.nonzero(loc.any(0))[0]
            bpos = np.full(d, -1, dtype=np.int64)
            bpos[bcol] = np.arange(len(bcol))
            um['bcol'] = torch.as_tensor(bcol if len(bcol) else np.zeros(1), dtype=torch.int32, device=self.device)
            um['bpos'] = torch.as_tensor(bpos, dtype=torch.int32, device=self.device)
            um['db'] = len(bcol)
        db = um['db']
        layout = self.cholesky_layout
        seq_fits = 1 <= db <= 16 and n_imgs >= 2 and (w + 1) * db <= 160 and ns <= 8 and \
            int(L.ba_chol_band_lds_bytes(db, w, ns)) <= 160 * 1024
        nsb = int(L.ba_chol_band_superblocks(db, w, ns, n_imgs)) if db >= 1 and n_imgs >= 2 else 0
        if layout == 'auto':
            layout = 'banded' if nsb > 0 or seq_fits else 'dense'
        mode = {'dense': 0, 'banded': 1, 'banded_sequential': 2}[layout]
        if mode == 2:
            nsb = 0
        lda = int(L.ba_chol_dense_lda(pa.n_u))
        nwork = int(L.ba_chol_work_doubles(mode, pa.n_u, n_imgs, db if mode else d, w, ns))
        info = ws('chol_info', (1,), torch.int32)
        ca = _lib.BaCholArgs(mode=mode, lda=lda, pair_idx=ptr(pidx), kind=ptr(um['kind']),
                             shared_u=ptr(um['shared_u']), n_shared=ns, w=w, db=db, bcol=ptr(um['bcol']),
                             bpos=ptr(um['bpos']), n_pairs=n_p, info=ptr(info),
                             work=ptr(ws('chol_work', (nwork,), torch.float64)))
        self.last['direct_A'] = None
        if mode == 0:
            self.last['direct_A'] = ws('chol_A', (lda, lda), torch.float64)   # S_u's lower triangle, then L
            ca.A = ptr(self.last['direct_A'])
            ca.Linv = ptr(ws('chol_Linv', (lda // 128, 128, 128), torch.float64))
        check(L.ba_reduced_solve(pa, ca, st))
        self.last['direct_call'] = (pa, ca)    # kept for re-timing the bare launch sequence
        self.last['direct'] = dict(layout=layout, w=w, db=db, n_shared=ns, superblocks=nsb if mode == 1 else 0,
                                   first_bad_pivot=None)
        return info

    def _direct_status(self, info):
        """The direct solve's status (one read per solve): True when every pivot was positive; else
        records the first bad pivot in last['direct'] and returns False (the caller then runs the PCG)."""
        bad = int(info.cpu())
        if bad != 2 ** 31 - 1:
            self.last['direct']['first_bad_pivot'] = bad
        return bad == 2 ** 31 - 1

    def _run_pcg(self, pa, plan, st):
        """ba_pcg_solve, replayed from HIP graphs captured once per argument set and kept with the plan.  The
        iterations go in chunks of PCG_CHUNK, one graph each, whose last kernel stores the loop's stopped flag
        to pinned host memory; the host reads chunk k's flag (after chunk k's event) while chunk k + 1 runs,
        and once the loop has stopped launches only the final decisions and the result (the reference checks
        its stopping rule after every iteration, bs:1216-1236).  The kernels skipped would have returned at
        once, so the result is the one of the whole sequence.  Where the loop ran to its cap the last time
        on this argument set, the whole sequence is replayed from one graph instead (chunks are tried again
        every eighth solve); so it is without a device-reachable flag, and launched directly with use_graph
        off."""
        L = lib()
        self.last['pcg_launched'] = int(pa.maxiter)    # iterations launched (those after a stop return at once)
        if not self.use_graph:
            check(L.ba_pcg_solve(pa, st))
            return
        graphs = plan.__dict__.setdefault('_pcg_graphs', {})
        key = bytes(pa)
        ent = graphs.get(key)
        if ent is None:
            if len(graphs) > 4:
                graphs.clear()
            ent = self._capture_pcg(pa)
            graphs[key] = ent
        ent['solves'] += 1
        if ent['chunks'] is None or not (ent['early'] or ent['solves'] % 8 == 1):
            # the loop ran to its cap on this argument set last time: the whole sequence, one graph (chunks
            # cost a graph launch and a flag store each); chunks are tried again every eighth solve
            ent['whole'].replay()
            return
        flags, bounds, chunks, fin = ent['flags'], ent['bounds'], ent['chunks'], ent['fin']
        events = []
        end = bounds[-1]
        for k, g in enumerate(chunks):
            g.replay()
            ev = torch.cuda.Event()
            ev.record()
            events.append(ev)
            if k >= 1:                                 # chunk k runs while chunk k - 1's flag is read
                events[k - 1].synchronize()
                if int(flags[k - 1]):                  # stopped before update bounds[k]: chunk k returns at once
                    end = bounds[k + 1]
                    break
        fin[end].replay()
        self.last['pcg_launched'] = end
        ent['early'] = end < bounds[-1]

    def _capture_pcg(self, pa):
        """The graphs of _run_pcg for one argument set: the whole sequence in one graph, and the iteration
        chunks (each storing its stopped flag) with the final decisions and result after each chunk."""
        L = lib()
        dev = self.device
        maxit = int(pa.maxiter)
        bounds = list(range(0, maxit, PCG_CHUNK)) + [maxit]
        flags = torch.zeros(max(len(bounds) - 1, 1), dtype=torch.int32, pin_memory=True)
        dptr = L.ba_host_mapped_ptr(ctypes.c_void_p(flags.data_ptr())) if maxit > PCG_CHUNK else None
        torch.cuda.synchronize(dev)

        def capture(fn):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                check(fn(stream_ptr(dev)))
            return g
        whole = capture(lambda s: L.ba_pcg_solve(pa, s))
        if not dptr:
            return dict(whole=whole, chunks=None, solves=0, early=False)
        chunks = [capture(lambda s, k=k: L.ba_pcg_solve_range(pa, bounds[k], bounds[k + 1], 0,
                                                               ctypes.c_void_p(dptr + 4 * k), s))
                  for k in range(len(bounds) - 1)]
        fin = {e: capture(lambda s, e=e: L.ba_pcg_solve_range(pa, e, e, 1, None, s)) for e in bounds[1:]}
        return dict(whole=whole, flags=flags, bounds=bounds, chunks=chunks, fin=fin, solves=0, early=False)

    def _add_z_prior(self, z_prior, lay, plan, S_pairs, e_img, dg_img):
        """Tangent-prior terms on the z-coefficient blocks before damping (bs:141-173)."""
        H_z, g_z = z_prior
        if H_z is None or g_z is None:
            return
        assert lay['hasZ'], 'the z unknowns of a prior are in the reduced system (with_z_by_prior)'
        C = self.n_zcf
        o = lay['d'] - C
        R = S_pairs.dtype
        H_z = H_z.to(device=S_pairs.device, dtype=R).contiguous()
        g_z = g_z.to(device=S_pairs.device, dtype=R).contiguous()
        assert g_z.shape == (self.imgs.n, C) and H_z.shape == (self.imgs.n, C, C)
        if len(e_img) != self.imgs.n:          # compacted images: the rows of the optimised ones
            idx = torch.as_tensor(self.imgs.true_idxs, device=S_pairs.device).long()
            gf = torch.zeros((len(e_img), C), dtype=R, device=S_pairs.device)
            Hf = torch.zeros((len(e_img), C, C), dtype=R, device=S_pairs.device)
            gf[idx], Hf[idx] = g_z, H_z
            g_z, H_z = gf, Hf
        diag = plan.workspace_cache.get('diag_pair')
        if diag is None:                       # the (i, i) block of each image, once per structure
            n_imgs = len(e_img)
            i1, i2 = plan.dev['pair_i1'][:plan.scalars['n_pairs']], plan.dev['pair_i2'][:plan.scalars['n_pairs']]
            pid = torch.nonzero(i1 == i2).squeeze(-1)
            diag = torch.full((n_imgs,), -1, dtype=torch.int32, device=S_pairs.device)
            diag[i1[pid].long()] = pid.to(torch.int32)
            if bool((diag < 0).any()):
                raise ValueError('z_prior: an image without observations has no block in the reduced system')
            plan.workspace_cache['diag_pair'] = diag
        check(lib().ba_add_z_prior(ptr(S_pairs), ptr(diag), ptr(e_img), ptr(dg_img), ptr(H_z), ptr(g_z), len(e_img),
                                   lay['d'], C, int(R == torch.float32), stream_ptr(S_pairs.device)))

    # ------------------------------------------------------------------ bs:228-248
    def unpack_delta_inplace(self, delta):
        sizes = [self.cams.n * N_FOC, self.nodes.n * N_TAU, self.imgs.n * self.n_zcf, self.tracks.n * 3]
        cum_sizes = torch.tensor(sizes, dtype=torch.int).cumsum(dim=0)
        assert delta.shape == (cum_sizes[-1],)
        dK, dP, dZ, dX = delta.tensor_split(cum_sizes[:-1])

        def expand(deriv, param, np_):
            deriv = deriv.view(param.n, np_)
            if param.true_idxs is not None:
                deriv2 = deriv.new_zeros((param.true_n, np_))
                deriv2[param.true_idxs] = deriv
                return deriv2
            return deriv

        return (expand(dK, self.cams, N_FOC), expand(dP, self.nodes, N_TAU), expand(dZ, self.imgs, self.n_zcf),
                expand(dX, self.tracks, 3))

    # ------------------------------------------------------------------ inspection helpers
    def point_blocks(self):
        """H_pp upper (n_tracks,6) and g_p (n_tracks,3) of the last solve_delta in track-id order
        (the device keeps them in chunk-track order), as fp64; tracks without observations hold zeros."""
        last = self.last
        plan = last['plan']
        T = self.tracks.true_n
        if last.get('path') == 'pairmajor':         # kept in track order
            return last['Hpp'][:T].to(torch.float64, copy=True), last['gp'][:T].to(torch.float64, copy=True)
        n_ct = plan.scalars['n_ctracks']
        pid = plan.dev['ct_pid'][:n_ct].long()
        H = torch.zeros((T, 6), dtype=torch.float64, device=self.device)
        g = torch.zeros((T, 3), dtype=torch.float64, device=self.device)
        H[pid] = last['Hpp'][:n_ct].to(torch.float64)
        g[pid] = last['gp'][:n_ct].to(torch.float64)
        return H, g

    def reduced_system_dense(self):
        """Dense S (reference unknown order, damped) and rhs of the last solve_delta, as fp64 (for tests)."""
        last = self.last
        um, lay, plan = last['unknowns'], last['lay'], last['plan']
        n_u, d = um['n_u'], lay['d']
        S_img_pairs = last['S_pairs']
        umap = um['umap'].long()
        S = torch.zeros((n_u, n_u), dtype=torch.float64, device=self.device)
        i1 = plan.dev['pair_i1'].long()[:plan.scalars['n_pairs']]
        i2 = plan.dev['pair_i2'].long()[:plan.scalars['n_pairs']]
        for p in range(len(i1)):
            r = umap[i1[p]]
            c = umap[i2[p]]
            blk = S_img_pairs[p].to(torch.float64)
            mr, mc = r >= 0, c >= 0
            sub = blk[mr][:, mc]
            S.index_put_((r[mr][:, None].expand(-1, int(mc.sum())), c[mc][None, :].expand(int(mr.sum()), -1)), sub,
                         accumulate=True)
            if i1[p] != i2[p]:
                S.index_put_((c[mc][:, None].expand(-1, int(mr.sum())), r[mr][None, :].expand(int(mc.sum()), -1)),
                             sub.T, accumulate=True)
        S += torch.diag(last['damp'].to(torch.float64))
        return S, last['rhs'].to(torch.float64)


def _param_state(J):
    """Identity of the parameter tensors a residual evaluation was computed from."""
    return tuple((t.data_ptr(), t._version) for t in (J.K, J.P_w2rig, J.z_coefs, J.pts3d, J.pix2d_dep, J.pids))
