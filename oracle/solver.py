"""Oracle restatement of the reference Gauss-Newton solver (test infrastructure only).

Restates ``GaussNewtonSolver`` (src/blast3r/inference/ba_solver.py, abbreviated
``bs`` below) as torch-CPU code with the same arithmetic and the same block
structure, without the reference's sparse-matrix class hierarchy:

  * unknown order [foc (n_cams x 2) | tau (n_nodes x 6) | zcf (n_imgs x C) | pts (T x 3)]
    (bs:119, bs:229-233);
  * W = clamp(w, 1e-6, 1e6) in fp32, g = (W*r).to(fp64) @ J, J *= sqrt(W) with the
    square root taken in fp32 (bs:123-132);
  * J^T J as a Schur matrix: leaves foc/tau/zcf/pts block-diagonal, cross blocks
    aggregated per unique (row, col) block pair (bs:854-924, bs:1063-1071);
  * per-leaf damping 1e-12 * max|diag(leaf)| (bs:575-582, bs:1188-1191); an all-off
    leaf (optim_*=False, a ZerosMat) becomes 1e-12 * I (bs:510-517);
  * reduced solve by Jacobi-preconditioned CG on S = A - B D^-1 C with
    M^-1 = 1/clamp(diag(A), 1e-12), tol 1e-6, maxiter 300, best-so-far return
    (bs:184-206, bs:1197-1238), or a dense direct solve of the same S;
  * back-substitution delta_p = D^-1 (g_p - C delta_c) and fp32 output (bs:182, bs:203).

Pinning (tests/test_oracle.py): every block against a materialised dense
J (``oracle.dense``): dense J^T W J and J^T W r, the Schur identity (full dense
solve == reduced solve + back-substitution), symmetry and PSD of S, the 7-DoF
similarity gauge in ker S, and converged PCG == direct solve.
"""
import torch

from .kernels import chol3x3_solve, obs_to_img

N_FOC = 2
N_TAU = 6

__all__ = ['Problem', 'NormalEquations', 'build_normal_equations', 'solve_reduced_pcg',
           'solve_reduced_direct', 'pcg', 'dense_schur', 'unpack_delta']


class _Param:
    """Mirrors bs:15-18: active count n, full count true_n, kept indices true_idxs."""
    def __init__(self, n):
        self.n = self.true_n = n
        self.true_idxs = None


class _BlockCOO:
    """Blocks (M, r, c) at block coordinates (rows, cols) of an (n_rows*r, n_cols*c) sub-matrix
    placed at (row_off, col_off) of a bigger matrix."""
    def __init__(self, blocks, rows, cols, row_off, col_off, n_rows, n_cols):
        self.blocks, self.rows, self.cols = blocks, rows.long(), cols.long()
        self.row_off, self.col_off = row_off, col_off
        self.n_rows, self.n_cols = n_rows, n_cols

    def matvec(self, x, out):
        r, c = self.blocks.shape[1:]
        xs = x[self.col_off: self.col_off + self.n_cols * c].view(-1, c)[self.cols]
        contrib = torch.einsum('nij,nj->ni', self.blocks, xs)
        out[self.row_off: self.row_off + self.n_rows * r].view(-1, r).index_add_(0, self.rows, contrib)

    def rmatvec(self, y, out):
        r, c = self.blocks.shape[1:]
        ys = y[self.row_off: self.row_off + self.n_rows * r].view(-1, r)[self.rows]
        contrib = torch.einsum('nij,ni->nj', self.blocks, ys)
        out[self.col_off: self.col_off + self.n_cols * c].view(-1, c).index_add_(0, self.cols, contrib)


def _aggregate(blocks, rows, cols, n_cols):
    """Sum blocks sharing the same (row, col); deterministic order (index_add_ on CPU)."""
    flat = rows.long() * n_cols + cols.long()
    uniq, inv = torch.unique(flat, return_inverse=True)
    out = torch.zeros((len(uniq),) + tuple(blocks.shape[1:]), dtype=blocks.dtype)
    out.index_add_(0, inv, blocks)
    return out, uniq // n_cols, uniq % n_cols


class Problem:
    """Observation structure shared by the oracle functions (from infos and pids)."""
    def __init__(self, infos, pids, n_cams, n_nodes, n_tracks, C):
        self.n_imgs = infos.shape[1]
        self.n_obs = len(pids)
        self.n_cams, self.n_nodes, self.n_tracks, self.C = n_cams, n_nodes, n_tracks, C
        self.img = obs_to_img(infos, self.n_obs)                      # kpt2img (bs:51)
        self.cam = infos[2].long()[self.img]
        self.node = infos[1].long()[self.img]
        self.pid = pids.long()
        self.cam_ids = infos[2].long()
        self.node_ids = infos[1].long()


class NormalEquations:
    """Damped normal equations in the reference's unknown order, split as A | B | D."""
    def __init__(self):
        self.leaves = {}      # name -> (n_active, b, b) blocks (damped)
        self.cross = []       # _BlockCOO inside A (upper part; lower applied as transpose)
        self.B = []           # _BlockCOO with rows in camera space, cols in point space
        self.sizes = {}


def _enable(status, blocks, cols, param, ent_of_obs):
    """Restates ``GaussNewtonSolver.enable`` (bs:72-108) on explicit per-obs blocks.

    Returns (blocks, cols, is_zero).  A bool tensor zeroes the observations of
    disabled entities and compacts the column indices.  For tracks the mask is
    applied per track (the reference indexes a track mask by image id at bs:98,
    which only matters for a tensor optim_X; the oracle uses per-track semantics).
    """
    if status is True:
        return blocks, cols, False
    if status is False:
        return blocks, cols, True
    assert isinstance(status, torch.Tensor) and status.dtype == torch.bool and status.shape == (param.n,)
    idxs = status.nonzero().squeeze(-1)
    if len(idxs) == 0:
        return blocks, cols, True
    new_map = torch.zeros(param.n, dtype=torch.long)
    new_map[idxs] = torch.arange(len(idxs))
    keep = status[ent_of_obs].to(blocks.dtype)
    blocks = blocks * keep.view(-1, *([1] * (blocks.ndim - 1)))
    cols = new_map[cols]
    param.n = len(idxs)
    param.true_idxs = idxs
    return blocks, cols, False


def build_normal_equations(prob, J_cam, J_zcf, J_pts, residuals, w_pts, optim_K=True, optim_P=True,
                           optim_Z=True, optim_X=True, no_grad_f_from_rz=False, clamp_w=(1e-6, 1e6),
                           dampen=1e-12, adaptive_dampen=True, z_prior=None):
    """g = J^T W r and damped J^T W J (bs:42-70, bs:110-177), blocks kept separate.

    z_prior = (H_z, g_z) adds the tangent-prior terms to the z-coefficient blocks and gradient
    before damping (bs:141-173); a switched-off z block becomes H_z (bs:163-164).

    Returns (NormalEquations, g, params) where g is the fp64 gradient in the
    (compacted) unknown order and params the four ``_Param`` counters.
    """
    dt = J_cam.dtype
    N = prob.n_obs
    C = J_zcf.shape[-1]
    cams, nodes, imgs, trks = (_Param(prob.n_cams), _Param(prob.n_nodes), _Param(prob.n_imgs),
                               _Param(prob.n_tracks))
    J_foc = J_cam[:, :, :2].clone()
    J_tau = J_cam[:, :, 2:].clone()
    Jz = J_zcf[:, 0, :].clone()                                   # row 2 only (stride 3, offset 2; bs:55)
    Jp = J_pts.clone()
    if no_grad_f_from_rz:                                          # bs:59-60
        J_foc[:, 2] = 0
    c_foc, c_tau, c_zcf, c_pts = prob.cam.clone(), prob.node.clone(), prob.img.clone(), prob.pid.clone()
    J_foc, c_foc, zf = _enable(optim_K, J_foc, c_foc, cams, prob.cam)
    J_tau, c_tau, zt = _enable(optim_P, J_tau, c_tau, nodes, prob.node)
    Jz, c_zcf, zz = _enable(optim_Z, Jz, c_zcf, imgs, prob.img)
    Jp, c_pts, zp = _enable(optim_X, Jp, c_pts, trks, prob.pid)

    n_f, n_t, n_z, n_p = cams.n * N_FOC, nodes.n * N_TAU, imgs.n * C, trks.n * 3
    off_t, off_z = n_f, n_f + n_t
    n_c = n_f + n_t + n_z

    # gradient (bs:123-129)
    W = w_pts.expand(-1, 3).clamp(min=clamp_w[0], max=clamp_w[1])
    Wr = (W * residuals).to(dt)                                    # (N, 3) fp32 product cast to fp64
    g = torch.zeros(n_c + n_p, dtype=dt)
    if not zf:
        g[:n_f].view(-1, 2).index_add_(0, c_foc, torch.einsum('nki,nk->ni', J_foc, Wr))
    if not zt:
        g[off_t:off_z].view(-1, 6).index_add_(0, c_tau, torch.einsum('nki,nk->ni', J_tau, Wr))
    if not zz:
        g[off_z:n_c].view(-1, C).index_add_(0, c_zcf, Jz * Wr[:, 2:3])
    if z_prior is not None:                                        # bs:150-155
        assert z_prior[1].shape == (imgs.n, C)
        g[off_z:n_c] += z_prior[1].to(dt).reshape(-1)
    if not zp:
        g[n_c:].view(-1, 3).index_add_(0, c_pts, torch.einsum('nki,nk->ni', Jp, Wr))

    # J *= sqrt(W) (bs:132), sqrt in fp32 then promoted
    sW = torch.sqrt(W).to(dt)
    J_foc = J_foc * sW[:, :, None]
    J_tau = J_tau * sW[:, :, None]
    Jz = Jz * sW[:, 2:3]
    Jp = Jp * sW[:, :, None]

    ne = NormalEquations()
    ne.sizes = dict(n_f=n_f, n_t=n_t, n_z=n_z, n_p=n_p, n_c=n_c, C=C)

    def gram_leaf(name, Jb, cols, n_ent, b, is_zero, extra=None):
        if is_zero and extra is not None:                          # ZerosMat replaced by H_z (bs:163-164)
            blocks = extra.to(dt).clone()
            val = dampen
            if adaptive_dampen:
                val = val * blocks.diagonal(dim1=-1, dim2=-2).abs().max() if n_ent else val
            ne.leaves[name] = blocks + val * torch.eye(b, dtype=dt)
            return
        if is_zero:                                                # ZerosMat.dampen_ (bs:510-517)
            blocks = torch.zeros((n_ent, b, b), dtype=dt)
            blocks += dampen * torch.eye(b, dtype=dt)
        else:
            per = torch.einsum('nki,nkj->nij', Jb, Jb) if Jb.ndim == 3 else Jb[:, :, None] * Jb[:, None, :]
            blocks = torch.zeros((n_ent, b, b), dtype=dt)
            blocks.index_add_(0, cols, per)                          # bs:919-924
            if extra is not None:                                    # bs:157-158, before damping
                blocks += extra.to(dt)
            val = dampen
            if adaptive_dampen:                                      # bs:579-581
                val = val * blocks.diagonal(dim1=-1, dim2=-2).abs().max() if n_ent else val
            blocks += val * torch.eye(b, dtype=dt)
        ne.leaves[name] = blocks

    gram_leaf('foc', J_foc, c_foc, cams.n, 2, zf)
    gram_leaf('tau', J_tau, c_tau, nodes.n, 6, zt)
    gram_leaf('zcf', Jz, c_zcf, imgs.n, C, zz, None if z_prior is None else z_prior[0])
    gram_leaf('pts', Jp, c_pts, trks.n, 3, zp)
    ne.leaf_offsets = dict(foc=0, tau=off_t, zcf=off_z, pts=n_c)

    # cross blocks inside A (upper triangle: foc-tau, foc-zcf, tau-zcf; bs:1069 recursively)
    def cross(J1, c1, off1, n1, z1, J2, c2, off2, n2, z2, row2_only_second=False, row2_only_first=False):
        if z1 or z2:
            return
        if row2_only_second:
            per = J1[:, 2, :, None] * J2[:, None, :]
        elif row2_only_first:
            per = J1[:, :, None] * J2[:, 2, None, :]
        else:
            per = torch.einsum('nki,nkj->nij', J1, J2)
        blocks, rows, cols = _aggregate(per, c1, c2, n2)
        ne.cross.append(_BlockCOO(blocks, rows, cols, off1, off2, n1, n2))

    cross(J_foc, c_foc, 0, cams.n, zf, J_tau, c_tau, off_t, nodes.n, zt)
    cross(J_foc, c_foc, 0, cams.n, zf, Jz, c_zcf, off_z, imgs.n, zz, row2_only_second=True)
    cross(J_tau, c_tau, off_t, nodes.n, zt, Jz, c_zcf, off_z, imgs.n, zz, row2_only_second=True)

    # B = H_cp blocks (camera rows, point cols), aggregated per unique (entity, track)
    def hcp(J1, c1, off1, n1, z1, row2_only=False):
        if z1 or zp:
            return
        per = (J1[:, :, None] * Jp[:, 2, None, :]) if row2_only else torch.einsum('nki,nkj->nij', J1, Jp)
        blocks, rows, cols = _aggregate(per, c1, c_pts, trks.n)
        ne.B.append(_BlockCOO(blocks, rows, cols, off1, 0, n1, trks.n))

    hcp(J_foc, c_foc, 0, cams.n, zf)
    hcp(J_tau, c_tau, off_t, nodes.n, zt)
    hcp(Jz, c_zcf, off_z, imgs.n, zz, row2_only=True)
    return ne, g, (cams, nodes, imgs, trks)


def _A_matvec(ne, v):
    s = ne.sizes
    out = torch.zeros(s['n_c'], dtype=v.dtype)
    for name in ('foc', 'tau', 'zcf'):
        blk = ne.leaves[name]
        off = ne.leaf_offsets[name]
        b = blk.shape[-1]
        seg = v[off: off + blk.shape[0] * b].view(-1, b)
        out[off: off + blk.shape[0] * b] += torch.einsum('nij,nj->ni', blk, seg).reshape(-1)
    for X in ne.cross:
        X.matvec(v, out)
        X.rmatvec(v, out)
    return out


def _B_matvec(ne, y):
    out = torch.zeros(ne.sizes['n_c'], dtype=y.dtype)
    for X in ne.B:
        X.matvec(y, out)
    return out


def _C_matvec(ne, v):
    out = torch.zeros(ne.sizes['n_p'], dtype=v.dtype)
    for X in ne.B:
        X.rmatvec(v, out)
    return out


def _D_solve(ne, y):
    D = ne.leaves['pts']
    return chol3x3_solve(D, y.view(-1, 3), 1e-12).reshape(-1)           # bs:589-599


def A_diag(ne):
    return torch.cat([ne.leaves[n].diagonal(dim1=-1, dim2=-2).reshape(-1) for n in ('foc', 'tau', 'zcf')])


def pcg(A_mv, b, M_mv=None, x0=None, tol=1e-6, maxiter=200, history=None):
    """Restates ``_pcg`` (bs:1197-1238): returns (x, iters, converged).

    ``history``, a list, receives the iterate after every update (x after k updates at index k - 1).
    """
    x = torch.zeros_like(b) if x0 is None else x0.clone()
    r = b - A_mv(x)
    z = M_mv(r) if M_mv is not None else r
    p = z.clone()
    rz_old = torch.dot(r, z)
    best = (float('inf'), x, 0)
    bnorm = torch.norm(b).clamp(min=1e-12)
    for k in range(1, maxiter + 1):
        Ap = A_mv(p)
        denom = torch.dot(p, Ap).clamp(min=1e-32)
        alpha = rz_old / denom
        x = x + alpha * p
        r = r - alpha * Ap
        if history is not None:
            history.append(x)
        r_norm = r.norm()
        if r_norm < best[0]:
            best = (r_norm, x, k)
        if torch.norm(r) <= tol * bnorm:
            return x, k, True
        z = M_mv(r) if M_mv is not None else r
        rz_new = torch.dot(r, z)
        if not rz_new.isfinite():
            break
        beta = rz_new / rz_old.clamp(min=1e-32)
        p = z + beta * p
        rz_old = rz_new
    return best[1], best[2], False


def reduced_rhs(ne, g):
    n_c = ne.sizes['n_c']
    g_c, g_p = g[:n_c], g[n_c:]
    return g_c - _B_matvec(ne, _D_solve(ne, g_p))                      # bs:188


def S_matvec(ne, v):
    return _A_matvec(ne, v) - _B_matvec(ne, _D_solve(ne, _C_matvec(ne, v)))   # bs:197-200


def solve_reduced_pcg(ne, g, tol=1e-6, maxiter=300):
    """``_solve_CG`` (bs:184-206). Returns (delta fp64, iters, converged)."""
    n_c = ne.sizes['n_c']
    g_p = g[n_c:]
    rhs = reduced_rhs(ne, g)
    diagA = A_diag(ne).clamp(min=1e-12)                                # bs:191-194
    delta_c, niter, conv = pcg(lambda v: S_matvec(ne, v), rhs, M_mv=lambda v: v / diagA, tol=tol, maxiter=maxiter)
    delta_p = _D_solve(ne, g_p - _C_matvec(ne, delta_c))               # bs:203
    return torch.cat([delta_c, delta_p]), niter, conv


def dense_A(ne):
    n_c = ne.sizes['n_c']
    A = torch.zeros((n_c, n_c), dtype=ne.leaves['foc'].dtype)
    eye = torch.eye(n_c, dtype=A.dtype)
    for j in range(n_c):                                                # small problems only
        A[:, j] = _A_matvec(ne, eye[j])
    return A


def dense_schur(ne):
    """Explicit S = A - B D^-1 C by applying the operator to unit vectors (tiny problems)."""
    n_c = ne.sizes['n_c']
    S = torch.zeros((n_c, n_c), dtype=ne.leaves['foc'].dtype)
    eye = torch.eye(n_c, dtype=S.dtype)
    for j in range(n_c):
        S[:, j] = S_matvec(ne, eye[j])
    return S


def solve_reduced_direct(ne, g, S=None):
    """Dense direct solve of the same reduced system + back-substitution."""
    n_c = ne.sizes['n_c']
    if S is None:
        S = dense_schur(ne)
    rhs = reduced_rhs(ne, g)
    delta_c = torch.linalg.solve(S, rhs)
    delta_p = _D_solve(ne, g[n_c:] - _C_matvec(ne, delta_c))
    return torch.cat([delta_c, delta_p])


def unpack_delta(delta, params, C):
    """Restates ``unpack_delta_inplace`` (bs:228-248): split and scatter masked entries back."""
    cams, nodes, imgs, trks = params
    sizes = [cams.n * N_FOC, nodes.n * N_TAU, imgs.n * C, trks.n * 3]
    dK, dP, dZ, dX = torch.split(delta, sizes)

    def expand(d, p, k):
        d = d.view(p.n, k)
        if p.true_idxs is not None:
            d2 = d.new_zeros((p.true_n, k))
            d2[p.true_idxs] = d
            return d2
        return d

    return expand(dK, cams, N_FOC), expand(dP, nodes, N_TAU), expand(dZ, imgs, C), expand(dX, trks, 3)
