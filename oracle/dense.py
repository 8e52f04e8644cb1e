"""Brute-force dense forms used to pin the oracle on tiny problems (test infrastructure only).

Nothing here follows the reference's block algorithms: J is materialised as a
dense (3N x n_params) matrix in the reference unknown order
[foc | tau | zcf | pts] (src/blast3r/inference/ba_solver.py:119), the normal
equations are formed by dense products, the Schur complement by a dense
inverse, and per-observation Jacobians by ``torch.func`` autodiff of an
independent fp64 residual written from the model equations
(src/blast3r/inference/engine.py:228-231 docstring; sfm_jacobian_rigs.cu:201-238).
"""
import torch
from torch.func import jacrev, vmap

from .kernels import exp_se3, obs_to_img

__all__ = ['residual_fp64', 'autodiff_jacobians', 'dense_jacobian', 'dense_normal_equations',
           'similarity_gauge_basis']


def _skew(w):
    z = torch.zeros((), dtype=w.dtype)
    return torch.stack([torch.stack([z, -w[2], w[1]]), torch.stack([w[2], z, -w[0]]),
                        torch.stack([-w[1], w[0], z])])


def _expm_se3_single(xi):
    H = torch.zeros((4, 4), dtype=xi.dtype)
    H = H.index_put((torch.arange(3)[:, None], torch.arange(3)[None, :]), _skew(xi[:3]))
    H = H.index_put((torch.arange(3), torch.full((3,), 3)), xi[3:])
    return torch.linalg.matrix_exp(H)


def residual_fp64(fxy, xi, zc, X, cx, cy, P_w2rig, P_rig2c, pix, std, dep, is_depth_log=True):
    """One observation's 3 residuals in fp64 under the left perturbation P <- exp(xi^) P."""
    P = _expm_se3_single(xi) @ P_w2rig
    X_rig = P[:3, :3] @ X + P[:3, 3]
    X_cam = P_rig2c[:3, :3] @ X_rig + P_rig2c[:3, 3]
    z = X_cam[2]
    p0 = (fxy[0] * X_cam[0] + cx * z) / z
    p1 = (fxy[1] * X_cam[1] + cy * z) / z
    g = (zc * dep).sum()
    fbar = 0.5 * (fxy[0] + fxy[1])
    r2 = fbar * (g - torch.log(z)) if is_depth_log else fbar * torch.log(g / z)
    return torch.stack([(p0 - pix[0]) / std[0], (p1 - pix[1]) / std[1], r2])


def autodiff_jacobians(infos, K, P_rig2c, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std, pix2d_dep,
                       is_depth_log=True):
    """Per-observation true derivatives (N,3,2), (N,3,6), (N,3,C), (N,3,3) at xi = 0."""
    d = torch.float64
    n = len(pids)
    img = obs_to_img(infos, n)
    node = infos[1].long()[img]
    cam = infos[2].long()[img]
    Kc = K.to(d)[cam]
    fxy = torch.stack([Kc[:, 0, 0], Kc[:, 1, 1]], 1)
    cx, cy = Kc[:, 0, 2], Kc[:, 1, 2]
    xi = torch.zeros((n, 6), dtype=d)
    zc = z_coefs.to(d)[img]
    X = pts3d.to(d)[pids.long()]
    f = lambda a, b, c, e, *rest: residual_fp64(a, b, c, e, *rest, is_depth_log=is_depth_log)
    jac = vmap(jacrev(f, argnums=(0, 1, 2, 3)))(fxy, xi, zc, X, cx, cy, P_w2rig.to(d)[node],
                                               P_rig2c.to(d)[cam], pix2d.to(d), pix2d_std.to(d),
                                               pix2d_dep.to(d))
    return jac


def dense_jacobian(J_cam, J_zcf, J_pts, infos, pids, n_cams, n_nodes, n_tracks):
    """Materialise J (3N x n_params) from per-observation blocks, reference unknown order."""
    n = J_cam.shape[0]
    C = J_zcf.shape[-1]
    n_imgs = infos.shape[1]
    img = obs_to_img(infos, n)
    node = infos[1].long()[img]
    cam = infos[2].long()[img]
    nf, nt, nz, npp = 2 * n_cams, 6 * n_nodes, C * n_imgs, 3 * n_tracks
    J = torch.zeros((3 * n, nf + nt + nz + npp), dtype=J_cam.dtype)
    for o in range(n):
        rows = slice(3 * o, 3 * o + 3)
        c, nd, i, t = int(cam[o]), int(node[o]), int(img[o]), int(pids[o])
        J[rows, 2 * c: 2 * c + 2] = J_cam[o, :, :2]
        J[rows, nf + 6 * nd: nf + 6 * nd + 6] = J_cam[o, :, 2:]
        J[3 * o + 2, nf + nt + C * i: nf + nt + C * i + C] = J_zcf[o, 0]
        J[rows, nf + nt + nz + 3 * t: nf + nt + nz + 3 * t + 3] = J_pts[o]
    return J


def dense_normal_equations(J, residuals, w_pts, sizes, dampen=1e-12, adaptive=True, clamp_w=(1e-6, 1e6)):
    """H = J^T W J + per-leaf damping, g = J^T W r, with dense products only.

    ``sizes`` = (n_foc, n_tau, n_zcf, n_pts) scalar counts of the four leaves.
    """
    W = w_pts.expand(-1, 3).clamp(min=clamp_w[0], max=clamp_w[1]).reshape(-1).to(J.dtype)
    r = residuals.reshape(-1).to(J.dtype)
    g = J.T @ (W * r)
    H = J.T @ (W[:, None] * J)
    off = 0
    for s in sizes:
        if s:
            dg = H.diagonal()[off: off + s]
            lam = dampen * (dg.abs().max() if adaptive else 1.0)
            idx = torch.arange(off, off + s)
            H[idx, idx] += lam
        off += s
    return H, g


def similarity_gauge_basis(P_w2rig, pts3d, z_coefs_cols, n_cams, C, beta_col=1):
    """Seven infinitesimal world-similarity directions in the full unknown space.

    World transform X -> (1+s) (X + w x X + v).  Under the reference update rules
    (P <- exp(-dP^) P, X <- X - dX, z <- z - dZ) a world rotation w / translation v /
    scale s maps to: dX = -(w x X + v + s X); for each node with R,t:
    the rig frame sees X_rig' = R X' + t' so the pose must absorb the change;
    d(tau) follows from X_rig' = X_rig (1 + s) with tau = -(R w ; R v - (R w) x t ... ).
    Computed numerically here by finite differences of the residual-free
    pose identity: for a world similarity G, P' = P G^-1 (scaled), which is
    linearised below.  Returns an (n_params x 7) fp64 matrix.
    """
    d = torch.float64
    n_nodes = P_w2rig.shape[0]
    T = pts3d.shape[0]
    nf, nt, nz, npp = 2 * n_cams, 6 * n_nodes, C * z_coefs_cols, 3 * T
    basis = torch.zeros((nf + nt + nz + npp, 7), dtype=d)
    R = P_w2rig[:, :3, :3].to(d)
    t = P_w2rig[:, :3, 3].to(d)
    X = pts3d.to(d)
    e = torch.eye(3, dtype=d)
    for k in range(7):
        w = e[k] if k < 3 else torch.zeros(3, dtype=d)
        v = e[k - 3] if 3 <= k < 6 else torch.zeros(3, dtype=d)
        s = 1.0 if k == 6 else 0.0
        # new world points X' = X + w x X + v + s X  ->  dX = -(X' - X)
        dXw = torch.cross(w.expand_as(X), X, dim=1) + v + s * X
        basis[nf + nt + nz:, k] = -dXw.reshape(-1)
        # new pose must satisfy R' X' + t' = (1+s)(R X + t) to first order
        # R' = exp(a^) R, t' = exp(a^) t + b + ...: with left increment (a, b):
        # (a x (R X + t) + b) + R (w x X + v + s X) = s (R X + t)
        # => a = -R w ; b = -R v + s t + (R w) x t  (rotation of t cancels)
        Rw = R @ w
        a = -Rw
        b = -(R @ v) + s * t + torch.cross(Rw.expand_as(t), t, dim=1)
        # update rule P <- exp(-dP^) P  =>  dP = -(a, b)
        basis[nf: nf + nt, k] = torch.cat([-a, -b], 1).reshape(-1)
        # scale: log-depth shifts by log(1+s) ~ s, absorbed by beta (z <- z - dZ => dZ = -s)
        if k == 6:
            zpart = torch.zeros((z_coefs_cols, C), dtype=d)
            zpart[:, beta_col] = -1.0
            basis[nf + nt: nf + nt + nz, k] = zpart.reshape(-1)
    return basis
