"""Oracle restatement of the reference ``cujac`` kernels (test infrastructure only).

Each function restates one entry point of
``src/blast3r/extensions/cujac/sfm_jacobian_rigs.cu`` (abbreviated ``.cu`` below)
as vectorised torch-CPU code.  Precision follows the reference: the residual
kernel is fp32 end to end (``.cu:129-259``), the Jacobian kernel computes in the
output dtype (fp64 on the solver path, ``.cu:323-509``) from fp32 inputs.

Pinning (see tests/test_oracle.py):
  * residuals: fp64 closed form of the projection, identity-pose on-axis point,
    z <= 1e-3 rows, textbook Huber/IRLS for pnorm=1, clip -> w_null.
  * jacobians: torch.autograd of an independent fp64 residual under the left
    perturbation P <- exp(xi^) P, separate fx/fy, z-coefs and X; the three
    quirks (g>0 gate, fp32-rounded J_k_f, r2 focal through fbar) separately.
  * chol3x3_solve: torch.linalg.solve on the symmetrised, jittered block.
  * blockcoo_matvec / fused_einsum_bki_bkj: dense materialisation.
  * exp_se3: closed-form SE(3) exponential (Rodrigues + V matrix).
"""
import torch

__all__ = ['obs_to_img', 'residuals_with_rigs', 'jacobians_with_rigs', 'chol3x3_solve',
           'blockcoo_matvec', 'fused_einsum_bki_bkj', 'skew_symmetric', 'hat_se3', 'exp_se3']


def obs_to_img(infos, n_obs):
    """Image index of every observation.

    Restates ``searchsorted`` (.cu:72-88): the largest ``a`` in [0, n_imgs) with
    cum[a-1] <= idx, i.e. an upper bound over cum[0..n_imgs-2].
    """
    cum = infos[0].long()
    idx = torch.arange(n_obs, dtype=torch.long)
    return torch.searchsorted(cum[:-1].contiguous(), idx, right=True)


def _poses(infos, K, P_rig2c, P_w2rig, n_obs, dtype):
    img = obs_to_img(infos, n_obs)
    node = infos[1].long()[img]
    cam = infos[2].long()[img]
    Kc = K.to(dtype)[cam]
    Prc = P_rig2c.to(dtype)[cam]          # stride-0 broadcast views index fine
    Pwr = P_w2rig.to(dtype)[node]
    return img, node, cam, Kc, Prc, Pwr


def residuals_with_rigs(infos, K, P_rig2c, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std, pix2d_dep,
                        is_depth_log, weight_z=1.0, pnorm=-1.0, max_pix_err=100.0, huber_delta=0.5,
                        w_pts_null=1e-16):
    """Per-observation residuals, Huber errors and IRLS weights, fp32.

    Restates ``residuals_with_rigs`` (.cu:1048-1101) and its kernel (.cu:129-259).
    Returns the (n_out, n_obs) SoA buffer transposed to (n_obs, n_out), n_out = 9
    when pnorm > 0 else 3 (.cu:1069-1075, :1100).  Rows with z <= 1e-3 stay zero
    (.cu:212).
    """
    assert (pnorm == -1) or (0 < pnorm <= 2), 'pnorm must be in {-1} U ]0,2]'   # .cu:1066
    f32 = torch.float32
    n_obs = len(pids)
    C = pix2d_dep.shape[1]
    assert C == z_coefs.shape[1]
    img, node, cam, Kc, Prc, Pwr = _poses(infos, K, P_rig2c, P_w2rig, n_obs, f32)
    X = pts3d.to(f32)[pids.long()]
    X_rig = torch.einsum('nij,nj->ni', Pwr[:, :3, :3], X) + Pwr[:, :3, 3]          # .cu:203
    X_cam = torch.einsum('nij,nj->ni', Prc[:, :3, :3], X_rig) + Prc[:, :3, 3]      # .cu:208
    z = X_cam[:, 2]
    valid = z.double() > 1e-3         # .cu:212: the fp32 depth against the double literal (1e-3f is kept)
    fx, cx, fy, cy = Kc[:, 0, 0], Kc[:, 0, 2], Kc[:, 1, 1], Kc[:, 1, 2]
    zs = torch.where(valid, z, torch.ones_like(z))
    p0 = (fx * X_cam[:, 0] + cx * X_cam[:, 2]) / zs                                  # .cu:217
    p1 = (fy * X_cam[:, 1] + cy * X_cam[:, 2]) / zs                                  # .cu:218
    r0 = (p0 - pix2d[:, 0]) / pix2d_std[:, 0]                                        # .cu:228
    r1 = (p1 - pix2d[:, 1]) / pix2d_std[:, 1]
    g = (z_coefs.to(f32)[img] * pix2d_dep.to(f32)).sum(1)                            # .cu:231-233
    avg_focal = 0.5 * (fx + fy)                                                      # .cu:234
    if is_depth_log:
        r2 = avg_focal * (g - torch.log(zs))                                          # .cu:236
    else:
        r2 = avg_focal * torch.log(g / zs)                                            # .cu:238
    res = torch.stack((r0, r1, r2), 0)
    n_out = 9 if pnorm > 0 else 3
    out = torch.zeros((n_out, n_obs), dtype=f32)
    out[:3] = torch.where(valid, res, torch.zeros_like(res))
    if pnorm > 0:
        delta = torch.tensor(huber_delta, dtype=f32)
        pn = torch.tensor(pnorm, dtype=f32)
        a = 0.5 * pn * torch.pow(delta, pn - 2)                                       # .cu:242
        b = torch.pow(delta, pn) - a * delta * delta                                  # .cu:243
        wz = torch.tensor([1.0, 1.0, weight_z], dtype=f32)
        M = torch.tensor(max_pix_err, dtype=f32)
        for i in range(3):
            r = res[i].abs()
            r = torch.where(r > M, M, r)                                               # .cu:251
            err = wz[i] * torch.where(r <= delta, a * r * r, torch.pow(r, pn) - b)     # .cu:252
            r = torch.where(r < delta, delta, r)                                       # .cu:255
            w = torch.where(r == M, torch.tensor(w_pts_null, dtype=f32), wz[i] * torch.pow(r, pn - 2))  # .cu:256
            out[3 + i] = torch.where(valid, err, torch.zeros_like(err))
            out[6 + i] = torch.where(valid, w, torch.zeros_like(w))
    return out.transpose(0, 1)


def jacobians_with_rigs(infos, K, P_rig2c, P_w2rig, z_coefs, pts3d, pids, pix2d_std, pix2d_dep,
                        is_depth_log, float64=False):
    """Explicit per-observation Jacobian blocks.

    Restates ``jacobians_with_rigs`` (.cu:1105-1148) and its kernel (.cu:323-509).
    Returns J_cam (N,3,8) with columns [fx, fy, wx, wy, wz, vx, vy, vz],
    J_zcf (N,1,C) and J_pts (N,3,3), zero for rows with z <= 1e-3 (.cu:408).
    """
    T = torch.float64 if float64 else torch.float32
    n_obs = len(pids)
    C = pix2d_dep.shape[1]
    img, node, cam, Kc, Prc, Pwr = _poses(infos, K, P_rig2c, P_w2rig, n_obs, T)
    X = pts3d.to(T)[pids.long()]
    R_rw, t_rw = Pwr[:, :3, :3], Pwr[:, :3, 3]
    R_cr, t_cr = Prc[:, :3, :3], Prc[:, :3, 3]
    X_rig = torch.einsum('nij,nj->ni', R_rw, X) + t_rw                               # .cu:392
    X_cam = torch.einsum('nij,nj->ni', R_cr, X_rig) + t_cr                           # .cu:397
    fx, cx, fy, cy = Kc[:, 0, 0], Kc[:, 0, 2], Kc[:, 1, 1], Kc[:, 1, 2]
    p0 = fx * X_cam[:, 0] + cx * X_cam[:, 2]                                          # .cu:403
    p1 = fy * X_cam[:, 1] + cy * X_cam[:, 2]
    z = X_cam[:, 2]
    valid = z.double() > 1e-3         # .cu:408: Tfloat depth against the double literal
    zs = torch.where(valid, z, torch.ones_like(z))
    inv_z = 1.0 / zs                                                                  # .cu:411
    inv_z2 = inv_z * inv_z
    avg_focal = 0.5 * (fx + fy)                                                       # .cu:413
    std = pix2d_std.to(T)
    Jpc = torch.zeros((n_obs, 3, 3), dtype=T)                                         # .cu:415-427
    Jpc[:, 0, 0] = fx * inv_z / std[:, 0]
    Jpc[:, 0, 2] = (cx * inv_z - p0 * inv_z2) / std[:, 0]
    Jpc[:, 1, 1] = fy * inv_z / std[:, 1]
    Jpc[:, 1, 2] = (cy * inv_z - p1 * inv_z2) / std[:, 1]
    Jpc[:, 2, 2] = -avg_focal * inv_z
    Jpr = Jpc @ R_cr                                                                  # .cu:441
    Jrt = torch.zeros((n_obs, 3, 6), dtype=T)                                         # .cu:444-453
    Jrt[:, 0, 1] = X_rig[:, 2]; Jrt[:, 0, 2] = -X_rig[:, 1]; Jrt[:, 0, 3] = 1
    Jrt[:, 1, 0] = -X_rig[:, 2]; Jrt[:, 1, 2] = X_rig[:, 0]; Jrt[:, 1, 4] = 1
    Jrt[:, 2, 0] = X_rig[:, 1]; Jrt[:, 2, 1] = -X_rig[:, 0]; Jrt[:, 2, 5] = 1
    J_tau = Jpr @ Jrt                                                                 # .cu:458
    J_pts = Jpr @ R_rw                                                                # .cu:463
    dep = pix2d_dep.to(T)
    # Tfloat guidance (.cu:466-468): each product z_c * dep_c is a float product, summed in Tfloat
    prod = (z_coefs.to(torch.float32)[img] * pix2d_dep.to(torch.float32)).to(T)
    g = torch.zeros(n_obs, dtype=T)
    for c in range(C):
        g = g + prod[:, c]
    J_cam = torch.zeros((n_obs, 3, 8), dtype=T)
    J_cam[:, 0, 0] = X_cam[:, 0] * inv_z / std[:, 0]                                  # .cu:473
    J_cam[:, 1, 1] = X_cam[:, 1] * inv_z / std[:, 1]                                  # .cu:477
    J_cam[:, :, 2:] = J_tau
    # J_k_f is gated on g > 0 and held in a float even on the fp64 path (.cu:481-489)
    if is_depth_log:
        jkf = 0.5 * (g + torch.log(inv_z))
    else:
        jkf = 0.5 * torch.log(g * inv_z)
    jkf = torch.where(g > 0, jkf, torch.zeros_like(jkf)).to(torch.float32).to(T)
    J_cam[:, 2, 0] = jkf
    J_cam[:, 2, 1] = jkf
    if is_depth_log:                                                                  # .cu:496-501
        J_zcf = avg_focal[:, None] * dep
    else:
        gs = torch.where(g != 0, g, torch.ones_like(g))
        J_zcf = torch.where((g != 0)[:, None], (avg_focal / gs)[:, None] * dep, torch.zeros_like(dep))
    J_zcf = J_zcf[:, None, :]
    m = valid.to(T)
    return J_cam * m[:, None, None], J_zcf * m[:, None, None], J_pts * m[:, None, None]


def chol3x3_solve(blocks, rhs, jitter=1e-12):
    """Batched 3x3 SPD solve; restates ``chol3x3_solve`` (.cu:1151-1169, kernel :560-634).

    Jitter on the diagonal, off-diagonals symmetrised by averaging, non-positive
    pivots get +jitter, then LL^T forward/back substitution.
    """
    A = blocks
    j = jitter
    a00, a11, a22 = A[:, 0, 0] + j, A[:, 1, 1] + j, A[:, 2, 2] + j                   # .cu:578-586
    a01 = (A[:, 0, 1] + A[:, 1, 0]) * 0.5                                             # .cu:590-595
    a02 = (A[:, 0, 2] + A[:, 2, 0]) * 0.5
    a12 = (A[:, 1, 2] + A[:, 2, 1]) * 0.5
    guard = lambda v: torch.where(v > 0, v, v + j)                                    # .cu:600, :609, :617
    l00 = torch.sqrt(guard(a00))
    l10 = a01 / l00
    l20 = a02 / l00
    l11 = torch.sqrt(guard(a11 - l10 * l10))
    l21 = (a12 - l10 * l20) / l11
    l22 = torch.sqrt(guard(a22 - l20 * l20 - l21 * l21))
    b = rhs
    z0 = b[:, 0] / l00                                                                 # .cu:621-628
    z1 = (b[:, 1] - l10 * z0) / l11
    z2 = (b[:, 2] - l20 * z0 - l21 * z1) / l22
    x2 = z2 / l22
    x1 = (z1 - l21 * x2) / l11
    x0 = (z0 - l10 * x1 - l20 * x2) / l00
    return torch.stack((x0, x1, x2), 1)


def blockcoo_matvec(blocks, row_indices, col_indices, x, HB1, WB1, transpose_blocks=False):
    """y = A x (or A^T x) for a block-COO matrix; restates ``blockcoo_matvec`` (.cu:1171-1219)."""
    N, bh, bw = blocks.shape
    in_len = HB1 * bh if transpose_blocks else WB1 * bw
    out_len = WB1 * bw if transpose_blocks else HB1 * bh
    assert x.numel() == in_len, 'x has wrong length for the provided shapes'
    r = row_indices.long()
    c = col_indices.long()
    if not transpose_blocks:
        xs = x.view(WB1, bw)[c]                                       # (N, bw)
        contrib = torch.einsum('nij,nj->ni', blocks, xs)              # (N, bh)
        y = torch.zeros((HB1, bh), dtype=blocks.dtype)
        y.index_add_(0, r, contrib)
    else:
        xs = x.view(HB1, bh)[r]
        contrib = torch.einsum('nij,ni->nj', blocks, xs)
        y = torch.zeros((WB1, bw), dtype=blocks.dtype)
        y.index_add_(0, c, contrib)
    return y.view(out_len)


def fused_einsum_bki_bkj(left, right):
    """out[b] = left[b]^T right[b]; restates ``fused_einsum_bki_bkj`` (.cu:1222-1250).

    The reference dispatches a fixed (I,J,K) list (.cu:969-1007); the oracle is
    the mathematical definition for any shape.
    """
    assert left.shape[0] == right.shape[0] and left.shape[1] == right.shape[1]
    return torch.einsum('bki,bkj->bij', left, right)


def skew_symmetric(w):
    """(B,3) -> (B,3,3) cross-product matrices; restates cujac/__init__.py:27-41."""
    wx, wy, wz = w.T
    res = w.new_zeros((len(w), 3, 3))
    res[:, 2, 1] = wx
    res[:, 1, 2] = -wx
    res[:, 2, 0] = -wy
    res[:, 0, 2] = wy
    res[:, 0, 1] = -wz
    res[:, 1, 0] = wz
    return res


def hat_se3(xi):
    """(B,6) [w|v] -> (B,4,4); restates cujac/__init__.py:43-54."""
    hat = xi.new_zeros((len(xi), 4, 4))
    hat[:, :3, :3] = skew_symmetric(xi[:, :3])
    hat[:, :3, 3] = xi[:, 3:]
    return hat


def exp_se3(xi):
    """SE(3) exponential via ``torch.matrix_exp`` of the hat matrix (cujac/__init__.py:56-58)."""
    return torch.matrix_exp(hat_se3(xi))
