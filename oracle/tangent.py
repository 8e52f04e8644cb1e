"""Oracle restatement of the dense tangent prior (test infrastructure only).

Follows ``_dense_tangent_prior_terms`` and ``confident_in_planar_regions``
(src/blast3r/inference/engine.py:15-179, :182-200, abbreviated ``en``) on CPU
torch, one image at a time, in the working dtype the reference uses:

  * the maps are subsampled at rows/columns s//2, s//2 + s, ... and the
    intrinsics follow (principal point minus s//2, first two rows / s);
  * combined log depth L = sum_c a_c L_c, D = exp(min(L, 80)), X = D K^-1 (u+.5, v+.5, 1)
    (en:76-87, utils/geometry.py:137-153);
  * unit tangents of X and of the reference pointmap X0 along rows (x) and
    columns (y), residuals r = t_hat - t0_hat, weights sqrt(max(Cw Cw', 0)) with Cw
    the planar confidence of X0's depth (en:98-130, en:182-200);
  * loss = weight * mean(w r^2) per direction and image (en:132-135);
  * Gauss-Newton terms w.r.t. z_coefs (en:141-172): dX/da_c = D L_c ray, projected
    orthogonally to t_hat and scaled by 1/|t| when the tangents are normalised.

The reference's quirks are kept: images whose subsampled width or channel count
is below 2 are skipped (en:75, ``min(L.shape[1:])``); the pointmap X0 stays in
its own dtype (fp32) even on the fp64 path; without normalisation X0 is
rescaled by the lower median of D / z0 and the tangents of X share X0's norms.

Pinned in tests/test_tangent.py: g and H against J^T r and J^T J of the
residuals differentiated by torch.autograd, zero loss and gradient when X equals
X0, the planar confidence on constant and affine maps and at borders.
"""
import torch
import torch.nn.functional as F


def planar_confidence(D0, alpha=1e4):
    """en:182-200: exp(-alpha (lx^2 + ly^2)), l = discrete Laplacians normalised by the 3x3 minimum."""
    assert D0.ndim == 2
    lx = 2 * D0
    lx[:, 1:] -= D0[:, :-1]
    lx[:, :-1] -= D0[:, 1:]
    ly = 2 * D0
    ly[1:, :] -= D0[:-1, :]
    ly[:-1, :] -= D0[1:, :]
    m = -F.max_pool2d(-D0[None, None], 3, stride=1, padding=1)
    m = m.squeeze().clip(min=1e-12)
    lx /= m
    ly /= m
    return torch.exp(-alpha * (lx * lx + ly * ly))


def _rays(H, W, Ks, dtype):
    """K^-1 (u + .5, v + .5, 1) on an H x W grid (utils/geometry.py:137-153)."""
    Ki = torch.linalg.inv(Ks)
    u = torch.arange(W, dtype=dtype) + 0.5
    v = torch.arange(H, dtype=dtype) + 0.5
    grid = torch.stack(torch.meshgrid(u, v, indexing='xy'), dim=-1)          # (H, W, 2)
    return grid @ Ki.T[:2, :] + Ki.T[2:, :]


def _image_terms(L, a, Ks, X0, weight, eps, normalize, dtype, compute_gn):
    """One image: (loss terms per direction, g, H) or None when the reference skips it."""
    Hs, Ws, C = L.shape
    if min(Ws, C) < 2:                                                        # en:75
        return None
    D = torch.exp(torch.einsum('c,hwc->hw', a, L).clamp(max=80))
    ray = _rays(Hs, Ws, Ks, dtype)
    X = ray * D[..., None]
    if not normalize:                                                         # en:89-95
        z0 = X0[..., 2]
        keep = z0 > 1e-6
        s = torch.median(D[keep] / z0[keep]) if keep.any() else D.new_tensor(1.0)
        X0 = s * X0
    terms = []
    g = torch.zeros(C, dtype=dtype) if compute_gn else None
    Hm = torch.zeros((C, C), dtype=dtype) if compute_gn else None
    Cw = planar_confidence(X0[:, :, 2])
    for dim in (0, 1):                                                        # rows (x), then columns (y)
        n = X.shape[dim] - 1
        if n <= 0:
            continue
        t = X.narrow(dim, 1, n) - X.narrow(dim, 0, n)
        t0 = X0.narrow(dim, 1, n) - X0.narrow(dim, 0, n)
        is0 = 1.0 / t0.norm(dim=-1, keepdim=True).clamp(min=eps)
        is_ = 1.0 / t.norm(dim=-1, keepdim=True).clamp(min=eps) if normalize else is0
        th = t * is_
        r = th - t0 * is0
        w = (Cw.narrow(dim, 1, n) * Cw.narrow(dim, 0, n)).clamp(min=0).sqrt()
        terms.append(weight * (w.unsqueeze(-1) * r.square()).mean())
        if not compute_gn:
            continue
        S = D.unsqueeze(0) * L.permute(2, 0, 1)                               # dD/da_c
        dX = S.unsqueeze(-1) * ray.unsqueeze(0)                              # (C, H, W, 3)
        dt = dX.narrow(dim + 1, 1, n) - dX.narrow(dim + 1, 0, n)
        if normalize:
            dt = (dt - th.unsqueeze(0) * (dt * th.unsqueeze(0)).sum(-1, keepdim=True)) * is_.unsqueeze(0)
        else:
            dt = dt * is_
        scale = weight / r.numel()
        wf = w.reshape(-1)
        dtf = dt.reshape(C, -1, 3)
        g += scale * torch.einsum('n,cnk,nk->c', wf, dtf, r.reshape(-1, 3))
        Hm += scale * torch.einsum('n,cnk,dnk->cd', wf, dtf, dtf)
    return terms, g, Hm


def tangent_prior_terms(cam_ids, K, z_coefs, log_depth_maps, pts3d_ref, weight_tan=0.0, tan_stride=4,
                        optim_Z0=True, dtype=torch.float32, compute_gn=True, normalize_tangents=True, eps=1e-4):
    """en:15-179 on CPU: (tan_loss, g_z (n_imgs, C) or None, H_z (n_imgs, C, C) or None)."""
    n_imgs, C = z_coefs.shape
    loss = torch.zeros((), dtype=dtype)
    g = torch.zeros((n_imgs, C), dtype=dtype) if compute_gn else None
    H = torch.zeros((n_imgs, C, C), dtype=dtype) if compute_gn else None
    if weight_tan <= 0:
        return loss, g, H
    s = tan_stride
    o = s // 2
    for i in range(n_imgs):
        Ks = K[int(cam_ids[i])].to(dtype).clone()
        Ks[:2, 2] -= o
        Ks[:2] /= s
        L = log_depth_maps[i][o::s, o::s].to(dtype)
        X0 = pts3d_ref[i][o::s, o::s]
        res = _image_terms(L, z_coefs[i].to(dtype), Ks, X0, float(weight_tan), eps, normalize_tangents, dtype,
                           compute_gn)
        if res is None:
            continue
        for term in res[0]:                                                   # en:132-135, in order
            loss = loss + term
        if compute_gn:
            g[i] += res[1]
            H[i] += res[2]
    if compute_gn and not optim_Z0 and C > 0:                                 # en:174-177
        g[:, 0] = 0
        H[:, 0, :] = 0
        H[:, :, 0] = 0
    return loss, g, H
