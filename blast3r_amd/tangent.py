"""Dense tangent prior on the device: drop-in for ``_dense_tangent_prior_terms`` and
``confident_in_planar_regions`` (src/blast3r/inference/engine.py:15-200).

Same arguments, defaults and results (tan_loss as a 0-d tensor of ``dtype``; g_z (n_imgs, C) and
H_z (n_imgs, C, C), or None when ``compute_gn`` is False).  Every image is handled by one launch
sequence of ``ba_tangent_prior`` in libba_hip.so, which reads each image's maps where they lie
(a list of per-image tensors, channel slices of wider maps, or one stacked tensor).  With
compute_gn, up to 24 z-coefficients are supported (the solver's own limit).
"""
import ctypes

import torch

from ._lib import BaTangentArgs, check, lib, ptr, stream_ptr

__all__ = ['dense_tangent_prior_terms', 'confident_in_planar_regions']


def _views(maps, what):
    if isinstance(maps, torch.Tensor):
        return list(maps.unbind(0)) if maps.dim() == 4 else [maps]
    return list(maps)


def _pixel_stride(m, c_min, what):
    """Floats between neighbouring pixels of an (H, W, >= c_min) fp32 view with contiguous channels and
    rows W pixels apart."""
    if m.dim() != 3 or m.shape[2] < c_min:
        raise ValueError(f'{what}: expected (H, W, {c_min}+) maps, got {tuple(m.shape)}')
    if m.dtype != torch.float32:
        raise ValueError(f'{what} must be fp32')
    H, W, Cm = m.shape
    if Cm > 1 and m.stride(2) != 1:
        raise ValueError(f'{what}: channels must be contiguous')
    ps = m.stride(1) if W > 1 else (m.stride(0) if H > 1 else Cm)
    if ps < Cm or (H > 1 and m.stride(0) != W * ps):
        raise ValueError(f'{what}: pixels must be evenly spaced, rows W pixels apart')
    return ps


def dense_tangent_prior_terms(rigs, K, z_coefs, log_depth_maps, conf, pts3d_ref, *, weight_tan=0.0, tan_stride=4,
                              optim_Z0=True, dtype=torch.float32, compute_gn=True, normalize_tangents=True,
                              eps=1e-4):
    """engine.py:15-179 on the device."""
    n_imgs, C = z_coefs.shape
    dev = z_coefs.device
    if weight_tan <= 0:
        return (z_coefs.new_zeros((), dtype=dtype),
                None if not compute_gn else z_coefs.new_zeros((n_imgs, C), dtype=dtype),
                None if not compute_gn else z_coefs.new_zeros((n_imgs, C, C), dtype=dtype))
    assert tan_stride >= 1
    assert None not in (log_depth_maps, conf, pts3d_ref)
    if dev.type != 'cuda':
        raise RuntimeError('the tangent prior runs in libba_hip.so: pass device tensors')
    if dtype not in (torch.float32, torch.float64):
        raise ValueError(f'dtype must be float32 or float64, got {dtype}')
    deps = _views(log_depth_maps, 'log_depth_maps')
    refs = _views(pts3d_ref, 'pts3d_ref')
    assert len(deps) == len(conf) == len(refs) == n_imgs
    for L in deps:
        assert L.ndim == 3 and L.shape[2] == C, f'expected log_depth_maps n_imgs x (H,W,C), got {tuple(L.shape)}'
    shapes = [tuple(L.shape[:2]) for L in deps]
    for L, X0 in zip(deps, refs):
        if tuple(X0.shape[:2]) != tuple(L.shape[:2]) or L.device != dev or X0.device != dev:
            raise ValueError('each pts3d_ref must match its depth map in size and device')
    dps = {_pixel_stride(L, C, 'log_depth_maps') for L in deps}
    rps = {_pixel_stride(X0, 3, 'pts3d_ref') for X0 in refs}
    if len(dps) != 1 or len(rps) != 1:
        raise ValueError('every map of a kind must share one pixel stride')
    H = max(s[0] for s in shapes)
    W = max(s[1] for s in shapes)
    hw = None
    if any(s != (H, W) for s in shapes):
        hw = torch.tensor(shapes, dtype=torch.int32).to(dev)
    dep_addr = torch.tensor([L.data_ptr() for L in deps], dtype=torch.int64).to(dev)
    ref_addr = torch.tensor([X0.data_ptr() for X0 in refs], dtype=torch.int64).to(dev)
    rigs = rigs.to(dev)
    cam_ids = rigs[2].to(torch.int32).contiguous()
    if len(cam_ids) != n_imgs or int(cam_ids.min()) < 0 or int(cam_ids.max()) >= len(K):
        raise ValueError('rigs[2] must hold a camera index of K for every image')
    Kc = K.detach().to(device=dev, dtype=torch.float32).contiguous()
    zc = z_coefs.detach().to(torch.float32).contiguous()
    loss = torch.empty((), dtype=dtype, device=dev)
    g = torch.empty((n_imgs, C), dtype=dtype, device=dev) if compute_gn else None
    Hz = torch.empty((n_imgs, C, C), dtype=dtype, device=dev) if compute_gn else None
    L_ = lib()
    nb = int(L_.ba_tangent_workspace_bytes(n_imgs, C, H, W, int(tan_stride), int(bool(normalize_tangents)),
                                           int(bool(compute_gn))))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
    a = BaTangentArgs(depth_addr=ptr(dep_addr), ref_addr=ptr(ref_addr), map_hw=ptr(hw), H=H, W=W,
                      depth_pix_stride=dps.pop(), ref_pix_stride=rps.pop(), K=ptr(Kc), cam_ids=ptr(cam_ids),
                      z_coefs=ptr(zc), n_imgs=n_imgs, C=C, tan_stride=int(tan_stride),
                      normalize=int(bool(normalize_tangents)), optim_Z0=int(bool(optim_Z0)),
                      fp64=int(dtype == torch.float64), compute_gn=int(bool(compute_gn)), weight=float(weight_tan),
                      eps=float(eps), loss=ptr(loss), g_z=ptr(g), H_z=ptr(Hz), workspace=ptr(ws), workspace_bytes=nb)
    check(L_.ba_tangent_prior(ctypes.byref(a), stream_ptr(dev)))
    return loss, g, Hz


def confident_in_planar_regions(D0, alpha=1e4):
    """engine.py:182-200 on the device, for one (H, W) fp32 map."""
    assert D0.ndim == 2
    if D0.device.type != 'cuda':
        raise RuntimeError('confident_in_planar_regions runs in libba_hip.so: pass a device tensor')
    if D0.dtype != torch.float32:
        raise ValueError('confident_in_planar_regions: the device version takes fp32 maps')
    x = D0.contiguous()
    out = torch.empty_like(x)
    check(lib().ba_planar_confidence(ptr(x), x.shape[0], x.shape[1], float(alpha), ptr(out), stream_ptr(x.device)))
    return out
