"""F sampling on the device: the multi-depth values of the observations.

Drop-in for ``bilinear_sampling`` (src/blast3r/utils/geometry.py:167-198) and
``gather_data_from_dense_tracks`` (src/blast3r/inference/tracks.py:841-873).  The reference runs
one ``F.grid_sample`` per view; here one launch of ``ba_sample_depth`` (libba_hip.so) samples every
observation of every view, reading each view's map where it lies (no stacked copy of the maps).
The arithmetic is that of torch's CPU ``grid_sample`` (bilinear, padding 'border',
align_corners=False), bit for bit.
"""
import ctypes

import numpy as np
import torch

from ._lib import BaSampleArgs, check, lib, stream_ptr
from .data import ObservedTracks

__all__ = ['prepare_sample', 'sample_depth_maps', 'bilinear_sampling', 'gather_data_from_dense_tracks', 'DEPTH_MODES']

DEPTH_MODES = ('log_multidepth', 'linear_multidepth')


def _map_geometry(m, C):
    """(H, W, pixel stride) of a map whose last dim holds its C channels contiguously."""
    if m.dim() != 3:
        raise ValueError(f'not a multi-depth map: got {m.dim()} dims')
    H, W, Cm = m.shape
    if Cm != C:
        raise ValueError(f'maps have different channel counts ({Cm} vs {C})')
    if C > 1 and m.stride(2) != 1:
        raise ValueError('map channels must be contiguous')
    ps = m.stride(1) if W > 1 else (m.stride(0) if H > 1 else C)
    if ps < C or (H > 1 and m.stride(0) != W * ps):
        raise ValueError('map pixels must be evenly spaced, rows W pixels apart, without overlap')
    return H, W, ps


def prepare_sample(maps, cum_nppi, pix2d, insert_ones=False, out=None):
    """Argument block of ba_sample_depth for sample_depth_maps (same arguments); returns
    (args, out, keep) where keep holds the device tensors args points into."""
    stacked = isinstance(maps, torch.Tensor) and maps.dim() == 4
    if isinstance(maps, torch.Tensor) and not stacked:
        maps = [maps]
    dev = pix2d.device
    if dev.type != 'cuda':
        raise RuntimeError('sample_depth_maps needs device tensors (the sampling runs in libba_hip.so)')
    views = list(maps.unbind(0)) if stacked else list(maps)
    if len(views) == 0:
        raise ValueError('no maps')
    C = views[0].shape[-1]
    for m in views:
        if m.dtype != torch.float32 or m.device != dev:
            raise ValueError('maps must be fp32 tensors on the device of pix2d')
    if stacked:
        geo = [_map_geometry(views[0], C)]
        if len(views) > 1 and maps.stride(0) <= 0:
            raise ValueError('stacked maps need a positive image stride')
    else:
        geo = [_map_geometry(m, C) for m in views]
    pix2d = pix2d.contiguous()
    if pix2d.dtype != torch.float32 or pix2d.dim() != 2 or pix2d.shape[1] != 2:
        raise ValueError('pix2d must be (n_obs, 2) fp32')
    cum_nppi = cum_nppi.to(device=dev, dtype=torch.int32).contiguous()
    if len(cum_nppi) != len(views):
        raise ValueError(f'{len(views)} maps for {len(cum_nppi)} images')
    n_obs = pix2d.shape[0]
    co = C + int(bool(insert_ones))
    if out is None:
        out = torch.empty((n_obs, co), dtype=torch.float32, device=dev)
    elif out.shape != (n_obs, co) or not out.is_contiguous() or out.dtype != torch.float32:
        raise ValueError(f'out must be a contiguous ({n_obs}, {co}) fp32 tensor')
    pss = {g[2] for g in geo}
    if len(pss) != 1:
        raise ValueError('maps must share one pixel stride')
    hw = {(g[0], g[1]) for g in geo}
    if stacked:                                   # image i at base + i * stride, formed on the device
        addr = maps.data_ptr() + torch.arange(len(views), dtype=torch.int64, device=dev) * (maps.stride(0) * 4)
    else:
        addr = torch.tensor([m.data_ptr() for m in views], dtype=torch.int64).to(dev)
    map_hw = None
    if len(hw) > 1:
        map_hw = torch.tensor([[g[0], g[1]] for g in geo], dtype=torch.int32).to(dev)
    H, W = next(iter(hw)) if len(hw) == 1 else (0, 0)
    a = BaSampleArgs(map_addr=addr.data_ptr(), map_hw=None if map_hw is None else map_hw.data_ptr(), H=H, W=W, Cm=C,
                     pix_stride=pss.pop(), insert_ones=int(bool(insert_ones)), cum_nppi=cum_nppi.data_ptr(),
                     n_imgs=len(views), pix2d=pix2d.data_ptr(), n_obs=n_obs, out=out.data_ptr())
    return a, out, (addr, map_hw, cum_nppi, pix2d, maps)


def sample_depth_maps(maps, cum_nppi, pix2d, insert_ones=False, out=None):
    """Bilinear samples of per-image maps at image-major observations.

    maps       list of (H_i, W_i, Cm) fp32 device tensors, one per image, or one (n_imgs, H, W, Cm)
               tensor; channel slices of wider maps (``raw[..., 2:]``) are read in place
    cum_nppi   (n_imgs,) int32 inclusive cumulative observation counts (``infos`` row 0)
    pix2d      (n_obs, 2) fp32 pixel coordinates
    insert_ones  also sample a constant-one channel at output column 1 (the stack of
               src/blast3r/inference/multidepth.py:53-54)
    returns    (n_obs, Cm + insert_ones) fp32
    """
    a, out, keep = prepare_sample(maps, cum_nppi, pix2d, insert_ones, out)
    if a.n_obs > 0:
        check(lib().ba_sample_depth(ctypes.byref(a), stream_ptr(pix2d.device)))
    return out


def bilinear_sampling(depth, pix2d, mode='bilinear', padding_mode='border'):
    """geometry.py:167-198 on the device.

    depth (*B, H, W, C), pix2d (*B, *P, 2) -> (*B, *P, C).  numpy inputs are copied to the current
    GPU and the result comes back as numpy, as the reference returns numpy for numpy inputs.
    Only mode='bilinear' with padding_mode='border' (the reference's defaults, the only ones on
    the BA path) is implemented; other modes raise NotImplementedError.
    """
    if mode != 'bilinear' or padding_mode != 'border':
        raise NotImplementedError(f'bilinear_sampling: only mode=bilinear, padding_mode=border ({mode}, {padding_mode})')
    to_numpy = isinstance(depth, np.ndarray) or isinstance(pix2d, np.ndarray)
    dev = next((t.device for t in (depth, pix2d) if isinstance(t, torch.Tensor) and t.is_cuda),
               torch.device('cuda', torch.cuda.current_device()))
    depth = torch.as_tensor(depth).to(dev, torch.float32)
    pix2d = torch.as_tensor(pix2d).to(dev, torch.float32)
    nb = depth.dim() - 3
    batch_dims = depth.shape[:nb]
    if tuple(depth.shape[:nb]) != tuple(pix2d.shape[:nb]):
        raise ValueError('depth and pix2d must have the same batch dimension')
    B = int(np.prod(batch_dims)) if nb else 1
    pix_shape = pix2d.shape[nb:-1]
    P = int(np.prod(pix_shape)) if len(pix_shape) else 1
    maps = depth.reshape(B, *depth.shape[nb:])
    pts = pix2d.reshape(B * P, 2)
    cum = torch.arange(1, B + 1, dtype=torch.int32, device=dev) * P
    res = sample_depth_maps(maps, cum, pts).view(*batch_dims, *pix_shape, depth.shape[-1])
    return res.cpu().numpy() if to_numpy else res


def gather_data_from_dense_tracks(views, tracks, tracks_std=None, device=None):
    """tracks.py:841-873: ObservedTracks from dense tracks and the views' multi-depth maps.

    tracks (n_tracks, n_views, 2), NaN where a track is not seen.  Observations come out
    image-major with track ids ascending inside an image; ``pix2d_dep`` is sampled from
    ``views[i][depth_mode]`` in one launch.  The result holds device tensors (the BA path's
    input).  As in the reference, passing ``tracks_std`` leaves ``pix2d_std`` as None, which
    ``ObservedTracks`` rejects.
    """
    if device is None:
        cands = [v[k] for v in views[:1] for k in DEPTH_MODES if k in v]
        device = cands[0].device if cands and isinstance(cands[0], torch.Tensor) and cands[0].is_cuda else \
            torch.device('cuda', torch.cuda.current_device())
    tr = torch.as_tensor(tracks).to(device)
    n_tracks, n_views, two = tr.shape
    assert two == 2
    valids = torch.isfinite(tr).all(-1)
    assert bool((valids.sum(1) >= 2).all())
    tr, valids = tr.transpose(0, 1), valids.T
    nppi = valids.sum(1)
    pids = torch.arange(n_tracks, dtype=torch.int32, device=device).expand(n_views, n_tracks)[valids]
    pix2d = tr[valids].to(torch.float32).contiguous()
    pix2d_std = torch.ones_like(pix2d) if tracks_std is None else None
    depth_mode, = [k for k in views[0] if k in DEPTH_MODES]
    maps = []
    for view in views:
        m = torch.as_tensor(view[depth_mode])
        if m.dim() != 3:
            raise AssertionError(f'not a multi-depth: got {m.dim()} dims')
        maps.append(m.to(device, torch.float32))
    pix2d_dep = sample_depth_maps(maps, torch.cumsum(nppi, 0), pix2d)
    return ObservedTracks(n_views, n_tracks, nppi, pids, pix2d, pix2d_std, pix2d_dep, depth_mode)
