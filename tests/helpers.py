"""Shared helpers for the test suite (tolerances are stated where they are used)."""
import torch

from blast3r_amd.synthetic import make_problem


def rel_err(a, b):
    """Norm-wise relative error ||a - b|| / ||b|| in fp64."""
    a = a.detach().to('cpu', torch.float64)
    b = b.detach().to('cpu', torch.float64)
    den = b.norm()
    return float((a - b).norm() / den) if den > 0 else float((a - b).norm())


def tiny_problem(cfg=0, n_frames=6, n_tracks=60, seed=None):
    return make_problem(cfg, n_frames=n_frames, n_tracks=n_tracks, seed=seed)


def opts(p):
    o = p.options
    return dict(weight_z=o['weight_z'], pnorm=o['pnorm'], clip_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
