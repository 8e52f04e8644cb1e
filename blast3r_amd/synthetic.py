"""Seeded synthetic bundle-adjustment problems in the reference's boundary layout.

Emits exactly the tensors ``lm_step`` receives (src/blast3r/inference/engine.py:206-219):
``infos`` (3, n_imgs) int32 = [inclusive cumsum of per-image counts, node ids,
cam ids] (src/blast3r/inference/rigs.py:50-51), image-major observations with
pid-ascending order inside an image (src/blast3r/inference/tracks.py:856-861),
``P_rig2cam`` as a stride-0 broadcast identity (src/blast3r/inference/rigs.py:231),
``pix2d_std`` = 1 (src/blast3r/inference/tracks.py:862) and the log-depth channel
stack [F0, 1, F1, ..., F_{K-1}] (src/blast3r/inference/multidepth.py:53-54).

Configs (numbering of the benchmark definition):
  0  32 frames, mono focal, circle of radius 3 m looking inward, 20k tracks x U{3..8}
  1  256 frames, smooth trajectory in a 20 m box, 200k tracks x U{3..10} in 24-frame neighbourhoods
  2  1024 frames, forward motion 0.05 m/frame, 1M tracks on contiguous windows U{4..12}
  3  4096 frames, per-frame focal U(350,900), 16 random neighbours, 3M tracks x U{3..12}
  4  config-2 scene, depth stitching: K=8 channels (C=9), omega=1, poses/focal fixed

The smooth channels F1.. are Gaussian random fields (sigma 0.1, correlation
length 32 px) built from random Fourier features on an 8-px lattice and
bilinearly sampled at the observations; channel 0 is the log of the true depth
of the observed point (config 4: with a per-frame affine error).  Every array is
produced on the CPU from ``numpy.random.Generator(PCG64(1000 + cfg))`` so both
sides of a parity test see identical tensors.
"""
from dataclasses import dataclass, field

import numpy as np
import torch

W_IMG, H_IMG = 512, 384


@dataclass
class BAProblem:
    cfg: int
    infos: torch.Tensor          # (3, n_imgs) int32
    K: torch.Tensor              # (n_cams, 3, 3) f32
    P_rig2cam: torch.Tensor      # (n_cams, 4, 4) f32, stride-0 broadcast
    P_w2rig: torch.Tensor        # (n_nodes, 4, 4) f32 (initial, perturbed)
    z_coefs: torch.Tensor        # (n_imgs, C) f32
    pts3d: torch.Tensor          # (n_tracks, 3) f32 (initial, perturbed)
    pids: torch.Tensor           # (n_obs,) int32
    pix2d: torch.Tensor          # (n_obs, 2) f32
    pix2d_std: torch.Tensor      # (n_obs, 2) f32
    pix2d_dep: torch.Tensor      # (n_obs, C) f32
    options: dict = field(default_factory=dict)
    truth: dict = field(default_factory=dict)

    @property
    def n_obs(self):
        return int(self.pids.shape[0])

    @property
    def n_tracks(self):
        return int(self.pts3d.shape[0])

    @property
    def n_imgs(self):
        return int(self.infos.shape[1])

    @property
    def C(self):
        return int(self.pix2d_dep.shape[1])

    def lm_inputs(self):
        """Positional/keyword arguments of ``lm_step`` in the reference order."""
        return dict(rigs=self.infos, pids=self.pids, pix2d=self.pix2d, pix2d_std=self.pix2d_std,
                    pix2d_dep=self.pix2d_dep, K=self.K, P_rig2cam=self.P_rig2cam, P_w2rig=self.P_w2rig,
                    z_coefs=self.z_coefs, pts3d=self.pts3d)

    def to(self, device):
        def mv(t):
            if t.stride(0) == 0:
                return t[:1].contiguous().to(device).expand(t.shape)
            return t.to(device)
        return BAProblem(self.cfg, *(mv(getattr(self, k)) for k in
                                     ('infos', 'K', 'P_rig2cam', 'P_w2rig', 'z_coefs', 'pts3d', 'pids', 'pix2d',
                                      'pix2d_std', 'pix2d_dep')), dict(self.options), dict(self.truth))


# ----------------------------------------------------------------------------- geometry helpers

def _rodrigues(w):
    """(n,3) axis-angle -> (n,3,3) rotation matrices, fp64."""
    th = np.linalg.norm(w, axis=1, keepdims=True)
    k = np.where(th > 1e-12, w / np.maximum(th, 1e-12), 0.0)
    Kx = np.zeros((len(w), 3, 3))
    Kx[:, 0, 1], Kx[:, 0, 2] = -k[:, 2], k[:, 1]
    Kx[:, 1, 0], Kx[:, 1, 2] = k[:, 2], -k[:, 0]
    Kx[:, 2, 0], Kx[:, 2, 1] = -k[:, 1], k[:, 0]
    s, c = np.sin(th)[:, :, None], np.cos(th)[:, :, None]
    return np.eye(3)[None] + s * Kx + (1 - c) * (Kx @ Kx)


def _look_at(centers, targets, up=np.array([0.0, -1.0, 0.0])):
    """World-to-camera rotations (camera z toward target, y down in image)."""
    z = targets - centers
    z /= np.linalg.norm(z, axis=1, keepdims=True)
    x = np.cross(-up[None], z)
    bad = np.linalg.norm(x, axis=1) < 1e-6
    x[bad] = np.cross(np.array([1.0, 0.0, 0.0]), z[bad])
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    y = np.cross(z, x)
    return np.stack([x, y, z], axis=1)          # rows = camera axes in world coords


def _w2c(R, centers):
    P = np.tile(np.eye(4), (len(R), 1, 1))
    P[:, :3, :3] = R
    P[:, :3, 3] = -np.einsum('nij,nj->ni', R, centers)
    return P


def _project(P, f, X):
    """P (n,4,4) world-to-cam, f (n,), X (n,3) -> pixels (n,2), depth (n,)."""
    Xc = np.einsum('nij,nj->ni', P[:, :3, :3], X) + P[:, :3, 3]
    z = Xc[:, 2]
    zs = np.where(np.abs(z) > 1e-9, z, 1e-9)
    u = f * Xc[:, 0] / zs + W_IMG / 2
    v = f * Xc[:, 1] / zs + H_IMG / 2
    return np.stack([u, v], 1), z


def _visible(uv, z, margin=0.0):
    return (z > 0.1) & (uv[:, 0] >= margin) & (uv[:, 0] < W_IMG - margin) & \
           (uv[:, 1] >= margin) & (uv[:, 1] < H_IMG - margin)


def _backproject(P, f, uv, depth):
    xc = np.stack([(uv[:, 0] - W_IMG / 2) / f * depth, (uv[:, 1] - H_IMG / 2) / f * depth, depth], 1)
    R, t = P[:, :3, :3], P[:, :3, 3]
    return np.einsum('nji,nj->ni', R, xc - t)


# ----------------------------------------------------------------------------- random fields

class _FieldBank:
    """Per (frame, channel) smooth Gaussian random field, sigma 0.1, correlation length 32 px.

    Random Fourier features of the squared-exponential kernel evaluated on an
    8-px lattice, then bilinear interpolation (half-pixel centres, border clamp).
    """
    STRIDE = 8
    N_FEAT = 32

    def __init__(self, rng, n_frames, n_ch, sigma=0.1, ell=32.0):
        gh, gw = H_IMG // self.STRIDE, W_IMG // self.STRIDE
        ys = (np.arange(gh) + 0.5) * self.STRIDE
        xs = (np.arange(gw) + 0.5) * self.STRIDE
        self.grid = np.zeros((n_frames, n_ch, gh, gw), dtype=np.float32)
        for f0 in range(0, n_frames, 64):
            f1 = min(n_frames, f0 + 64)
            om = rng.normal(0.0, 1.0 / ell, size=(f1 - f0, n_ch, self.N_FEAT, 2))
            ph = rng.uniform(0, 2 * np.pi, size=(f1 - f0, n_ch, self.N_FEAT))
            # cos(w_x x + w_y y + ph) on the separable lattice = Re(e^{i (w_y y + ph)} e^{i w_x x}):
            # a sum over features of outer products, one complex matrix product per (frame, channel)
            ey = np.exp(1j * (om[..., 1, None] * ys + ph[..., None]))          # (f, c, r, gh)
            ex = np.exp(1j * (om[..., 0, None] * xs))                           # (f, c, r, gw)
            val = sigma * np.sqrt(2.0 / self.N_FEAT) * np.matmul(ey.transpose(0, 1, 3, 2), ex).real
            self.grid[f0:f1] = val.astype(np.float32)
        self.gh, self.gw = gh, gw
        self.grid_hwc = np.ascontiguousarray(self.grid.transpose(0, 2, 3, 1))   # channel-last for gathers

    def sample(self, frame, uv):
        """Bilinear sample of every channel at pixels uv (n,2) of frames (n,) -> (n, n_ch)."""
        x = uv[:, 0] / self.STRIDE - 0.5
        y = uv[:, 1] / self.STRIDE - 0.5
        x = np.clip(x, 0, self.gw - 1)
        y = np.clip(y, 0, self.gh - 1)
        x0 = np.minimum(np.floor(x).astype(np.int64), self.gw - 2)
        y0 = np.minimum(np.floor(y).astype(np.int64), self.gh - 2)
        ax = (x - x0)[:, None]
        ay = (y - y0)[:, None]
        g = self.grid_hwc
        v00 = g[frame, y0, x0]
        v01 = g[frame, y0, x0 + 1]
        v10 = g[frame, y0 + 1, x0]
        v11 = g[frame, y0 + 1, x0 + 1]
        return ((1 - ay) * ((1 - ax) * v00 + ax * v01) + ay * ((1 - ax) * v10 + ax * v11)).astype(np.float32)


# ----------------------------------------------------------------------------- scenes

_SPEC = {
    0: dict(F=32, T=20_000, mmin=3, mmax=8, outl=0.10, KF=4, mono=True),
    1: dict(F=256, T=200_000, mmin=3, mmax=10, outl=0.05, KF=4, mono=True),
    2: dict(F=1024, T=1_000_000, mmin=4, mmax=12, outl=0.08, KF=4, mono=True),
    3: dict(F=4096, T=3_000_000, mmin=3, mmax=12, outl=0.10, KF=4, mono=False),
    4: dict(F=1024, T=1_000_000, mmin=4, mmax=12, outl=0.08, KF=8, mono=True),
}


def _scene_circle(rng, F):
    th = 2 * np.pi * np.arange(F) / F
    C = np.stack([3 * np.cos(th), rng.normal(0, 0.1, F), 3 * np.sin(th)], 1)
    R = _look_at(C, np.zeros_like(C))
    R = _rodrigues(rng.normal(0, np.deg2rad(5.0) / np.sqrt(3), (F, 3))) @ R
    return _w2c(R, C)


def _scene_smooth(rng, F, box=20.0):
    """Smooth random trajectory in a box; a scaled-down problem is a prefix of the 256-frame path."""
    Fn = max(F, 256)
    t = np.arange(Fn) / 255.0
    C = np.zeros((Fn, 3))
    for k in range(3):
        a = rng.normal(0, 1, 4)
        ph = rng.uniform(0, 2 * np.pi, 4)
        C[:, k] = sum(a[j] * np.sin(2 * np.pi * (j + 1) * t + ph[j]) for j in range(4))
    C -= C.min(0)
    C *= (box * 0.6) / np.maximum(C.max(0), 1e-9)
    C += box * 0.2
    tang = np.gradient(C, axis=0)
    yaw = rng.normal(0, 0.3, 1) + 0.5 * np.sin(2 * np.pi * t * 3)
    dirn = tang / np.linalg.norm(tang, axis=1, keepdims=True)
    dirn = dirn + 0.5 * np.stack([np.cos(yaw), np.zeros_like(yaw), np.sin(yaw)], 1)
    C, dirn = C[:F], dirn[:F]
    R = _look_at(C, C + dirn)
    return _w2c(R, C)


def _scene_forward(rng, F, step=0.05):
    t = np.arange(F)
    C = np.stack([0.5 * np.sin(2 * np.pi * t / 400.0), 0.1 * np.sin(2 * np.pi * t / 170.0), step * t], 1)
    d = np.stack([0.05 * np.cos(2 * np.pi * t / 300.0), np.zeros(F), np.ones(F)], 1)
    R = _look_at(C, C + d)
    return _w2c(R, C)


def _scene_sphere(rng, F, radius=4.0):
    v = rng.normal(0, 1, (F, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    C = radius * v
    R = _look_at(C, np.zeros_like(C))
    R = _rodrigues(np.concatenate([np.zeros((F, 2)), rng.uniform(-np.pi, np.pi, (F, 1))], 1)) @ R
    return _w2c(R, C)


def _sample_tracks(rng, cfg, P, f_img, T, mmin, mmax, neigh=None):
    """Return (frame per obs, track id per obs, world points (T,3)), rejection-sampled in batches."""
    F = len(P)
    m = rng.integers(mmin, mmax + 1, size=T)
    X = np.zeros((T, 3))
    frames_of = np.full((T, mmax), -1, dtype=np.int64)
    todo = np.arange(T)
    for _ in range(400):
        if not len(todo):
            break
        sel = todo[:2_000_000]
        n = len(sel)
        mt = m[sel]
        if cfg in (2, 4):
            start = rng.integers(0, F - mt + 1)
            center = start + mt // 2
            depth = rng.uniform(2.0, 30.0, n)
            uv = np.stack([rng.uniform(32, W_IMG - 32, n), rng.uniform(32, H_IMG - 32, n)], 1)
            Xn = _backproject(P[center], f_img[center], uv, depth)
            cand = np.minimum(start[:, None] + np.arange(mmax)[None], F - 1)
        elif cfg == 0:
            Xn = rng.uniform(-2, 2, (n, 3))
            cand = np.tile(np.arange(F), (n, 1))
        elif cfg == 1:
            center = rng.integers(0, F, n)
            depth = rng.uniform(2.0, 15.0, n)
            uv = np.stack([rng.uniform(0, W_IMG, n), rng.uniform(0, H_IMG, n)], 1)
            Xn = _backproject(P[center], f_img[center], uv, depth)
            lo = np.clip(center - 12, 0, max(F - 24, 0))
            cand = np.minimum(lo[:, None] + np.arange(min(24, F))[None], F - 1)
        else:
            seedf = rng.integers(0, F, n)
            Xn = rng.normal(0, 0.5, (n, 3))
            cand = np.concatenate([seedf[:, None], neigh[seedf]], 1)
        Kc = cand.shape[1]
        uvk, zk = _project(P[cand.ravel()], f_img[cand.ravel()], np.repeat(Xn, Kc, 0))
        vis = _visible(uvk, zk, 1.0).reshape(n, Kc)
        if cfg in (2, 4):
            need = np.arange(mmax)[None] < mt[:, None]
            ok = (vis | ~need).all(1)
            chosen = np.where(need, cand, -1)
        else:
            keys = rng.random((n, Kc))
            keys[~vis] = 2.0
            order = np.argsort(keys, 1)[:, :mmax]
            pick = np.take_along_axis(cand, order, 1)
            need = np.arange(mmax)[None] < mt[:, None]
            ok = vis.sum(1) >= mt
            chosen = np.where(need, pick, -1)
        good = sel[ok]
        X[good] = Xn[ok]
        frames_of[good] = chosen[ok]
        todo = np.concatenate([sel[~ok], todo[2_000_000:]])
    if len(todo):
        raise RuntimeError('synthetic track sampling did not converge')
    frames_of = np.sort(np.where(frames_of < 0, np.iinfo(np.int64).max, frames_of), 1)
    valid = frames_of != np.iinfo(np.int64).max
    frames = frames_of[valid]
    tids = np.repeat(np.arange(T), valid.sum(1))
    return frames, tids, X


def make_problem(cfg=0, n_frames=None, n_tracks=None, seed=None, huber_delta=2.0, dtype=torch.float32,
                 n_channels=None, track_len=None, depth_mode='log'):
    """Build one benchmark configuration (optionally scaled down in frames/tracks).  n_channels (K_F,
    giving C = K_F + 1 z-coefficients) and track_len (min, max images per track) override the
    configuration's own values, for the wide and long-track cases of the tests.  depth_mode='lin'
    gives linear depth channels (the reference's 'lin' mode, r2 = fbar log(g / z), which has no ones
    channel, multidepth.py:53-54): channel 0 the depth (for config 4 with the per-frame error applied
    in log space), the others the random fields, with the same C columns."""
    assert depth_mode in ('log', 'lin')
    spec = dict(_SPEC[cfg])
    if n_channels is not None:
        spec['KF'] = int(n_channels)
    if track_len is not None:
        spec['mmin'], spec['mmax'] = int(track_len[0]), int(track_len[1])
    F = int(n_frames or spec['F'])
    T = int(n_tracks or spec['T'])
    rng = np.random.Generator(np.random.PCG64(1000 + cfg if seed is None else seed))
    neigh = None
    if cfg == 0:
        P = _scene_circle(rng, F)
    elif cfg == 1:
        P = _scene_smooth(rng, F)
    elif cfg in (2, 4):
        P = _scene_forward(rng, F)
    else:
        P = _scene_sphere(rng, F)
        neigh = np.stack([rng.choice(np.delete(np.arange(F), i), size=min(16, F - 1), replace=False)
                           for i in range(F)])
    if spec['mono']:
        f_cam = np.array([rng.uniform(400, 800)])
        f_img = np.repeat(f_cam, F)
    else:
        f_cam = rng.uniform(350, 900, F)
        f_img = f_cam
    mmax = min(spec['mmax'], F)
    mmin = min(spec['mmin'], mmax)
    frames, tids, X = _sample_tracks(rng, cfg, P, f_img, T, mmin, mmax, neigh)

    # image-major order, pid ascending inside an image
    order = np.lexsort((tids, frames))
    frames, tids = frames[order], tids[order]
    N = len(frames)
    uv, z = _project(P[frames], f_img[frames], X[tids])
    pix = uv + rng.normal(0, 1.0, (N, 2))
    outl = rng.random(N) < spec['outl']
    pix[outl] = np.stack([rng.uniform(0, W_IMG, outl.sum()), rng.uniform(0, H_IMG, outl.sum())], 1)

    KF = spec['KF']
    C = KF + 1
    fields = _FieldBank(rng, F, KF - 1 + (depth_mode == 'lin'))     # lin: no ones channel, one more field
    dep = np.zeros((N, C), dtype=np.float32)
    logz = np.log(np.maximum(z, 1e-6))
    if cfg == 4:
        a = rng.normal(1.0, 0.1, F)
        b = rng.normal(0.0, 0.2, F)
        logz = a[frames] * logz + b[frames]
    smp = fields.sample(frames, np.clip(pix, 0, [W_IMG - 1e-3, H_IMG - 1e-3]))
    if depth_mode == 'log':
        dep[:, 0] = logz
        dep[:, 1] = 1.0
        dep[:, 2:] = smp
    else:
        dep[:, 0] = np.exp(logz)
        dep[:, 1:] = smp

    nppi = np.bincount(frames, minlength=F)
    n_cams = 1 if spec['mono'] else F
    infos = np.stack([np.cumsum(nppi), np.arange(F), np.zeros(F) if spec['mono'] else np.arange(F)]).astype(np.int32)

    # initial values
    fixed_cams = cfg == 4
    if fixed_cams:
        P0 = P.copy()
        f0 = f_cam.copy()
    else:
        dR = _rodrigues(rng.normal(0, 0.1 / np.sqrt(3), (F, 3)))
        P0 = P.copy()
        P0[:, :3, :3] = dR @ P[:, :3, :3]
        P0[:, :3, 3] = P[:, :3, 3] + rng.normal(0, 0.2 / np.sqrt(3), (F, 3))
        P0[0] = P[0]
        f0 = f_cam * (1.0 + rng.normal(0, 0.02, len(f_cam)))
    X0 = X + rng.normal(0, 0.05, X.shape)
    Kmat = np.zeros((n_cams, 3, 3))
    Kmat[:, 0, 0] = f0
    Kmat[:, 1, 1] = f0
    Kmat[:, 0, 2] = W_IMG / 2
    Kmat[:, 1, 2] = H_IMG / 2
    Kmat[:, 2, 2] = 1
    zc = np.zeros((F, C), dtype=np.float32)
    zc[:, 0] = 1.0

    t32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    options = dict(weight_z=(1.0 if cfg == 4 else 1e-4), huber_delta=huber_delta, pnorm=1.0,
                   clip_pix_err=100.0, optim_K=not fixed_cams, optim_P=not fixed_cams, optim_Z=True,
                   optim_X=True, depth_mode=depth_mode)
    truth = dict(P_w2rig=t32(P), pts3d=t32(X), f=t32(f_cam), frames=torch.from_numpy(frames.astype(np.int64)))
    return BAProblem(cfg=cfg,
                     infos=torch.from_numpy(infos),
                     K=t32(Kmat),
                     P_rig2cam=torch.eye(4).view(1, 4, 4).expand(n_cams, 4, 4),
                     P_w2rig=t32(P0),
                     z_coefs=t32(zc),
                     pts3d=t32(X0),
                     pids=torch.from_numpy(tids.astype(np.int32)),
                     pix2d=t32(pix),
                     pix2d_std=torch.ones((N, 2), dtype=torch.float32),
                     pix2d_dep=torch.from_numpy(dep),
                     options=options, truth=truth)
