"""F sampling: oracle pins (CPU) and parity of ba_sample_depth with the oracle (GPU).

The reference samples the multi-depth maps with torch's grid_sample (bilinear, padding 'border',
align_corners=False; src/blast3r/utils/geometry.py:167-198), called once per view by
gather_data_from_dense_tracks (src/blast3r/inference/tracks.py:841-873).

Bars:
  * oracle vs torch CPU grid_sample, called the way geometry.py calls it: bit-for-bit equal;
  * GPU kernel vs oracle: bit-for-bit equal (same fp32 roundings; integer layout work exact);
  * GPU kernel vs torch's grid_sample on the GPU: |diff| <= 1e-5 * max(1, |value|) on smooth maps
    (the north-star fp32 tolerance; torch's GPU build may contract its arithmetic differently).
"""
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sampling as osmp

f32 = np.float32


def torch_reference(fmap, pix):
    """geometry.py:183-196 as the reference evaluates it (torch, here on the CPU)."""
    d = torch.as_tensor(fmap)[None]
    H, W = fmap.shape[:2]
    p = torch.as_tensor(pix).reshape(1, 1, -1, 2)
    grid = p * p.new([2 / W, 2 / H]) - 1
    r = F.grid_sample(d.permute(0, 3, 1, 2), grid.to(d.device), mode='bilinear', padding_mode='border',
                      align_corners=False)
    return r.permute(0, 2, 3, 1).reshape(-1, fmap.shape[2])


def _maps(rng, H, W, C, kind):
    if kind == 'rand':
        return (rng.random((H, W, C), dtype=f32) * 4 - 2).astype(f32)
    if kind == 'int':
        return rng.integers(-8, 8, (H, W, C)).astype(f32)
    y, x = np.mgrid[0:H, 0:W]
    return np.stack([np.sin(x / 17 + c) + np.cos(y / 13 - c) for c in range(C)], -1).astype(f32)


def _points(rng, H, W, n):
    pix = np.stack([rng.uniform(-20, W + 20, n), rng.uniform(-20, H + 20, n)], 1).astype(f32)
    k = max(n // 20, 1)
    pix[:k, 0] = 0
    pix[k:2 * k, 0] = W
    pix[2 * k:3 * k, 1] = H
    pix[3 * k:4 * k] = [W - 0.5, H - 0.5]
    pix[4 * k:8 * k] = np.round(pix[4 * k:8 * k] * 4) / 4          # quarter-pixel lattice
    return pix


# ---------------------------------------------------------------------------------- oracle pins

@pytest.mark.parametrize('H,W,C', [(384, 512, 5), (37, 53, 3), (1, 7, 2), (5, 1, 1), (64, 48, 9)])
@pytest.mark.parametrize('kind', ['rand', 'smooth', 'int'])
def test_oracle_equals_torch_grid_sample(H, W, C, kind):
    rng = np.random.default_rng(H * 1000 + W * 10 + C)
    m = _maps(rng, H, W, C, kind)
    pix = _points(rng, H, W, 4000)
    np.testing.assert_array_equal(osmp.bilinear_sample(m, pix), torch_reference(m, pix).numpy())


def _round_to_f32(q):
    """Correctly rounded (ties to even) fp32 of an exact rational."""
    r = np.float32(float(q))
    cands = [np.nextafter(r, f32(-np.inf)), r, np.nextafter(r, f32(np.inf))]
    dist = [abs(Fraction(float(c)) - q) for c in cands]
    best = min(dist)
    ties = [c for c, dd in zip(cands, dist) if dd == best]
    if len(ties) == 1:
        return ties[0]
    return next(c for c in ties if int(np.array(c).view(np.uint32)) & 1 == 0)


def test_fma32_single_rounding():
    """fma32 rounds once: checked against exact rational arithmetic, including two cases built so
    that rounding the fp64 sum to fp32 would land on a tie the exact sum is not on (A * B = 2^47 + 28
    for the fp32 mantissas A, B below)."""
    A, B = 12041362, 11687838
    assert A * B == 2 ** 47 + 28
    a, b = f32(A * 2.0 ** -48), f32(B * 2.0 ** -23)
    c = f32(1 + 2.0 ** -22)
    cases = [(a, b, c), (-a, b, c), (-a, b, -c), (a, b, -c)]
    rng = np.random.default_rng(5)
    for _ in range(400):
        x, y, z = (f32(v) for v in rng.normal(size=3) * 10.0 ** rng.integers(-6, 6, size=3))
        cases.append((x, y, z))
    for x, y, z in cases:
        exact = Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z))
        assert osmp.fma32(x, y, z) == _round_to_f32(exact), (x, y, z)
    # the two tie cases differ from the naive double rounding
    naive = f32(np.float64(a) * np.float64(b) + np.float64(c))
    assert osmp.fma32(a, b, c) != naive
    assert osmp.fma32(a, b, c) == f32(1 + 3 * 2.0 ** -23)
    assert osmp.fma32(-a, b, c) == f32(1 + 2.0 ** -23)


def test_oracle_pixel_centres_power_of_two():
    """At the centre (j + 0.5, i + 0.5) of a texel of a power-of-two map the sample is the texel."""
    rng = np.random.default_rng(1)
    m = _maps(rng, 64, 128, 4, 'rand')
    i, j = np.meshgrid(np.arange(64), np.arange(128), indexing='ij')
    pix = np.stack([j.ravel() + 0.5, i.ravel() + 0.5], 1).astype(f32)
    np.testing.assert_array_equal(osmp.bilinear_sample(m, pix), m.reshape(-1, 4))


def test_oracle_affine_map_interior():
    """Bilinear interpolation reproduces an affine map v = a + b x + c y (x, y texel coordinates)
    inside the pixel-centre hull, up to fp32 rounding."""
    H, W = 384, 512
    y, x = np.mgrid[0:H, 0:W].astype(np.float64)
    coef = [(0.3, 0.01, -0.02), (-1.0, 0.002, 0.005)]
    m = np.stack([a + b * x + c * y for a, b, c in coef], -1).astype(f32)
    rng = np.random.default_rng(2)
    pix = np.stack([rng.uniform(0.5, W - 0.5, 5000), rng.uniform(0.5, H - 0.5, 5000)], 1).astype(f32)
    got = osmp.bilinear_sample(m, pix).astype(np.float64)
    px, py = pix[:, 0].astype(np.float64) - 0.5, pix[:, 1].astype(np.float64) - 0.5
    want = np.stack([a + b * px + c * py for a, b, c in coef], -1)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)


def test_oracle_border_clamp():
    """Points beyond the map return the nearest border texel (padding_mode='border')."""
    rng = np.random.default_rng(3)
    m = _maps(rng, 8, 16, 3, 'rand')                 # power-of-two sizes: the texel centre 0.5 maps to 0 exactly
    pix = np.array([[-5, -5], [100, -3], [-1, 100], [50, 50], [0.25, 0.5], [16, 0.5]], f32)
    want = np.stack([m[0, 0], m[0, 15], m[7, 0], m[7, 15], m[0, 0], m[0, 15]])
    np.testing.assert_array_equal(osmp.bilinear_sample(m, pix), want)


def test_oracle_dense_tracks_layout():
    """tracks.py:846-862 on a hand-written case: image-major, track ids ascending in an image."""
    nan = np.nan
    tracks = np.array([
        [[1, 2], [3, 4], [nan, nan]],
        [[nan, 0], [5, 6], [7, 8]],
        [[9, 10], [nan, nan], [11, 12]],
    ], np.float32)
    nppi, pids, pix = osmp.dense_tracks_layout(tracks)
    np.testing.assert_array_equal(nppi, [2, 2, 2])
    np.testing.assert_array_equal(pids, [0, 2, 0, 1, 1, 2])
    np.testing.assert_array_equal(pix, [[1, 2], [9, 10], [3, 4], [5, 6], [7, 8], [11, 12]])


def test_oracle_ones_channel_stack():
    raw = np.arange(24, dtype=f32).reshape(2, 3, 4)
    st = osmp.stack_log_multidepth(raw)
    assert st.shape == (2, 3, 5)
    np.testing.assert_array_equal(st[..., 0], raw[..., 0])
    np.testing.assert_array_equal(st[..., 1], 1)
    np.testing.assert_array_equal(st[..., 2:], raw[..., 1:])


# ---------------------------------------------------------------------------------- GPU parity

DEV = 'cuda:0'


def _ragged_case(rng, n_imgs, H, W, C, mean_obs, sizes=None):
    nppi = rng.integers(0, 2 * mean_obs + 1, n_imgs)
    nppi[rng.integers(0, n_imgs)] = 0
    maps, pix = [], []
    for i in range(n_imgs):
        h, w = sizes[i] if sizes is not None else (H, W)
        maps.append(_maps(rng, h, w, C, 'rand'))
        pix.append(_points(rng, h, w, int(nppi[i])) if nppi[i] else np.zeros((0, 2), f32))
    return maps, nppi, np.concatenate(pix)


def _run(maps, nppi, pix, insert_ones=False, dev_maps=None):
    from blast3r_amd.sampling import sample_depth_maps
    dm = dev_maps if dev_maps is not None else [torch.from_numpy(m).to(DEV) for m in maps]
    cum = torch.from_numpy(np.cumsum(nppi)).to(DEV, torch.int32)
    out = sample_depth_maps(dm, cum, torch.from_numpy(pix).to(DEV), insert_ones=insert_ones)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize('C', [1, 3, 4, 5, 9, 16, 17, 24])
@pytest.mark.parametrize('insert_ones', [False, True])
def test_sample_depth_matches_oracle(C, insert_ones):
    print(f'sample_depth C={C} insert_ones={insert_ones}', flush=True)
    rng = np.random.default_rng(100 + C)
    maps, nppi, pix = _ragged_case(rng, 7, 48, 64, C, 300)
    got = _run(maps, nppi, pix, insert_ones)
    want = osmp.sample_images(maps, nppi, pix, insert_ones=insert_ones)
    assert got.shape == want.shape
    np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
def test_sample_depth_per_image_sizes_and_strided_maps():
    print('sample_depth per-image sizes / strided maps', flush=True)
    rng = np.random.default_rng(7)
    sizes = [(30, 40), (1, 9), (17, 1), (64, 48), (5, 5)]
    maps, nppi, pix = _ragged_case(rng, 5, 0, 0, 4, 200, sizes=sizes)
    got = _run(maps, nppi, pix)
    np.testing.assert_array_equal(got, osmp.sample_images(maps, nppi, pix))
    # channel slices of wider maps are read in place (raw[..., 2:] of a 6-channel map)
    wide = [np.concatenate([_maps(rng, 30, 40, 2, 'rand'), m], -1) for m in
            [_maps(rng, 30, 40, 4, 'rand') for _ in range(3)]]
    nppi = np.array([50, 0, 70])
    pix = np.concatenate([_points(rng, 30, 40, n) for n in nppi if n])
    dev = [torch.from_numpy(w).to(DEV)[..., 2:] for w in wide]
    got = _run(None, nppi, pix, insert_ones=True, dev_maps=dev)
    np.testing.assert_array_equal(got, osmp.sample_images([w[..., 2:] for w in wide], nppi, pix, insert_ones=True))


@pytest.mark.gpu
def test_sample_depth_edge_cases():
    print('sample_depth edge cases', flush=True)
    from blast3r_amd.sampling import sample_depth_maps
    m = torch.rand(4, 5, 3, device=DEV)
    empty = sample_depth_maps([m], torch.zeros(1, dtype=torch.int32, device=DEV),
                              torch.zeros((0, 2), device=DEV))
    assert empty.shape == (0, 3)
    # the C ABI rejects bad arguments with an error, before any launch
    import ctypes
    from blast3r_amd._lib import BaSampleArgs, check, lib, stream_ptr
    out = torch.empty((1, 3), device=DEV)
    addr = torch.tensor([m.data_ptr()], dtype=torch.int64, device=DEV)
    cum = torch.ones(1, dtype=torch.int32, device=DEV)
    pix = torch.zeros((1, 2), device=DEV)
    for bad in (dict(insert_ones=2), dict(Cm=0), dict(pix_stride=2), dict(H=0)):
        kw = dict(map_addr=addr.data_ptr(), map_hw=None, H=4, W=5, Cm=3, pix_stride=0, insert_ones=0,
                  cum_nppi=cum.data_ptr(), n_imgs=1, pix2d=pix.data_ptr(), n_obs=1, out=out.data_ptr())
        kw.update(bad)
        with pytest.raises(RuntimeError):
            check(lib().ba_sample_depth(ctypes.byref(BaSampleArgs(**kw)), stream_ptr(DEV)))
    with pytest.raises(ValueError):
        sample_depth_maps([m, torch.rand(4, 5, 2, device=DEV)], torch.ones(2, dtype=torch.int32, device=DEV),
                          torch.zeros((1, 2), device=DEV))
    # one observation in a single-texel map
    one = torch.full((1, 1, 2), 3.5, device=DEV)
    r = sample_depth_maps([one], torch.ones(1, dtype=torch.int32, device=DEV), torch.tensor([[7.0, -2.0]], device=DEV))
    assert r.tolist() == [[3.5, 3.5]]


@pytest.mark.gpu
def test_sample_depth_vs_torch_gpu_grid_sample():
    """Against torch's own grid_sample on the GPU (the call the reference makes)."""
    print('sample_depth vs torch GPU grid_sample', flush=True)
    rng = np.random.default_rng(11)
    m = _maps(rng, 384, 512, 5, 'smooth')
    pix = _points(rng, 384, 512, 20000)
    got = _run([m], np.array([len(pix)]), pix)
    ref = torch_reference(torch.from_numpy(m).to(DEV), torch.from_numpy(pix).to(DEV)).cpu().numpy()
    assert np.all(np.abs(got - ref) <= 1e-5 * np.maximum(1, np.abs(ref)))


@pytest.mark.gpu
def test_bilinear_sampling_api():
    """geometry.py:167-198 interface: batch dims, numpy in -> numpy out."""
    print('bilinear_sampling api', flush=True)
    from blast3r_amd.sampling import bilinear_sampling
    rng = np.random.default_rng(12)
    depth = rng.random((2, 3, 20, 30, 4), dtype=f32)
    pix = _points(rng, 20, 30, 2 * 3 * 7 * 5).reshape(2, 3, 7, 5, 2)
    got = bilinear_sampling(depth, pix)
    assert isinstance(got, np.ndarray) and got.shape == (2, 3, 7, 5, 4)
    for b0 in range(2):
        for b1 in range(3):
            want = osmp.bilinear_sample(depth[b0, b1], pix[b0, b1].reshape(-1, 2)).reshape(7, 5, 4)
            np.testing.assert_array_equal(got[b0, b1], want)
    t = bilinear_sampling(torch.from_numpy(depth[0, 0]).to(DEV), torch.from_numpy(pix[0, 0]).to(DEV))
    assert isinstance(t, torch.Tensor) and t.shape == (7, 5, 4)
    with pytest.raises(NotImplementedError):
        bilinear_sampling(depth, pix, mode='nearest')


@pytest.mark.gpu
def test_gather_data_from_dense_tracks():
    print('gather_data_from_dense_tracks', flush=True)
    from blast3r_amd.sampling import gather_data_from_dense_tracks
    rng = np.random.default_rng(13)
    n_tracks, n_views, H, W = 500, 6, 40, 50
    tracks = np.stack([rng.uniform(0, W, (n_tracks, n_views)), rng.uniform(0, H, (n_tracks, n_views))], -1)
    tracks = tracks.astype(f32)
    hide = rng.random((n_tracks, n_views)) < 0.4
    hide[:, :2] = False                                             # every track seen at least twice
    tracks[hide] = np.nan
    views = [{'log_multidepth': torch.from_numpy(_maps(rng, H, W, 5, 'rand')).to(DEV)} for _ in range(n_views)]
    trk = gather_data_from_dense_tracks(views, tracks)
    nppi, pids, pix = osmp.dense_tracks_layout(tracks)
    np.testing.assert_array_equal(trk.nppi.cpu().numpy(), nppi)
    np.testing.assert_array_equal(trk.pids.cpu().numpy(), pids)
    np.testing.assert_array_equal(trk.pix2d.cpu().numpy(), pix)
    np.testing.assert_array_equal(trk.pix2d_std.cpu().numpy(), np.ones_like(pix))
    want = osmp.sample_images([v['log_multidepth'].cpu().numpy() for v in views], nppi, pix)
    np.testing.assert_array_equal(trk.pix2d_dep.cpu().numpy(), want)
    assert trk.depth_mode == 'log_multidepth'


@pytest.mark.gpu
def test_sample_depth_full_size_config2():
    """Config-2 scale: 1024 maps of 384 x 512 x 5 (4 GB) and ~8M image-major observations.  Every
    row is checked against the oracle on a seeded subset of 40 images (bit-exact), and the ones
    channel of the stacked maps samples to 1 within one rounding everywhere."""
    print('sample_depth full size config 2', flush=True)
    from blast3r_amd.sampling import sample_depth_maps
    g = torch.Generator(device=DEV).manual_seed(21)
    F_, H, W, K = 1024, 384, 512, 4
    maps = torch.rand((F_, H, W, K + 1), device=DEV, generator=g)
    maps[..., 1] = 1.0
    nppi = torch.randint(6000, 9600, (F_,), device=DEV, generator=g)
    n = int(nppi.sum())
    pix = torch.stack([torch.rand(n, device=DEV, generator=g) * (W + 4) - 2,
                       torch.rand(n, device=DEV, generator=g) * (H + 4) - 2], 1)
    cum = torch.cumsum(nppi, 0).to(torch.int32)
    out = sample_depth_maps(maps, cum, pix)
    raw_out = sample_depth_maps(torch.cat([maps[..., :1], maps[..., 2:]], -1), cum, pix, insert_ones=True)
    torch.cuda.synchronize()
    assert torch.equal(out, raw_out)
    assert float((out[:, 1] - 1).abs().max()) <= 1e-6            # four rounded weights summed in fp32
    cum_h = np.concatenate([[0], cum.cpu().numpy()])
    rng = np.random.default_rng(22)
    for i in rng.choice(F_, 40, replace=False):
        s, e = cum_h[i], cum_h[i + 1]
        want = osmp.bilinear_sample(maps[i].cpu().numpy(), pix[s:e].cpu().numpy())
        np.testing.assert_array_equal(out[s:e].cpu().numpy(), want)
