"""Oracle restatement of the F-sampling step (test infrastructure only).

Restates, in numpy fp32:
  * ``bilinear_sampling`` (src/blast3r/utils/geometry.py:167-198): the pixel (x, y) goes to the
    grid coordinate g = x * fl32(2/W) - 1 (:188; ``pix2d.new([2/imW, 2/imH])`` rounds the Python
    double to fp32; product and difference are separate torch ops, so each rounds), then
    ``F.grid_sample(mode='bilinear', padding_mode='border', align_corners=False)`` (:189-193) maps
    it back to the source index fma(g + 1, W, -1) / 2, clamps it to [0, W-1] and sums the four
    neighbouring texels weighted nw, ne, sw, se in that order with fused multiply-adds, skipping
    corners past the last row or column.  The two fused steps are the roundings of torch's CPU
    grid_sample (fma32 below is an exact single-rounding fma);
  * ``gather_data_from_dense_tracks`` (src/blast3r/inference/tracks.py:841-873): image-major
    observations from dense (n_tracks, n_views, 2) tracks with NaN for "not seen", track ids
    ascending within an image, and the per-view samples concatenated;
  * the channel stack [F0, 1, F1, ...] of src/blast3r/inference/multidepth.py:53-54.

Pinning (tests/test_sampling.py): bit-for-bit equality with torch CPU ``F.grid_sample`` called the
way geometry.py calls it, on random and smooth maps with points inside, on and beyond the border;
fma32 against exact rational arithmetic on cases built to round on a tie; pixel centres of
power-of-two maps return the texel exactly; an affine map is reproduced exactly in the interior
up to fp32 rounding; points beyond the border return the border texel; the layout of
``gather_data_from_dense_tracks`` against a hand-written case.
"""
import numpy as np

__all__ = ['fma32', 'src_index', 'bilinear_sample', 'sample_images', 'stack_log_multidepth', 'dense_tracks_layout']

f32 = np.float32


def fma32(a, b, c):
    """fp32 a*b + c with one rounding (ties to even).

    The fp32 product is exact in fp64; the fp64 sum s is then rounded once more to fp32, which can
    differ from a single rounding only when s falls exactly on an fp32 tie while the exact sum does
    not; that case is detected with the exact error of the fp64 sum (TwoSum) and resolved toward it.
    """
    a, b, c = np.broadcast_arrays(*(np.asarray(x, dtype=f32).astype(np.float64) for x in (a, b, c)))
    p = a * b
    s = p + c
    bp = s - p
    err = (p - (s - bp)) + (c - bp)                     # p + c = s + err exactly
    r = s.astype(f32)
    r64 = r.astype(np.float64)
    other = np.where(s > r64, np.nextafter(r, f32(np.inf)), np.nextafter(r, f32(-np.inf))).astype(np.float64)
    tie = (s == (r64 + other) / 2) & (s != r64) & (err != 0)
    hi, lo = np.maximum(r64, other), np.minimum(r64, other)
    return np.where(tie, np.where(err > 0, hi, lo), r64).astype(f32)


def src_index(pix, size):
    """grid coordinate and grid_sample's unnormalise + border clamp, in fp32."""
    pix = np.asarray(pix, dtype=f32)
    g = pix * f32(2.0 / size) - f32(1)                                  # geometry.py:188
    i = fma32(g + f32(1), f32(size), f32(-1)) * f32(0.5)                # align_corners=False
    return np.fmin(f32(size - 1), np.fmax(i, f32(0)))                   # padding_mode='border'


def bilinear_sample(fmap, pix):
    """fmap (H, W, C) fp32, pix (n, 2) -> (n, C) fp32 (one view of geometry.py:167-198)."""
    fmap = np.asarray(fmap, dtype=f32)
    pix = np.asarray(pix, dtype=f32).reshape(-1, 2)
    H, W, C = fmap.shape
    ix, iy = src_index(pix[:, 0], W), src_index(pix[:, 1], H)
    fx0, fy0 = np.floor(ix), np.floor(iy)
    e, w = (fx0 + f32(1)) - ix, ix - fx0
    s, n = (fy0 + f32(1)) - iy, iy - fy0
    wnw, wne, wsw, wse = e * s, w * s, e * n, w * n
    x0, y0 = fx0.astype(np.int64), fy0.astype(np.int64)
    xin, yin = x0 + 1 < W, y0 + 1 < H
    xe, ys = np.where(xin, x0 + 1, x0), np.where(yin, y0 + 1, y0)
    v = fmap[y0, x0] * wnw[:, None]
    v = np.where(xin[:, None], fma32(fmap[y0, xe], wne[:, None], v), v)
    v = np.where(yin[:, None], fma32(fmap[ys, x0], wsw[:, None], v), v)
    v = np.where((xin & yin)[:, None], fma32(fmap[ys, xe], wse[:, None], v), v)
    return v.astype(f32)


def stack_log_multidepth(raw):
    """multidepth.py:53-54: (H, W, K) -> (H, W, K + 1) with a ones channel at index 1."""
    raw = np.asarray(raw, dtype=f32)
    return np.concatenate((raw[..., :1], np.ones_like(raw[..., :1]), raw[..., 1:]), -1)


def sample_images(maps, nppi, pix2d, insert_ones=False):
    """Image-major samples: observation rows of image i come from maps[i] (tracks.py:865-872)."""
    nppi = np.asarray(nppi, dtype=np.int64)
    pix2d = np.asarray(pix2d, dtype=f32).reshape(-1, 2)
    out, start = [], 0
    for m, cnt in zip(maps, nppi):
        m = stack_log_multidepth(m) if insert_ones else np.asarray(m, dtype=f32)
        out.append(bilinear_sample(m, pix2d[start:start + cnt]))
        start += cnt
    assert start == len(pix2d)
    C = out[0].shape[1] if out else 0
    return np.concatenate(out) if out else np.zeros((0, C), f32)


def dense_tracks_layout(tracks):
    """tracks.py:846-862: (nppi, pids, pix2d) of dense (n_tracks, n_views, 2) tracks, image-major."""
    tracks = np.asarray(tracks)
    n_tracks, n_views, two = tracks.shape
    assert two == 2
    valids = np.isfinite(tracks).all(-1)
    assert (valids.sum(1) >= 2).all()
    tr, va = tracks.swapaxes(0, 1), valids.T
    nppi = va.sum(1)
    pids = np.broadcast_to(np.arange(n_tracks, dtype=np.int32), va.shape)[va]
    return nppi, pids, tr[va]
