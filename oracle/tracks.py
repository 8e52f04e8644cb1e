"""Oracle restatement of the ObservedTracks structure edits (test infrastructure only).

Follows src/blast3r/inference/tracks.py:19-127 on CPU torch, on plain tuples
``(nppi, pids, pix2d, pix2d_std, pix2d_dep)`` of one image-major observation set:

  * ``img_slices`` / ``img_id``   tracks.py:31, :45-54 (delimiters assigned, not added)
  * ``select``                   ``tracks[idx]`` for an index tensor, tracks.py:66-74
  * ``merge``                    ``old | new``, tracks.py:84-102
  * ``to_dense``                 tracks.py:104-114
  * ``remove``                   tracks.py:116-127 (torch.isin, torch.unique + inverse)

Pinned in tests/test_tracks.py by relations that tie the functions to each other
and to closed forms (to_dense of a merge is the two dense arrays side by side,
remove is a column selection of to_dense, img_id against repeat_interleave and a
known answer for empty images, select against one-image views).
"""
import torch


def img_slices(nppi):
    cum = torch.cumsum(nppi.to(torch.int64), -1).tolist()
    return [slice(i, j) for i, j in zip([0] + cum[:-1], cum)]


def img_id(nppi, n_rows):
    """tracks.py:45-49."""
    res = torch.zeros(n_rows, dtype=torch.int32)
    res[torch.cumsum(nppi, -1)[:-1].long()] = 1
    return torch.cumsum(res, -1)


def select(obs, idx):
    """tracks.py:70-74."""
    nppi, pids, pix, std, dep = obs
    sl = img_slices(nppi)
    cat = lambda arr: torch.cat([arr[sl[int(i)]] for i in idx])
    return nppi[idx], cat(pids), cat(pix), cat(std), cat(dep)


def merge(old, n_tracks_old, new):
    """tracks.py:84-102 (old has one image less than new)."""
    nppi_o, pids_o, pix_o, std_o, dep_o = old
    nppi_n, pids_n, pix_n, std_n, dep_n = new
    assert len(nppi_o) + 1 == len(nppi_n)
    nppi = nppi_n.clone()
    nppi[:-1] += nppi_o
    parts = ([], [], [], [])
    for s1, s2 in zip(img_slices(nppi_o) + [slice(0, 0)], img_slices(nppi_n)):
        for k, (a, b) in enumerate(((pids_o, pids_n + n_tracks_old), (pix_o, pix_n), (std_o, std_n), (dep_o, dep_n))):
            parts[k].append(a[s1])
            parts[k].append(b[s2])
    return (nppi,) + tuple(torch.cat(p) for p in parts)


def to_dense(obs, n_tracks, n_imgs=None):
    """tracks.py:104-114: (n_tracks, n_imgs, 2)."""
    nppi, pids, pix = obs[0], obs[1], obs[2]
    n_imgs = len(nppi) if n_imgs is None else n_imgs
    res = torch.full((n_imgs, n_tracks, 2), float('nan'))
    for i, sl in enumerate(img_slices(nppi)):
        res[i, pids[sl].long()] = pix[sl]
    return res.transpose(0, 1)


def remove(obs, bad):
    """tracks.py:116-127: ((nppi, pids, pix, std, dep), old_to_keep)."""
    nppi, pids, pix, std, dep = obs
    bad = torch.as_tensor(bad)
    ok = ~torch.isin(pids, bad)
    nppi2 = torch.tensor([int(ok[sl].sum()) for sl in img_slices(nppi)], dtype=torch.int32)
    old_to_keep, pids2 = torch.unique(pids[ok], return_inverse=True)
    return (nppi2, pids2.int(), pix[ok], std[ok], dep[ok]), old_to_keep
