"""Observation-structure plan for the fused kernels (built once, reused every LM iteration).

The reference rebuilds the same structure on every call with bincount /
torch.unique / index_add_ (src/blast3r/inference/ba_solver.py:51-56, :877-909,
:968-974).  Here the native planner in ba_plan.cpp orders tracks, packs them
into 128-observation chunks and groups chunks into batches whose camera-pair
blocks fit one workgroup; the arrays are uploaded once and the per-observation
inputs are permuted into that slot order once per data tensor.
"""
import ctypes
import threading
import weakref

import numpy as np
import torch

from ._lib import check, lib, stream_ptr

# array / scalar ids (ba_plan.h)
ARRAYS = ['chunk_obs', 'chunk_meta', 'slot_info', 'ct_pid', 'ct_first', 'ct_m', 'ct_mask', 'b_chunk_ptr', 'b_imgs',
          'b_nimgs', 'b_slot_ptr', 'slot_pair', 'slot_gpair', 'pair_i1', 'pair_i2', 'pair_ptr', 'pair_src',
          'row_ptr', 'row_ent', 'img_ptr', 'img_src', 'chunk_slots', 'chunk_ent', 'chunk_eptr',
          'b_pos_slot', 'slot_src', 's_pid', 's_img', 'b_order']
SCALARS = ['n_chunks', 'n_batches', 'n_slots', 'n_pairs', 'n_ctracks', 'L', 'chunk', 'max_slots_used',
           'max_chunks_per_batch', 'n_pair_terms']
CHUNK = 128
MAX_LOCAL = 16
_append_lock = threading.Lock()
MAX_SLOTS = 96


class _HostArrays:
    """A plan's arrays on the host, exported on first use (from the host plan while it lives, else from
    the device)."""

    def __init__(self, plan):
        self._plan = weakref.ref(plan)
        self._d = {}

    def __getitem__(self, name):
        if name not in self._d:
            pl = self._plan()
            n = pl.sizes[name]
            # an append (another thread) edits the host plan in place and then takes it from this plan:
            # read it under the same lock, or from the device once it is gone
            arr = None
            with _append_lock:
                if pl._h:
                    arr = pl._host_view(ARRAYS.index(name), n).copy()
            self._d[name] = arr if arr is not None else pl.dev[name][:n].cpu().numpy()
        return self._d[name]

    def __contains__(self, name):
        return name in ARRAYS

    def keys(self):
        return list(ARRAYS)


class BAPlan:
    """Device-resident plan for one (infos, pids) structure.  The host planner's state is kept (`_h`) so
    that the structure `old | new` can be planned from this one (BAPlan.appended), until that is done once."""
    kind = 'batched'

    def __init__(self, infos, pids, n_tracks, device=None, max_local_imgs=MAX_LOCAL, max_slots=MAX_SLOTS,
                 max_batch_obs=0, _parent=None, _chain=None):
        device = device or pids.device
        cum = np.ascontiguousarray(infos[0].detach().cpu().numpy().astype(np.int32, copy=False))
        self.node_ids = np.ascontiguousarray(infos[1].detach().cpu().numpy().astype(np.int64))
        self.cam_ids = np.ascontiguousarray(infos[2].detach().cpu().numpy().astype(np.int64))
        self.n_imgs = int(cum.shape[0])
        self.n_obs = int(pids.shape[0])
        self.n_tracks = int(n_tracks)
        self.options = dict(max_local_imgs=int(max_local_imgs), max_slots=int(max_slots), max_batch_obs=int(max_batch_obs))
        L = lib()
        if _parent is None:
            p = np.ascontiguousarray(pids.detach().cpu().numpy().astype(np.int32, copy=False))
            h = L.ba_plan_create(cum.ctypes.data_as(ctypes.c_void_p), self.n_imgs, p.ctypes.data_as(ctypes.c_void_p),
                                 self.n_obs, self.n_tracks, int(max_local_imgs), int(max_slots), int(max_batch_obs))
        else:
            # one append per link of the chain (each consumes the previous host plan); the parent's device
            # arrays serve the final plan: per array the shortest stable prefix, per image the summed id shift
            if self.n_imgs != _parent.n_imgs + len(_chain) or \
                    any(len(c) != _parent.n_imgs + q + 1 for q, (c, _, _) in enumerate(_chain)):
                raise RuntimeError('structure plan failed: not an append (each link adds one image)')
            h = _parent._h
            stable = np.full(len(ARRAYS), np.iinfo(np.int64).max, dtype=np.int64)
            shift = np.zeros(max(self.n_imgs, 1), dtype=np.int32)
            n_im = _parent.n_imgs
            for q, (add_cnt, add_pids, n_tr) in enumerate(_chain):
                n_im += 1
                h2 = L.ba_plan_append(ctypes.c_void_p(h), add_cnt.ctypes.data_as(ctypes.c_void_p), n_im,
                                      add_pids.ctypes.data_as(ctypes.c_void_p), int(add_pids.shape[0]), int(n_tr))
                if not h2:
                    # a failed append leaves its input as it was: at q == 0 that is the parent's host plan,
                    # which stays appendable; later, an intermediate plan that only this chain holds
                    if q:
                        L.ba_plan_destroy(ctypes.c_void_p(h))
                    raise RuntimeError('structure plan failed: ' + (L.ba_plan_last_error() or b'').decode())
                _parent._h = None if q == 0 else _parent._h       # consumed by ba_plan_append
                h = h2
                st = np.zeros(len(ARRAYS), dtype=np.int64)
                sh = np.zeros(n_im, dtype=np.int32)
                check(L.ba_plan_stable(h, st.ctypes.data_as(ctypes.c_void_p), sh.ctypes.data_as(ctypes.c_void_p)))
                stable = np.minimum(stable, st)
                shift[:n_im] += sh[:n_im]
        if not h:
            raise RuntimeError('structure plan failed: ' + (L.ba_plan_last_error() or b'').decode())
        self._h = h
        sc = np.zeros(len(SCALARS), dtype=np.int64)
        sz = np.zeros(len(ARRAYS), dtype=np.int64)
        check(L.ba_plan_query(h, sc.ctypes.data_as(ctypes.c_void_p), sz.ctypes.data_as(ctypes.c_void_p)))
        self.scalars = {k: int(v) for k, v in zip(SCALARS, sc)}
        if _parent is None:
            stable = np.zeros(len(ARRAYS), dtype=np.int64)
            shift = np.zeros(max(self.n_imgs, 1), dtype=np.int32)
        self.device = torch.device(device)
        self.dev = {}
        self.sizes = {name: int(sz[i]) for i, name in enumerate(ARRAYS)}
        for i, name in enumerate(ARRAYS):
            n, keep = int(sz[i]), int(stable[i]) if _parent is not None else 0
            host = self._host_view(i, n)
            t = torch.empty(max(n, 1), dtype=torch.int32, device=self.device)
            if n == 0:
                t.zero_()                      # never hand a null pointer to a kernel for an empty array
            if keep:
                t[:keep].copy_(_parent.dev[name][:keep])
            if n > keep:
                t[keep:n].copy_(torch.from_numpy(host[keep:n]))
            self.dev[name] = t[:n] if n else t
        if _parent is not None and shift.any():
            # the kept chunks' observation ids, brought to the merged structure's numbering
            sh = torch.from_numpy(shift).to(self.device)
            for name in ('chunk_obs', 'slot_src'):
                keep = int(stable[ARRAYS.index(name)])
                if self.device.type == 'cuda':
                    check(L.ba_plan_shift_ids(ctypes.c_void_p(self.dev[name].data_ptr()),
                                              ctypes.c_void_p(self.dev['s_img'].data_ptr()),
                                              ctypes.c_void_p(sh.data_ptr()), keep, stream_ptr(self.device)))
                else:
                    self.dev[name][:keep] += sh[self.dev['s_img'][:keep].long()]
        self.stable_prefix = {name: int(stable[i]) for i, name in enumerate(ARRAYS)} if _parent is not None else None
        self.host = _HostArrays(self)
        self.L = int(max_local_imgs)
        self._cum = cum
        self.slot_index = self.dev['slot_src'] if self.sizes['slot_src'] else self.dev['slot_src'][:0]
        self._slot_cache = {}
        self._ws = {}
        self.workspace_cache = {}      # derived per-structure arrays (e.g. each image's diagonal block)

    def _host_view(self, which, n):
        """Array `which` of the host plan, in place (numpy view; valid while the host plan lives)."""
        if n == 0:
            return np.zeros(0, dtype=np.int32)
        addr = lib().ba_plan_array(ctypes.c_void_p(self._h), which)
        return np.ctypeslib.as_array((ctypes.c_int32 * n).from_address(addr))

    @property
    def appendable(self):
        return self._h is not None

    @classmethod
    def appended(cls, parent, infos, pids, n_tracks, add_cnt, add_pids):
        """Plan of `parent`'s structure with one image and new tracks appended (`old | new`): add_cnt
        (n_imgs + 1,) new observations per image, add_pids their track ids, image by image.  Equal to
        BAPlan(infos, pids, n_tracks), array for array; consumes the parent's host state."""
        return cls.appended_chain(parent, infos, pids, n_tracks, [(add_cnt, add_pids, n_tracks)])

    @classmethod
    def appended_chain(cls, parent, infos, pids, n_tracks, links):
        """As appended, over several appends in a row (`((old | a) | b) | ...`): links lists, oldest first,
        each append's (add_cnt, add_pids, n_tracks after it)."""
        chain = [(np.ascontiguousarray(c, dtype=np.int32), np.ascontiguousarray(p, dtype=np.int32), int(t))
                 for c, p, t in links]
        with _append_lock:             # ba_plan_append consumes the parent's host plan: one append at a time
            if parent._h is None:
                raise RuntimeError('the parent plan was already appended to')
            return cls(infos, pids, n_tracks, device=parent.device, _parent=parent, _chain=chain, **parent.options)

    def __del__(self):
        h, self._h = getattr(self, '_h', None), None
        if h:
            try:
                lib().ba_plan_destroy(ctypes.c_void_p(h))
            except Exception:
                pass

    @property
    def obs_img(self):
        """Image of every observation (host array)."""
        counts = np.diff(np.concatenate([[0], self._cum.astype(np.int64)]))
        return np.repeat(np.arange(self.n_imgs, dtype=np.int32), counts)

    # ------------------------------------------------------------------ data
    def slot_data(self, pix2d, pix2d_std, pix2d_dep):
        """pix2d, pix2d_std, pix2d_dep permuted into slot order (cached per tensor version)."""
        # identity by weak reference (a new tensor may reuse a freed one's address with version 0)
        ts = (pix2d, pix2d_std, pix2d_dep)
        key = tuple((t._version, tuple(t.shape), t.data_ptr()) for t in ts)
        refs = self._slot_cache.get('refs')
        if refs is not None and self._slot_cache['key'] == key and all(r() is t for r, t in zip(refs, ts)):
            return self._slot_cache['val']
        if self.slot_index.numel():
            val = (pix2d.index_select(0, self.slot_index).contiguous(),
                   pix2d_std.index_select(0, self.slot_index).contiguous(),
                   pix2d_dep.index_select(0, self.slot_index).contiguous())
        else:
            val = (torch.zeros((1, 2), device=self.device), torch.ones((1, 2), device=self.device),
                   torch.zeros((1, max(1, pix2d_dep.shape[1])), device=self.device))
        self._slot_cache = {'key': key, 'refs': tuple(weakref.ref(t) for t in ts), 'val': val}
        return val

    def workspace(self, name, shape, dtype):
        t = self._ws.get(name)
        n = int(np.prod(shape)) if len(shape) else 1
        if t is None or t.numel() < max(n, 1) or t.dtype != dtype:
            t = torch.empty(max(n, 1), dtype=dtype, device=self.device)
            self._ws[name] = t
        return t[:n].view(shape) if n else t[:0]


PM_ARRAYS = ['run_ptr', 'run_obs', 'run_trk', 'run_img', 'img_run_ptr', 'trk_run_ptr', 'trk_run', 'trk_obs_ptr',
             'trk_obs', 'obs_img', 'pair_i1', 'pair_i2', 'row_ptr', 'row_ent', 'diag_pair', 'term_ptr', 'term',
             'pair_sched']
PM_SCALARS = ['n_runs', 'n_pairs', 'n_terms', 'max_terms', 'max_track_runs']


class _DeviceArrays:
    """A plan's arrays on the host, copied from its device arrays on first use."""

    def __init__(self, plan):
        self._plan = weakref.ref(plan)
        self._d = {}

    def __getitem__(self, name):
        if name not in self._d:
            pl = self._plan()
            self._d[name] = pl.dev[name][:pl.sizes[name]].cpu().numpy()
        return self._d[name]

    def __contains__(self, name):
        return name in PM_ARRAYS

    def keys(self):
        return list(PM_ARRAYS)


class PMPlan:
    """Device-resident pair-major plan for one (infos, pids) structure: runs (the observations of one track
    in one image), the tracks' runs and observations in image order, and the image pairs with their (run,
    run) terms.  No limit on track length or co-visibility.  Built on the GPU for CUDA inputs
    (ba_pm_dplan_create), on the host otherwise (ba_pm_plan_create, host_planner=True forces it); the two
    give the same arrays."""
    kind = 'pairmajor'

    def __init__(self, infos, pids, n_tracks, device=None, host_planner=False):
        device = torch.device(device or pids.device)
        self.node_ids = np.ascontiguousarray(infos[1].detach().cpu().numpy().astype(np.int64))
        self.cam_ids = np.ascontiguousarray(infos[2].detach().cpu().numpy().astype(np.int64))
        self.n_imgs = int(infos.shape[1])
        self.n_obs = int(pids.shape[0])
        self.n_tracks = int(n_tracks)
        self.device = device
        self._ws = {}
        self.workspace_cache = {}
        if device.type == 'cuda' and not host_planner:
            self._build_on_device(infos, pids)
            return
        cum = np.ascontiguousarray(infos[0].detach().cpu().numpy().astype(np.int32, copy=False))
        p = np.ascontiguousarray(pids.detach().cpu().numpy().astype(np.int32, copy=False))
        L = lib()
        h = L.ba_pm_plan_create(cum.ctypes.data_as(ctypes.c_void_p), self.n_imgs, p.ctypes.data_as(ctypes.c_void_p),
                                self.n_obs, self.n_tracks)
        if not h:
            raise RuntimeError('pair-major structure plan failed: ' + (L.ba_plan_last_error() or b'').decode())
        try:
            sc = np.zeros(len(PM_SCALARS), dtype=np.int64)
            sz = np.zeros(len(PM_ARRAYS), dtype=np.int64)
            check(L.ba_pm_plan_query(h, sc.ctypes.data_as(ctypes.c_void_p), sz.ctypes.data_as(ctypes.c_void_p)))
            self.scalars = {k: int(v) for k, v in zip(PM_SCALARS, sc)}
            self.host = {}
            for i, name in enumerate(PM_ARRAYS):
                arr = np.empty(int(sz[i]), dtype=np.int32)
                check(L.ba_pm_plan_export(h, i, arr.ctypes.data_as(ctypes.c_void_p)))
                self.host[name] = arr
        finally:
            L.ba_pm_plan_destroy(h)
        self.sizes = {k: int(v.shape[0]) for k, v in self.host.items()}
        self.dev = {k: torch.from_numpy(v).to(self.device) for k, v in self.host.items()}
        for k in PM_ARRAYS:     # never hand a null pointer to a kernel for an empty array
            if self.dev[k].numel() == 0:
                self.dev[k] = torch.zeros(1, dtype=torch.int32, device=self.device)

    def _build_on_device(self, infos, pids):
        """ba_pm_dplan_create on the device's current stream; its arrays are copied into torch tensors (the
        plan is then released), and the host copies are made on first use."""
        L = lib()
        dev = self.device
        cum = infos[0].to(device=dev, dtype=torch.int32).contiguous()
        p = pids.to(device=dev, dtype=torch.int32).contiguous()
        st = stream_ptr(dev)
        h = L.ba_pm_dplan_create(ctypes.c_void_p(cum.data_ptr()), self.n_imgs, ctypes.c_void_p(p.data_ptr()),
                                 self.n_obs, self.n_tracks, st)
        if not h:
            raise RuntimeError('pair-major structure plan failed: ' + (L.ba_pm_dplan_last_error() or b'').decode())
        try:
            sc = np.zeros(len(PM_SCALARS), dtype=np.int64)
            sz = np.zeros(len(PM_ARRAYS), dtype=np.int64)
            check(L.ba_pm_dplan_query(h, sc.ctypes.data_as(ctypes.c_void_p), sz.ctypes.data_as(ctypes.c_void_p)))
            self.scalars = {k: int(v) for k, v in zip(PM_SCALARS, sc)}
            self.sizes = {k: int(sz[i]) for i, k in enumerate(PM_ARRAYS)}
            self.dev = {}
            for i, name in enumerate(PM_ARRAYS):
                t = torch.zeros(max(int(sz[i]), 1), dtype=torch.int32, device=dev)
                check(L.ba_pm_dplan_copy(h, i, ctypes.c_void_p(t.data_ptr()), st))
                self.dev[name] = t
            torch.cuda.current_stream(dev).synchronize()
        finally:
            L.ba_pm_dplan_destroy(h)
        self.host = _DeviceArrays(self)

    workspace = BAPlan.workspace


class SpanProfile:
    """How far apart the images of one track lie, for the path choice of GaussNewtonSolver(path='auto'):
    the median over the observed tracks of (last image - first image + 1).  The batched plan packs tracks
    in (first image, last image) order into batches of at most MAX_LOCAL images, which holds many tracks
    per batch only where tracks are windows of nearby images; where the median span is several batches
    wide (tracks on random neighbours of a large collection), the batched plan is not built at all.
    Computed on the device for device inputs (a scatter min / max per track); holds no arrays."""
    kind = 'span'

    def __init__(self, infos, pids, n_tracks):
        dev = pids.device
        cum = infos[0].to(device=dev, dtype=torch.int64)
        counts = torch.diff(cum, prepend=cum.new_zeros(1))
        img = torch.repeat_interleave(torch.arange(len(cum), device=dev), counts)
        T = max(int(n_tracks), 1)
        p = pids.to(torch.int64)
        lo = torch.full((T,), len(cum), dtype=torch.int64, device=dev).scatter_reduce_(0, p, img, 'amin')
        hi = torch.full((T,), -1, dtype=torch.int64, device=dev).scatter_reduce_(0, p, img, 'amax')
        span = (hi - lo + 1)[hi >= 0]
        self.median_span = int(span.median()) if span.numel() else 0


# ---------------------------------------------------------------------- cache
_cache_lock = threading.Lock()
_cache = {}


def _prune():
    """Drop plans whose pids tensor is gone: they can no longer be looked up, and each holds its
    workspaces (GB-scale at large sizes)."""
    for k in list(_cache):
        live = [ent for ent in _cache[k] if ent[0]() is not None]
        if live:
            _cache[k] = live
        else:
            del _cache[k]


_lineage = {}
_MAX_CHAIN = 64


class _Lineage:
    """How the structure with track ids `ref()` was made by `old | new` (tracks.py:84-102): the new
    observations per image and the new tracks' ids (device tensors, read only if a plan is needed), the
    track counts, the parent structure's appendable plans when it had any (held here, since the parent
    structure itself is usually dropped right after the merge; get_plan adds a plan made after the merge),
    a weak reference to the parent's ids, and the parent's own record if it was a merge result too (so that
    several merges in a row can be planned from the last planned structure)."""
    __slots__ = ('ref', 'version', 'parent_ref', 'parent_version', 'parent_n_tracks', 'add_nppi', 'add_pids',
                 'n_tracks', 'plans', 'parent', 'depth')

    def plan_for(self, key):
        """The parent structure's appendable plan for this key (call with _cache_lock held)."""
        for k, plan in self.plans:
            if k == key[2:] and plan.appendable:
                return plan
        ppids = self.parent_ref()
        if ppids is None or ppids._version != self.parent_version:
            return None
        for ref, version, k, m, iref, iversion, plan in _cache.get(id(ppids), []):
            if ref() is ppids and version == ppids._version and k[2:] == key[2:] and isinstance(plan, BAPlan) \
                    and plan.appendable:
                return plan
        return None


def note_append(pids, parent_pids, parent_n_tracks, add_nppi, add_pids, n_tracks):
    """Records that the structure with track ids `pids` is `old | new` of the one with `parent_pids`:
    add_nppi (n_imgs + 1,) new observations per image, add_pids the new tracks' ids before the shift by
    parent_n_tracks, image by image, n_tracks the merged count."""
    with _cache_lock:
        for k in [k for k, v in _lineage.items() if v.ref() is None]:
            del _lineage[k]
        rec = _Lineage()
        rec.ref, rec.version = weakref.ref(pids), pids._version
        rec.parent_ref, rec.parent_version = weakref.ref(parent_pids), parent_pids._version
        rec.parent_n_tracks, rec.add_nppi, rec.add_pids, rec.n_tracks = int(parent_n_tracks), add_nppi, add_pids, \
            int(n_tracks)
        rec.plans = [(k[2:], plan) for ent in _cache.get(id(parent_pids), [])
                     for ref, version, k, m, iref, iversion, plan in (ent,)
                     if ref() is parent_pids and version == parent_pids._version and isinstance(plan, BAPlan)
                     and plan.appendable]
        parent = _lineage.get(id(parent_pids))
        if parent is not None and (parent.ref() is not parent_pids or parent.version != parent_pids._version
                                   or parent.depth >= _MAX_CHAIN):
            parent = None
        rec.parent = parent
        rec.depth = 1 if parent is None else parent.depth + 1
        _lineage[id(pids)] = rec
        while parent is not None:          # plans kept only for appends: their workspaces are made again if used
            if parent.parent_ref() is None:
                for _, plan in parent.plans:
                    plan._ws, plan._slot_cache = {}, {}
            parent = parent.parent


def _appended_plan(infos, pids, n_tracks, key):
    """The batched plan of `pids` from the plan of an earlier structure, when the lineage says the structures
    between are appends (`old | new`, one image each): the nearest one that had a plan."""
    links = []
    with _cache_lock:
        rec = _lineage.get(id(pids))
        if rec is None or rec.ref() is not pids or rec.version != pids._version:
            return None
        parent = None
        while rec is not None:
            links.append(rec)
            parent = rec.plan_for(key)
            if parent is not None:
                break
            rec = rec.parent
    if parent is None:
        return None
    links.reverse()                                    # oldest first
    chain, counts = [], np.diff(np.concatenate([[0], parent._cum.astype(np.int64)]))
    for ln in links:
        add_nppi = ln.add_nppi.detach().cpu().numpy().astype(np.int64)
        if len(add_nppi) != len(counts) + 1:
            return None
        counts = np.concatenate([counts, [0]]) + add_nppi
        chain.append((add_nppi, ln.add_pids.detach().cpu().numpy().astype(np.int64) + ln.parent_n_tracks,
                      ln.n_tracks))
    cum = infos[0].detach().cpu().numpy().astype(np.int64)
    if chain[-1][2] != int(n_tracks) or len(cum) != len(counts) or not np.array_equal(cum, np.cumsum(counts)):
        return None
    try:
        plan = BAPlan.appended_chain(parent, infos, pids, n_tracks, chain)
    except RuntimeError:
        return None
    with _cache_lock:                                  # the parent's host plan is consumed: let it go
        for ln in links:
            ln.plans = [(k, p) for k, p in ln.plans if p is not parent]
    return plan


def get_plan(infos, pids, n_tracks, kind='batched', **kw):
    """Plan for this structure (kind 'batched': BAPlan, 'pairmajor': PMPlan, 'span': SpanProfile): reused while the same
    pids tensor (unmodified) and the same per-image counts / node / cam ids come back, rebuilt otherwise
    (a batched plan from its parent's, when note_append recorded the structure as `old | new` of a cached one).  The ids are compared by
    content unless the very infos tensor of the cached plan comes back unmodified (torch's version
    counter), which needs no device-to-host read."""
    key = (int(n_tracks), tuple(pids.shape), kind, tuple(sorted(kw.items())))
    with _cache_lock:
        for ent in _cache.get(id(pids), []):
            ref, version, k, m, iref, iversion, plan = ent
            if ref() is pids and version == pids._version and k == key and iref() is infos and \
                    iversion == infos._version:
                return plan
    meta = infos.detach().cpu().numpy().tobytes()
    with _cache_lock:
        _prune()
        for ent in _cache.get(id(pids), []):
            ref, version, k, m, iref, iversion, plan = ent
            if ref() is pids and version == pids._version and k == key and m == meta:
                return plan
    plan = None
    if kind == 'batched':
        plan = _appended_plan(infos, pids, n_tracks, key)
    if plan is None:
        make = {'pairmajor': PMPlan, 'batched': BAPlan, 'span': SpanProfile}[kind]
        plan = make(infos, pids, n_tracks, **kw)
    with _cache_lock:
        if sum(1 for v in _cache.values() for ent in v if not isinstance(ent[6], SpanProfile)) > 8:
            _cache.clear()
        _cache.setdefault(id(pids), []).append((weakref.ref(pids), pids._version, key, meta, weakref.ref(infos),
                                                infos._version, plan))
        if isinstance(plan, BAPlan):     # planned after a merge: its children keep it past this structure's end
            for rec in _lineage.values():
                if rec.parent_ref() is pids and rec.parent_version == pids._version:
                    rec.plans.append((key[2:], plan))
    return plan
