"""ctypes binding of libba_hip.so (declarations in include/ba_hip.h).

The library is loaded lazily on first use and never replaced by a Python or
CPU implementation: if it is missing the call raises RuntimeError, exactly like
the reference's stub module does when its extension is not compiled
(src/blast3r/extensions/cujac/__init__.py:7-16).
"""
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, 'libba_hip.so')

_lib = None
_lock = threading.Lock()

c_int = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f = ctypes.c_float
c_d = ctypes.c_double
c_p = ctypes.c_void_p


class BaHuber(ctypes.Structure):
    _fields_ = [('weight_z', c_f), ('pnorm', c_f), ('max_pix_err', c_f), ('huber_delta', c_f),
                ('w_pts_null', c_f), ('is_depth_log', c_int)]


class BaLayout(ctypes.Structure):
    _fields_ = [('d', c_int), ('C', c_int), ('off_tau', c_int), ('off_zcf', c_int), ('hasK', c_int), ('hasP', c_int),
                ('hasZ', c_int), ('no_grad_f_from_rz', c_int), ('optim_Z0', c_int), ('optim_Z_1st_cam', c_int),
                ('wmin', c_f), ('wmax', c_f), ('dampen', c_d), ('adaptive', c_int), ('x_off', c_int)]


_LIN_FIELDS = [
    ('infos', c_p), ('n_imgs', c_int),
    ('chunk_obs', c_p), ('chunk_meta', c_p), ('slot_info', c_p),
    ('ct_pid', c_p), ('ct_first', c_p), ('ct_m', c_p), ('ct_mask', c_p),
    ('b_chunk_ptr', c_p), ('b_imgs', c_p), ('b_nimgs', c_p), ('b_slot_ptr', c_p), ('slot_pair', c_p),
    ('L', c_int),
    ('s_pix', c_p), ('s_std', c_p), ('s_dep', c_p), ('s_pid', c_p), ('s_img', c_p),
    ('K', c_p), ('P_rig2cam', c_p), ('P_rig2cam_stride', c_i64), ('P_w2rig', c_p), ('z_coefs', c_p), ('pts3d', c_p),
    ('enK', c_p), ('enP', c_p), ('enZ', c_p), ('enX', c_p),
    ('hp', BaHuber), ('lay', BaLayout),
    ('Hpp', c_p), ('gp', c_p), ('chunk_max', c_p), ('lam_p', c_p),
    ('partials', c_p), ('img_partials', c_p),
    ('dc', c_p), ('umap', c_p), ('dX', c_p), ('dX64', c_p),
    ('n_chunks', c_i64), ('n_batches', c_i64), ('n_pairs', c_i64),
    ('pair_ptr', c_p), ('pair_src', c_p), ('img_ptr', c_p), ('img_src', c_p),
    ('S_pairs', c_p), ('e_img', c_p), ('dg_img', c_p),
    ('r_in', c_p), ('w_in', c_p), ('r_s0', c_i64), ('r_s1', c_i64), ('w_s0', c_i64), ('w_s1', c_i64),
    ('ct_pt', c_p), ('n_ctracks', c_i64), ('core', c_p),
    ('chunk_slots', c_p), ('chunk_ent', c_p), ('chunk_eptr', c_p), ('b_pos_slot', c_p), ('pfac', c_p),
    ('b_order', c_p), ('work_ctr', c_p), ('dc_img', c_p), ('real32', c_int),
]


class BaLinArgs(ctypes.Structure):
    _fields_ = _LIN_FIELDS


class BaPcgArgs(ctypes.Structure):
    _fields_ = [('n_u', c_i64), ('n_imgs', c_int), ('d', c_int), ('umap', c_p), ('inv_ptr', c_p), ('inv_src', c_p),
                ('leaf', c_p), ('row_ptr', c_p), ('row_ent', c_p), ('pair_i1', c_p), ('pair_i2', c_p),
                ('S_pairs', c_p), ('e_img', c_p), ('dg_img', c_p), ('dampen', c_d), ('adaptive', c_int),
                ('maxiter', c_int), ('tol', c_d),
                ('rhs', c_p), ('diagA', c_p), ('damp', c_p), ('x', c_p), ('xbest', c_p), ('r', c_p), ('z', c_p),
                ('p', c_p), ('y_img', c_p), ('partials', c_p), ('state', c_p), ('istate', c_p),
                ('S_rows', c_p), ('n_row_ent', c_i64), ('row_u', c_p), ('long_u', c_p), ('n_long', c_i64),
                ('long_ptr', c_p), ('long_idx', c_p), ('img_part', c_p), ('src1', c_p), ('long_rng', c_p),
                ('row_cap', c_int), ('real32', c_int)]

class BaPmArgs(ctypes.Structure):
    _fields_ = [('infos', c_p), ('n_imgs', c_int), ('n_tracks', c_int),
                ('run_ptr', c_p), ('run_obs', c_p), ('run_trk', c_p), ('run_img', c_p), ('img_run_ptr', c_p),
                ('trk_run_ptr', c_p), ('trk_run', c_p), ('trk_obs_ptr', c_p), ('trk_obs', c_p), ('obs_img', c_p),
                ('pair_i1', c_p), ('pair_i2', c_p), ('diag_pair', c_p), ('term_ptr', c_p), ('term', c_p),
                ('pair_sched', c_p), ('n_obs', c_i64), ('n_runs', c_i64), ('n_pairs', c_i64),
                ('pids', c_p), ('pix2d', c_p), ('pix2d_std', c_p), ('pix2d_dep', c_p),
                ('K', c_p), ('P_rig2cam', c_p), ('P_rig2cam_stride', c_i64), ('P_w2rig', c_p), ('z_coefs', c_p),
                ('pts3d', c_p), ('enK', c_p), ('enP', c_p), ('enZ', c_p), ('enX', c_p),
                ('hp', BaHuber), ('lay', BaLayout),
                ('r_in', c_p), ('w_in', c_p), ('r_s0', c_i64), ('r_s1', c_i64), ('w_s0', c_i64), ('w_s1', c_i64),
                ('pobs', c_p), ('wobs', c_p), ('jslots', c_p), ('vslots', c_p), ('yrun', c_p), ('Hpp', c_p), ('gp', c_p), ('tmax', c_p), ('lam_p', c_p), ('pfac', c_p), ('V', c_p),
                ('S_pairs', c_p), ('e_img', c_p), ('dg_img', c_p), ('dc_img', c_p), ('dX', c_p), ('dX64', c_p),
                ('real32', c_int)]


class BaCholArgs(ctypes.Structure):
    _fields_ = [('mode', c_int), ('A', c_p), ('lda', c_i64), ('Linv', c_p), ('pair_idx', c_p), ('kind', c_p),
                ('shared_u', c_p), ('n_shared', c_int), ('w', c_int), ('db', c_int), ('bcol', c_p), ('bpos', c_p),
                ('n_pairs', c_i64), ('info', c_p),
                ('work', c_p)]


PCG_LONG_LIST = 32          # BA_PCG_LONG_LIST in include/ba_hip.h
PCG_BLOCK = 256             # unknowns per block of the PCG update launch (long_ptr granularity)


class BaSampleArgs(ctypes.Structure):
    _fields_ = [('map_addr', c_p), ('map_hw', c_p), ('H', c_int), ('W', c_int), ('Cm', c_int), ('pix_stride', c_int),
                ('insert_ones', c_int),
                ('cum_nppi', c_p), ('n_imgs', c_i64), ('pix2d', c_p), ('n_obs', c_i64), ('out', c_p)]


class BaObsSet(ctypes.Structure):
    _fields_ = [('pids', c_p), ('pix2d', c_p), ('pix2d_std', c_p), ('pix2d_dep', c_p), ('nppi', c_p), ('n_imgs', c_i64)]


class BaGatherArgs(ctypes.Structure):
    _fields_ = [('a', BaObsSet), ('b', BaObsSet), ('sel_a', c_p), ('sel_b', c_p), ('pid_shift_b', c_int), ('C', c_int),
                ('n_out', c_i64), ('n_rows', c_i64), ('pids', c_p), ('pix2d', c_p), ('pix2d_std', c_p),
                ('pix2d_dep', c_p), ('nppi', c_p), ('total', c_p), ('workspace', c_p)]


class BaRemoveArgs(ctypes.Structure):
    _fields_ = [('in_', BaObsSet), ('n_rows', c_i64), ('n_tracks', c_i64), ('C', c_int), ('bad_int64', c_int),
                ('bad', c_p), ('n_bad', c_i64), ('pids', c_p), ('pix2d', c_p), ('pix2d_std', c_p), ('pix2d_dep', c_p),
                ('nppi', c_p), ('old_to_keep', c_p), ('counts', c_p), ('workspace', c_p)]


class BaTangentArgs(ctypes.Structure):
    _fields_ = [('depth_addr', c_p), ('ref_addr', c_p), ('map_hw', c_p), ('H', c_int), ('W', c_int),
                ('depth_pix_stride', c_int), ('ref_pix_stride', c_int), ('K', c_p), ('cam_ids', c_p), ('z_coefs', c_p),
                ('n_imgs', c_i64), ('C', c_int), ('tan_stride', c_int), ('normalize', c_int), ('optim_Z0', c_int),
                ('fp64', c_int), ('compute_gn', c_int), ('weight', c_d), ('eps', c_d), ('loss', c_p), ('g_z', c_p),
                ('H_z', c_p), ('workspace', c_p), ('workspace_bytes', c_i64)]


# name -> (restype, argtypes)
_SIGS = {
    'ba_last_error': (ctypes.c_char_p, []),
    'ba_version': (c_int, []),
    'ba_residuals': (c_int, [c_p, c_int, c_p, c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_int, c_int,
                             c_f, c_f, c_f, c_f, c_f, c_p, c_p]),
    'ba_jacobians': (c_int, [c_p, c_int, c_p, c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_int, c_int, c_int,
                             c_p, c_p, c_p, c_p]),
    'ba_chol3x3_solve': (c_int, [c_p, c_p, c_p, c_i64, c_d, c_int, c_p]),
    'ba_blockcoo_workspace_size': (c_i64, [c_i64, c_i64]),
    'ba_blockcoo_matvec': (c_int, [c_p, c_int, c_int, c_p, c_p, c_int, c_i64, c_p, c_p, c_i64, c_i64, c_int, c_int,
                                   c_p, c_i64, c_p]),
    'ba_einsum_bki_bkj': (c_int, [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_p, c_i64, c_int, c_int, c_int, c_int, c_p]),
    'ba_exp_se3': (c_int, [c_p, c_p, c_i64, c_p]),
    'ba_plan_create': (c_p, [c_p, c_int, c_p, c_i64, c_int, c_int, c_int, c_i64]),
    'ba_plan_query': (c_int, [c_p, c_p, c_p]),
    'ba_plan_export': (c_int, [c_p, c_int, c_p]),
    'ba_plan_destroy': (None, [c_p]),
    'ba_plan_last_error': (ctypes.c_char_p, []),
    'ba_pm_dplan_create': (c_p, [c_p, c_int, c_p, c_i64, c_int, c_p]),
    'ba_pm_dplan_query': (c_int, [c_p, c_p, c_p]),
    'ba_pm_dplan_array': (c_p, [c_p, c_int]),
    'ba_pm_dplan_copy': (c_int, [c_p, c_int, c_p, c_p]),
    'ba_pm_dplan_destroy': (None, [c_p]),
    'ba_pm_dplan_last_error': (ctypes.c_char_p, []),
    'ba_plan_append': (c_p, [c_p, c_p, c_int, c_p, c_i64, c_int]),
    'ba_plan_array': (c_p, [c_p, c_int]),
    'ba_plan_stable': (c_int, [c_p, c_p, c_p]),
    'ba_plan_shift_ids': (c_int, [c_p, c_p, c_p, c_i64, c_p]),
    'ba_abi_sizeof': (c_i64, [ctypes.c_char_p]),
    'ba_linearize_schur': (c_int, [ctypes.POINTER(BaLinArgs), c_p]),
    'ba_linearize_stage': (c_int, [ctypes.POINTER(BaLinArgs), c_int, c_p]),
    'ba_backsubstitute': (c_int, [ctypes.POINTER(BaLinArgs), c_p]),
    'ba_pcg_solve': (c_int, [ctypes.POINTER(BaPcgArgs), c_p]),
    'ba_pcg_solve_range': (c_int, [ctypes.POINTER(BaPcgArgs), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, c_p,
                                   c_p]),
    'ba_host_mapped_ptr': (c_p, [c_p]),
    'ba_pcg_partials_size': (c_i64, [c_i64]),
    'ba_apply_update': (c_int, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_f, c_f, c_int, c_int, c_int, c_int, c_i64,
                                c_p, c_p, c_p, c_p, c_p]),
    'ba_objective_workspace_bytes': (c_i64, [c_i64]),
    'ba_objective': (c_int, [c_p, c_i64, c_int, c_p, c_p, c_p]),
    'ba_objective_noalloc': (c_int, [c_p, c_i64, c_int, c_p, c_p]),
    'ba_chol_dense_lda': (c_i64, [c_i64]),
    'ba_pm_plan_create': (c_p, [c_p, c_int, c_p, c_i64, c_int]),
    'ba_pm_plan_query': (c_int, [c_p, c_p, c_p]),
    'ba_pm_plan_export': (c_int, [c_p, c_int, c_p]),
    'ba_pm_plan_destroy': (None, [c_p]),
    'ba_pm_linearize_schur': (c_int, [ctypes.POINTER(BaPmArgs), c_p]),
    'ba_pm_linearize_stage': (c_int, [ctypes.POINTER(BaPmArgs), c_int, c_p]),
    'ba_pm_backsubstitute': (c_int, [ctypes.POINTER(BaPmArgs), c_p]),
    'ba_pm_slot_doubles': (c_i64, [c_i64, c_int, c_int]),
    'ba_chol_band_lds_bytes': (c_i64, [c_int, c_int, c_int]),
    'ba_chol_work_doubles': (c_i64, [c_int, c_i64, c_int, c_int, c_int, c_int]),
    'ba_chol_band_superblocks': (c_int, [c_int, c_int, c_int, c_int]),
    'ba_reduced_solve': (c_int, [ctypes.POINTER(BaPcgArgs), ctypes.POINTER(BaCholArgs), c_p]),
    'ba_nonfinite_flags': (c_int, [c_p, c_p, c_int, c_p, c_p]),
    'ba_stream_triad': (c_int, [c_p, c_p, c_p, ctypes.c_double, c_i64, c_p]),
    'ba_sample_depth': (c_int, [ctypes.POINTER(BaSampleArgs), c_p]),
    'ba_tracks_gather': (c_int, [ctypes.POINTER(BaGatherArgs), c_p]),
    'ba_tracks_remove': (c_int, [ctypes.POINTER(BaRemoveArgs), c_p]),
    'ba_tracks_to_dense': (c_int, [c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_p, c_p, c_p]),
    'ba_tracks_img_id': (c_int, [c_p, c_i64, c_i64, c_p, c_p, c_p]),
    'ba_tracks_workspace_bytes': (c_i64, [c_i64, c_i64, c_i64]),
    'ba_tangent_prior': (c_int, [ctypes.POINTER(BaTangentArgs), c_p]),
    'ba_tangent_workspace_bytes': (c_i64, [c_i64, c_int, c_int, c_int, c_int, c_int, c_int]),
    'ba_planar_confidence': (c_int, [c_p, c_int, c_int, c_f, c_p, c_p]),
    'ba_add_z_prior': (c_int, [c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_int, c_int, c_int, c_p]),
}

EXPORTED = tuple(_SIGS)


ABI_STRUCTS = {'ba_huber': BaHuber, 'ba_layout': BaLayout, 'ba_lin_args': BaLinArgs, 'ba_pm_args': BaPmArgs,
               'ba_pcg_args': BaPcgArgs, 'ba_chol_args': BaCholArgs, 'ba_sample_args': BaSampleArgs,
               'ba_obs_set': BaObsSet, 'ba_gather_args': BaGatherArgs, 'ba_remove_args': BaRemoveArgs,
               'ba_tangent_args': BaTangentArgs}


def _check_abi(L):
    """Every argument struct here has the library's size (a field missing on one side would hand
    the kernels shifted pointers)."""
    bad = [(n, ctypes.sizeof(cls), int(L.ba_abi_sizeof(n.encode()))) for n, cls in ABI_STRUCTS.items()
           if ctypes.sizeof(cls) != int(L.ba_abi_sizeof(n.encode()))]
    if bad:
        raise RuntimeError(f'libba_hip.so struct layout differs from the Python binding: {bad}')


def lib():
    """The loaded library (raises RuntimeError when it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f'libba_hip.so is not built ({LIB_PATH}); run `python -m blast3r_amd.build` '
                                   'or __graft_entry__.build()')
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                f = getattr(L, name)
                f.restype = res
                f.argtypes = args
            _check_abi(L)
            _lib = L
    return _lib


def check(status):
    if status != 0:
        msg = lib().ba_last_error()
        raise RuntimeError((msg or b'libba_hip error').decode())


def stream_ptr(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    """Raw device pointer of a tensor (None -> NULL); a host tensor raises instead of handing a
    host address to a kernel."""
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError(f'expected a device tensor for a kernel argument, got one on {t.device}')
    return ctypes.c_void_p(t.data_ptr())
