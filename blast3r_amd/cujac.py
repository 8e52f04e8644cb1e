"""Drop-in for the reference's ``blast3r.extensions.cujac`` module on MI355X.

Same names, argument meaning and error behaviour as
src/blast3r/extensions/cujac/__init__.py:18-58 and the pybind table of
sfm_jacobian_rigs.cu:1254-1275 (``.cu`` below); every call runs a kernel of
libba_hip.so on the current stream.  Input checks mirror the reference's
TORCH_CHECKs (.cu:10-15, :1013-1044) and raise RuntimeError.
"""
import torch

from . import _lib
from ._lib import check, lib, ptr, stream_ptr

__all__ = ['compute_residuals_with_rigs', 'compute_jacobians_with_rigs', 'chol3x3_solve', 'blockcoo_matvec',
           'fused_einsum_bki_bkj', 'skew_symmetric', 'hat_se3', 'exp_se3']


def _req(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _dev(name, t):
    _req(t.is_cuda, f'{name} is not on CUDA device')


def _cont(name, t, nd, last=None):
    _dev(name, t)
    _req(t.is_contiguous(), f'{name} is not memory-contiguous')
    _req(t.dim() == nd, f'{name}.ndim should be == {nd}, not {t.dim()}')
    if last is not None:
        _req(t.shape[-1] == last, f'{name}.shape[-1] should be == {last}, not {t.shape[-1]}')


def _dtype(name, t, dt):
    _req(t.dtype == dt, f'{name} must be {dt}, got {t.dtype}')


def check_inputs(infos, K, P_rig2c, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std, pix2d_dep):
    """Restates check_inputs (.cu:1013-1044); returns (n_imgs, n_obs, C)."""
    _cont('infos', infos, 2)
    _cont('K', K, 3, 3)
    _dev('P_rig2c', P_rig2c)
    _req(P_rig2c.dim() == 3 and P_rig2c.stride(1) == 4 and P_rig2c.stride(2) == 1,
         'P_rig2c should be (N,4,4) and contiguous inside 4x4 blocks')
    _cont('P_w2rig', P_w2rig, 3, 4)
    _cont('z_coefs', z_coefs, 2)
    _cont('pts3d', pts3d, 2, 3)
    _cont('pids', pids, 1)
    _cont('pix2d', pix2d, 2, 2)
    _cont('pix2d_std', pix2d_std, 2, 2)
    _cont('pix2d_dep', pix2d_dep, 2)
    _req(infos.shape[0] == 3, 'infos should have 3 rows = [nkpt_cum, node_ids, cam_ids]')
    for n, t in (('infos', infos), ('pids', pids)):
        _dtype(n, t, torch.int32)
    for n, t in (('K', K), ('P_rig2c', P_rig2c), ('P_w2rig', P_w2rig), ('z_coefs', z_coefs), ('pts3d', pts3d),
                 ('pix2d', pix2d), ('pix2d_std', pix2d_std), ('pix2d_dep', pix2d_dep)):
        _dtype(n, t, torch.float32)
    C = pix2d_dep.shape[1]
    _req(C == z_coefs.shape[1], 'Number of Z coefs is not consistent')
    return infos.shape[1], pids.shape[0], C


def compute_residuals_with_rigs(infos, K, P_rig2c, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std, pix2d_dep,
                                is_depth_log, weight_z=1.0, pnorm=-1.0, max_pix_err=100.0, huber_delta=0.5,
                                w_pts_nul=1e-16):
    """residuals_with_rigs (.cu:1048-1101): (n_obs, 9) view of an (9, n_obs) buffer (3 when pnorm <= 0)."""
    n_imgs, n_obs, C = check_inputs(infos, K, P_rig2c, P_w2rig, z_coefs, pts3d, pids, pix2d, pix2d_std, pix2d_dep)
    _req(pnorm == -1 or (0 < pnorm <= 2), 'pnorm must be in {-1} U ]0,2]')
    n_out = 9 if pnorm > 0 else 3
    out = torch.empty((n_out, n_obs), dtype=torch.float32, device=pids.device)
    check(lib().ba_residuals(ptr(infos), n_imgs, ptr(K), ptr(P_rig2c), P_rig2c.stride(0), ptr(P_w2rig),
                             ptr(z_coefs), ptr(pts3d), ptr(pids), ptr(pix2d), ptr(pix2d_std), ptr(pix2d_dep), n_obs,
                             C, int(bool(is_depth_log)), float(weight_z), float(pnorm), float(max_pix_err),
                             float(huber_delta), float(w_pts_nul), ptr(out), stream_ptr(pids.device)))
    return out.transpose(0, 1)


def compute_jacobians_with_rigs(infos, K, P_rig2c, P_w2rig, z_coefs, pts3d, pids, pix2d_std, pix2d_dep,
                                is_depth_log, float64=False):
    """jacobians_with_rigs (.cu:1105-1148): [J_cam (N,3,8), J_zcf (N,1,C), J_pts (N,3,3)]."""
    n_imgs, n_obs, C = check_inputs(infos, K, P_rig2c, P_w2rig, z_coefs, pts3d, pids, pix2d_std, pix2d_std,
                                    pix2d_dep)
    dt = torch.float64 if float64 else torch.float32
    dev = pids.device
    J_pts = torch.empty((n_obs, 3, 3), dtype=dt, device=dev)
    J_cam = torch.empty((n_obs, 3, 8), dtype=dt, device=dev)
    J_zcf = torch.empty((n_obs, 1, C), dtype=dt, device=dev)
    check(lib().ba_jacobians(ptr(infos), n_imgs, ptr(K), ptr(P_rig2c), P_rig2c.stride(0), ptr(P_w2rig), ptr(z_coefs),
                             ptr(pts3d), ptr(pids), ptr(pix2d_std), ptr(pix2d_dep), n_obs, C,
                             int(bool(is_depth_log)), int(bool(float64)), ptr(J_cam), ptr(J_zcf), ptr(J_pts),
                             stream_ptr(dev)))
    return [J_cam, J_zcf, J_pts]


def chol3x3_solve(blocks, rhs, jitter=1e-12):
    """chol3x3_solve (.cu:1151-1169)."""
    _req(blocks.is_cuda, 'blocks must be CUDA tensor')
    _req(rhs.is_cuda, 'rhs must be CUDA tensor')
    _req(blocks.is_contiguous(), 'blocks must be contiguous')
    _req(rhs.is_contiguous(), 'rhs must be contiguous')
    _req(blocks.dim() == 3 and blocks.shape[1] == 3 and blocks.shape[2] == 3, 'blocks must have shape [N,3,3]')
    _req(rhs.dim() == 2 and rhs.shape[1] == 3 and rhs.shape[0] == blocks.shape[0], 'rhs must have shape [N,3]')
    _req(blocks.dtype == rhs.dtype, 'dtype mismatch between blocks and rhs')
    _req(blocks.dtype in (torch.float32, torch.float64), 'only float32/float64 supported')
    out = torch.empty_like(rhs)
    check(lib().ba_chol3x3_solve(ptr(blocks), ptr(rhs), ptr(out), blocks.shape[0], float(jitter),
                                 int(blocks.dtype == torch.float64), stream_ptr(blocks.device)))
    return out


def blockcoo_matvec(blocks, row_indices, col_indices, x, HB1, WB1, transpose_blocks=False):
    """blockcoo_matvec (.cu:1171-1219): y = A x, or A^T x when transpose_blocks."""
    _req(blocks.is_cuda and x.is_cuda, 'blocks and x must be CUDA tensors')
    _req(row_indices.is_cuda and col_indices.is_cuda, 'indices must be CUDA tensors')
    _req(blocks.is_contiguous(), 'blocks must be contiguous [N,bh,bw]')
    _req(x.is_contiguous(), 'x must be contiguous')
    _req(blocks.dim() == 3, 'blocks must be [N,bh,bw]')
    _req(row_indices.dim() == 1 and col_indices.dim() == 1 and row_indices.shape[0] == blocks.shape[0]
         and col_indices.shape[0] == blocks.shape[0], 'indices must be [N] and match blocks.size(0)')
    _req(blocks.dtype == x.dtype, 'dtype mismatch')
    _req(col_indices.dtype == row_indices.dtype, 'index dtypes must match')
    _req(row_indices.dtype in (torch.int32, torch.int64), 'Only int32/int64 indicessupported')
    _req(blocks.dtype in (torch.float32, torch.float64), 'Only float32/float64 supported')
    N, bh, bw = blocks.shape
    in_len = HB1 * bh if transpose_blocks else WB1 * bw
    out_len = WB1 * bw if transpose_blocks else HB1 * bh
    _req(x.numel() == in_len, 'x has wrong length for the provided shapes')
    y = torch.empty(out_len, dtype=blocks.dtype, device=blocks.device)
    L = lib()
    nbytes = L.ba_blockcoo_workspace_size(N, int(WB1 if transpose_blocks else HB1))
    if nbytes < 0:
        raise RuntimeError(L.ba_last_error().decode())
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=blocks.device)
    check(L.ba_blockcoo_matvec(ptr(blocks), bh, bw, ptr(row_indices.contiguous()),
                               ptr(col_indices.contiguous()), int(row_indices.dtype == torch.int64), N, ptr(x),
                               ptr(y), int(HB1), int(WB1), int(bool(transpose_blocks)),
                               int(blocks.dtype == torch.float64), ptr(ws), int(nbytes), stream_ptr(blocks.device)))
    return y


def fused_einsum_bki_bkj(left, right):
    """fused_einsum_bki_bkj (.cu:1222-1250) for every (I, J, K)."""
    _req(left.is_cuda and right.is_cuda, 'tensors must be CUDA')
    _req(left.dim() == 3 and right.dim() == 3, 'expected [B,K,I] and [B,K,J]')
    _req(left.shape[0] == right.shape[0], 'B mismatch')
    _req(left.shape[1] == right.shape[1], 'K mismatch')
    _req(left.dtype == right.dtype, 'dtype mismatch')
    _req(left.stride(2) == 1, f'left must have stride(2)==1 (got {left.stride(2)})')
    _req(right.stride(2) == 1, f'right must have stride(2)==1 (got {right.stride(2)})')
    _req(left.dtype in (torch.float32, torch.float64), 'only float32/float64 supported')
    B, K, I = left.shape
    J = right.shape[2]
    out = torch.empty((B, I, J), dtype=left.dtype, device=left.device)
    check(lib().ba_einsum_bki_bkj(ptr(left), left.stride(0), left.stride(1), ptr(right), right.stride(0),
                                  right.stride(1), ptr(out), B, K, I, J, int(left.dtype == torch.float64),
                                  stream_ptr(left.device)))
    return out


def skew_symmetric(w, device=None):
    """(B,3) -> (B,3,3) (cujac/__init__.py:27-41)."""
    wx, wy, wz = w.T
    res = w.new_zeros((len(w), 3, 3))
    res[:, 2, 1] = wx
    res[:, 1, 2] = -wx
    res[:, 2, 0] = -wy
    res[:, 0, 2] = wy
    res[:, 0, 1] = -wz
    res[:, 1, 0] = wz
    return res


def hat_se3(xi):
    """(B,6) -> (B,4,4) (cujac/__init__.py:43-54)."""
    hat = xi.new_zeros((len(xi), 4, 4))
    hat[:, :3, :3] = skew_symmetric(xi[:, :3])
    hat[:, :3, 3] = xi[:, 3:]
    return hat


def exp_se3(xi):
    """SE(3) exponential (cujac/__init__.py:56-58), closed form on the device."""
    _dev('xi', xi)
    _req(xi.dim() == 2 and xi.shape[1] == 6 and xi.dtype == torch.float32, 'xi must be (B,6) float32')
    xi = xi.contiguous()
    out = torch.empty((xi.shape[0], 4, 4), dtype=torch.float32, device=xi.device)
    check(lib().ba_exp_se3(ptr(xi), ptr(out), xi.shape[0], stream_ptr(xi.device)))
    return out
