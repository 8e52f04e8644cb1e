"""ba_objective_noalloc (the objective entry point that allocates nothing and keeps its partial sums
in the library's per-GPU scratch array) against ba_objective through the C ABI: bit-identical loss
and reproj_score on two calls in a row, the second with a smaller input (the scratch keeps the first
call's contents, which the second must not see), with and without the Huber error rows, and a size
beyond the 32-bit selection rank rejected with an error before any launch."""
import ctypes

import pytest
import torch

from blast3r_amd._lib import lib, stream_ptr

pytestmark = pytest.mark.gpu
DEV = 'cuda:0'


def _pair(res, n, has_err):
    L = lib()
    st = stream_ptr(DEV)
    ws = torch.empty(int(L.ba_objective_workspace_bytes(n)), dtype=torch.uint8, device=DEV)
    ref = torch.full((2,), 7.0, dtype=torch.float32, device=DEV)
    got = torch.full((2,), -7.0, dtype=torch.float32, device=DEV)
    assert L.ba_objective(res.data_ptr(), n, has_err, ws.data_ptr(), ref.data_ptr(), st) == 0
    assert L.ba_objective_noalloc(res.data_ptr(), n, has_err, got.data_ptr(), st) == 0
    torch.cuda.synchronize()
    return ref.cpu(), got.cpu()


@pytest.mark.parametrize('has_err', [1, 0])
def test_noalloc_objective_matches_workspace_entry_point(has_err):
    gen = torch.Generator(device='cpu').manual_seed(3 + has_err)
    for n in (1_000_003, 70_001, 1):                    # the later calls are smaller
        print(f'ba_objective_noalloc n={n} has_err={has_err}', flush=True)
        rows = 9 if has_err else 3
        res = (torch.randn((rows, n), generator=gen) * 3.0).to(DEV)
        res[:, ::17] *= 50.0                            # a heavy tail, as outliers give
        ref, got = _pair(res, n, has_err)
        assert torch.equal(ref.view(torch.int32)[1:], got.view(torch.int32)[1:]), (n, ref, got)
        if has_err:
            assert torch.equal(ref.view(torch.int32), got.view(torch.int32)), (n, ref, got)
            want = res[3:6].double().mean()
            assert abs(float(got[0]) - float(want)) <= 1e-6 * abs(float(want))
        e = res[:2].norm(dim=0).sort().values
        n80 = n * 80 // 100
        if n80:
            assert abs(float(got[1]) - float(e[:n80].double().mean())) <= 1e-6 * float(e[:n80].double().mean())


def test_noalloc_objective_rejects_rank_overflow():
    L = lib()
    out = torch.zeros(2, dtype=torch.float32, device=DEV)
    rc = L.ba_objective_noalloc(None, 6_000_000_000, 1, out.data_ptr(), stream_ptr(DEV))
    assert rc != 0
    assert b'32 bits' in L.ba_last_error()
