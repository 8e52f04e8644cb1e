"""Writes tests/golden/pcg_golden.npz: input/output vectors of the reference `_pcg`.

`_pcg` (src/blast3r/inference/ba_solver.py:1197-1238) fixes the iterate sequence, the
stopping rule and the best-so-far choice of the reduced solve; nothing but the reference
itself pins that control flow.  This script imports the reference module from
/root/reference (pure torch: the cujac kernels it also imports are stubs that raise only
when called, and `_pcg` calls none of them) and records its outputs on small seeded
systems.  It is run by hand in the build container only; the tests read the .npz.
"""
import os
import sys

import numpy as np
import torch

REF = '/root/reference/src'


def cases():
    g = torch.Generator().manual_seed(7)
    out = []

    def spd(n, cond):
        Q, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
        ev = torch.logspace(0, np.log10(cond), n, dtype=torch.float64)
        return (Q * ev) @ Q.T

    A = spd(30, 1e3)
    b = torch.randn(30, generator=g, dtype=torch.float64)
    out.append(('converges', A, b, 1e-6, 200))
    out.append(('maxiter_hit', A, b, 1e-6, 5))
    A2 = spd(40, 1e9)
    b2 = torch.randn(40, generator=g, dtype=torch.float64)
    out.append(('ill_conditioned', A2, b2, 1e-10, 25))
    A3 = spd(12, 10.0)
    A3[0, 0] = -5.0                                  # indefinite: CG can go wrong, best-so-far matters
    b3 = torch.randn(12, generator=g, dtype=torch.float64)
    out.append(('indefinite', A3, b3, 1e-8, 30))
    out.append(('zero_rhs', A, torch.zeros(30, dtype=torch.float64), 1e-6, 50))
    return out


def main():
    sys.path.insert(0, REF)
    from blast3r.inference.ba_solver import _pcg
    data = {}
    for name, A, b, tol, maxiter in cases():
        d = A.diagonal().clamp(min=1e-12)
        x, k, conv = _pcg(lambda v: A @ v, b, M_mv=lambda v: v / d, tol=tol, maxiter=maxiter)
        data[f'{name}/A'] = A.numpy()
        data[f'{name}/b'] = b.numpy()
        data[f'{name}/tol'] = np.float64(tol)
        data[f'{name}/maxiter'] = np.int64(maxiter)
        data[f'{name}/x'] = x.numpy()
        data[f'{name}/iters'] = np.int64(k)
        data[f'{name}/converged'] = np.bool_(bool(conv))
        print(f'{name}: iters={k} converged={bool(conv)} |x|={float(x.norm()):.6g}')
    np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)), 'pcg_golden.npz'), **data)


if __name__ == '__main__':
    main()
