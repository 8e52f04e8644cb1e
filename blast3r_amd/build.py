"""Builds libba_hip.so in-tree with hipcc for gfx950 (no JIT, no torch extension machinery).

The library is plain C ABI (include/ba_hip.h); Python reaches it through ctypes.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, 'csrc')
LIB = os.path.join(HERE, 'libba_hip.so')
SOURCES = ['ba_compat.hip', 'ba_schur.hip', 'ba_pcg.hip', 'ba_chol.hip', 'ba_update.hip', 'ba_sample.hip', 'ba_tracks.hip', 'ba_tangent.hip',
           'ba_pmplan.hip', 'ba_plan.cpp']
ARCH = os.environ.get('BA_OFFLOAD_ARCH', 'gfx950')

HIPCC_FLAGS = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}',
               # no packed fp32 instructions: some of their forms have given wrong results on these GPUs
               '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
               '-I', os.path.join(ROOT, 'include'), '-I', CSRC, '-Wno-unused-result']


def _hipcc():
    for c in (os.environ.get('HIPCC'), '/opt/rocm/bin/hipcc', 'hipcc'):
        if c and (os.path.sep not in c or os.path.exists(c)):
            return c
    raise RuntimeError('hipcc not found')


def build(verbose=False, jobs=None):
    """Compile every source and link libba_hip.so next to this file. Always rebuilds."""
    hipcc = _hipcc()
    objdir = os.path.join(HERE, '_build')
    os.makedirs(objdir, exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        obj = os.path.join(objdir, src + '.o')
        objs.append(obj)
        if src.endswith('.cpp'):
            cmd = ['g++', '-O3', '-std=c++17', '-fPIC', '-pthread', '-I', os.path.join(ROOT, 'include'), '-I', CSRC, '-c', path,
                   '-o', obj]
        else:
            cmd = [hipcc] + HIPCC_FLAGS + ['-c', path, '-o', obj]
        if verbose:
            print(' '.join(cmd), flush=True)
        procs.append((src, cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, cmd, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors='replace')
        if p.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text)
    if failed:
        msg = '\n'.join(f'--- {s}\n{t}' for s, t in failed)
        raise RuntimeError(f'HIP build failed:\n{msg}')
    tmp = LIB + '.tmp'
    cmd = [hipcc, '-shared', f'--offload-arch={ARCH}', '-fPIC', '-pthread', '-o', tmp] + objs
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError('link failed:\n' + r.stdout.decode(errors='replace'))
    os.replace(tmp, LIB)
    return LIB


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
