"""Code generation check of the MFMA kernels (CPU only: hipcc cross-compiles gfx950 here).

An MFMA result read back from its accumulator registers (v_accvgpr_read, or any instruction
naming the register) needs a number of wait states after the v_mfma that writes it.  The compiler
inserts them in straight-line code, but one loop shape of the pair kernel had the accumulators
copied out at the loop head with only 5 wait states after the MFMA at the loop end (the back
edge): the result read back was stale in its last element, which the pair-major parity tests
caught.  This test compiles the MFMA sources to assembly and requires at least MIN_WAIT wait states
(instructions, s_nop n counting n + 1) between every v_mfma_f64 and a read of its destination
registers, along straight-line code and across loop back edges.
"""
import os
import re
import subprocess

import pytest

from blast3r_amd import build as B

MIN_WAIT = 10
MFMA_SOURCES = ['ba_schur.hip', 'ba_chol.hip']


def _asm(src, tmp_path):
    out = str(tmp_path / (src + '.s'))
    cmd = [B._hipcc()] + [f for f in B.HIPCC_FLAGS if f not in ('-fPIC',)] + \
        ['-S', '--cuda-device-only', os.path.join(B.CSRC, src), '-o', out]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-2000:]
    return open(out).read()


def _functions(asm):
    cur, body = None, []
    for line in asm.split('\n'):
        m = re.match(r'^(_Z\w+):', line)
        if m:
            if cur:
                yield cur, body
            cur, body = m.group(1), []
            continue
        t = line.split(';')[0].strip()
        if cur and t and not (t.startswith('.') and not t.startswith('.LBB')):
            body.append(t)
        if cur and line.startswith('.Lfunc_end'):
            yield cur, body
            cur = None
    if cur:
        yield cur, body


def _mfma_dest(t):
    m = re.match(r'v_mfma_f64\S*\s+([av])\[(\d+):(\d+)\]', t)
    return (m.group(1), int(m.group(2)), int(m.group(3))) if m else None


def _reads(t, kind, reg):
    """Does instruction t read register kind+reg (outside an MFMA's own accumulator operand)?"""
    if t.startswith('v_mfma') or t.startswith('.LBB') or t.startswith('s_'):
        return False
    ops = t.split(None, 1)[1] if ' ' in t else ''
    parts = [p.strip() for p in ops.split(',')]
    srcs = parts[1:] if not t.startswith(('global_store', 'buffer_store', 'ds_write', 'flat_store')) else parts
    for p in srcs:
        m = re.match(rf'{kind}\[(\d+):(\d+)\]', p)
        if m and int(m.group(1)) <= reg <= int(m.group(2)):
            return True
        if p == f'{kind}{reg}':
            return True
    return False


def _wait(t):
    m = re.match(r's_nop\s+(\d+)', t)
    return int(m.group(1)) + 1 if m else (0 if t.startswith('.LBB') else 1)


def _violations(body):
    bad = []
    for k, t in enumerate(body):
        dst = _mfma_dest(t)
        if not dst:
            continue
        kind, lo, hi = dst
        for reg in range(lo, hi + 1):
            # straight-line successors, and the loop head after a back edge to an earlier label
            w = 0
            for j in range(k + 1, min(len(body), k + 64)):
                u = body[j]
                if _reads(u, kind, reg):
                    if w < MIN_WAIT:
                        bad.append((t, u, w))
                    break
                if _mfma_dest(u) and _mfma_dest(u)[0] == kind and _mfma_dest(u)[1] <= reg <= _mfma_dest(u)[2]:
                    break
                m = re.match(r's_(?:cbranch\w*|branch)\s+(\.LBB\w+)$', u)
                if m:
                    lab = m.group(1)
                    heads = [i for i, x in enumerate(body) if x.split(':')[0] == lab]
                    if heads and heads[0] < j:
                        w2 = w + 1
                        for i in range(heads[0] + 1, min(len(body), heads[0] + 64)):
                            v = body[i]
                            if _reads(v, kind, reg):
                                if w2 < MIN_WAIT:
                                    bad.append((t, v, w2))
                                break
                            if _mfma_dest(v) or v.startswith('s_cbranch') or v.startswith('s_branch'):
                                break
                            w2 += _wait(v)
                    if u.startswith('s_branch'):
                        break
                w += _wait(u)
                if w >= 64:
                    break
    return bad


def test_scanner_finds_a_short_back_edge():
    """The scanner itself: a loop whose head reads the accumulator 5 wait states after the MFMA at
    its end (the shape that gave stale results) is flagged; with s_nop padding it is not."""
    body = ['.LBB0_1:', 's_nop 3', 'v_accvgpr_read_b32 v9, a7', 'v_mov_b32_e32 v1, v2',
            'v_mfma_f64_16x16x4_f64 a[0:7], v[2:3], v[4:5], a[0:7]', 's_cbranch_vccnz .LBB0_1', 's_endpgm']
    assert _violations(body)
    ok = list(body)
    ok[1] = 's_nop 15'
    assert not _violations(ok)
    straight = ['v_mfma_f64_16x16x4_f64 a[0:7], v[2:3], v[4:5], a[0:7]', 's_nop 1', 'v_accvgpr_read_b32 v9, a7']
    assert _violations(straight)


@pytest.mark.parametrize('src', MFMA_SOURCES)
def test_mfma_results_read_after_enough_wait_states(src, tmp_path):
    asm = _asm(src, tmp_path)
    n_mfma = asm.count('v_mfma_f64')
    assert n_mfma > 0
    bad = {}
    for name, body in _functions(asm):
        v = _violations(body)
        if v:
            bad[name] = v[:3]
    assert not bad, bad


def _vregs(text):
    """VGPRs named in an instruction's operand text (v5, v[4:7])."""
    regs = set()
    for m in re.finditer(r'\bv\[(\d+):(\d+)\]|\bv(\d+)\b', text):
        if m.group(3) is not None:
            regs.add(int(m.group(3)))
        else:
            regs.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return regs


def _lds_asm_violations(lines):
    """LDS reads tagged `ba_pf` are issued from inline asm, so the compiler does not wait for them:
    no instruction may name one of their destination registers before the next `ba_pw` wait (an
    `s_waitcnt lgkmcnt(0)`), and none may still be pending at a label or branch."""
    bad, pending = [], {}
    for ln in lines:
        t = ln.strip()
        if not t or t.startswith(';') or (t.startswith('.') and not t.startswith('.LBB')):
            continue
        if t.endswith('ba_pw'):
            if not t.startswith('s_waitcnt lgkmcnt(0)'):
                bad.append(('wait is not lgkmcnt(0)', t))
            pending = {}
            continue
        if pending and (t.startswith('.LBB') or t.startswith(('s_branch', 's_cbranch', 's_endpgm', 's_setpc'))):
            bad.append(('read pending at ' + t.split()[0], sorted(pending)))
            pending = {}
            continue
        parts = t.split(';')[0].split(None, 1)
        ops = parts[1] if len(parts) > 1 else ''
        hit = _vregs(ops) & set(pending)
        if hit:
            bad.append((t, {r: pending[r] for r in sorted(hit)}))
        if t.endswith('ba_pf'):
            for r in _vregs(ops.split(',')[0]):
                pending[r] = t
    return bad


def test_lds_asm_scanner_flags_an_early_use():
    ok = ['ds_read_b64 v[8:9], v0 ; ba_pf', 's_waitcnt lgkmcnt(0) ; ba_pw',
          'v_mfma_f64_16x16x4_f64 v[58:65], v[8:9], v[6:7], v[58:65]']
    assert not _lds_asm_violations(ok)
    early = ['ds_read_b64 v[8:9], v0 ; ba_pf', 'v_mov_b64_e32 v[4:5], v[8:9]', 's_waitcnt lgkmcnt(0) ; ba_pw']
    assert _lds_asm_violations(early)
    crossing = ['ds_read_b64 v[8:9], v0 ; ba_pf', 's_cbranch_scc0 .LBB0_1', 's_waitcnt lgkmcnt(0) ; ba_pw']
    assert _lds_asm_violations(crossing)
    clobber = ['ds_read_b64 v[8:9], v0 ; ba_pf', 'ds_read_b64 v[8:9], v1 ; ba_pf', 's_waitcnt lgkmcnt(0) ; ba_pw']
    assert _lds_asm_violations(clobber)
    weak = ['ds_read_b64 v[8:9], v0 ; ba_pf', 's_waitcnt lgkmcnt(1) ; ba_pw']
    assert _lds_asm_violations(weak)


def test_schur_asm_lds_reads_untouched_until_their_wait(tmp_path):
    """The MFMA phase of k_schur reads LDS through inline asm (so that the compiler does not make it
    wait for the next chunk's global_load_lds copies); in the compiled kernel every such read's
    destination is left alone until the explicit lgkmcnt(0) wait that follows it."""
    asm = _asm('ba_schur.hip', tmp_path)
    assert asm.count('ba_pf') > 0 and asm.count('ba_pw') > 0
    funcs, cur = {}, None
    for line in asm.split('\n'):
        m = re.match(r'^(_Z\w+):', line)
        if m:
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur:
            funcs[cur].append(line)
    bad = {name: v[:3] for name, lines in funcs.items() for v in [_lds_asm_violations(lines)] if v}
    assert not bad, bad
