"""Benchmark of the bundle-adjustment linearize + Schur path on one MI355X.

A "step" is one fused linearize + Schur-reduce pass (ba_linearize_schur: point
blocks, camera-pair Schur blocks, rhs, deterministic reductions) over the whole
synthetic problem, inputs resident in HBM.  The default workload is benchmark
config 2: 1024 frames, 1M tracks on contiguous windows of 4..12 frames
(~8M observations), log-depth with K=4 channels (C=5 z-coefficients), focal +
pose + depth coefficients + points optimised.

Prints one JSON line: value = observations per second of the linearize + Schur
pass; LM iterations per second of the full lm_step are reported beside it, as
are the roofline of the dominant kernel (k_schur, timed with events on its own
launch stream), the pass's algorithmic bytes against its counter traffic (the
committed rocprofv3 summaries under profiles/), the pair-major path on config 3
(random co-visibility, 22.5 M observations) and the CPU oracle on the same
workload (fp64 and fp32 passes, one lm_step with a capped PCG).
"""
import argparse
import json
import os
import sys
import time

import torch


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--config', type=int, default=2)
    ap.add_argument('--frames', type=int, default=None)
    ap.add_argument('--tracks', type=int, default=None)
    ap.add_argument('--lm-steps', type=int, default=3)
    ap.add_argument('--cpu-baseline', type=int, default=1)
    ap.add_argument('--sampling', type=int, default=1,
                    help='also time the F-sampling kernel on maps of the configuration (1 = yes)')
    ap.add_argument('--layout', type=int, default=1,
                    help='also time the observation-structure edits (old | new merge, remove, plan rebuild)')
    ap.add_argument('--tangent', type=int, default=1,
                    help='also time the dense tangent prior on maps of the configuration (1 = yes)')
    ap.add_argument('--reduced-solve', type=int, default=1,
                    help='also time the reduced-system Cholesky (ba_reduced_solve, dense and banded) on the config')
    ap.add_argument('--pm-config', type=int, default=3,
                    help='also time the pair-major path on this configuration at full size (-1 = no)')
    ap.add_argument('--copy-probe', action='store_true',
                    help='run a 256 MiB fill and a 256 MiB kernel copy (calibrates FETCH_SIZE / WRITE_SIZE counters)')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one MI355X: multi-GPU runs are not part of this build '
              '(the path would shard by track, with one all-reduce of the reduced system)',
              file=sys.stderr)
        sys.exit(2)

    from blast3r_amd import cujac
    from blast3r_amd._lib import check, lib
    from blast3r_amd.ba_solver import GaussNewtonSolver
    from blast3r_amd import engine
    from blast3r_amd.synthetic import make_problem

    dev = torch.device('cuda:0')
    t0 = time.time()
    prob = make_problem(args.config, n_frames=args.frames, n_tracks=args.tracks)
    log(f'[bench] generated cfg {args.config}: {prob.n_imgs} frames, {prob.n_tracks} tracks, {prob.n_obs} obs, '
        f'C={prob.C} in {time.time() - t0:.1f}s')
    g = prob.to(dev)
    o = prob.options
    hp = dict(weight_z=o['weight_z'], pnorm=o['pnorm'], max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d,
                                            g.pix2d_std, g.pix2d_dep, True, hp['weight_z'], hp['pnorm'],
                                            hp['max_pix_err'], hp['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    gs = GaussNewtonSolver(len(g.K), len(g.P_w2rig), prob.n_imgs, prob.n_tracks, dev, dtype=torch.float64)
    J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                             g.pix2d_dep, True, optim_K=o['optim_K'], optim_P=o['optim_P'], pix2d=g.pix2d, hp=hp)
    from blast3r_amd.ba_solver import _param_state
    res._ba_state = _param_state(J)
    t0 = time.time()
    ctx = gs.prepare(J, res, w)
    torch.cuda.synchronize()
    log(f'[bench] plan + slot data in {time.time() - t0:.1f}s: {ctx["plan"].scalars}')
    a, st = ctx['args'], ctx['stream']
    L = lib()
    pm_path = ctx['path'] == 'pairmajor'          # config 3 (random co-visibility) or d > 15

    def step(ev=None):
        # events bracket the dominant kernel: k_schur (batched stage 1) or k_pm_pairs (pair-major stage 1)
        if pm_path:
            check(L.ba_pm_linearize_stage(a, 0, st))
        else:
            check(L.ba_linearize_stage(a, 0, st))
        if ev is not None:
            ev[0].record()
        if pm_path:
            check(L.ba_pm_linearize_stage(a, 1, st))
        else:
            check(L.ba_linearize_stage(a, 1, st))
        if ev is not None:
            ev[1].record()
        if not pm_path:
            check(L.ba_linearize_stage(a, 2, st))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(evs[k])
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    schur_ms = sum(e0.elapsed_time(e1) for e0, e1 in evs) / args.steps
    n_obs = prob.n_obs
    value = n_obs / (ms_step * 1e-3)
    kname = 'k_pm_pairs' if pm_path else 'k_schur'
    log(f'[bench] linearize+Schur {ms_step:.3f} ms/step ({ctx["path"]} path), {kname} {schur_ms:.3f} ms -> '
        f'{value:.4g} obs/s')

    if args.copy_probe:
        # byte-counter calibration: a fill (writes 256 MiB) and a kernel copy (reads 256 MiB,
        # writes 256 MiB); tensor copy_ may go to a DMA engine, so the copy is an elementwise kernel
        src = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()

    # roofline of the dominant kernel (k_schur): fp64 MFMA-bound; algorithmic bytes of the pass
    sc = ctx['plan'].scalars
    d, C = ctx['lay']['d'], prob.C
    T = prob.n_tracks
    # pair terms: every pair of observations of a track, self pairs included (batched k_schur forms
    # them all); the pair-major k_pm_pairs forms the off-diagonal ones (its runs pass the rest)
    pair_terms = sc['n_terms'] + n_obs if pm_path else sc['n_pair_terms']
    kernel_terms = sc['n_terms'] if pm_path else sc['n_pair_terms']
    alg = algorithmic_counts(prob, ctx['lay'], pair_terms, sc['n_pairs'])
    kalg = algorithmic_counts(prob, ctx['lay'], kernel_terms, sc['n_pairs'])
    achieved_tf = kalg['flops_dense'] / (schur_ms * 1e-3) / 1e12
    achieved_gbs = alg['bytes'] / (ms_step * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic(args.config, kname)
    pass_traffic = pass_counter_traffic(args.config, PM_PASS_KERNELS if pm_path else PASS_KERNELS)

    # full LM iterations
    lm_ms = lm_ms_direct = None
    if args.lm_steps > 0:
        kw = dict(dtype=torch.float64,
                  weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=o['pnorm'], optim_K=o['optim_K'],
                  optim_P=o['optim_P'])
        engine.lm_step(**g.lm_inputs(), **kw)          # warm (plan cached after this)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.lm_steps):
            engine.lm_step(**g.lm_inputs(), **kw)
        torch.cuda.synchronize()
        lm_ms = (time.perf_counter() - t0) * 1e3 / args.lm_steps
        log(f'[bench] lm_step {lm_ms:.2f} ms')
        # the same step with the reduced system solved directly (solver='cholesky': the reference's
        # _solve_dense_S, ba_solver.py:208-226, in place of its default _solve_CG)
        engine.lm_step(**g.lm_inputs(), **kw, solver='cholesky')
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.lm_steps):
            engine.lm_step(**g.lm_inputs(), **kw, solver='cholesky')
        torch.cuda.synchronize()
        lm_ms_direct = (time.perf_counter() - t0) * 1e3 / args.lm_steps
        log(f'[bench] lm_step with the direct reduced solve {lm_ms_direct:.2f} ms')

    # the reference's default solver precision (GaussNewtonSolver dtype=torch.float32, what lm_step uses
    # without dtype): the same pass in fp32 on the path the solver picks, its dominant kernel against the
    # fp32 MFMA peak, and lm_step called without dtype
    fp32 = None
    if args.lm_steps > 0:
        gs32 = GaussNewtonSolver(len(g.K), len(g.P_w2rig), prob.n_imgs, prob.n_tracks, dev, dtype=torch.float32)
        J32 = gs32.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                                     g.pix2d_dep, True, optim_K=o['optim_K'], optim_P=o['optim_P'], pix2d=g.pix2d,
                                     hp=hp)
        res._ba_state = _param_state(J32)
        ctx32 = gs32.prepare(J32, res, w)
        a32, pm32 = ctx32['args'], ctx32['path'] == 'pairmajor'
        stage = L.ba_pm_linearize_stage if pm32 else L.ba_linearize_stage

        def step32(ev=None):
            check(stage(a32, 0, st))
            if ev is not None:
                ev[0].record()
            check(stage(a32, 1, st))
            if ev is not None:
                ev[1].record()
            if not pm32:
                check(stage(a32, 2, st))
        for _ in range(args.warmup):
            step32()
        ev32 = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(args.steps):
            step32(ev32[k])
        torch.cuda.synchronize()
        ms32 = (time.perf_counter() - t0) * 1e3 / args.steps
        k32_ms = sum(e0.elapsed_time(e1) for e0, e1 in ev32) / args.steps
        k32_tf = kalg['flops_dense'] / (k32_ms * 1e-3) / 1e12 if not pm32 else None
        del gs32, J32, ctx32
        kw32 = {k: v for k, v in kw.items() if k != 'dtype'}
        engine.lm_step(**g.lm_inputs(), **kw32)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.lm_steps):
            engine.lm_step(**g.lm_inputs(), **kw32)
        torch.cuda.synchronize()
        lm32_ms = (time.perf_counter() - t0) * 1e3 / args.lm_steps
        kn32 = 'k_pm_pairs' if pm32 else 'k_schur'
        log(f'[bench] fp32 solver ({"pairmajor" if pm32 else "batched"} path): linearize+Schur {ms32:.3f} ms, {kn32} '
            f'{k32_ms:.3f} ms; lm_step without dtype {lm32_ms:.2f} ms')
        fp32 = {'note': 'GaussNewtonSolver(dtype=torch.float32), what lm_step uses without dtype (the reference default)',
                'path': 'pairmajor' if pm32 else 'batched', 'ms_per_step': ms32, 'obs_per_s': n_obs / (ms32 * 1e-3),
                'kernel': kn32, 'kernel_ms': k32_ms,
                'kernel_fp32_tflops': k32_tf, 'kernel_fp32_frac': (k32_tf / 157.3) if k32_tf else None,
                'lm_ms_per_iter': lm32_ms, 'lm_iters_per_s': 1e3 / lm32_ms}

    red = bench_reduced_solve(prob, g, dev, args.warmup) if args.reduced_solve else None
    smp = bench_sampling(prob, g, dev, args.steps, args.warmup, args.config) if args.sampling else None
    lay = bench_layout(prob, g, dev, args.steps, args.warmup) if args.layout else None
    tan = bench_tangent(prob, g, dev, args.steps, args.warmup) if args.tangent else None

    pm = bench_pairmajor(args.pm_config, dev, args.steps, args.warmup) if args.pm_config >= 0 else None

    cpu = None
    if args.cpu_baseline:
        cpu = cpu_baseline(args.config, prob)
        log(f'[bench] cpu baseline {cpu}')

    triad = stream_triad(dev)
    log(f'[bench] STREAM triad (fp64, 3 x 1 GiB): {triad:.0f} GB/s achievable')
    line = {
        'metric': 'BA linearize+Schur obs/sec & LM iters/sec at 1024 frames; % HBM roofline',
        'value': value, 'unit': 'obs/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
        'ms_per_step': ms_step, 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f64',
        'data': 'synthetic (seeded generator, benchmark config %d)' % args.config,
        'config': {'workload': f'cfg{args.config}: {prob.n_imgs} frames, {T} tracks, {n_obs} observations, '
                               f'C={C}, d={d} image-level parameters, {ctx["path"]} path', 'frames': prob.n_imgs,
                   'tracks': T, 'observations': n_obs, 'C': C, 'path': ctx['path']},
        'lm_iters_per_s': (1e3 / lm_ms) if lm_ms else None,
        'lm_iters_per_s_direct_solve': (1e3 / lm_ms_direct) if lm_ms_direct else None,
        'lm_ms_per_iter': lm_ms,
        'fp32_solver': fp32,
        'roofline': {'bound': 'mfma', 'achieved': achieved_tf, 'peak': 78.6, 'unit': 'TFLOP/s',
                     'frac': achieved_tf / 78.6, 'traffic': traffic, 'kernel': kname,
                     'kernel_ms': schur_ms, 'flops_per_launch': kalg['flops_dense'], 'd_alg': kalg['d_alg'],
                     'pair_terms': kernel_terms,
                     'flops_rule': ('6 d_alg^2 per pair of observations of a track in two images (the off-diagonal '
                                    'terms)' if pm_path else
                                    '6 d_alg^2 per pair of observations of a track (sum over tracks of m(m+1)/2)'),
                     'structured_flops_per_launch': kalg['flops_structured'],
                     'structured_achieved': kalg['flops_structured'] / (schur_ms * 1e-3) / 1e12,
                     'structured_rule': kalg['structured_rule'], 'traffic_source': traffic_src},
        'hbm_roofline': {'achieved': achieved_gbs, 'peak': 8000.0, 'unit': 'GB/s', 'frac': achieved_gbs / 8000.0,
                         'bytes_per_step': alg['bytes'], 'bytes_rule': alg['bytes_rule'],
                         'scope': 'linearize + Schur pass (all stage kernels)', 'achievable_triad': triad,
                         'pass_counter_traffic': pass_traffic['bytes'] if pass_traffic else None,
                         'pass_counter_traffic_over_alg': (pass_traffic['bytes'] / alg['bytes']) if pass_traffic
                         else None,
                         'pass_counter_kernels': pass_traffic['kernels'] if pass_traffic else None},
        'pairmajor': pm,
        'reduced_solve': red,
        'cpu_baseline': cpu,
        'f_sampling': smp,
        'layout': lay,
        'tangent_prior': tan,
    }
    print(json.dumps(line), flush=True)


def bench_layout(prob, g, dev, steps, warmup):
    """Observation-structure edits of the online pipeline at the configuration's size: `old | new`
    (tracks.py:84-102) with old = every observation of the configuration and new = one more frame
    whose 1000 tracks are seen in the last 12 frames, then `remove` of 1% of the tracks
    (tracks.py:116-127) and the rebuild of the structure plan for the merged set; the plan of `old | new`
    made from the old set's plan (ba_plan_append, wall clock with the device copies).  The bare gather
    launch sequence (ba_tracks_gather) is timed with events on its stream; algorithmic bytes per
    output row: one row read and written, 2 (4 + 8 + 8 + 4 C)."""
    import ctypes
    from blast3r_amd._lib import BaGatherArgs, check, lib, ptr, stream_ptr
    from blast3r_amd.data import ObservedTracks, _obs_set, _workspace
    from blast3r_amd.plan import BAPlan
    C, n_imgs, T = prob.C, prob.n_imgs, prob.n_tracks
    cum = g.infos[0].long()
    nppi = torch.diff(torch.cat([cum.new_zeros(1), cum])).to(torch.int32)
    old = ObservedTracks(n_imgs, T, nppi, g.pids, g.pix2d, g.pix2d_std, g.pix2d_dep, 'log_multidepth')
    gen = torch.Generator(device=dev).manual_seed(11)
    nppi_n = torch.zeros(n_imgs + 1, dtype=torch.int32, device=dev)
    nppi_n[-12:] = 1000 * 8 // 12
    m = int(nppi_n.sum())
    new = ObservedTracks(n_imgs + 1, 1000, nppi_n,
                         torch.randint(0, 1000, (m,), device=dev, dtype=torch.int32, generator=gen),
                         torch.rand((m, 2), device=dev, generator=gen) * 500, torch.ones((m, 2), device=dev),
                         torch.rand((m, C), device=dev, generator=gen), 'log_multidepth')
    # the bare launch sequence, arguments prepared once
    sa, ka = _obs_set(old)
    sb, kb = _obs_set(new)
    n_rows = old.n_kpts + new.n_kpts
    out = [torch.empty(n_rows, dtype=torch.int32, device=dev), torch.empty((n_rows, 2), device=dev),
           torch.empty((n_rows, 2), device=dev), torch.empty((n_rows, C), device=dev),
           torch.empty(n_imgs + 1, dtype=torch.int32, device=dev), torch.empty(1, dtype=torch.int64, device=dev)]
    sel_a = torch.cat([torch.arange(n_imgs, dtype=torch.int32), torch.tensor([-1], dtype=torch.int32)]).to(dev)
    sel_b = torch.arange(n_imgs + 1, dtype=torch.int32, device=dev)
    ws = _workspace(dev, n_rows, 0, n_imgs + 1)
    a = BaGatherArgs(a=sa, b=sb, sel_a=ptr(sel_a), sel_b=ptr(sel_b), pid_shift_b=T, C=C, n_out=n_imgs + 1,
                     n_rows=n_rows, pids=ptr(out[0]), pix2d=ptr(out[1]), pix2d_std=ptr(out[2]), pix2d_dep=ptr(out[3]),
                     nppi=ptr(out[4]), total=ptr(out[5]), workspace=ptr(ws))
    L, st = lib(), stream_ptr(dev)
    for _ in range(warmup):
        check(L.ba_tracks_gather(ctypes.byref(a), st))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        check(L.ba_tracks_gather(ctypes.byref(a), st))
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    gbs = n_rows * 2 * (20 + 4 * C) / (ms * 1e-3) / 1e9
    # the Python operations, outputs allocated per call (host waits for the row count, as the reference)
    t0 = time.perf_counter()
    merged = old | new
    torch.cuda.synchronize()
    merge_ms = (time.perf_counter() - t0) * 1e3
    # the structure plan of the merged set, made from the old set's plan (ba_plan_append), as the solver's
    # next lm_step makes it: the old plan is the one the pass above used
    from blast3r_amd.plan import get_plan
    get_plan(g.infos, g.pids, T, device=dev)
    infos_m = torch.stack([torch.cumsum(merged.nppi.long(), 0), torch.arange(n_imgs + 1, device=dev),
                           torch.zeros(n_imgs + 1, dtype=torch.long, device=dev)]).to(torch.int32)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan_m = get_plan(infos_m, merged.pids, merged.n_tracks, device=dev)
    torch.cuda.synchronize()
    append_ms = (time.perf_counter() - t0) * 1e3
    appended = plan_m.stable_prefix is not None
    kept_frac = plan_m.stable_prefix['chunk_ent'] / max(1, plan_m.sizes['chunk_ent']) if appended else 0.0
    del plan_m
    bad = torch.randperm(T + 1000, device=dev, generator=gen)[:(T + 1000) // 100]
    merged.remove(bad)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    kept, _ = merged.remove(bad)
    torch.cuda.synchronize()
    remove_ms = (time.perf_counter() - t0) * 1e3
    infos = torch.stack([torch.cumsum(kept.nppi.long(), 0), torch.arange(n_imgs + 1, device=dev),
                         torch.zeros(n_imgs + 1, dtype=torch.long, device=dev)]).to(torch.int32)
    t0 = time.perf_counter()
    BAPlan(infos, kept.pids, kept.n_tracks)
    torch.cuda.synchronize()
    plan_s = time.perf_counter() - t0
    log(f'[bench] layout: gather {ms:.3f} ms ({gbs:.0f} GB/s algorithmic, {n_rows} rows); old | new {merge_ms:.2f} ms, '
        f'plan of old | new {append_ms:.2f} ms ({"appended, " if appended else "full, "}{kept_frac:.3f} of the MFMA '
        f'entries kept), remove 1% {remove_ms:.2f} ms, plan rebuild {plan_s:.3f} s')
    return {'gather_ms': ms, 'rows': n_rows, 'bytes_per_row': 2 * (20 + 4 * C),
            'roofline': {'bound': 'hbm', 'achieved': gbs, 'peak': 8000.0, 'unit': 'GB/s', 'frac': gbs / 8000.0,
                         'kernel': 'ba_tracks_gather (k_gather_rows + offsets)',
                         'traffic': measured_traffic(2, 'k_gather_rows')[0] if prob.n_imgs == 1024 else None},
            'merge_call_ms': merge_ms, 'remove_call_ms': remove_ms, 'plan_rebuild_s': plan_s,
            'plan_append_ms': append_ms, 'plan_appended': appended, 'plan_append_kept_frac': kept_frac}


def stream_triad(dev, n=1 << 27, reps=10):
    """Achievable HBM bandwidth: ba_stream_triad (a = b + s c, fp64) over three 1 GiB arrays, the best
    of `reps` launches timed with events on the launch stream; 24 bytes moved per element."""
    from blast3r_amd._lib import check, lib, stream_ptr
    a = torch.empty(n, dtype=torch.float64, device=dev)
    b = torch.ones(n, dtype=torch.float64, device=dev)
    c = torch.full((n,), 2.0, dtype=torch.float64, device=dev)
    L, st = lib(), stream_ptr(dev)
    stream = torch.cuda.current_stream(dev)
    best = None
    for r in range(reps + 2):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        check(L.ba_stream_triad(a.data_ptr(), b.data_ptr(), c.data_ptr(), 0.5, n, st))
        e1.record(stream)
        torch.cuda.synchronize()
        if r >= 2:
            ms = e0.elapsed_time(e1)
            best = ms if best is None else min(best, ms)
    assert float(a[0]) == 2.0 and float(a[-1]) == 2.0
    del a, b, c
    return 24 * n / (best * 1e-3) / 1e9


def bench_tangent(prob, g, dev, steps, warmup):
    """Dense tangent prior (ba_tangent_prior) at the configuration's size: one (384, 512, C) log-depth
    map and one (384, 512, 3) reference pointmap per frame, stride 4 (engine.py defaults): the
    fp32 loss of every line-search objective and the fp64 Gauss-Newton terms of every step.  The
    bare launch sequences are timed with events on their stream.  Algorithmic bytes: the sampled
    pixels' C + 3 floats (the kernel reads each once; the cache lines around them come along)."""
    import ctypes
    from blast3r_amd._lib import BaTangentArgs, check, lib, ptr, stream_ptr
    H, W, C, s = 384, 512, prob.C, 4
    n = prob.n_imgs
    gen = torch.Generator(device=dev).manual_seed(13)
    yy, xx = torch.meshgrid(torch.arange(H, device=dev, dtype=torch.float32),
                            torch.arange(W, device=dev, dtype=torch.float32), indexing='ij')
    plane = 3.0 + 0.004 * xx + 0.003 * yy
    maps = torch.empty((n, H, W, C), device=dev)
    maps[..., 0] = torch.log(plane)
    maps[..., 1:] = 0.05 * torch.rand((n, H, W, C - 1), device=dev, generator=gen)
    Kc = g.K[0]
    ray = torch.stack([(xx + 0.5 - Kc[0, 2]) / Kc[0, 0], (yy + 0.5 - Kc[1, 2]) / Kc[1, 1], torch.ones_like(xx)], -1)
    refs = (ray * plane[..., None]).expand(n, H, W, 3).contiguous()
    cam_ids = g.infos[2].to(torch.int32).contiguous()
    Kd = g.K.contiguous()
    zc = g.z_coefs.contiguous()
    dep_addr = maps.data_ptr() + torch.arange(n, device=dev, dtype=torch.int64) * (H * W * C * 4)
    ref_addr = refs.data_ptr() + torch.arange(n, device=dev, dtype=torch.int64) * (H * W * 3 * 4)
    L, st = lib(), stream_ptr(dev)
    res = {}
    for name, gn, fp64 in (('loss_fp32', 0, 0), ('gauss_newton_fp64', 1, 1)):
        loss = torch.empty((), dtype=torch.float64 if fp64 else torch.float32, device=dev)
        gz = torch.empty((n, C), dtype=torch.float64, device=dev)
        hz = torch.empty((n, C, C), dtype=torch.float64, device=dev)
        nb = int(L.ba_tangent_workspace_bytes(n, C, H, W, s, 1, gn))
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        a = BaTangentArgs(depth_addr=ptr(dep_addr), ref_addr=ptr(ref_addr), map_hw=None, H=H, W=W,
                          depth_pix_stride=C, ref_pix_stride=3, K=ptr(Kd), cam_ids=ptr(cam_ids), z_coefs=ptr(zc),
                          n_imgs=n, C=C, tan_stride=s, normalize=1, optim_Z0=1, fp64=fp64, compute_gn=gn, weight=0.5,
                          eps=1e-4, loss=ptr(loss), g_z=ptr(gz), H_z=ptr(hz), workspace=ptr(ws), workspace_bytes=nb)
        for _ in range(warmup):
            check(L.ba_tangent_prior(ctypes.byref(a), st))
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            check(L.ba_tangent_prior(ctypes.byref(a), st))
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        pts = n * ((H - s // 2 + s - 1) // s) * ((W - s // 2 + s - 1) // s)
        gbs = pts * 4 * (C + 3) / (ms * 1e-3) / 1e9
        traffic = measured_traffic(2, 'k_tan_tile_gn' if gn else 'k_tan_tile_loss')[0] if n == 1024 else None
        res[name] = {'ms': ms, 'grid_points': pts, 'algorithmic_GBps': gbs, 'traffic_per_launch': traffic}
    log(f"[bench] tangent prior: loss {res['loss_fp32']['ms']:.3f} ms, GN terms {res['gauss_newton_fp64']['ms']:.3f} ms "
        f"({res['loss_fp32']['grid_points']} grid points, {n} maps of {H}x{W}x{C})")
    return res


def bench_sampling(prob, g, dev, steps, warmup, cfg):
    """F sampling (ba_sample_depth) at the configuration's size: one (384, 512, C) fp32 map per
    frame (C = K + 1 channels with the ones channel stacked, as the reference's maps are) and the
    configuration's observations.  Algorithmic bytes per observation: pixel 8 + four texels 16 C
    read + row 4 C written.  Beside it, the reference's own call sequence on the same GPU (one
    torch grid_sample per frame, geometry.py:183-196)."""
    import torch.nn.functional as F
    import ctypes
    from blast3r_amd._lib import check, lib, stream_ptr
    from blast3r_amd.sampling import prepare_sample
    H, W, C = 384, 512, prob.C
    gen = torch.Generator(device=dev).manual_seed(5)
    maps = torch.rand((prob.n_imgs, H, W, C), device=dev, generator=gen)
    cum = g.infos[0].contiguous()
    pix = g.pix2d.contiguous()
    a, out, keep = prepare_sample(maps, cum, pix)
    L, st = lib(), stream_ptr(dev)
    for _ in range(warmup):
        check(L.ba_sample_depth(ctypes.byref(a), st))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        check(L.ba_sample_depth(ctypes.byref(a), st))
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # the reference's loop (one grid_sample per frame) on the same inputs, for comparison
    cum_h = [0] + g.infos[0].tolist()
    scale = pix.new_tensor([2 / W, 2 / H])

    def ref_loop():
        res = []
        for i in range(prob.n_imgs):
            p = pix[cum_h[i]:cum_h[i + 1]].reshape(1, 1, -1, 2)
            r = F.grid_sample(maps[i:i + 1].permute(0, 3, 1, 2), p * scale - 1, mode='bilinear',
                              padding_mode='border', align_corners=False)
            res.append(r.permute(0, 2, 3, 1).reshape(-1, C))
        return torch.cat(res)

    ref_loop()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        ref_loop()
    torch.cuda.synchronize()
    ref_ms = (time.perf_counter() - t0) * 1e3 / 3
    bytes_alg = prob.n_obs * (8 + 16 * C + 4 * C)
    gbs = bytes_alg / (ms * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic(cfg, 'k_sample')
    log(f'[bench] F sampling {ms:.3f} ms ({prob.n_obs / (ms * 1e-3):.4g} obs/s, {gbs:.0f} GB/s algorithmic); '
        f'torch grid_sample per frame {ref_ms:.2f} ms')
    del maps
    return {'kernel': 'k_sample', 'ms': ms, 'obs_per_s': prob.n_obs / (ms * 1e-3),
            'roofline': {'bound': 'hbm', 'achieved': gbs, 'peak': 8000.0, 'unit': 'GB/s', 'frac': gbs / 8000.0,
                         'bytes_per_launch': bytes_alg, 'traffic': traffic, 'traffic_source': traffic_src},
            'maps': f'{prob.n_imgs} x {H} x {W} x {C} fp32 (uniform random values)',
            'torch_grid_sample_per_frame_ms': ref_ms}


def algorithmic_counts(prob, lay, n_pair_terms, n_pairs):
    """Algorithmic flops and bytes of one linearize + Schur pass.

    d_alg is the per-image block the reduced system needs: 6 pose + C depth coefficients + 2 focal
    parameters when every image has its own camera; a focal shared by all images (mono) is a border
    of 2 unknowns accumulated per track, not per image pair, so it is not in d_alg.
      dense flops: 6 d_alg^2 per pair of observations of one track (S_ij -= V_i V_j^T with V d x 3),
        summed over tracks as m(m+1)/2 pairs;
      structured flops: the same products with the depth-coefficient block of V of rank one (the
        z-coefficient Jacobian is dep_c times one row): per pair 2 x (3*36 pose-pose + 2*(18 + 6C)
        pose-depth + (3 + C^2) depth-depth [+ per-image focal: 12 + 2*36 + 2*(6 + 2C)]) MACs for
        the enabled blocks;
      bytes: per observation pid 4 + pix 8 + std 8 + dep 4C read, per track point 12 + H_pp^-1 24
        + g_p 12, per reduced block 4 d_alg^2 written once, per image 4 d_alg."""
    C = prob.C
    hasP, hasZ = bool(lay['hasP']), bool(lay['hasZ'])
    per_image_K = bool(lay['hasK']) and len(prob.K) == prob.n_imgs and prob.n_imgs > 1
    d_alg = 6 * hasP + C * hasZ + 2 * per_image_K
    mac = 0
    if hasP:
        mac += 3 * 36
    if hasP and hasZ:
        mac += 2 * (18 + 6 * C)
    if hasZ:
        mac += 3 + C * C
    if per_image_K:
        mac += 12 + (2 * 36 if hasP else 0) + (2 * (6 + 2 * C) if hasZ else 0)
    return {'d_alg': d_alg,
            'flops_dense': n_pair_terms * 6 * d_alg * d_alg,
            'flops_structured': n_pair_terms * 2 * mac,
            'structured_rule': f'{2 * mac} flops per pair (rank-one depth block; pose {hasP}, depth {hasZ}, '
                               f'per-image focal {per_image_K})',
            'bytes': prob.n_obs * (20 + 4 * C) + prob.n_tracks * 48 + n_pairs * 4 * d_alg * d_alg
            + prob.n_imgs * 4 * d_alg,
            'bytes_rule': 'N (20 + 4C) + T 48 + N_blk 4 d_alg^2 + F 4 d_alg'}


PASS_KERNELS = ['k_track_pp', 'k_point_factor', 'k_schur', 'k_pair_reduce', 'k_img_reduce']
PM_PASS_KERNELS = ['k_pm_obs', 'k_pm_track', 'k_point_factor', 'k_pm_runs', 'k_pm_diag', 'k_pm_pairs']


def pass_counter_traffic(cfg, kernels_of_pass=PASS_KERNELS):
    """HBM bytes of one linearize + Schur pass from the committed counter summaries of its kernels
    (None unless every one is present)."""
    tot, kernels = 0, {}
    for k in kernels_of_pass:
        b, _ = measured_traffic(cfg, k)
        if b is None:
            return None
        tot += b
        kernels[k] = b
    return {'bytes': tot, 'kernels': kernels}


def bench_pairmajor(cfg, dev, steps, warmup):
    """The pair-major linearize + Schur pass (ba_pm_linearize_schur) on configuration `cfg` at full
    size, inputs resident: observations per second of the pass (HIP events around the launches on
    their stream) and one full lm_step.  Configuration 3 (random co-visibility) is where the solver
    chooses this path."""
    from blast3r_amd import cujac, engine
    from blast3r_amd._lib import check, lib
    from blast3r_amd.ba_solver import GaussNewtonSolver, _param_state
    from blast3r_amd.synthetic import make_problem
    t0 = time.time()
    prob = make_problem(cfg)
    g = prob.to(dev)
    o = prob.options
    hp = dict(weight_z=o['weight_z'], pnorm=o['pnorm'], max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d,
                                            g.pix2d_std, g.pix2d_dep, True, hp['weight_z'], hp['pnorm'],
                                            hp['max_pix_err'], hp['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    gs = GaussNewtonSolver(len(g.K), len(g.P_w2rig), prob.n_imgs, prob.n_tracks, dev, dtype=torch.float64,
                               path='pairmajor')
    J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                             g.pix2d_dep, True, optim_K=o['optim_K'], optim_P=o['optim_P'], pix2d=g.pix2d, hp=hp)
    res._ba_state = _param_state(J)
    ctx = gs.prepare(J, res, w)
    torch.cuda.synchronize()
    sc = ctx['plan'].scalars
    log(f'[bench] pair-major cfg {cfg}: {prob.n_obs} obs, generated + planned in {time.time() - t0:.1f}s: {sc}')
    a, st = ctx['args'], ctx['stream']
    L = lib()
    for _ in range(warmup):
        check(L.ba_pm_linearize_schur(a, st))
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        check(L.ba_pm_linearize_schur(a, st))
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # the dominant kernel alone (stage 1 of the pass: k_pm_pairs, the off-diagonal pair blocks)
    e0.record(stream)
    for _ in range(steps):
        check(L.ba_pm_linearize_stage(a, 1, st))
    e1.record(stream)
    torch.cuda.synchronize()
    pairs_ms = e0.elapsed_time(e1) / steps
    kw = dict(dtype=torch.float64,
              weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=o['pnorm'], optim_K=o['optim_K'],
              optim_P=o['optim_P'])
    engine.lm_step(**g.lm_inputs(), **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n_lm = 2
    for _ in range(n_lm):
        engine.lm_step(**g.lm_inputs(), **kw)
    torch.cuda.synchronize()
    lm_ms = (time.perf_counter() - t0) * 1e3 / n_lm
    # the structure plan built on the device (a structure change), after the build above warmed it
    from blast3r_amd.plan import PMPlan
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    PMPlan(g.infos, g.pids, prob.n_tracks, device=dev)
    torch.cuda.synchronize()
    plan_ms = (time.perf_counter() - t0) * 1e3
    # the reference's default solver precision (GaussNewtonSolver dtype=torch.float32): the same pass in
    # fp32, and lm_step called without dtype
    gs32 = GaussNewtonSolver(len(g.K), len(g.P_w2rig), prob.n_imgs, prob.n_tracks, dev, dtype=torch.float32)
    J32 = gs32.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                                 g.pix2d_dep, True, optim_K=o['optim_K'], optim_P=o['optim_P'], pix2d=g.pix2d, hp=hp)
    ctx32 = gs32.prepare(J32, res, w)
    a32 = ctx32['args']
    for _ in range(warmup):
        check(L.ba_pm_linearize_schur(a32, st))
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        check(L.ba_pm_linearize_schur(a32, st))
    e1.record(stream)
    torch.cuda.synchronize()
    ms32 = e0.elapsed_time(e1) / steps
    kw32 = {k: v for k, v in kw.items() if k != 'dtype'}
    engine.lm_step(**g.lm_inputs(), **kw32)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_lm):
        engine.lm_step(**g.lm_inputs(), **kw32)
    torch.cuda.synchronize()
    lm32_ms = (time.perf_counter() - t0) * 1e3 / n_lm
    del gs32, J32, ctx32
    log(f'[bench] pair-major cfg {cfg}: device plan {plan_ms:.1f} ms; fp32 pass {ms32:.3f} ms, fp32 lm_step '
        f'{lm32_ms:.2f} ms')
    alg = algorithmic_counts(prob, ctx['lay'], sc['n_terms'] + prob.n_obs, sc['n_pairs'])
    v_bytes = sc['n_terms'] * 2 * 3 * (16 if ctx['lay']['d'] <= 15 else 32) * 8
    d_pm = ctx['lay']['d']
    n_diag = int((ctx['plan'].dev['diag_pair'][:prob.n_imgs] >= 0).sum())
    pairs_alg = sc['n_runs'] * 3 * d_pm * 8 + (sc['n_pairs'] - n_diag) * d_pm * d_pm * 8
    pairs_traffic, src = measured_traffic(cfg, 'k_pm_pairs')
    log(f'[bench] pair-major cfg {cfg}: linearize+Schur {ms:.3f} ms -> {prob.n_obs / (ms * 1e-3):.4g} obs/s; '
        f'lm_step {lm_ms:.2f} ms')
    res = {'config': f'cfg{cfg}: {prob.n_imgs} frames, {prob.n_tracks} tracks, {prob.n_obs} observations, C={prob.C}, '
                     f'd={ctx["lay"]["d"]}',
           'ms_per_step': ms, 'obs_per_s': prob.n_obs / (ms * 1e-3), 'lm_ms_per_iter': lm_ms,
           'lm_iters_per_s': 1e3 / lm_ms, 'runs': sc['n_runs'], 'pairs': sc['n_pairs'], 'pair_terms': sc['n_terms'],
           'plan_device_ms': plan_ms,
           'fp32_solver': {'note': 'GaussNewtonSolver(dtype=torch.float32), the reference default lm_step uses',
                           'ms_per_step': ms32, 'obs_per_s': prob.n_obs / (ms32 * 1e-3), 'lm_ms_per_iter': lm32_ms,
                           'lm_iters_per_s': 1e3 / lm32_ms},
           'hbm_roofline': {'achieved': alg['bytes'] / (ms * 1e-3) / 1e9, 'peak': 8000.0, 'unit': 'GB/s',
                            'frac': alg['bytes'] / (ms * 1e-3) / 1e9 / 8000.0, 'bytes_per_step': alg['bytes'],
                            'bytes_rule': alg['bytes_rule']},
           'k_pm_pairs': {'bound': 'hbm', 'v_bytes_per_launch': v_bytes,
                          'v_rule': 'two V rows (3 x dp fp64, dp = 16 for d <= 15) read per pair term',
                          'traffic': pairs_traffic, 'traffic_source': src, 'kernel_ms': pairs_ms},
           'roofline': {'kernel': 'k_pm_pairs', 'bound': 'hbm', 'kernel_ms': pairs_ms,
                        'achieved': pairs_alg / (pairs_ms * 1e-3) / 1e9, 'peak': 8000.0, 'unit': 'GB/s',
                        'frac': pairs_alg / (pairs_ms * 1e-3) / 1e9 / 8000.0, 'traffic': pairs_traffic,
                        'algorithmic_bytes': pairs_alg,
                        'rule': 'algorithmic bytes: every run\'s V (3 x d fp64) read once and every off-diagonal '
                                'S block (d x d fp64) written once, over the kernel time',
                        'requested_bytes': v_bytes,
                        'requested_rate_gbs': v_bytes / (pairs_ms * 1e-3) / 1e9,
                        'fp64_tflops': alg['flops_dense'] * sc['n_terms'] / (sc['n_terms'] + prob.n_obs)
                        / (pairs_ms * 1e-3) / 1e12,
                        'fp64_frac': alg['flops_dense'] * sc['n_terms'] / (sc['n_terms'] + prob.n_obs)
                        / (pairs_ms * 1e-3) / 78.6e12,
                        'fp64_rule': '6 d_alg^2 per off-diagonal term'}}
    del gs, J, ctx, g, prob
    torch.cuda.empty_cache()
    return res


def measured_traffic(cfg, kernel='k_schur'):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary of this workload
    (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter on a plain copy of known size),
    or None when no summary for this configuration is present."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'profiles', f'{kernel}_cfg{cfg}_pmc.json')
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        rec = json.load(f)
    return rec['hbm_bytes_per_launch'], os.path.relpath(path, os.path.dirname(os.path.abspath(__file__)))


def bench_reduced_solve(prob, g, dev, warmup, reps=5):
    """The reduced-system Cholesky (ba_reduced_solve, solver='cholesky') on the configuration's
    damped reduced system, banded (block cyclic reduction where it applies), banded by one workgroup, and
    dense layouts: the bare launch sequence (assembly of S_u from the image-pair blocks, factorisation,
    both triangular sweeps) timed with events on its stream, beside the device PCG's solve.  fp64 flops:
    dense n^3/3 + 2 n^2; banded n b^2 + 4 n b with b the scalar bandwidth (w + 1) d_band (the band
    factor's own count: the cyclic reduction issues more, 128^3 x ~7 per super-block and level).
    Beside them, the reference's own call (torch.linalg.solve, ba_solver.py:220) on the same dense S_u
    (rebuilt as L L^T from the dense factor) on the same GPU."""
    from blast3r_amd._lib import check, lib
    from blast3r_amd.ba_solver import GaussNewtonSolver
    o = prob.options
    hp = dict(weight_z=o['weight_z'], pnorm=o['pnorm'], max_pix_err=o['clip_pix_err'], huber_delta=o['huber_delta'])
    from blast3r_amd import cujac
    out = cujac.compute_residuals_with_rigs(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d,
                                            g.pix2d_std, g.pix2d_dep, True, hp['weight_z'], hp['pnorm'],
                                            hp['max_pix_err'], hp['huber_delta'])
    res, err, w = out.view(-1, 3, 3).unbind(dim=1)
    L = lib()
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    result = {}
    for layout in ('banded', 'banded_sequential', 'dense'):
        gs = GaussNewtonSolver(len(g.K), len(g.P_w2rig), prob.n_imgs, prob.n_tracks, dev, dtype=torch.float64, solver='cholesky',
                               cholesky_layout=layout)
        J = gs.compute_jacobians(g.infos, g.K, g.P_rig2cam, g.P_w2rig, g.z_coefs, g.pts3d, g.pids, g.pix2d_std,
                                 g.pix2d_dep, True, optim_K=o['optim_K'], optim_P=o['optim_P'], pix2d=g.pix2d, hp=hp)
        try:
            gs.solve_delta(J, res, w)
        except RuntimeError as e:
            result[layout] = {'error': str(e)}
            continue
        info = gs.last['direct']
        if info is None or info.get('first_bad_pivot') is not None or info['layout'] != layout:
            result[layout] = {'error': f'not run as {layout}: {info}'}
            continue
        pa, ca = gs.last['direct_call']
        for _ in range(warmup):
            check(L.ba_reduced_solve(pa, ca, st))
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            check(L.ba_reduced_solve(pa, ca, st))
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        n = int(pa.n_u)
        if layout == 'dense':
            flops = n ** 3 / 3 + 2 * n * n
        else:
            b = (info['w'] + 1) * info['db']
            flops = n * b * b + 4 * n * b
        result[layout] = {'ms': ms, 'unknowns': n, 'flops': flops, 'achieved_tflops': flops / (ms * 1e-3) / 1e12,
                          'frac_of_fp64_peak': flops / (ms * 1e-3) / 1e12 / 78.6, 'w': info['w'], 'd_band': info['db'],
                          'shared': info['n_shared'], 'superblocks': info.get('superblocks', 0)}
        log(f'[bench] reduced solve ({layout}): {ms:.2f} ms for {n} unknowns, '
            f'{flops / (ms * 1e-3) / 1e12:.2f} TFLOP/s fp64' +
            (f', {info["superblocks"]} super-blocks' if info.get('superblocks') else ''))
        if layout == 'dense':
            # the reference's call on the same system: S_u = L L^T from the factor just computed
            Lt = torch.tril(gs.last['direct_A'][:n, :n])
            S = Lt @ Lt.T
            rhs = torch.randn(n, 1, dtype=torch.float64, device=dev)
            for _ in range(max(1, warmup)):
                torch.linalg.solve(S, rhs)
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(reps):
                torch.linalg.solve(S, rhs)
            e1.record(stream)
            torch.cuda.synchronize()
            ms_t = e0.elapsed_time(e1) / reps
            result['torch_linalg_solve'] = {'ms': ms_t, 'unknowns': n,
                                            'call': 'torch.linalg.solve(S, rhs), ba_solver.py:220'}
            log(f'[bench] reference call torch.linalg.solve on the same {n} x {n} S_u: {ms_t:.2f} ms')
            del S, Lt
        del gs, J
    torch.cuda.empty_cache()
    return result


def host_cpu():
    """Model name and logical CPU count of this host (the CPU baseline's machine)."""
    model = None
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    return {'model': model, 'logical_cpus': os.cpu_count()}


CPU_PCG_CAP = 5


def cpu_baseline(cfg, prob=None):
    """The oracle (torch-CPU restatement of the reference's path) on the full configuration, on this
    host's CPU share (OMP_NUM_THREADS when set, as on the GPU boxes, else every logical CPU):
      * value: observations per second of one linearize + Schur-rhs pass in fp64 (residuals, fp64
        Jacobians, normal equations, reduced rhs), the reference's solver dtype;
      * fp32: the same pass with fp32 Jacobians and normal equations;
      * lm_step: one full oracle lm_step (objective, linearisation, Schur, PCG capped at CPU_PCG_CAP
        iterations, back-substitution, line search) -- LM iterations per second at that cap, and the
        time of one PCG iteration (one S v product of the Schur operator plus the vector work), from
        which the 300-iteration step is estimated.
    About 20-60 s of CPU work at configuration 2."""
    import oracle.kernels as ok
    import oracle.solver as osol
    import oracle.engine as oeng
    from blast3r_amd.synthetic import make_problem
    threads = int(os.environ.get('OMP_NUM_THREADS') or 0) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    p = prob if prob is not None else make_problem(cfg)
    o = p.options

    def npass(float64):
        t0 = time.perf_counter()
        loss, res, w = oeng.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                      p.pix2d_std, p.pix2d_dep, True, o['weight_z'], o['pnorm'], o['clip_pix_err'],
                                      o['huber_delta'])
        Jc, Jz, Jp = ok.jacobians_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids,
                                            p.pix2d_std, p.pix2d_dep, True, float64=float64)
        pr = osol.Problem(p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks, p.C)
        ne, g, params = osol.build_normal_equations(pr, Jc, Jz, Jp, res, w, optim_K=o['optim_K'], optim_P=o['optim_P'])
        rhs = osol.reduced_rhs(ne, g)
        dt = time.perf_counter() - t0
        return dt, ne, rhs

    dt64, ne, rhs = npass(True)
    # one PCG iteration's operator: S v plus the preconditioner and vector updates
    v = torch.randn(rhs.shape[0], dtype=torch.float64)
    t0 = time.perf_counter()
    osol.S_matvec(ne, v)
    t_mv = time.perf_counter() - t0
    del ne
    dt32, ne32, _ = npass(False)
    del ne32
    kw = dict(dtype=torch.float64,
              weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=o['pnorm'], clip_pix_err=o['clip_pix_err'],
              optim_K=o['optim_K'], optim_P=o['optim_P'])
    t0 = time.perf_counter()
    _, st, info = oeng.lm_step(**p.lm_inputs(), **kw, pcg_maxiter=CPU_PCG_CAP)
    t_lm = time.perf_counter() - t0
    est300 = t_lm + (300 - CPU_PCG_CAP) * t_mv
    return {'value': p.n_obs / dt64, 'unit': 'obs/s', 'cores': threads, 'kind': 'port',
            'sample': f'the full cfg{cfg} workload ({p.n_imgs} frames, {p.n_tracks} tracks, {p.n_obs} obs): one '
                      f'fp64 pass of residuals, Jacobians, normal equations and Schur rhs in the oracle ({dt64:.2f} s), '
                      f'the fp32 variant ({dt32:.2f} s), one S v product ({t_mv:.2f} s) and one oracle lm_step with '
                      f'PCG capped at {CPU_PCG_CAP} iterations ({t_lm:.2f} s, {info["trials"]} line-search trials)',
            'host': host_cpu(), 'threads': threads,
            'fp32_obs_per_s': p.n_obs / dt32,
            'lm_step_s_at_pcg_cap': t_lm, 'pcg_cap': CPU_PCG_CAP, 'lm_iters_per_s_at_pcg_cap': 1.0 / t_lm,
            'pcg_iteration_s': t_mv, 'lm_step_s_estimated_300_pcg': est300,
            'lm_iters_per_s_estimated_300_pcg': 1.0 / est300}


if __name__ == '__main__':
    main()
