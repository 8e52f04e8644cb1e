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
launch stream) and the CPU oracle timed on a bounded sample of the same
workload.
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
    ap.add_argument('--copy-probe', action='store_true',
                    help='run a 256 MiB fill and a 256 MiB kernel copy (calibrates FETCH_SIZE / WRITE_SIZE counters)')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one MI355X: multi-GPU runs are not part of this build '
              '(the path would shard by track with one all-reduce of the reduced system; see DESIGN.md)',
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
    gs = GaussNewtonSolver(len(g.K), len(g.P_w2rig), prob.n_imgs, prob.n_tracks, dev)
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

    def step(ev=None):
        check(L.ba_linearize_stage(a, 0, st))
        if ev is not None:
            ev[0].record()
        check(L.ba_linearize_stage(a, 1, st))
        if ev is not None:
            ev[1].record()
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
    log(f'[bench] linearize+Schur {ms_step:.3f} ms/step, k_schur {schur_ms:.3f} ms -> {value:.4g} obs/s')

    if args.copy_probe:
        # byte-counter calibration: a fill (writes 256 MiB) and a kernel copy (reads 256 MiB,
        # writes 256 MiB); tensor copy_ may go to a DMA engine, so the copy is an elementwise kernel
        src = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()

    # roofline of the dominant kernel (k_schur): fp64 MFMA-bound.  Algorithmic flops per launch =
    # 6 d^2 per (track, image pair) term and per observation (the J_c^T J_c term), d = image-level
    # parameters; algorithmic bytes of the whole linearize + Schur pass = per observation
    # pid 4 + pix 8 + std 8 + dep 4C, per track point 12 + H_pp^-1 24 + g_p 12, per reduced
    # block d^2 fp64 written once, per image g_c d fp64.
    sc = ctx['plan'].scalars
    d, C = ctx['lay']['d'], prob.C
    T = prob.n_tracks
    bytes_alg = n_obs * (20 + 4 * C) + T * 48 + sc['n_pairs'] * d * d * 8 + prob.n_imgs * d * 8
    flops_pairs = (sc['n_pair_terms'] + n_obs) * 6 * d * d
    achieved_tf = flops_pairs / (schur_ms * 1e-3) / 1e12
    achieved_gbs = bytes_alg / (ms_step * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic(args.config)

    # full LM iterations
    lm_ms = None
    if args.lm_steps > 0:
        kw = dict(weight_z=o['weight_z'], huber_delta=o['huber_delta'], pnorm=o['pnorm'], optim_K=o['optim_K'],
                  optim_P=o['optim_P'])
        engine.lm_step(**g.lm_inputs(), **kw)          # warm (plan cached after this)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.lm_steps):
            engine.lm_step(**g.lm_inputs(), **kw)
        torch.cuda.synchronize()
        lm_ms = (time.perf_counter() - t0) * 1e3 / args.lm_steps
        log(f'[bench] lm_step {lm_ms:.2f} ms')

    smp = bench_sampling(prob, g, dev, args.steps, args.warmup, args.config) if args.sampling else None
    lay = bench_layout(prob, g, dev, args.steps, args.warmup) if args.layout else None
    tan = bench_tangent(prob, g, dev, args.steps, args.warmup) if args.tangent else None

    cpu = None
    if args.cpu_baseline:
        cpu = cpu_baseline(args.config)
        log(f'[bench] cpu baseline {cpu}')

    triad = stream_triad(dev)
    log(f'[bench] STREAM triad (fp64, 3 x 1 GiB): {triad:.0f} GB/s achievable')
    line = {
        'metric': 'BA linearize+Schur obs/sec & LM iters/sec at 1024 frames; % HBM roofline',
        'value': value, 'unit': 'obs/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
        'ms_per_step': ms_step, 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f64',
        'data': 'synthetic (seeded generator, benchmark config %d)' % args.config,
        'config': {'workload': f'cfg{args.config}: {prob.n_imgs} frames, {T} tracks, {n_obs} observations, '
                               f'C={C}, d={d} image-level parameters', 'frames': prob.n_imgs, 'tracks': T,
                   'observations': n_obs, 'C': C},
        'lm_iters_per_s': (1e3 / lm_ms) if lm_ms else None,
        'lm_ms_per_iter': lm_ms,
        'roofline': {'bound': 'mfma', 'achieved': achieved_tf, 'peak': 78.6, 'unit': 'TFLOP/s',
                     'frac': achieved_tf / 78.6, 'traffic': traffic, 'kernel': 'k_schur',
                     'kernel_ms': schur_ms, 'flops_per_launch': flops_pairs, 'traffic_source': traffic_src},
        'hbm_roofline': {'achieved': achieved_gbs, 'peak': 8000.0, 'unit': 'GB/s', 'frac': achieved_gbs / 8000.0,
                         'bytes_per_step': bytes_alg, 'scope': 'linearize + Schur pass (all stage kernels)',
                         'achievable_triad': triad},
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
    (tracks.py:116-127) and the rebuild of the structure plan for the merged set.  The bare gather
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
        f'remove 1% {remove_ms:.2f} ms, plan rebuild {plan_s:.3f} s')
    return {'gather_ms': ms, 'rows': n_rows, 'bytes_per_row': 2 * (20 + 4 * C),
            'roofline': {'bound': 'hbm', 'achieved': gbs, 'peak': 8000.0, 'unit': 'GB/s', 'frac': gbs / 8000.0,
                         'kernel': 'ba_tracks_gather (k_gather_rows + offsets)',
                         'traffic': measured_traffic(2, 'k_gather_rows')[0] if prob.n_imgs == 1024 else None},
            'merge_call_ms': merge_ms, 'remove_call_ms': remove_ms, 'plan_rebuild_s': plan_s}


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


def cpu_baseline(cfg, reps=3):
    """Oracle (torch-CPU restatement of the reference's linearisation + normal equations + Schur
    rhs) on the full configuration, timed on this host over `reps` passes (about 10-30 s of CPU
    work at configuration 2)."""
    import oracle.kernels as ok
    import oracle.solver as osol
    import oracle.engine as oeng
    from blast3r_amd.synthetic import make_problem
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    p = make_problem(cfg)
    o = p.options
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        loss, res, w = oeng.objective(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids, p.pix2d,
                                      p.pix2d_std, p.pix2d_dep, True, o['weight_z'], o['pnorm'], o['clip_pix_err'],
                                      o['huber_delta'])
        Jc, Jz, Jp = ok.jacobians_with_rigs(p.infos, p.K, p.P_rig2cam, p.P_w2rig, p.z_coefs, p.pts3d, p.pids,
                                            p.pix2d_std, p.pix2d_dep, True, float64=True)
        prob = osol.Problem(p.infos, p.pids, len(p.K), len(p.P_w2rig), p.n_tracks, p.C)
        ne, g, params = osol.build_normal_equations(prob, Jc, Jz, Jp, res, w, optim_K=o['optim_K'],
                                                    optim_P=o['optim_P'])
        osol.reduced_rhs(ne, g)
        times.append(time.perf_counter() - t0)
        del Jc, Jz, Jp, ne, g, params
    dt = sum(times) / len(times)
    return {'value': p.n_obs / dt, 'unit': 'obs/s', 'cores': threads, 'kind': 'port',
            'sample': f'the full cfg{cfg} workload ({p.n_imgs} frames, '
                      f'{p.n_tracks} tracks, {p.n_obs} obs), {reps} passes of residuals, fp64 Jacobians, normal '
                      f'equations and Schur rhs in the oracle: {sum(times):.1f} s in total, {dt:.2f} s per pass'}


if __name__ == '__main__':
    main()
