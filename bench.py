"""Benchmark: graph-captured training step and forward render on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--no-cpu-baseline]

Headline (`value`): training iterations per second at G=100k (clustered), 1264x832, K=128,
8 orbit cameras round-robin (one camera per step), fp32: each step is geometry fwd, binning,
fused splat fwd, L1+SSIM loss gradient, fused splat bwd (+theta bwd, per-slot gradients),
slot gather + geometry bwd + Adam, replayed as one HIP graph per camera.  Inputs are resident
on the GPU before the timed region; the timed region is exactly K steps between two
synchronisations.

Also reported: forward fps (geometry + binning + splat, graph replay) for the same scene, the
G=2000 128x128, G=10k 800x800 and G=1M 1920x1072 numbers, per-kernel times from HIP events on
the launch stream, the roofline of the dominant kernel, and the CPU oracle (PyTorch-CPU
restatement of the reference path) timed on this host's cores, and on one thread, on bounded
samples of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "tt-splat_amd"), ROOT]

METRIC = "train it/s + render fps (G2k res128, G100k 1264×832), % of HBM/VALU roofline"
PEAK_FP32_TFLOPS = 157.3      # MI355X published FP32 vector/matrix peak
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
FLOP_PER_PAIR = {"splat_fwd": 22.0, "splat_bwd": 44.0}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--config", default="c4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--kernel-reps", type=int, default=100)
    ap.add_argument("--no-small", action="store_true", help="skip the G=2000 128x128 run")
    ap.add_argument("--no-c3", action="store_true", help="skip the G=10k 800x800 run")
    ap.add_argument("--no-c5", action="store_true", help="skip the G=1M 1920x1072 batch run")
    ap.add_argument("--c5-batches", type=int, default=3)
    ap.add_argument("--no-sh", action="store_true",
                    help="skip the SH degree 3 run of the headline workload")
    ap.add_argument("--no-mcmc", action="store_true",
                    help="skip the MCMC density-control run of the headline workload")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB 5 times (a known-size "
                         "kernel to calibrate hardware byte counters against)")
    return ap.parse_args()


def load_traffic(kernel, cfg_name):
    """HBM bytes per launch of `kernel` on this workload, measured with rocprofv3 PMC counters
    (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy) and recorded in
    profiles/traffic.json; None when no measurement is recorded."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f).get(f"{kernel}/{cfg_name}")
    return None if rec is None else rec.get("bytes_per_launch")


def sh_rest_init(torch, G, seed, scale=0.1):
    """Synthetic SH rest coefficients [G,15,3] (seeded normal draws)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(G, 15, 3, generator=g) * scale


def build_step(cfg, torch, TrainStep, batch=1, sh_degree=0, mcmc=None):
    """TrainStep for the configuration; targets are the GPU render of the seed-1 set (with
    sh_degree > 0: SH rest coefficients drawn from seeds 4 (target) and 3 (trained set))."""
    cams = cfg.cameras()
    P0 = cfg.params(seed=0)
    zero = torch.zeros(cfg.H, cfg.W, 3, device="cuda")
    sh_t = dict(sh_degree=sh_degree, sh_rest=sh_rest_init(torch, cfg.G, 4)) if sh_degree else {}
    sh_0 = dict(sh_degree=sh_degree, sh_rest=sh_rest_init(torch, cfg.G, 3)) if sh_degree else {}
    tgt_maker = TrainStep(cfg.params(seed=1), cams, [zero] * len(cams), K=cfg.K, S=cfg.S,
                          k=cfg.k, dtype=cfg.dtype, **sh_t)
    targets = []
    for ci in range(len(cams)):
        targets.append(tgt_maker.forward(ci).clone())
    del tgt_maker, zero
    ts = TrainStep(P0, cams, targets, K=cfg.K, S=cfg.S, k=cfg.k, batch=batch, dtype=cfg.dtype,
                   mcmc=mcmc, **sh_0)
    return ts


def time_train(ts, steps, warmup, torch):
    ncam = ts.n_steps
    ts.capture()
    for i in range(warmup):
        ts.step(i % ncam)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ts.step((warmup + i) % ncam)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def time_forward(ts, steps, warmup, torch):
    ncam = len(ts.cams)
    graphs = []
    for ci in range(ncam):
        ts.forward(ci)
    torch.cuda.synchronize()
    for ci in range(ncam):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ts.forward(ci)
        graphs.append(g)
    for i in range(warmup):
        graphs[i % ncam].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        graphs[i % ncam].replay()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def time_kernels(ts, reps, torch, kernels):
    """Average duration of each kernel group at the current state (camera 0), from HIP events
    recorded on the stream the kernels are launched on."""
    ts.enqueue(0)                       # bring every buffer to a consistent step state
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    P_save, m_save, v_save, s_save = (t.clone() for t in (ts.P, ts.m, ts.v, ts.step_block))
    cam = ts.cams[0]
    sh = dict(sh_rest=ts.sh, sh_degree=ts.sh_degree)
    shs = [ts.sh, ts.sh_m, ts.sh_v] if ts.sh is not None else []
    saved_sh = [t.clone() for t in shs]
    jobs = {
        "geom_fwd": lambda: kernels.geom_fwd(ts.P, cam, proj=ts.proj, keep=ts.keep, **sh),
        "binning": lambda: kernels.assign_bins(ts.proj[:, 0:2], ts.keep, ts.H, ts.W, ts.S, ts.K,
                                               ts.span, 1, ts.bin_ws, ts.idx, ts.valid,
                                               ts.count, ts.ncand, ts.inv, ts.order),
        "splat_fwd": (lambda: kernels.splat_fwd_mx(ts.proj, ts.idx, ts.valid, ts.bg, ts.H, ts.W,
                                                   ts.S, ts.k, ts.image, ts.den, ts.order,
                                                   bf16=True))
        if ts.dtype == "bf16" else
        (lambda: kernels.splat_fwd(ts.proj, ts.idx, ts.valid, ts.bg, ts.H, ts.W, ts.S, ts.k,
                                   ts.image, ts.den, ts.order)),
        "loss_grad": lambda: kernels.loss_grad(ts.image, ts.targets[0], ts.lam, ts.gimage,
                                               ts.partials, ts.loss_ws),
        "splat_bwd": lambda: kernels.splat_bwd(ts.proj, ts.idx, ts.valid, ts.bg, ts.H, ts.W,
                                               ts.S, ts.k, ts.image, ts.den, ts.gimage,
                                               ts.gslot, order=ts.order),
        "geom_bwd_adam": lambda: kernels.geom_bwd_adam(ts.P, cam, ts.gslot, ts.inv, ts.m, ts.v,
                                                       ts.lr, ts.step_block, sh_m=ts.sh_m,
                                                       sh_v=ts.sh_v, lr_sh=ts.lr_sh, **sh),
    }
    if ts.batch > 1:
        del jobs["geom_bwd_adam"]
        jobs["geom_bwd_accum"] = lambda: kernels.geom_bwd_accum(ts.P, cam, ts.gslot, ts.inv,
                                                                ts.gacc, 1.0 / ts.batch,
                                                                gacc_sh=ts.gacc_sh, **sh)
    out = {}
    for name, fn in jobs.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        e1.synchronize()
        out[name] = e0.elapsed_time(e1) / reps * 1e3      # microseconds per launch
    # restore the state the measurement perturbed
    for dst, src in zip((ts.P, ts.m, ts.v, ts.step_block, *shs),
                        (P_save, m_save, v_save, s_save, *saved_sh)):
        dst.copy_(src)
    if ts.gacc is not None:
        ts.gacc.zero_()
    if ts.gacc_sh is not None:
        ts.gacc_sh.zero_()
    ts.forward(0)
    torch.cuda.synchronize()
    return out


def splat_bytes(ts, torch):
    """Algorithmic HBM bytes of one fused splat launch at the current bins: per tile
    40 B per valid slot (theta 6 + col 3 + oc 1, fp32) + 4 B per slot of the bin table,
    12 B per pixel of image; the backward adds 16 B per pixel (dL/dC, den) and 36 B per valid
    slot (the slot's 9 gradients)."""
    nvalid = int(ts.count.long().sum())
    T, P = ts.tmap.T, ts.H * ts.W
    fwd = 40 * nvalid + 4 * ts.K * T + 12 * P
    return fwd, fwd + 16 * P + 36 * nvalid


def run_c3(args, torch, scenes, TrainStep):
    cfg = scenes.CONFIGS["c3"]
    ts = build_step(cfg, torch, TrainStep)
    n = 300
    its = n / time_train(ts, n, 30, torch)
    fps = n / time_forward(ts, n, 30, torch)
    return dict(c3_train_its=its, c3_train_ms=1e3 / its, c3_fwd_fps=fps, c3_fwd_ms=1e3 / fps)


def run_sh(args, torch, scenes, kernels, TrainStep):
    """The headline workload with view-dependent colour: SH degree 3 (45 rest coefficients per
    gaussian, trained with Adam in the fused geometry backward)."""
    cfg = scenes.CONFIGS[args.config]
    ts = build_step(cfg, torch, TrainStep, sh_degree=3)
    n = 300
    its = n / time_train(ts, n, 30, torch)
    fps = n / time_forward(ts, n, 30, torch)
    kt = time_kernels(ts, 50, torch, kernels)
    return dict(sh3_train_its=its, sh3_fwd_fps=fps,
                sh3_kernel_us={k: kt[k] for k in ("geom_fwd", "geom_bwd_adam")},
                sh3_note="SH degree 3 view-dependent colour on the same workload")


MCMC_OPTS = dict(lambda_o=0.01, lambda_s=0.01, noise_lr=5e5, relocate_every=100,
                 dead_thr=0.005, offset=0.005, seed=1)


def run_mcmc(args, torch, scenes, TrainStep):
    """The headline workload with fixed-count MCMC density control (spike/mcmc.py defaults:
    regulariser 0.01/0.01, SGLD noise_lr 5e5, relocation every 100 steps, threshold 0.005),
    starting with a seeded 10 % of the gaussians dead (opacity 1e-3): train it/s over 300 steps
    (3 relocations inside the timed region), then one relocation of a fresh 10 % dead set timed
    with HIP events (state restored before each repetition)."""
    import math
    cfg = scenes.CONFIGS[args.config]
    ts = build_step(cfg, torch, TrainStep, mcmc=MCMC_OPTS)
    g = torch.Generator().manual_seed(5)
    dead = (torch.rand(cfg.G, generator=g) < 0.1).cuda()
    dead_op = math.log(1e-3 / (1 - 1e-3))
    ts.P[dead, 13] = dead_op
    n = 300
    its = n / time_train(ts, n, 30, torch)
    relocated = int(ts.relocations)
    snap = ts.P.clone()
    snap[dead, 13] = dead_op
    stream = torch.cuda.current_stream()
    reps, total_ms = 20, 0.0
    for _ in range(reps):
        ts.P.copy_(snap)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        ts.reloc_graph.replay()
        e1.record(stream)
        e1.synchronize()
        total_ms += e0.elapsed_time(e1)
    return dict(mcmc_train_its=its, mcmc_relocate_us=total_ms / reps * 1e3,
                mcmc_relocate_moved=int(ts.moved), mcmc_relocations_in_run=relocated,
                mcmc_opts=MCMC_OPTS)


def run_c5(args, torch, scenes, kernels, TrainStep):
    """G=1M clustered, 1920x1072, K=256: batches of 64 views (fwd + bwd of every view, mean
    gradient, one Adam update), one graph per batch."""
    cfg = scenes.CONFIGS["c5"]
    ts = build_step(cfg, torch, TrainStep, batch=len(cfg.cameras()))
    nb = max(1, args.c5_batches)
    t_batch = time_train(ts, nb, 1, torch) / nb
    # forward only, all 64 views, one graph
    for ci in range(len(ts.cams)):
        ts.forward(ci)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for ci in range(len(ts.cams)):
            ts.forward(ci)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(nb):
        g.replay()
    torch.cuda.synchronize()
    t_fwd = (time.perf_counter() - t0) / nb
    # overflow over the batch: candidates beyond the budget K
    cand = over = kept = 0
    for ci in range(len(ts.cams)):
        ts.forward(ci)
        nc = ts.ncand.long()
        cand += int(nc.sum())
        over += int((nc - ts.K).clamp(min=0).sum())
        kept += int(ts.count.long().sum())
    kt = time_kernels(ts, 20, torch, kernels)
    bf, bb = splat_bytes(ts, torch)
    nv = len(ts.cams)
    return dict(
        c5_views_per_batch=nv, c5_batch_ms=t_batch * 1e3, c5_train_views_per_s=nv / t_batch,
        c5_fwd_views_per_s=nv / t_fwd, c5_overflow_rate=over / max(cand, 1),
        c5_candidates_per_view=cand / nv, c5_kept_per_view=kept / nv,
        c5_kernel_us_view0=kt,
        c5_binning_gaussians_per_s=cfg.G / (kt["binning"] * 1e-6),
        c5_splat_fwd_GBs=bf / (kt["splat_fwd"] * 1e-6) / 1e9,
        c5_splat_bwd_GBs=bb / (kt["splat_bwd"] * 1e-6) / 1e9,
        c5_dtype="bf16 render forward, fp32 backward/params/Adam",
        c5_crop="1080 rows cropped to 1072 (whole 16-px tiles)")


def cpu_baseline(cfg, seconds, torch):
    """The oracle's training step (autograd through the PyTorch-CPU restatement of the
    reference path, torch.optim-equivalent Adam) on this host, camera 0, bounded sample."""
    from oracle import binning as obin
    from oracle import pipeline as opipe
    from oracle import splat as osplat
    cam = cfg.cameras()[0].as_dict()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    P = cfg.params(seed=0)
    with torch.no_grad():
        tgt = osplat.render_binned(cfg.params(seed=1), cam, tmap, K=cfg.K, k=cfg.k)
    m = torch.zeros_like(P)
    v = torch.zeros_like(P)
    lr = torch.full((14,), 1e-3)
    lr[:3] = 1.6e-4
    opipe.train_step(P, m, v, 1, cam, tmap, tgt, lr, K=cfg.K, k=cfg.k)     # warm-up
    n, t0 = 0, time.perf_counter()
    while n < 2 or time.perf_counter() - t0 < seconds:
        opipe.train_step(P, m, v, n + 2, cam, tmap, tgt, lr, K=cfg.K, k=cfg.k)
        n += 1
    dt = time.perf_counter() - t0
    nf, t1 = 0, time.perf_counter()
    with torch.no_grad():
        while nf < 2 or time.perf_counter() - t1 < seconds / 3:
            osplat.render_binned(P, cam, tmap, K=cfg.K, k=cfg.k)
            nf += 1
    df = time.perf_counter() - t1
    cores = torch.get_num_threads()
    # the same train step on one thread (a shorter bounded sample)
    torch.set_num_threads(1)
    try:
        n1, t2 = 0, time.perf_counter()
        while n1 < 1 or time.perf_counter() - t2 < seconds / 3:
            opipe.train_step(P, m, v, n + n1 + 2, cam, tmap, tgt, lr, K=cfg.K, k=cfg.k)
            n1 += 1
        d1 = time.perf_counter() - t2
    finally:
        torch.set_num_threads(cores)
    return dict(value=n / dt, unit="it/s", cores=cores, kind="port",
                sample=f"{n} oracle train steps ({dt:.1f} s) + {nf} forwards ({df:.1f} s) "
                       f"after 1 warm-up, {cfg.name} camera 0",
                fwd_fps=nf / df,
                one_thread=dict(value=n1 / d1, unit="it/s", cores=1,
                                sample=f"{n1} oracle train steps ({d1:.1f} s)"))


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on exactly one GPU: the training step has no multi-GPU path "
              "(one process, one device); run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from ttsplat import kernels, scenes
    from ttsplat.step import TrainStep

    cfg = scenes.CONFIGS[args.config]
    torch.cuda.set_device(0)
    ts = build_step(cfg, torch, TrainStep)
    train_s = time_train(ts, args.steps, args.warmup, torch)
    its = args.steps / train_s
    fwd_s = time_forward(ts, args.steps, args.warmup, torch)
    fps = args.steps / fwd_s
    loss_last = float(ts.loss())
    kt = time_kernels(ts, args.kernel_reps, torch, kernels)
    pairs = int(ts.count.long().sum()) * ts.S * ts.S
    rows = {}
    for name in ("splat_fwd", "splat_bwd"):
        flops = FLOP_PER_PAIR[name] * pairs
        tfl = flops / (kt[name] * 1e-6) / 1e12
        rows[name] = dict(us=kt[name], tflops=tfl, frac=tfl / PEAK_FP32_TFLOPS)
    dom = max(("splat_fwd", "splat_bwd"), key=lambda n: kt[n])
    roofline = dict(bound="valu", kernel=dom, achieved=rows[dom]["tflops"], peak=PEAK_FP32_TFLOPS,
                    unit="TFLOP/s", frac=rows[dom]["frac"], traffic=load_traffic(dom, cfg.name),
                    flops_per_launch=FLOP_PER_PAIR[dom] * pairs, pairs_per_launch=pairs,
                    us_per_launch=kt[dom])
    # the small configuration (G=2000, 128x128)
    its2 = fps2 = None
    if not args.no_small:
        small = scenes.CONFIGS["c2"]
        ts2 = build_step(small, torch, TrainStep)
        its2 = 1000 / time_train(ts2, 1000, 50, torch)
        fps2 = 1000 / time_forward(ts2, 1000, 50, torch)
    extra_c3 = {} if args.no_c3 else run_c3(args, torch, scenes, TrainStep)
    extra_c5 = {} if args.no_c5 else run_c5(args, torch, scenes, kernels, TrainStep)
    extra_sh = {} if args.no_sh else run_sh(args, torch, scenes, kernels, TrainStep)
    extra_mc = {} if args.no_mcmc else run_mcmc(args, torch, scenes, TrainStep)
    if args.copy_mib:
        src = torch.ones(args.copy_mib * (1 << 18), device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(cfg, args.cpu_seconds, torch)
    out = {
        "metric": METRIC,
        "value": its,
        "unit": "it/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": train_s / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": f"{cfg.name}: training step, G={cfg.G} "
                               f"{'clustered' if cfg.means == 'clustered' else 'uniform'} "
                               f"gaussians, {cfg.W}x{cfg.H}, K={cfg.K}, S={cfg.S}, k={cfg.k}, "
                               f"{len(ts.cams)} orbit cameras round-robin, one per step",
                   "G": cfg.G, "W": cfg.W, "H": cfg.H, "K": cfg.K, "S": cfg.S},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": {
            f"{cfg.name}_fwd_fps": fps,
            f"{cfg.name}_loss_after_steps": loss_last,
            "kernel_us": kt,
            "kernel_roofline": rows,
            "overflow_tiles": int((ts.ncand > ts.K).sum()),
            "pairs_kept": int(ts.count.long().sum()),
            "candidates": int(ts.ncand.long().sum()),
            "c2_train_its": its2,
            "c2_fwd_fps": fps2,
            "c2_note": "G=2000 128x128, bf16 render forward (matrix cores), fp32 params/Adam",
            **extra_c3,
            **extra_c5,
            **extra_sh,
            **extra_mc,
        },
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
