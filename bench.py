"""Benchmark: graph-captured training step and forward render on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--no-cpu-baseline]

Headline (`value`): training iterations per second at G=100k (clustered), 1264x832, K=128,
8 orbit cameras round-robin (one camera per step), fp32: each step is geometry fwd, binning,
fused splat fwd, L1+SSIM loss gradient, fused splat bwd (+theta bwd, per-slot gradients),
slot gather + geometry bwd + Adam, captured as HIP graphs of 8 consecutive steps (one per
starting camera; a remainder of K mod 8 steps replays one-step graphs); inside such a graph one
launch joins each step's geometry bwd + Adam to the next step's geometry fwd and binning count
pass (the step seam).  Inputs are resident on
the GPU before the timed region; the timed region is exactly K steps between two
synchronisations.

Also reported: forward fps (geometry + binning + splat, graphs of 8 renders) for the same
scene, the same training at the reference trainer's default bin cadence (bins rebuilt every 5th
step), the G=2000 128x128, G=10k 800x800 and G=1M 1920x1072 numbers, per-kernel times from HIP
events on the launch stream, the roofline of the dominant kernel, and the CPU oracle
(PyTorch-CPU restatement of the reference path) timed on this host's cores, and on one thread,
on bounded samples of the same workload.

Clock state: before any timed region the GPU replays the forward graphs for ~1.5 s (no state
change), so every timed region runs at steady clocks; a cold GPU measures several percent slower
for the first second.  Per-kernel times are HIP events on the launch stream around replays of a
graph of 20 back-to-back launches, camera 0 (and each of the 8 cameras for the splat kernels,
with their pair counts, so the roofline fraction can be recomputed from a profile of the same
run, whose kernel durations these agree with: no host time between the launches); each is the
best of 3 such averages taken after ~20 ms of warm-up replays of the same graph.

Roofline convention: every kernel of the training step gets a row (`extra.kernel_roofline`)
with the roof that bounds it and its algorithmic units, and `roofline` is the row of the step's
slowest single-kernel launch (HIP events, camera 0; the geometry + binning call launches four
kernels and its row covers the four together):
- splat forward / backward: the reference's algorithmic flops per (pixel, valid slot) pair --
  22 forward, 44 backward (the GEMM form of tools/m3_perf.py:80, Phi.theta 12 + relu^2 2 +
  WSR 8, and the transposed contractions) -- against the 157.3 TFLOP/s FP32 peak (1024 SIMDs
  x 64 lanes x 2 flop per 2 cycles at 2.4 GHz; without packed FP32, which this build does not
  emit, back-to-back wave64 FMAs measured 2.7 cycles each at the nominal clock on gfx950, so
  about 0.74 of the peak is what FMAs alone reach): bound "valu";
- the loss gradient: 1056 flop per pixel (3 channels: the separable filters of the forward
  and transposed passes) against the same FP32 peak, bound "valu" (1056 flop per 36 algorithmic
  bytes lies right of the FP32/HBM ridge); its HBM fraction at 36 bytes per pixel (image and
  target in, gradient out) is reported beside it;
- geometry forward + binning and geometry backward + Adam: algorithmic HBM bytes against
  8 TB/s, bound "hbm" (the byte counts are in kernel_bytes below).
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
LOSS_FLOP_PER_PIXEL = 1056.0  # 3 channels x (5 + 3) filtered quantities x 2 passes x 11 taps x 2
LOSS_BYTES_PER_PIXEL = 36.0   # image and target in, dL/dimage out (fp32, 3 channels)
# the step's single-kernel launches (roofline picks the slowest of them, with geom_seam -- the
# launch that joins two steps -- when the step has it); geom_fwd_binning is one call of four
# kernels (geometry + the binning's count pass, column scan, scatter, select) and gets its own
# row as a group
STEP_KERNELS = ("splat_fwd", "loss_grad", "splat_bwd", "geom_bwd_adam")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--config", default="c4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="rough total of the oracle's timed CPU samples over all configurations")
    ap.add_argument("--kernel-reps", type=int, default=100)
    ap.add_argument("--no-small", action="store_true",
                    help="skip the G=2000 128x128 runs (c1 forward, c2 3000-iteration training)")
    ap.add_argument("--no-c3", action="store_true", help="skip the G=10k 800x800 run")
    ap.add_argument("--no-c5", action="store_true", help="skip the G=1M 1920x1072 batch run")
    ap.add_argument("--c5-batches", type=int, default=3)
    ap.add_argument("--no-sh", action="store_true",
                    help="skip the SH degree 3 run of the headline workload")
    ap.add_argument("--no-mcmc", action="store_true",
                    help="skip the MCMC density-control run of the headline workload")
    ap.add_argument("--no-bin5", action="store_true",
                    help="skip the run at the reference trainer's bin cadence (every 5 steps)")
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


def build_step(cfg, torch, TrainStep, batch=1, sh_degree=0, mcmc=None, bin_every=1):
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
                   mcmc=mcmc, bin_every=bin_every, **sh_0)
    return ts


def time_train(ts, steps, warmup, torch, run_len=8):
    ncam = ts.n_steps
    ts.capture(run_len=run_len)
    ts.run(0, warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ts.run(warmup % ncam, steps)     # exactly `steps` steps, in graphs of ts.run_len steps
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def time_forward(ts, steps, warmup, torch, run_len=8):
    """Forward renders of the cameras round-robin: graphs of run_len consecutive renders (one
    per starting camera), one-render graphs for a remainder; exactly `steps` renders timed.  A
    render bins without the inverse table, which only the backward reads."""
    ncam = len(ts.cams)
    single, runs = [], []
    for ci in range(ncam):
        ts.forward(ci, grads=False)
    torch.cuda.synchronize()
    for ci in range(ncam):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ts.forward(ci, grads=False)
        single.append(g)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for j in range(run_len):
                ts.forward((ci + j) % ncam, grads=False)
        runs.append(g)

    def render(start, n):
        i = 0
        while n - i >= run_len:
            runs[(start + i) % ncam].replay()
            i += run_len
        for j in range(i, n):
            single[(start + j) % ncam].replay()

    render(0, warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    render(warmup % ncam, steps)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def warm_clocks(ts, torch, seconds=1.5):
    """Forward graph replays of every camera for `seconds` (reads the state, changes nothing
    the training reads), so the following timed regions start at steady GPU clocks."""
    graphs = []
    for ci in range(len(ts.cams)):
        ts.forward(ci)
    torch.cuda.synchronize()
    for ci in range(len(ts.cams)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ts.forward(ci)
        graphs.append(g)
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            graphs[i % len(graphs)].replay()
            i += 1
        torch.cuda.synchronize()
    return i


def graph_time(fn, reps, torch, per_graph=20, samples=3, warm_ms=20.0):
    """Microseconds per launch of fn(): per_graph launches captured back to back in one HIP graph
    (no host work between them), the graph replayed until about reps launches have run, between
    two HIP events on the stream the launches run on; the smallest of `samples` such averages,
    taken after about warm_ms of replays.  The host work before a measurement (eager calls,
    capture) leaves the GPU idle for milliseconds and its clock drops: without the warm-up the
    first kernel timed after it read up to 2 us slow.  Timing eager launches instead would add
    the host's per-call time to every kernel shorter than it."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g.replay()
    e1.record(stream)
    e1.synchronize()
    n_warm = int(warm_ms / max(e0.elapsed_time(e1), 1e-3))
    for _ in range(min(n_warm, 1000)):
        g.replay()
    n = max(1, reps // per_graph)
    best = float("inf")
    for _ in range(samples):
        e0.record(stream)
        for _ in range(n):
            g.replay()
        e1.record(stream)
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) / (n * per_graph) * 1e3)
    del g
    return best


def step_splat_jobs(ts, kernels, gimage):
    """The fused splat forward and backward as the training step launches them after a rebin:
    on the slot records for 16x16 tiles, else on proj / idx / valid."""
    if ts.use_rec:
        fwd = ((lambda: kernels.splat_fwd_mx_rec(ts.slot_rec, ts.pos_count, ts.order, ts.bg,
                                                 ts.H, ts.W, ts.S, ts.k, ts.image, ts.den,
                                                 bf16=True))
               if ts.dtype == "bf16" else
               (lambda: kernels.splat_fwd_rec(ts.slot_rec, ts.pos_count, ts.order, ts.bg, ts.H,
                                              ts.W, ts.S, ts.k, ts.image, ts.den)))
        bwd = lambda: kernels.splat_bwd_rec(ts.slot_rec, ts.pos_count, ts.order, ts.bg, ts.H,
                                            ts.W, ts.S, ts.k, ts.image, ts.den, gimage, ts.gslot)
    else:
        fwd = ((lambda: kernels.splat_fwd_mx(ts.proj, ts.idx, ts.valid, ts.bg, ts.H, ts.W, ts.S,
                                             ts.k, ts.image, ts.den, ts.order, bf16=True))
               if ts.dtype == "bf16" else
               (lambda: kernels.splat_fwd(ts.proj, ts.idx, ts.valid, ts.bg, ts.H, ts.W, ts.S,
                                          ts.k, ts.image, ts.den, ts.order)))
        bwd = lambda: kernels.splat_bwd(ts.proj, ts.idx, ts.valid, ts.bg, ts.H, ts.W, ts.S,
                                        ts.k, ts.image, ts.den, gimage, ts.gslot, order=ts.order)
    return fwd, bwd


def time_splat_per_camera(ts, reps, torch, kernels):
    """Fused splat forward / backward of every camera: HIP-event microseconds per launch and the
    (pixel, valid slot) pairs of that camera's bins (the state is the current one; the
    backward's input image gradient is a fixed random field)."""
    gim = torch.randn(ts.H, ts.W, 3, generator=torch.Generator().manual_seed(11)).cuda()
    rows = []
    for ci in range(len(ts.cams)):
        ts.forward(ci)
        torch.cuda.synchronize()
        pairs = int(ts.count.long().sum()) * ts.S * ts.S
        rec = dict(camera=ci, pairs=pairs)
        fwd, bwd = step_splat_jobs(ts, kernels, gim)
        jobs = {"splat_fwd": fwd, "splat_bwd": bwd}
        for name, fn in jobs.items():
            rec[name + "_us"] = graph_time(fn, reps, torch)
        rows.append(rec)
    ts.forward(0)
    torch.cuda.synchronize()
    return rows


def time_kernels(ts, reps, torch, kernels):
    """Average duration of each kernel group at the current state (camera 0), from HIP events
    around graph replays of its launches (graph_time)."""
    ts.enqueue(0)                       # bring every buffer to a consistent step state
    torch.cuda.synchronize()
    P_save, m_save, v_save, s_save = (t.clone() for t in (ts.P, ts.m, ts.v, ts.step_block))
    cam = ts.cams[0]
    sh = dict(sh_rest=ts.sh, sh_degree=ts.sh_degree)
    shs = [ts.sh, ts.sh_m, ts.sh_v] if ts.sh is not None else []
    saved_sh = [t.clone() for t in shs]
    fwd, bwd = step_splat_jobs(ts, kernels, ts.gimage)
    jobs = {
        "geom_fwd": lambda: kernels.geom_fwd(ts.P, cam, proj=ts.proj, keep=ts.keep, **sh),
        "binning": lambda: kernels.assign_bins(ts.proj[:, 0:2], ts.keep, ts.H, ts.W, ts.S, ts.K,
                                               ts.span, 1, ts.bin_ws, ts.idx, ts.valid,
                                               ts.count, ts.ncand, ts.inv, ts.order),
        # what the step launches: the geometry forward carrying the binning's count pass, then
        # the other binning kernels (writing the slot records the splat kernels then read)
        "geom_fwd_binning": lambda: kernels.geom_fwd_assign_bins(
            ts.P, cam, ts.H, ts.W, ts.S, ts.K, ts.span, proj=ts.proj, keep=ts.keep,
            workspace=ts.bin_ws, idx=ts.idx, valid=ts.valid, count=ts.count, ncand=ts.ncand,
            inv=ts.inv, order=ts.order, slot_rec=ts.slot_rec, pos_count=ts.pos_count, **sh),
        "splat_fwd": fwd,
        "loss_grad": lambda: kernels.loss_grad_stats(ts.image, ts.targets[0], ts.target_stats[0],
                                                     ts.lam, ts.gimage, ts.partials),
        "splat_bwd": bwd,
        "geom_bwd_adam": lambda: kernels.geom_bwd_adam(ts.P, cam, ts.gslot, ts.inv, ts.m, ts.v,
                                                       ts.lr, ts.step_block, sh_m=ts.sh_m,
                                                       sh_v=ts.sh_v, lr_sh=ts.lr_sh, **sh),
    }
    if ts.seamed:
        # the step seam: camera 0's backward + Adam and camera 1's geometry forward + count pass
        # in one launch (what the step's graphs launch between two steps)
        cam_f = ts.cams[1 % len(ts.cams)]
        jobs["geom_seam"] = lambda: kernels.geom_bwd_adam_fwd_count(
            ts.P, cam, cam_f, ts.gslot, ts.inv, ts.m, ts.v, ts.lr, ts.step_block, ts.proj,
            ts.keep, ts.H, ts.W, ts.S, ts.K, ts.span, workspace=ts.bin_ws)
    if ts.batch > 1:
        del jobs["geom_bwd_adam"]
        jobs["geom_bwd_accum"] = lambda: kernels.geom_bwd_accum(ts.P, cam, ts.gslot, ts.inv,
                                                                ts.gacc, 1.0 / ts.batch,
                                                                gacc_sh=ts.gacc_sh, **sh)
    out = {}
    for name, fn in jobs.items():
        out[name] = graph_time(fn, reps, torch)          # microseconds per launch
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


def kernel_bytes(ts):
    """Algorithmic HBM bytes of the step's geometry/binning and backward/Adam launches:
    geom_fwd_binning reads params (56 B/gaussian) and writes proj (48) and keep (1), the bin
    table (idx + valid, 5 B per slot), count, ncand and order (12 B per tile), the inverse table
    (36 B/gaussian) and one 48-byte slot record per kept slot; geom_bwd_adam reads params, m, v
    and the inverse table and writes params, m, v (56 B each per gaussian), and gathers 36 B per
    kept slot; the step seam (geom_seam) moves geom_bwd_adam's bytes and writes the next view's
    proj and keep (its forward reads the parameters it has just written, not HBM)."""
    G, T, K = ts.G, ts.tmap.T, ts.K
    nvalid = int(ts.count.long().sum())
    fwd = G * (56 + 48 + 1 + 36) + 5 * T * K + 12 * T + 48 * nvalid
    bwd = G * (6 * 56 + 36) + 36 * nvalid
    out = {"geom_fwd_binning": fwd, "geom_bwd_adam": bwd}
    if ts.seamed:
        out["geom_seam"] = bwd + G * (48 + 1)
    return out


def roofline_rows(ts, kt, pairs, cfg_name):
    """One roofline row per kernel of the step (camera 0 durations)."""
    rows = {}
    for name in ("splat_fwd", "splat_bwd"):
        flops = FLOP_PER_PAIR[name] * pairs
        tfl = flops / (kt[name] * 1e-6) / 1e12
        rows[name] = dict(us=kt[name], bound="valu", achieved=tfl, peak=PEAK_FP32_TFLOPS,
                          unit="TFLOP/s", frac=tfl / PEAK_FP32_TFLOPS,
                          flops_per_launch=flops, pairs_per_launch=pairs)
    npix = ts.H * ts.W
    tfl = LOSS_FLOP_PER_PIXEL * npix / (kt["loss_grad"] * 1e-6) / 1e12
    gbs = LOSS_BYTES_PER_PIXEL * npix / (kt["loss_grad"] * 1e-6) / 1e9
    rows["loss_grad"] = dict(us=kt["loss_grad"], bound="valu", achieved=tfl,
                             peak=PEAK_FP32_TFLOPS, unit="TFLOP/s", frac=tfl / PEAK_FP32_TFLOPS,
                             flops_per_launch=LOSS_FLOP_PER_PIXEL * npix, hbm_gbs=gbs,
                             hbm_frac=gbs / PEAK_HBM_GBS)
    for name, nbytes in kernel_bytes(ts).items():
        gbs = nbytes / (kt[name] * 1e-6) / 1e9
        rows[name] = dict(us=kt[name], bound="hbm", achieved=gbs, peak=PEAK_HBM_GBS, unit="GB/s",
                          frac=gbs / PEAK_HBM_GBS, bytes_per_launch=nbytes,
                          launches=4 if name == "geom_fwd_binning" else 1)
    for name, row in rows.items():
        row["traffic"] = load_traffic(name, cfg_name)
    return rows


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


def run_bin_every(args, torch, scenes, TrainStep, every=5):
    """The headline workload at the reference trainer's default bin cadence (--bin-every 5,
    tools/resident_traced.py:103,683): bins rebuilt on every 5th step and reused between, as
    graphs of 8 consecutive steps per starting camera and cadence phase.  Reported beside the
    headline, which rebins every step."""
    cfg = scenes.CONFIGS[args.config]
    ts = build_step(cfg, torch, TrainStep, bin_every=every)
    n = 300
    its = n / time_train(ts, n, 30, torch)
    return {f"bin_every{every}_train_its": its,
            f"bin_every{every}_note": f"bins rebuilt every {every}th step (the reference "
                                      f"trainer's default cadence); the headline rebins every "
                                      f"step"}


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
    t_batch = time_train(ts, nb, 1, torch, run_len=1) / nb   # one graph per 64-view batch
    # forward only (renders: no inverse table), all 64 views, one graph
    for ci in range(len(ts.cams)):
        ts.forward(ci, grads=False)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for ci in range(len(ts.cams)):
            ts.forward(ci, grads=False)
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


def cpu_threads():
    """(host cores, cores this process may run on, threads used): the oracle uses every core
    of the process's CPU share (capped by OMP_NUM_THREADS when the launcher sets it)."""
    host = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = host
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return host, avail, (min(avail, omp) if omp > 0 else avail)


def _rate(fn, seconds, min_n=1):
    """(calls, seconds) of fn repeated for at least `seconds` and `min_n` calls."""
    n, t0 = 0, time.perf_counter()
    while n < min_n or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
    return n, time.perf_counter() - t0


def cpu_baseline(args, torch, scenes, kernels):
    """The oracle -- the PyTorch-CPU restatement of the reference path (geometry, assign_bins,
    gather, einsum WSR; autograd backward, the restated L1+SSIM loss, Adam) -- timed on this
    host's cores, camera 0 of each configuration, bounded samples (the reference's own idiom:
    warm-up, then repeated calls timed with perf_counter, tools/m3_perf.py:47-56).  Also the
    dense arm-A render (spike/render.py) at G=2000, one-thread rows, and the bin-table
    agreement between the GPU and the oracle when each starts from the parameters."""
    from oracle import binning as obin
    from oracle import geometry as ogeo
    from oracle import pipeline as opipe
    from oracle import splat as osplat
    host, avail, use = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(use)
    sec = args.cpu_seconds
    rows = {}
    lr = torch.full((14,), 1e-3)
    lr[:3] = 1.6e-4
    plan = (("c1", sec * 0.06, sec * 0.06), ("c1_ref", sec * 0.06, sec * 0.06),
            ("c3", sec * 0.1, sec * 0.15), ("c4", sec * 0.12, sec * 0.3), ("c5", 0.0, 0.0))
    for name, fsec, tsec in plan:
        cfg = scenes.CONFIGS[name]
        cam = cfg.cameras()[0].as_dict()
        tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
        P = cfg.params(seed=0)
        with torch.no_grad():
            tgt = osplat.render_binned(cfg.params(seed=1), cam, tmap, K=cfg.K, k=cfg.k,
                                       span=cfg.span)
            nf, df = _rate(lambda: osplat.render_binned(P, cam, tmap, K=cfg.K, k=cfg.k,
                                                        span=cfg.span), fsec, 3)
        m, v = torch.zeros_like(P), torch.zeros_like(P)
        it = [0]

        def step():
            it[0] += 1
            opipe.train_step(P, m, v, it[0], cam, tmap, tgt, lr, K=cfg.K, k=cfg.k, span=cfg.span)
        step()                                       # warm-up (the target render warmed up
        nt, dt = _rate(step, tsec, 3)                # the forward); at least 3 timed samples
        rows[name] = dict(fwd_fps=nf / df, fwd_ms=df / nf * 1e3, train_its=nt / dt,
                          train_ms=dt / nt * 1e3, sample=f"{nf} forwards, {nt} train steps")
    rows["c2"] = dict(rows["c1_ref"], note="the c2 shape (G=2000, 128x128, S=16, k=4) in fp32: "
                                           "the oracle has no bf16 mode")
    # the dense arm-A render (spike/render.py:14-49) at G=2000, 128x128, k=9
    cfg = scenes.CONFIGS["c1"]
    cam = cfg.cameras()[0].as_dict()
    P = cfg.params(seed=0)
    with torch.no_grad():
        osplat.render_dense(P, cam, k=cfg.k)
        nd, dd = _rate(lambda: osplat.render_dense(P, cam, k=cfg.k), sec * 0.04, 2)
    rows["c1_dense_fwd_fps"] = nd / dd
    # one thread
    torch.set_num_threads(1)
    try:
        one = {}
        for name, tsec in (("c1_ref", sec * 0.05), ("c4", 0.0)):
            cfg = scenes.CONFIGS[name]
            cam = cfg.cameras()[0].as_dict()
            tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
            P = cfg.params(seed=0)
            with torch.no_grad():
                tgt = osplat.render_binned(cfg.params(seed=1), cam, tmap, K=cfg.K, k=cfg.k)
            m, v = torch.zeros_like(P), torch.zeros_like(P)
            one_step = lambda: opipe.train_step(P, m, v, 1, cam, tmap, tgt, lr, K=cfg.K,
                                                k=cfg.k)
            one_step()                               # warm-up, then at least 3 timed samples
            n1, d1 = _rate(one_step, tsec, 3)
            one[name] = dict(train_its=n1 / d1, train_ms=d1 / n1 * 1e3, steps=n1)
    finally:
        torch.set_num_threads(use)
    # bin tables: GPU geometry + binning vs oracle geometry + binning, each from the parameters
    agree = {}
    for name in ("c1_ref", "c3", "c4", "c5"):
        cfg = scenes.CONFIGS[name]
        camo = cfg.cameras()[5 if name == "c5" else 0]
        P = cfg.params(seed=0)
        proj, keep = kernels.geom_fwd(P.cuda(), camo.device_block("cuda"))
        idx, valid, _, ncand = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S,
                                                   cfg.K, cfg.span)
        pr = ogeo.project_params(P, camo.as_dict())
        tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
        ridx, rvalid = obin.assign_bins(pr["mu2d"].detach(), pr["keep"], tmap, 1, cfg.K,
                                        cfg.span, stable=True)
        diff = (idx.cpu().long() != ridx).any(1) | (valid.cpu().bool() != rvalid).any(1)
        agree[name] = dict(tiles=tmap.T, tiles_differ=int(diff.sum()),
                           pairs=int(ncand.long().sum()))
    # below 32768 pairs the reference's argsort is an introsort: G=2000 128x128 against the
    # reference order on the GPU's own centres
    cfg = scenes.CONFIGS["c1_ref"]
    camo = cfg.cameras()[0]
    proj, keep = kernels.geom_fwd(cfg.params(seed=0).cuda(), camo.device_block("cuda"))
    idx, valid, _, _ = kernels.assign_bins(proj[:, 0:2], keep, cfg.H, cfg.W, cfg.S, cfg.K,
                                           cfg.span)
    mu, kp = proj[:, 0:2].cpu(), keep.cpu().bool()
    tmap = obin.TileMap(cfg.H, cfg.W, cfg.S)
    ridx, rvalid = obin.assign_bins(mu, kp, tmap, 1, cfg.K, cfg.span, stable=False)
    ic, vc = idx.cpu().long(), valid.cpu().bool()
    reordered = (ic != ridx).any(1) | (vc != rvalid).any(1)
    set_diff, swapped = 0, 0
    for t in torch.nonzero(reordered).flatten().tolist():
        a, b = set(ic[t][vc[t]].tolist()), set(ridx[t][rvalid[t]].tolist())
        if a != b:
            set_diff += 1
            swapped += len(a - b)
    intro = dict(tiles=tmap.T, tie_tiles=len(obin.tie_tiles(mu, kp, tmap, 1, cfg.span)),
                 tiles_ordered_differently=int(reordered.sum()),
                 tiles_with_different_kept_set=set_diff, gaussians_swapped=swapped)
    torch.set_num_threads(prev)
    c4 = rows["c4"]
    return dict(value=c4["train_its"], unit="it/s", cores=use, kind="port",
                sample=f"oracle train steps and forwards, camera 0 of each configuration, about "
                       f"{sec:.0f} s of CPU work in all; headline: c4 {c4['sample']}",
                host_cores=host, cores_available=avail, fwd_fps=c4["fwd_fps"], rows=rows,
                one_thread=dict(cores=1, value=one["c4"]["train_its"], unit="it/s", rows=one),
                bins_from_parameters=agree, bins_reference_order_g2000=intro)


def small_configs(torch, scenes, TrainStep):
    """G=2000, 128x128: forward fps as configured (fp32, 32x32 tiles, k=9) and in the
    reference's own constants (16x16 tiles, k=4); the c2 training run for its 3000 iterations
    (bf16 render forward, fp32 Adam), wall-clock it/s and the final loss, beside the oracle's
    own 3000-step run of that shape (fp32, recorded in tests/golden/c2_oracle_trajectory.json)."""
    out = {}
    for name in ("c1", "c1_ref"):
        cfg = scenes.CONFIGS[name]
        ts = build_step(cfg, torch, TrainStep)
        out[f"{name}_fwd_fps"] = 1000 / time_forward(ts, 1000, 100, torch)
        del ts
    out["c1_note"] = "c1: fp32, S=32, k=9 as configured; c1_ref: S=16, k=4 (reference constants)"
    cfg = scenes.CONFIGS["c2"]
    ts = build_step(cfg, torch, TrainStep)
    ts.capture()
    ts.step(0)
    torch.cuda.synchronize()
    loss0 = float(ts.loss())
    t0 = time.perf_counter()
    ts.run(0, 2999)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    out.update(c2_train_its=2999 / dt, c2_iterations=3000, c2_seconds_3000=dt * 3000 / 2999,
               c2_loss_first=loss0, c2_loss_final=float(ts.loss()),
               c2_fwd_fps=1000 / time_forward(ts, 1000, 100, torch),
               c2_note="G=2000 128x128, bf16 render forward (matrix cores), fp32 params/Adam, "
                       "target = GPU bf16 render of the seed-1 set")
    path = os.path.join(ROOT, "tests", "golden", "c2_oracle_trajectory.json")
    if os.path.exists(path):
        with open(path) as f:
            rec = json.load(f)
        out.update(c2_oracle_loss_final=rec["final_loss"],
                   c2_oracle_loss_first=rec["loss_at"]["1"],
                   c2_oracle_note="oracle (fp32 CPU) 3000-step run, target = oracle render of "
                                  "the seed-1 set")
    return out


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
    warm_clocks(ts, torch)
    train_s = time_train(ts, args.steps, args.warmup, torch)
    its = args.steps / train_s
    fwd_s = time_forward(ts, args.steps, args.warmup, torch)
    fps = args.steps / fwd_s
    loss_last = float(ts.loss())
    kt = time_kernels(ts, args.kernel_reps, torch, kernels)
    per_cam = time_splat_per_camera(ts, max(10, args.kernel_reps // 2), torch, kernels)
    pairs = per_cam[0]["pairs"]
    rows = roofline_rows(ts, kt, pairs, cfg.name)
    dom = max(STEP_KERNELS + (("geom_seam",) if ts.seamed else ()), key=lambda n: kt[n])
    roofline = dict(rows[dom], kernel=dom, camera=0,
                    convention="the step's slowest single-kernel launch (HIP-event duration over graph "
                               "replays of 20 launches, camera 0, the best of 3 averages after "
                               "20 ms of warm-up replays) against its bound: algorithmic "
                               "flops (splat 22/44 per pixel-slot pair, loss 1056 per pixel) over "
                               "157.3 TFLOP/s FP32, reached on the VALU without packed FP32, or "
                               "algorithmic bytes over 8 TB/s HBM; every kernel's row in "
                               "extra.kernel_roofline")
    if dom in ("splat_fwd", "splat_bwd"):
        all_pairs = sum(r["pairs"] for r in per_cam)
        all_us = sum(r[dom + "_us"] for r in per_cam)
        roofline["frac_all_cameras"] = (FLOP_PER_PAIR[dom] * all_pairs / (all_us * 1e-6) / 1e12
                                        / PEAK_FP32_TFLOPS)
    small = {} if args.no_small else small_configs(torch, scenes, TrainStep)
    extra_c3 = {} if args.no_c3 else run_c3(args, torch, scenes, TrainStep)
    extra_c5 = {} if args.no_c5 else run_c5(args, torch, scenes, kernels, TrainStep)
    extra_sh = {} if args.no_sh else run_sh(args, torch, scenes, kernels, TrainStep)
    extra_mc = {} if args.no_mcmc else run_mcmc(args, torch, scenes, TrainStep)
    extra_b5 = {} if args.no_bin5 else run_bin_every(args, torch, scenes, TrainStep)
    if args.copy_mib:
        src = torch.ones(args.copy_mib * (1 << 18), device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args, torch, scenes, kernels)
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
            "splat_per_camera": per_cam,
            "overflow_tiles": int((ts.ncand > ts.K).sum()),
            "pairs_kept": int(ts.count.long().sum()),
            "candidates": int(ts.ncand.long().sum()),
            **small,
            **extra_c3,
            **extra_c5,
            **extra_sh,
            **extra_mc,
            **extra_b5,
        },
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
