"""Device-resident, graph-captured training step (the traced step of tools/resident_traced.py).

The reference allocates every persistent buffer first (tools/resident_traced.py:222-296),
captures the step as ttnn traces (:551-567) and replays them per iteration (:667-757), with
host binning/loss/scatter round trips in between.  Here one step is, on one stream and with no
host round trip:

    geom_fwd_assign_bins (geometry + Adam step advance + the binning's count pass in one
             kernel, then 3 binning kernels, + inverse table and tile order)
             -> splat_fwd -> loss_grad_stats (1 kernel) -> splat_bwd (theta bwd, per-slot gradients)
             -> geom_bwd_adam (slot gather-reduce + geometry bwd + Adam)

captured once per camera into a HIP graph (torch.cuda.CUDAGraph) and replayed.  The step
counter and Adam bias corrections live in device memory, so replays need no re-capture.
All buffers are allocated in __init__; a replay allocates nothing.
"""
import torch

from . import kernels
from .binned import TileMap
from .kernels import F32, I32, U8

DEFAULT_LR = 1e-3
MEANS_LR = 1.6e-4


def lr_vector(lr=DEFAULT_LR, means_lr=MEANS_LR, device="cuda"):
    """Per-column learning rates for the [G,14] block: means get means_lr, the rest lr."""
    v = torch.full((14,), float(lr), dtype=F32)
    v[0:3] = float(means_lr)
    return v.to(device)


class TrainStep:
    """Owns params [G,14], Adam moments and every work buffer for training against one or more
    (camera, target) pairs.

    dtype = "bf16": the render forward is the bf16 variant (matrix-core splat with bf16 weights
    and colours, fp32 accumulation); geometry, binning, loss, backward and Adam stay fp32
    (the reference's bf16 device path keeps its parameters and Adam state in fp32).
    batch = 1: step(i) is one full training step on camera i (one Adam update per view, the
    round-robin loop of tools/resident_traced.py:667-757).
    batch = B > 1: the views are grouped into consecutive batches of B; step(i) renders and
    backpropagates every view of batch i, accumulating the mean gradient, then applies one Adam
    update (the full-batch loop of spike/train.py:21-33 over B views).
    sh_degree = 1..3: view-dependent colour (the SHD > 0 mode of tools/resident_traced.py:237-264):
    sh_rest is spike's color_rest [G,15,3] (zeros if omitted), trained with Adam at lr_sh
    (default: the colour learning rate / 20, as the reference); the direction is constant in
    the backward, as there.
    mcmc = dict(...): fixed-count MCMC density control (spike/mcmc.py; the reference's device
    step flags --lambda-o, --lambda-s, --noise-lr, --relocate-every, --dead-thr,
    tools/resident_traced.py:124-130): the regulariser gradient and the SGLD step run inside the
    step's geometry backward + Adam kernel; every `relocate_every` steps (after step i > 0 with
    i % relocate_every == 0, counted by step()) a captured relocation graph moves dead slots
    onto live gaussians.  Random draws come from Philox keyed by `seed` and the device step
    number, so replays are reproducible.

    depth_weight = dict(beta0=1.0, tau0=None, lr_bt=0.02): the depth-weight occlusion lever
    (tools/resident_traced.py --depth-weight, :138-140,333-337,418-426,503-512): the opacity is
    multiplied by sigmoid(beta (tau - z_cam)); beta and tau live on the device and take an Adam
    step (learning rate lr_bt) after every step; tau0 = None uses the median camera depth of
    the gaussians camera 0 keeps, as the reference refines it at warm-up.
    keep_grad = True (batch = 1): the fused backward also stores each step's dL/dparams [G,14]
    in self.gparams (the gradient Adam was given).
    bin_every = N (batch = 1): the reference trainer's bin cadence (--bin-every, default 5 there,
    tools/resident_traced.py:103,683): step() rebins only on steps whose running count is a
    multiple of N (and on the step after an MCMC relocation); the other steps run geometry,
    splat, loss, backward and Adam on the bins last computed -- one bin table for all cameras,
    as in that trainer.  Each camera gets a graph with and one without the binning kernels.
    run(i, n) is n step() calls from step i on; without relocation it replays graphs that each
    hold run_len consecutive steps (one graph launch per run_len steps; with bin_every = N, one
    graph per starting camera and cadence phase).
    random_bg = True: the reference trainer's --random-bg (tools/resident_traced.py:182-185,
    671-674): targets are straight RGBA [H,W,4] (spike's load_blender(keep_alpha=True)); every
    view backward first draws a background colour (Philox keyed by bg_seed, the device step
    count and the view; the reference draws torch.rand(3) on the host), composites the target
    over it and renders with it as the numerator background c_b (w_b unchanged).  eval_psnr()
    renders on white, as the reference evaluates.
    target_stats: the loss needs each target's SSIM statistics.  "per_view" keeps one set per
    view, computed once (36 bytes per pixel per view: 2.3 GB for 100 views at 800x800; the
    targets must not change after construction); "per_step" keeps one set and recomputes it from
    the current target at every view backward, as the reference's recompute_gt_stats does on each
    view switch (tools/resident_traced.py:320-325,677-678).  random_bg implies "per_step".
    seam: run()'s multi-step graphs join each step's geometry backward + Adam to the next
    step's geometry forward + binning count pass in one launch (see seamed).  None (default):
    when that pays, G >= kernels.SEAM_MIN_G; True: whenever the step allows it; False: never."""

    MCMC_DEFAULTS = dict(lambda_o=0.0, lambda_s=0.0, noise_lr=0.0, relocate_every=0,
                         dead_thr=0.005, offset=0.005, seed=0)
    DEPTH_DEFAULTS = dict(beta0=1.0, tau0=None, lr_bt=0.02)

    def __init__(self, params, cameras, targets, K=128, S=16, k=4.0, lr=None, w_b_raw=-3.0,
                 c_b=(1.0, 1.0, 1.0), lambda_ssim=0.2, span=None, device="cuda", batch=1,
                 dtype="fp32", sh_degree=0, sh_rest=None, lr_sh=None, mcmc=None,
                 depth_weight=None, keep_grad=False, bin_every=1, random_bg=False, bg_seed=0,
                 target_stats="per_view", seam=None):
        dev = torch.device(device)
        if dtype not in ("fp32", "bf16"):
            raise ValueError(f"dtype must be 'fp32' or 'bf16', got {dtype!r}")
        if dtype == "bf16" and S != 16:
            raise ValueError("the bf16 render variant runs on 16x16 tiles")
        self.dtype = dtype
        self.dev = dev
        self.G = params.shape[0]
        self.H, self.W = cameras[0].H, cameras[0].W
        self.K, self.S, self.k, self.lam = K, S, float(k), float(lambda_ssim)
        self.tmap = TileMap(self.H, self.W, S, device=dev)
        self.span = span or self.tmap.span
        T = self.tmap.T
        G, H, W = self.G, self.H, self.W
        # parameters and optimiser state
        self.P = params.to(dev, F32).contiguous().clone()
        self.m = torch.zeros(G, 14, device=dev, dtype=F32)
        self.v = torch.zeros(G, 14, device=dev, dtype=F32)
        self.step_block = kernels.adam_state(dev)
        self.lr = (lr_vector(device=dev) if lr is None else torch.as_tensor(lr, dtype=F32).to(dev)).contiguous()
        self.sh_degree = int(sh_degree)
        if not 0 <= self.sh_degree <= 3:
            raise ValueError(f"sh_degree must be in [0, 3], got {sh_degree}")
        if self.sh_degree > 0:
            rest = (torch.zeros(G, kernels.SH_REST, 3) if sh_rest is None else sh_rest)
            self.sh = kernels.sh_rest_layout(rest.to(dev, F32))
            self.sh_m = torch.zeros_like(self.sh)
            self.sh_v = torch.zeros_like(self.sh)
            lrs = float(self.lr[10]) / 20.0 if lr_sh is None else float(lr_sh)
            self.lr_sh = torch.tensor([lrs], dtype=F32, device=dev)
        else:
            self.sh = self.sh_m = self.sh_v = self.lr_sh = None
        unknown = set(mcmc or {}) - set(self.MCMC_DEFAULTS)
        if unknown:
            raise ValueError(f"unknown mcmc options {sorted(unknown)}")
        self.mc = {**self.MCMC_DEFAULTS, **(mcmc or {})}
        self._it = 0
        if self.mc["relocate_every"]:
            self.reloc_ws = kernels.relocate_workspace(G, dev)
            self.moved = torch.zeros(1, device=dev, dtype=I32)
            self.relocations = torch.zeros(1, device=dev, dtype=torch.int64)
        self.reloc_graph = None
        w_b = torch.nn.functional.softplus(torch.tensor(float(w_b_raw)))
        self.dw = self.dw_state = self.lr_bt = self.gdw = None
        if depth_weight is not None:
            unknown = set(depth_weight) - set(self.DEPTH_DEFAULTS)
            if unknown:
                raise ValueError(f"unknown depth_weight options {sorted(unknown)}")
            dwo = {**self.DEPTH_DEFAULTS, **depth_weight}
            tau0 = dwo["tau0"]
            if tau0 is None:                 # median camera depth of the kept gaussians
                pr, kp = kernels.geom_fwd(self.P, cameras[0].device_block(dev))
                z = pr[:, 5][kp.bool()]
                tau0 = float(z.median()) if z.numel() else float(pr[:, 5].median())
            self.dw = torch.tensor([float(dwo["beta0"]), tau0], dtype=F32, device=dev)
            self.dw_state = torch.zeros(4, dtype=F32, device=dev)
            self.lr_bt = torch.tensor([float(dwo["lr_bt"])], dtype=F32, device=dev)
            self.gdw = torch.zeros(G, 2, dtype=F32, device=dev)
            self.dw_ws = kernels.depth_weight_workspace(G, dev)
        self.bg = torch.tensor([float(w_b), *c_b], dtype=F32, device=dev)
        self.bg_white = torch.tensor([float(w_b), 1.0, 1.0, 1.0], dtype=F32, device=dev)
        self.random_bg, self.bg_seed = bool(random_bg), int(bg_seed)
        if seam not in (None, True, False):
            raise ValueError(f"seam must be None, True or False, got {seam!r}")
        self.seam = seam
        if target_stats not in ("per_view", "per_step"):
            raise ValueError(f"target_stats must be 'per_view' or 'per_step', got {target_stats!r}")
        self.stats_mode = "per_step" if self.random_bg else target_stats
        # per-view inputs
        self.cams = [c.device_block(dev) for c in cameras]
        if len(targets) != len(self.cams):
            raise ValueError("one target image per camera is required")
        self.targets = self.rgba_pm = self.target_buf = None
        if self.random_bg:
            for t in targets:
                if tuple(t.shape) != (H, W, 4):
                    raise ValueError(f"random_bg needs RGBA targets [{H},{W},4], got "
                                     f"{tuple(t.shape)}")
            self.rgba_pm = [kernels.rgba_premult(t.cpu()).to(dev) for t in targets]
            self.target_buf = torch.empty(H, W, 3, device=dev, dtype=F32)
        else:
            self.targets = [t.to(dev, F32).contiguous() for t in targets]
        if self.stats_mode == "per_view":
            self.target_stats = [kernels.loss_stats(t) for t in self.targets]
        else:
            self.target_stats = None
            self.stats_buf = torch.empty(kernels.loss_stats_numel(H, W), device=dev, dtype=F32)
        # work buffers
        self.proj = torch.empty(G, 12, device=dev, dtype=F32)
        self.keep = torch.empty(G, device=dev, dtype=U8)
        self.bin_ws = kernels.bin_workspace(G, H, W, S, dev)
        self.idx = torch.empty(T, K, device=dev, dtype=I32)
        self.valid = torch.empty(T, K, device=dev, dtype=U8)
        self.count = torch.empty(T, device=dev, dtype=I32)
        self.ncand = torch.empty(T, device=dev, dtype=I32)
        self.order = torch.empty(T, device=dev, dtype=I32)
        self.inv = torch.empty(G, 9, device=dev, dtype=I32)
        # 16x16-tile steps that rebin: the binning also writes the slot records (each kept
        # slot's projection record, tiles in dispatch order) and the splat kernels read those
        # instead of order -> idx -> proj; steps that reuse older bins read proj itself
        self.use_rec = self.S == 16
        self.slot_rec = (torch.empty(T, K, 12, device=dev, dtype=F32) if self.use_rec
                         else None)
        self.pos_count = torch.empty(T, device=dev, dtype=I32) if self.use_rec else None
        self.gslot = torch.zeros(T, K, 9, device=dev, dtype=F32)
        self.image = torch.empty(H, W, 3, device=dev, dtype=F32)
        self.den = torch.empty(H, W, device=dev, dtype=F32)
        self.gimage = torch.empty(H, W, 3, device=dev, dtype=F32)
        self.partials = torch.empty(kernels.loss_partials_count(H, W)[0], device=dev, dtype=F32)
        self.batch = int(batch)
        if self.batch < 1 or len(self.cams) % self.batch:
            raise ValueError(f"{len(self.cams)} views do not split into batches of {batch}")
        self.gacc = torch.zeros(G, 14, device=dev, dtype=F32) if self.batch > 1 else None
        if keep_grad and self.batch > 1:
            raise ValueError("keep_grad keeps the per-view gradient: batch must be 1")
        # dL/dparams of the last step (written by the fused backward + Adam kernel)
        self.gparams = torch.zeros(G, 14, device=dev, dtype=F32) if keep_grad else None
        self.gacc_sh = (torch.zeros_like(self.sh) if self.batch > 1 and self.sh_degree > 0
                        else None)
        self.bin_every = int(bin_every)
        if self.bin_every < 1:
            raise ValueError(f"bin_every must be >= 1, got {bin_every}")
        if self.bin_every > 1 and self.batch > 1:
            raise ValueError("bin_every > 1 reuses one bin table across steps: batch must be 1")
        self._force_rebin = False
        self.graphs = {}
        self.run_graphs = {}
        self.run_len = 1

    @property
    def color_rest(self):
        """The SH rest coefficients in spike's layout [G,15,3] (None without SH)."""
        return None if self.sh is None else kernels.sh_rest_model(self.sh)

    # ---------------------------------------------------------------------------------
    def forward(self, ci=0, advance=False, rebin=True, grads=True):
        """Geometry + binning + fused splat for camera ci into self.image.  advance=True: the
        geometry launch also advances the Adam step block (a training step's first kernel).
        rebin=False: the bins last computed are reused (the binning kernels are not run).
        grads=False: a render only -- the binning skips the inverse table (gaussian -> slots)
        and the splat kernel the per-pixel den, which only the backward reads (self.den is
        left as it was).  A forward that rebins replaces the shared bin table (with
        grads=False, without its inverse table), so the next step() rebins whatever its
        bin_every count says."""
        self._forward(ci, advance, rebin, grads)
        if rebin:
            self._force_rebin = True
        return self.image

    def _forward(self, ci, advance=False, rebin=True, grads=True, camera=None, bg=None):
        """forward() as a training step enqueues it (no forced rebin); camera: a [16] device
        camera block to render instead of camera ci's; bg: a [4] background block instead of
        self.bg."""
        adv = self.step_block if advance else None
        cam = self.cams[ci] if camera is None else camera
        bgb = self.bg if bg is None else bg
        if rebin:   # one call: the binning's count pass rides on the geometry launch
            kernels.geom_fwd_assign_bins(self.P, cam, self.H, self.W, self.S, self.K,
                                         self.span, proj=self.proj, keep=self.keep,
                                         sh_rest=self.sh, sh_degree=self.sh_degree,
                                         depth_bt=self.dw, advance=adv,
                                         workspace=self.bin_ws, idx=self.idx, valid=self.valid,
                                         count=self.count, ncand=self.ncand,
                                         inv=self.inv if grads else None,
                                         order=self.order, slot_rec=self.slot_rec,
                                         pos_count=self.pos_count)
        else:
            kernels.geom_fwd(self.P, cam, proj=self.proj, keep=self.keep,
                             sh_rest=self.sh, sh_degree=self.sh_degree, depth_bt=self.dw,
                             advance=adv)
        return self._splat_forward(bgb, rebin, grads)

    def _splat_forward(self, bgb, rebin=True, grads=True):
        """The fused splat forward on the bins last computed (on the slot records when they were
        just rebuilt): self.image, and self.den when grads."""
        if self.dtype == "bf16" and rebin and self.use_rec:
            kernels.splat_fwd_mx_rec(self.slot_rec, self.pos_count, self.order, bgb, self.H,
                                     self.W, self.S, self.k, self.image, self.den, bf16=True,
                                     write_den=grads)
        elif self.dtype == "bf16":
            kernels.splat_fwd_mx(self.proj, self.idx, self.valid, bgb, self.H, self.W,
                                 self.S, self.k, self.image, self.den, self.order, bf16=True)
        elif rebin and self.use_rec:
            kernels.splat_fwd_rec(self.slot_rec, self.pos_count, self.order, bgb, self.H,
                                  self.W, self.S, self.k, self.image, self.den,
                                  write_den=grads)
        else:
            kernels.splat_fwd(self.proj, self.idx, self.valid, bgb, self.H, self.W, self.S,
                              self.k, self.image, self.den, self.order)
        return self.image

    @property
    def n_steps(self):
        """Number of distinct steps (views for batch = 1, batches otherwise)."""
        return len(self.cams) // self.batch

    def _loss_target(self, ci):
        """The target of view ci and its SSIM statistics (recomputed in "per_step" mode)."""
        if self.stats_mode == "per_view":
            return self.targets[ci], self.target_stats[ci]
        tgt = self.target_buf if self.random_bg else self.targets[ci]
        kernels.loss_stats(tgt, self.stats_buf)
        return tgt, self.stats_buf

    def _view_backward(self, ci, advance=False, rebin=True):
        """Forward, loss gradient and fused splat backward of camera ci (slot gradients).  With
        random_bg the view's background is drawn and its target composited first (before the
        step advance inside the geometry launch: the draw is keyed by the completed steps)."""
        if self.random_bg:
            kernels.composite_random_bg(self.rgba_pm[ci], self.step_block, ci, self.bg_seed,
                                        self.bg, self.target_buf)
        self._forward(ci, advance, rebin)
        self._loss_and_splat_backward(ci, rebin)

    def _loss_and_splat_backward(self, ci, rebin=True):
        """Loss gradient of view ci's render, then the fused splat backward (slot gradients)."""
        tgt, stats = self._loss_target(ci)
        kernels.loss_grad_stats(self.image, tgt, stats, self.lam, self.gimage, self.partials)
        if rebin and self.use_rec:
            kernels.splat_bwd_rec(self.slot_rec, self.pos_count, self.order, self.bg, self.H,
                                  self.W, self.S, self.k, self.image, self.den, self.gimage,
                                  self.gslot)
        else:
            kernels.splat_bwd(self.proj, self.idx, self.valid, self.bg, self.H, self.W, self.S,
                              self.k, self.image, self.den, self.gimage, self.gslot,
                              order=self.order)

    def enqueue(self, i=0, rebin=True):
        """Enqueue training step i (camera i, or batch i) on the current stream; rebin=False
        reuses the bins last computed (batch = 1 only)."""
        sh = dict(sh_rest=self.sh, sh_degree=self.sh_degree)
        mc = self.mc
        if self.batch == 1:
            self._view_backward(i, advance=True, rebin=rebin)   # step advance rides on geom_fwd
            self._geometry_backward_adam(i)
            return
        scale = 1.0 / self.batch
        for ci in range(i * self.batch, (i + 1) * self.batch):
            self._view_backward(ci)
            kernels.geom_bwd_accum(self.P, self.cams[ci], self.gslot, self.inv, self.gacc, scale,
                                   gacc_sh=self.gacc_sh, depth_bt=self.dw, gacc_depth=self.gdw,
                                   **sh)
        kernels.adam_advance(self.step_block)
        if mc["lambda_o"] or mc["lambda_s"]:
            kernels.mcmc_reg_grad(self.P, self.gacc, mc["lambda_o"], mc["lambda_s"])
        kernels.adam(self.P, self.m, self.v, self.gacc, self.lr, self.step_block)
        if mc["noise_lr"]:
            kernels.sgld_noise(self.P, self.lr, mc["noise_lr"], self.step_block, mc["seed"])
        kernels.zero_(self.gacc)
        if self.sh_degree > 0:
            kernels.adam_flat(self.sh, self.sh_m, self.sh_v, self.gacc_sh, self.lr_sh,
                              self.step_block)
            kernels.zero_(self.gacc_sh)
        if self.dw is not None:
            kernels.depth_weight_adam(self.gdw, self.dw, self.dw_state, self.lr_bt,
                                      self.step_block, self.dw_ws)
            kernels.zero_(self.gdw)

    def _geometry_backward_adam(self, i):
        """Slot gather + geometry backward + Adam of step i (camera i, batch = 1)."""
        sh = dict(sh_rest=self.sh, sh_degree=self.sh_degree)
        mc = self.mc
        kernels.geom_bwd_adam(self.P, self.cams[i], self.gslot, self.inv, self.m, self.v,
                              self.lr, self.step_block, gparams=self.gparams,
                              sh_m=self.sh_m, sh_v=self.sh_v,
                              lr_sh=self.lr_sh, lambda_o=mc["lambda_o"],
                              lambda_s=mc["lambda_s"], noise_lr=mc["noise_lr"],
                              seed=mc["seed"], depth_bt=self.dw, gdepth=self.gdw, **sh)
        if self.dw is not None:
            kernels.depth_weight_adam(self.gdw, self.dw, self.dw_state, self.lr_bt,
                                      self.step_block, self.dw_ws)

    @property
    def seam_possible(self):
        """Whether the step has a seam launch: the plain step (batch = 1, rebinning every step
        on 16 x 16 tiles, no SH, depth weight or MCMC) with 0 < G <= kernels.SEAM_MAX_G."""
        mc = self.mc
        return (self.batch == 1 and self.bin_every == 1 and self.use_rec
                and self.sh_degree == 0 and self.dw is None
                and not (mc["lambda_o"] or mc["lambda_s"] or mc["noise_lr"]
                         or mc["relocate_every"])
                and 0 < self.P.shape[0] <= kernels.SEAM_MAX_G)

    @property
    def seamed(self):
        """Whether run() joins consecutive steps at the seam: step i's geometry backward + Adam
        and step i+1's geometry forward + binning count pass in one launch (seam_possible, and
        seam=True or, by default, G >= kernels.SEAM_MIN_G: a seam block carries 512 gaussians
        through both halves, so with few blocks the two launches' wider spread wins)."""
        if not self.seam_possible or self.seam is False:
            return False
        return self.seam is True or self.P.shape[0] >= kernels.SEAM_MIN_G

    def enqueue_seamed(self, ci, n):
        """Enqueue n training steps from camera ci (as n enqueue() calls would run them, with
        the same results) where each step's backward + Adam and the next step's geometry forward
        + binning count pass share one launch; the next step's Adam step advance then rides on
        its binning's column scan.  Requires self.seamed."""
        if not self.seam_possible:
            raise ValueError("this step configuration has no seam launch (see "
                             "TrainStep.seam_possible)")
        ns = self.n_steps
        self._view_backward(ci % ns, advance=True, rebin=True)
        for j in range(n - 1):
            cb, cf = (ci + j) % ns, (ci + j + 1) % ns
            kernels.geom_bwd_adam_fwd_count(self.P, self.cams[cb], self.cams[cf], self.gslot,
                                            self.inv, self.m, self.v, self.lr, self.step_block,
                                            self.proj, self.keep, self.H, self.W, self.S, self.K,
                                            self.span, workspace=self.bin_ws,
                                            gparams=self.gparams)
            if self.random_bg:   # drawn before the step advance, as in enqueue()
                kernels.composite_random_bg(self.rgba_pm[cf], self.step_block, cf, self.bg_seed,
                                            self.bg, self.target_buf)
            kernels.assign_bins_counted(self.proj, self.keep, self.H, self.W, self.S, self.K,
                                        self.span, self.bin_ws, self.idx, self.valid, self.count,
                                        self.ncand, inv=self.inv, order=self.order,
                                        slot_rec=self.slot_rec, pos_count=self.pos_count,
                                        advance=self.step_block)
            self._splat_forward(self.bg)
            self._loss_and_splat_backward(cf)
        self._geometry_backward_adam((ci + n - 1) % ns)

    def enqueue_relocate(self):
        """Enqueue one MCMC relocation (dead slots onto live gaussians, moments reset)."""
        mc = self.mc
        kernels.relocate(self.P, self.m, self.v, self.step_block, mc["dead_thr"], mc["offset"],
                         mc["seed"], self.reloc_ws, self.moved, self.sh, self.sh_m, self.sh_v)
        self.relocations += self.moved

    def capture(self, cams=None, run_len=8):
        """Capture one HIP graph per camera.  A warm-up step runs eagerly first (so every
        kernel's code object is resident) and its effect on the state is rolled back.  Without
        relocation and with all cameras, run_len > 1 also captures, for every starting step and
        every phase of the bin cadence (the running step count mod bin_every), one graph of
        run_len consecutive steps (used by run())."""
        cams = range(self.n_steps) if cams is None else cams
        live = [self.P, self.m, self.v, self.step_block, self.bg]
        if self.sh is not None:
            live += [self.sh, self.sh_m, self.sh_v]
        if self.dw is not None:
            live += [self.dw, self.dw_state, self.gdw]
        state = [t.clone() for t in live]
        variants = (True, False) if self.bin_every > 1 else (True,)
        side = torch.cuda.Stream(device=self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(side):
            for ci in cams:
                for rebin in variants:
                    self.enqueue(ci, rebin)
            if self.mc["relocate_every"]:
                self.enqueue_relocate()
            if run_len > 1 and self.seamed:   # the seam launch's first call, outside capture
                self.enqueue_seamed(0, 2)
        torch.cuda.current_stream(self.dev).wait_stream(side)
        for dst, src in zip(live, state):
            dst.copy_(src)
        if self.mc["relocate_every"]:
            self.relocations.zero_()
        torch.cuda.synchronize(self.dev)
        for ci in cams:
            for rebin in variants:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    self.enqueue(ci, rebin)
                self.graphs[(ci, rebin)] = g
        if self.mc["relocate_every"]:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.enqueue_relocate()
            self.reloc_graph = g
        self.run_graphs, self.run_len = {}, 1
        if (run_len > 1 and not self.mc["relocate_every"]
                and list(cams) == list(range(self.n_steps))):
            for c in cams:
                for ph in range(self.bin_every):
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g):
                        if self.seamed:
                            self.enqueue_seamed(c, run_len)
                        else:
                            for j in range(run_len):
                                self.enqueue((c + j) % self.n_steps,
                                             (ph + j) % self.bin_every == 0)
                    self.run_graphs[(c, ph)] = g
            self.run_len = run_len
        torch.cuda.synchronize(self.dev)

    def run(self, ci=0, n=1):
        """n training steps: step ci, ci + 1, ... (mod n_steps), as n step() calls would run
        them; whole runs of run_len steps replay one captured graph each (the one for their
        first step and the bin cadence's phase there), the rest and a step that must rebin out
        of cadence (after forward() or eval_psnr()) run as step() calls."""
        i = 0
        while i < n:
            c = (ci + i) % self.n_steps
            g = None
            if n - i >= self.run_len and not self._force_rebin:
                g = self.run_graphs.get((c, self._it % self.bin_every))
            if g is not None:
                g.replay()
                self._it += self.run_len
                i += self.run_len
            else:
                self.step(c)
                i += 1

    def step(self, ci=0):
        """Training step ci: camera ci, or batch ci (graph replay when captured, else eager).
        With bin_every = N the bins are recomputed on every N-th step() call (counting from the
        first) and after a relocation, and reused otherwise."""
        rebin = self._it % self.bin_every == 0 or self._force_rebin
        self._force_rebin = False
        g = self.graphs.get((ci, rebin))
        if g is not None:
            g.replay()
        else:
            self.enqueue(ci, rebin)
        every = self.mc["relocate_every"]
        if every and self._it > 0 and self._it % every == 0:
            if self.reloc_graph is not None:
                self.reloc_graph.replay()
            else:
                self.enqueue_relocate()
            self._force_rebin = True     # relocated gaussians move: the next step rebins
        self._it += 1

    @torch.no_grad()
    def eval_psnr(self, cameras, images):
        """Mean PSNR over (camera, image) pairs of the binned device render, on a white
        background (c_b = 1: the reference's evaluation of its trainer, tools/resident_traced.py:
        768-783; psnr as spike/metrics.py:10-12, on clamped images).  images: [H,W,3], or RGBA
        [H,W,4] composited over white.  Each view is binned and rendered on its own; the next
        step() rebins.  Parameters and optimiser state are untouched."""
        if len(cameras) != len(images) or not cameras:
            raise ValueError("eval_psnr needs one image per camera")
        vals = []
        for cam, img in zip(cameras, images):
            if (cam.H, cam.W) != (self.H, self.W):
                raise ValueError(f"eval camera is {cam.W}x{cam.H}, the step renders "
                                 f"{self.W}x{self.H}")
            self._forward(0, rebin=True, grads=False, camera=cam.device_block(self.dev),
                          bg=self.bg_white)
            gt = torch.as_tensor(img).to(self.dev, F32)
            if gt.shape[-1] == 4:
                gt = gt[..., :3] * gt[..., 3:4] + (1.0 - gt[..., 3:4])
            mse = (self.image.clamp(0.0, 1.0) - gt.clamp(0.0, 1.0)).pow(2).mean()
            vals.append(float(-10.0 * torch.log10(mse.clamp(min=1e-12))))
        self._force_rebin = True
        return sum(vals) / len(vals)

    def loss(self):
        """Loss of the last step (a device scalar; reading it synchronises)."""
        return kernels.loss_from_partials(self.partials, self.H, self.W, self.lam)

    @property
    def steps_done(self):
        return int(self.step_block[0].item())
