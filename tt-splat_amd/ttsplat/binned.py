"""Binned poly-splat render on the GPU, with the reference's entry points.

Mirrors tools/m4_train_binned.py:
  K_POLY                      :39
  TileMap(H, W)               :60-72   (adds the tile side S; the reference fixes S=16)
  assign_bins(mu2d, keep, tmap, R, K)  :75-127  -> idx[T,K] int64 (0 in empty slots), valid bool
  theta_u_gathered            :130-143 (here from the per-gaussian records + bins)
  _operands(model, cam, tmap, R, K, cached_bins)  :189-212 (returns its 5-tuple)
  _DevRenderBinned            :154-186 (autograd op on pre-gathered operands)
  render_binned_device(model, cam, tmap, R, K, cached_bins, return_bins)  :215-219
The model is duck-typed as in the reference (means3d, quats, log_scales, opacity_raw, color_dc,
w_b_raw, c_b), or is a ttsplat.model.GaussianModel holding the [G,14] block directly.
Every op runs in libttsplat; tensors must live on a GPU.
"""
import torch
import torch.nn.functional as F

from . import kernels
from .kernels import F32

K_POLY = 4.0


class TileMap:
    """Tile geometry for S x S tiles (tools/m4_train_binned.py:60-72)."""

    def __init__(self, H, W, S=16, device="cuda"):
        if S not in (16, 32):
            raise ValueError(f"tile side must be 16 or 32, got {S}")
        if H % S or W % S:
            raise ValueError(f"image {H}x{W} is not a multiple of the tile side {S}")
        self.H, self.W, self.S = H, W, S
        self.nty, self.ntx = H // S, W // S
        self.T = self.nty * self.ntx
        p = torch.arange(S * S)
        lx = (p % S).float() + 0.5
        ly = (p // S).float() + 0.5
        self.Phi = torch.stack([lx * lx, ly * ly, lx * ly, lx, ly, torch.ones_like(lx)], -1).to(device)
        t = torch.arange(self.T)
        ty, tx = t // self.ntx, t % self.ntx
        self.origins = torch.stack([(tx * S).float(), (ty * S).float()], 1).to(device)
        row = ty[:, None] * S + (p // S)[None, :]
        col = tx[:, None] * S + (p % S)[None, :]
        self.gidx = (row * W + col).reshape(-1).to(device)
        self.span = 2048 if S == 16 else 8192


def params_of(model):
    """The [G,14] parameter block of a model (differentiable concatenation of the reference's
    separate tensors, or the model's own block)."""
    P = getattr(model, "params", None)
    if isinstance(P, torch.Tensor) and P.dim() == 2 and P.shape[1] == 14:
        return P
    op = model.opacity_raw.reshape(-1, 1)
    return torch.cat([model.means3d, model.quats, model.log_scales, model.color_dc, op], dim=1)


def _checked_bins(bins, G):
    """Cached bins from the caller: int32/uint8 device copies, gaussian ids checked to lie in
    [0, G) (the kernels index the per-gaussian records with them)."""
    idx32 = bins[0].to(torch.int32).contiguous()
    v8 = bins[1].to(torch.uint8).contiguous()
    if idx32.numel() and (int(idx32.min()) < 0 or int(idx32.max()) >= G):
        raise ValueError(f"bin indices must lie in [0, {G})")
    return idx32, v8


def background(model, device):
    """bg block [w_b, c_b r, g, b] with w_b = softplus(w_b_raw) (spike/render.py:28)."""
    w_b = F.softplus(torch.as_tensor(model.w_b_raw, dtype=F32, device=device).reshape(1))
    c_b = torch.as_tensor(model.c_b, dtype=F32, device=device).reshape(3)
    return torch.cat([w_b, c_b]).contiguous()


@torch.no_grad()
def assign_bins(mu2d, keep, tmap, R=1, K=128, span=None):
    """Per-tile gaussian lists (tools/m4_train_binned.py:75-127) in the reference layout:
    idx[T,K] int64 with 0 in empty slots, valid[T,K] bool."""
    mu2d = mu2d.detach()
    if mu2d.dtype != F32:
        mu2d = mu2d.float()
    if mu2d.stride(-1) != 1:
        mu2d = mu2d.contiguous()
    keep = keep.detach().to(torch.uint8).contiguous()
    idx, valid, _, _ = kernels.assign_bins(mu2d, keep, tmap.H, tmap.W, tmap.S, K,
                                           span or tmap.span, R)
    return idx.long(), valid.bool()


def project(model, cam, blur_eps=kernels.BLUR, near=kernels.NEAR):
    """Geometry forward on the GPU: returns the proj record [G,12] and keep [G] uint8."""
    P = params_of(model).detach().contiguous()
    return kernels.geom_fwd(P, cam.device_block(P.device), near, blur_eps)


@torch.no_grad()
def theta_u_gathered(proj, idx, valid, tmap, k=K_POLY):
    """theta_u[T,6,K], color_o_t[T,K,3], o_col_t[T,K,1] for the given bins
    (tools/m4_train_binned.py:130-143 with the gathers of :207-211)."""
    idx32, v8 = _checked_bins((idx, valid), proj.shape[0])
    th, col, oc = kernels.theta_gather(proj, idx32, v8, tmap.H, tmap.W, tmap.S, k)
    return th, col, oc[..., None]


@torch.no_grad()
def _operands(model, cam, tmap, R=1, K=128, cached_bins=None, k=K_POLY):
    """Geometry + binning + gather (tools/m4_train_binned.py:189-212), values only.
    Returns (theta_u, color_o_t, o_col_t, w_b, (idx, valid))."""
    proj, keep = project(model, cam)
    if cached_bins is None:
        idx32, v8, _, _ = kernels.assign_bins(proj[:, 0:2], keep, tmap.H, tmap.W, tmap.S, K,
                                              tmap.span, R)
        bins = (idx32.long(), v8.bool())
    else:
        bins = cached_bins
        idx32, v8 = _checked_bins(bins, proj.shape[0])
    th, col, oc = kernels.theta_gather(proj, idx32, v8, tmap.H, tmap.W, tmap.S, k)
    w_b = F.softplus(torch.as_tensor(model.w_b_raw, dtype=F32, device=proj.device))
    return th, col, oc[..., None], w_b, bins


def _dev_render_forward(ctx, operand_dtype, theta_u, color_o, o_col, w_b, Phi, H, W):
    S = int(round(Phi.shape[0] ** 0.5))
    dev = theta_u.device
    bg = torch.cat([torch.as_tensor(w_b, dtype=F32, device=dev).reshape(1),
                    torch.as_tensor(ctx.c_b, dtype=F32, device=dev).reshape(3)]).contiguous()
    dt = torch.bfloat16 if theta_u.dtype == torch.bfloat16 else operand_dtype
    th = theta_u.detach().to(dt).contiguous()
    col = color_o.detach().to(dt).contiguous()
    oc = o_col.detach().to(dt).reshape(th.shape[0], th.shape[2]).contiguous()
    img, den = kernels.splat_fwd_theta(th, col, oc, bg, H, W, S)
    ctx.save_for_backward(th, col, oc, bg, img, den)
    ctx.meta = (H, W, S, o_col.shape, theta_u.dtype, color_o.dtype, o_col.dtype)
    return img


class DevRenderBinned(torch.autograd.Function):
    """Splat forward/backward on pre-gathered operands (tools/m4_train_binned.py:154-186).

    forward(theta_u[T,6,K], color_o[T,K,3], o_col[T,K,1], w_b, Phi, gidx, c_b, H, W) -> img[H,W,3];
    backward returns (gtheta_u, gcolor_o, go_col, gw_b).  Phi/gidx describe the tile map
    (only its tile side is used: the kernel evaluates Phi itself).  fp32 operands (bf16 input
    tensors run the bf16 entry points); gradients come back in each input's dtype."""

    @staticmethod
    def forward(ctx, theta_u, color_o, o_col, w_b, Phi, gidx, c_b, H, W):
        ctx.c_b = c_b
        return _dev_render_forward(ctx, F32, theta_u, color_o, o_col, w_b, Phi, H, W)

    @staticmethod
    def backward(ctx, gimg):
        th, col, oc, bg, img, den = ctx.saved_tensors
        H, W, S, oc_shape, dth, dcol, doc = ctx.meta
        gwb = torch.empty(th.shape[0], device=th.device, dtype=F32)
        gth, gcol, goc = kernels.splat_bwd_theta(th, col, oc, bg, H, W, S, img, den,
                                                 gimg.float().contiguous(), gwb)
        return (gth.to(dth), gcol.to(dcol), goc.reshape(oc_shape).to(doc), gwb.sum(), None, None,
                None, None, None)


class _DevRenderBinned(DevRenderBinned):
    """The reference's own class (tools/m4_train_binned.py:154-186): operands uploaded as bf16
    (`up`, :42-43), the bf16 render variant; fp32 arithmetic on the bf16-rounded operands.  The
    rounding of theta loses precision as in the reference (:36): 3.6e-2 rel L2 against fp32
    operands on the 128x128 64-tile scene."""

    @staticmethod
    def forward(ctx, theta_u, color_o, o_col, w_b, Phi, gidx, c_b, H, W):
        ctx.c_b = c_b
        return _dev_render_forward(ctx, torch.bfloat16, theta_u, color_o, o_col, w_b, Phi, H, W)


class BinnedRender(torch.autograd.Function):
    """Whole binned render as one differentiable op of the [G,14] parameter block:
    geometry -> (given bins) -> fused splat; backward: fused splat bwd with theta bwd into
    per-slot gradients -> slot->gaussian reduce (through the inverse table when the bins came
    with one, else an atomic scatter) -> geometry bwd."""

    @staticmethod
    def forward(ctx, P, camera, bg, idx32, v8, inv, H, W, S, k):
        Pc = P.detach().contiguous()
        proj, keep = kernels.geom_fwd(Pc, camera)
        img, den = kernels.splat_fwd(proj, idx32, v8, bg, H, W, S, k)
        ctx.save_for_backward(Pc, camera, bg, idx32, v8, proj, img, den)
        ctx.inv = inv
        ctx.meta = (H, W, S, k)
        return img

    @staticmethod
    def backward(ctx, gimg):
        Pc, camera, bg, idx32, v8, proj, img, den = ctx.saved_tensors
        H, W, S, k = ctx.meta
        gwb = torch.empty(idx32.shape[0], device=Pc.device, dtype=F32)
        gslot = kernels.splat_bwd(proj, idx32, v8, bg, H, W, S, k, img, den,
                                  gimg.float().contiguous(), gwb=gwb)
        if ctx.inv is not None:
            grad9 = kernels.slot_reduce(gslot, ctx.inv)
        else:
            grad9 = kernels.slot_scatter(gslot, idx32, v8, Pc.shape[0])
        gP = kernels.geom_bwd(Pc, camera, grad9)
        gbg = torch.zeros(4, device=Pc.device, dtype=F32)
        gbg[0] = gwb.sum()
        return gP, None, gbg, None, None, None, None, None, None, None


def render_binned_device(model, cam, tmap, R=1, K=128, cached_bins=None, return_bins=False,
                         k=K_POLY):
    """Binned render of `model` from `cam` (tools/m4_train_binned.py:215-219), differentiable
    w.r.t. the model's parameters.  Bins are recomputed unless cached_bins is given."""
    P = params_of(model)
    dev = P.device
    camera = cam.device_block(dev)
    inv = None
    if cached_bins is None:
        proj, keep = kernels.geom_fwd(P.detach().contiguous(), camera)
        inv = torch.empty(P.shape[0], 9, device=dev, dtype=torch.int32)
        idx32, v8, _, _ = kernels.assign_bins(proj[:, 0:2], keep, tmap.H, tmap.W, tmap.S, K,
                                              tmap.span, R, inv=inv)
        bins = (idx32.long(), v8.bool())
    else:
        bins = cached_bins
        idx32, v8 = _checked_bins(bins, P.shape[0])
    img = BinnedRender.apply(P, camera, background(model, dev), idx32, v8, inv, tmap.H, tmap.W,
                             tmap.S, float(k))
    return (img, bins) if return_bins else img
