"""Typed wrappers over the libttsplat C ABI.

Each wrapper validates device, dtype, contiguity and shape of every tensor, then enqueues the
kernel on the current torch stream.  Nothing here allocates unless an output is not supplied
(out=None); the graph-captured training step passes every buffer in.
"""
import ctypes

import torch

from . import _lib
from ._lib import call, ptr, require, stream

F32, I32, U8 = torch.float32, torch.int32, torch.uint8

NEAR, BLUR = 0.2, 0.3          # tools/geom_device.py:25
BETA1, BETA2, EPS = 0.9, 0.999, 1e-8   # tools/resident_traced.py:92


def _aligned16(t, name):
    """The kernels read [G,12] records as float4: the base address must be 16-byte aligned."""
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must start on a 16-byte boundary")
    return t


def version():
    v = _lib.load().tts_version()
    return (v >> 16, v & 0xFFFF)


# ------------------------------------------------------------------------------- geometry --
SH_REST = 15   # rest coefficients per channel (SH degrees 1-3)


def sh_rest_layout(color_rest):
    """spike's color_rest [G,15,3] -> the library's coefficient-major rest block [15,3,G]."""
    if color_rest.dim() != 3 or tuple(color_rest.shape[1:]) != (SH_REST, 3):
        raise ValueError(f"color_rest must be [G,{SH_REST},3], got {tuple(color_rest.shape)}")
    return color_rest.permute(1, 2, 0).contiguous()


def sh_rest_model(rest):
    """The library's rest block [15,3,G] -> spike's color_rest layout [G,15,3]."""
    return rest.permute(2, 0, 1).contiguous()


def _sh_check(sh_rest, sh_degree, G, dev):
    if not 0 <= int(sh_degree) <= 3:
        raise ValueError(f"sh_degree must be in [0, 3], got {sh_degree}")
    if int(sh_degree) > 0:
        if sh_rest is None:
            raise ValueError("sh_degree > 0 needs the rest coefficients sh_rest [15,3,G]")
        require(sh_rest, "sh_rest", F32, (SH_REST, 3, G), dev)


def _dw_check(depth_bt, dev):
    if depth_bt is not None:
        require(depth_bt, "depth_bt", F32, (2,), dev)


def geom_fwd(params, camera, near=NEAR, blur=BLUR, proj=None, keep=None, sh_rest=None,
             sh_degree=0, depth_bt=None, advance=None, b1=None, b2=None):
    """Projection + activations -> proj[G,12], keep[G].  sh_degree > 0: view-dependent colour
    from the rest coefficients sh_rest [15,3,G] (sh_rest_layout of spike's color_rest).
    depth_bt (device (beta, tau)): the depth weight sigmoid(beta (tau - z_cam)) on the opacity.
    advance (a training step's Adam step block): advanced in the same launch, as
    adam_advance(advance, b1, b2) would."""
    G = params.shape[0]
    dev = params.device
    require(params, "params", F32, (G, 14))
    require(camera, "camera", F32, (16,), dev)
    _sh_check(sh_rest, sh_degree, G, dev)
    _dw_check(depth_bt, dev)
    proj = torch.empty(G, 12, device=dev, dtype=F32) if proj is None else proj
    keep = torch.empty(G, device=dev, dtype=U8) if keep is None else keep
    _aligned16(require(proj, "proj", F32, (G, 12), dev), "proj")
    require(keep, "keep", U8, (G,), dev)
    if advance is not None:
        require(advance, "advance", I32, (4,), dev)
    if sh_degree > 0 or depth_bt is not None or advance is not None:
        call("tts_geom_fwd_ex", ptr(params), ptr(sh_rest), int(sh_degree), ptr(depth_bt), G,
             ptr(camera), near, blur, ptr(proj), ptr(keep), ptr(advance),
             BETA1 if b1 is None else b1, BETA2 if b2 is None else b2, stream())
    else:
        call("tts_geom_fwd", ptr(params), G, ptr(camera), near, blur, ptr(proj), ptr(keep),
             stream())
    return proj, keep


def geom_bwd(params, camera, grad9, near=NEAR, blur=BLUR, out=None, sh_rest=None, sh_degree=0,
             gsh_out=None, depth_bt=None, depth_zgrad=False, gdepth=None, sh_dirgrad=False):
    """grad9[G,9] -> dL/dparams[G,14].  With sh_degree > 0 also dL/dsh_rest [15,3,G]; with
    depth_bt also dL/d(beta, tau) per gaussian [G,2] (depth_zgrad: plus the gradient through
    z_cam into the means; sh_dirgrad: plus the SH colour's gradient through its view direction
    into the means, as spike's dense autograd has them).  Returns gparams, or a tuple
    (gparams, gsh, gdepth) when either extension is on (absent parts None)."""
    G = params.shape[0]
    dev = params.device
    require(params, "params", F32, (G, 14))
    require(camera, "camera", F32, (16,), dev)
    require(grad9, "grad9", F32, (G, 9), dev)
    _sh_check(sh_rest, sh_degree, G, dev)
    _dw_check(depth_bt, dev)
    out = torch.empty(G, 14, device=dev, dtype=F32) if out is None else out
    require(out, "gparams", F32, (G, 14), dev)
    if sh_degree > 0 or depth_bt is not None:
        gsh = None
        if sh_degree > 0:
            gsh = torch.empty(SH_REST, 3, G, device=dev, dtype=F32) if gsh_out is None else gsh_out
            require(gsh, "gsh_out", F32, (SH_REST, 3, G), dev)
        gdw = None
        if depth_bt is not None:
            gdw = torch.empty(G, 2, device=dev, dtype=F32) if gdepth is None else gdepth
            require(gdw, "gdepth", F32, (G, 2), dev)
        flags = (1 if depth_zgrad else 0) | (2 if sh_dirgrad and sh_degree > 0 else 0)
        call("tts_geom_bwd_ex", ptr(params), ptr(sh_rest), int(sh_degree), ptr(depth_bt),
             flags, G, ptr(camera), near, blur, ptr(grad9), ptr(out), ptr(gsh), ptr(gdw),
             stream())
        return out, gsh, gdw
    call("tts_geom_bwd", ptr(params), G, ptr(camera), near, blur, ptr(grad9), ptr(out), stream())
    return out


# -------------------------------------------------------------------------------- binning --
def bin_workspace(G, H, W, S, device):
    """Zero-initialised workspace for assign_bins (kept zeroed by the library)."""
    n = _lib.load().tts_bin_workspace_bytes(G, H, W, S)
    return torch.zeros(max(n, 1), device=device, dtype=U8)


def assign_bins(mu2d, keep, H, W, S=16, K=128, span=2048, R=1, workspace=None, idx=None,
                valid=None, count=None, ncand=None, inv=None, order=None):
    """mu2d: [G,2] fp32 (or any [G,>=2] row-contiguous view, e.g. the proj record),
    keep: [G] uint8 or bool.  Returns idx[T,K] int32, valid[T,K] uint8, count[T], ncand[T];
    the inverse table inv[G,9] and the heaviest-first tile order[T] are written when buffers are
    passed."""
    G = mu2d.shape[0]
    dev = mu2d.device
    if not mu2d.is_cuda or mu2d.dtype != F32 or mu2d.dim() != 2 or mu2d.shape[1] < 2 \
            or mu2d.stride(1) != 1:
        raise ValueError("mu2d must be a [G,>=2] fp32 GPU tensor with unit column stride")
    if keep.dtype == torch.bool:
        keep = keep.view(U8)
    require(keep, "keep", U8, (G,), dev)
    if S not in (16, 32) or H % S or W % S:
        raise ValueError(f"tile side {S} must be 16 or 32 and divide {H}x{W}")
    T = (H // S) * (W // S)
    idx = torch.empty(T, K, device=dev, dtype=I32) if idx is None else idx
    valid = torch.empty(T, K, device=dev, dtype=U8) if valid is None else valid
    count = torch.empty(T, device=dev, dtype=I32) if count is None else count
    ncand = torch.empty(T, device=dev, dtype=I32) if ncand is None else ncand
    require(idx, "idx", I32, (T, K), dev)
    require(valid, "valid", U8, (T, K), dev)
    require(count, "count", I32, (T,), dev)
    require(ncand, "ncand", I32, (T,), dev)
    if inv is not None:
        require(inv, "inv", I32, (G, 9), dev)
    if order is not None:
        require(order, "order", I32, (T,), dev)
    workspace = bin_workspace(G, H, W, S, dev) if workspace is None else workspace
    call("tts_assign_bins", ptr(mu2d), mu2d.stride(0), ptr(keep), 1, G, H, W, S, R, K, span,
         ptr(idx), ptr(valid), ptr(count), ptr(ncand), ptr(inv), ptr(order), ptr(workspace),
         workspace.numel(), stream())
    return idx, valid, count, ncand


def geom_fwd_assign_bins(params, camera, H, W, S=16, K=128, span=2048, R=1, near=NEAR,
                         blur=BLUR, proj=None, keep=None, sh_rest=None, sh_degree=0,
                         depth_bt=None, advance=None, b1=None, b2=None, workspace=None, idx=None,
                         valid=None, count=None, ncand=None, inv=None, order=None,
                         slot_rec=None, pos_count=None):
    """geom_fwd then assign_bins on proj's means and keep, as one call (for G <= 131072 the
    binning's count pass runs inside the geometry launch).  Returns (proj, keep, idx, valid,
    count, ncand); inv and order are written when buffers are passed, and with order the slot
    records slot_rec [T,K,12] (proj[idx] of every kept slot, tiles in dispatch order) and
    pos_count [T] (their kept counts) when those are passed."""
    G = params.shape[0]
    dev = params.device
    require(params, "params", F32, (G, 14))
    require(camera, "camera", F32, (16,), dev)
    _sh_check(sh_rest, sh_degree, G, dev)
    _dw_check(depth_bt, dev)
    proj = torch.empty(G, 12, device=dev, dtype=F32) if proj is None else proj
    keep = torch.empty(G, device=dev, dtype=U8) if keep is None else keep
    _aligned16(require(proj, "proj", F32, (G, 12), dev), "proj")
    require(keep, "keep", U8, (G,), dev)
    if advance is not None:
        require(advance, "advance", I32, (4,), dev)
    if S not in (16, 32) or H % S or W % S:
        raise ValueError(f"tile side {S} must be 16 or 32 and divide {H}x{W}")
    T = (H // S) * (W // S)
    idx = torch.empty(T, K, device=dev, dtype=I32) if idx is None else idx
    valid = torch.empty(T, K, device=dev, dtype=U8) if valid is None else valid
    count = torch.empty(T, device=dev, dtype=I32) if count is None else count
    ncand = torch.empty(T, device=dev, dtype=I32) if ncand is None else ncand
    require(idx, "idx", I32, (T, K), dev)
    require(valid, "valid", U8, (T, K), dev)
    require(count, "count", I32, (T,), dev)
    require(ncand, "ncand", I32, (T,), dev)
    if inv is not None:
        require(inv, "inv", I32, (G, 9), dev)
    if order is not None:
        require(order, "order", I32, (T,), dev)
    if (slot_rec is None) != (pos_count is None) or (slot_rec is not None and order is None):
        raise ValueError("slot_rec and pos_count go together, and need order")
    if slot_rec is not None:
        _aligned16(require(slot_rec, "slot_rec", F32, (T, K, 12), dev), "slot_rec")
        require(pos_count, "pos_count", I32, (T,), dev)
    workspace = bin_workspace(G, H, W, S, dev) if workspace is None else workspace
    call("tts_geom_fwd_assign_bins", ptr(params), ptr(sh_rest), int(sh_degree), ptr(depth_bt),
         G, ptr(camera), near, blur, ptr(proj), ptr(keep), ptr(advance),
         BETA1 if b1 is None else b1, BETA2 if b2 is None else b2, H, W, S, R, K, span,
         ptr(idx), ptr(valid), ptr(count), ptr(ncand), ptr(inv), ptr(order), ptr(slot_rec),
         ptr(pos_count), ptr(workspace), workspace.numel(), stream())
    return proj, keep, idx, valid, count, ncand


SEAM_MAX_G = 131072   # count blocks of 512 gaussians: the seam launch's limit
# below this the two launches are as fast or faster (train it/s at 1264x832, seam vs two
# launches: G = 10k +0.1 %, 25k +0.6 %, 50k +1.6 %, 100k +2.8 %; 800x800, G = 10k -1.7 %)
SEAM_MIN_G = 32768


def geom_bwd_adam_fwd_count(params, camera_bwd, camera_fwd, gslot, inv, m, v, lr, step, proj,
                            keep, H, W, S=16, K=128, span=2048, R=1, workspace=None,
                            gparams=None, near=NEAR, blur=BLUR, b1=BETA1, b2=BETA2, eps=EPS):
    """The seam between two training steps, one launch: geom_bwd_adam (camera_bwd) and then
    the next step's geometry forward (camera_fwd, into proj / keep) with its binning's count
    pass into workspace -- finish that binning with assign_bins_counted on the same workspace.
    Equals geom_bwd_adam followed by geom_fwd_assign_bins; plain steps only (no SH, depth weight
    or MCMC terms) and G <= SEAM_MAX_G."""
    G = params.shape[0]
    dev = params.device
    if not 0 < G <= SEAM_MAX_G:
        raise ValueError(f"the seam launch takes 0 < G <= {SEAM_MAX_G}, got {G}")
    for t, n in ((params, "params"), (m, "m"), (v, "v")):
        require(t, n, F32, (G, 14), dev)
    require(camera_bwd, "camera_bwd", F32, (16,), dev)
    require(camera_fwd, "camera_fwd", F32, (16,), dev)
    require(inv, "inv", I32, (G, 9), dev)
    if gslot.dim() != 3 or gslot.shape[2] != 9:
        raise ValueError("gslot must be [T,K,9]")
    require(gslot, "gslot", F32, tuple(gslot.shape), dev)
    require(lr, "lr", F32, (14,), dev)
    require(step, "step", I32, (4,), dev)
    if gparams is not None:
        require(gparams, "gparams", F32, (G, 14), dev)
    _aligned16(require(proj, "proj", F32, (G, 12), dev), "proj")
    require(keep, "keep", U8, (G,), dev)
    if S not in (16, 32) or H % S or W % S:
        raise ValueError(f"tile side {S} must be 16 or 32 and divide {H}x{W}")
    workspace = bin_workspace(G, H, W, S, dev) if workspace is None else workspace
    call("tts_geom_bwd_adam_fwd_count", ptr(params), G, ptr(camera_bwd), ptr(camera_fwd), near,
         blur, ptr(gslot), ptr(inv), ptr(gparams), ptr(m), ptr(v), ptr(lr), ptr(step), b1, b2,
         eps, ptr(proj), ptr(keep), H, W, S, R, K, span, ptr(workspace), workspace.numel(),
         stream())
    return workspace


def assign_bins_counted(proj, keep, H, W, S, K, span, workspace, idx, valid, count, ncand,
                        inv=None, order=None, slot_rec=None, pos_count=None, advance=None, R=1,
                        b1=BETA1, b2=BETA2):
    """The rest of geom_fwd_assign_bins after geom_bwd_adam_fwd_count ran its count pass into
    workspace (column scan, scatter, select): the same idx, valid, count, ncand, inv, order and
    slot records.  advance: the Adam step block, advanced by the column scan."""
    G = proj.shape[0]
    dev = proj.device
    if not 0 < G <= SEAM_MAX_G:
        raise ValueError(f"the seam launch takes 0 < G <= {SEAM_MAX_G}, got {G}")
    _aligned16(require(proj, "proj", F32, (G, 12), dev), "proj")
    require(keep, "keep", U8, (G,), dev)
    T = (H // S) * (W // S)
    require(idx, "idx", I32, (T, K), dev)
    require(valid, "valid", U8, (T, K), dev)
    require(count, "count", I32, (T,), dev)
    require(ncand, "ncand", I32, (T,), dev)
    if inv is not None:
        require(inv, "inv", I32, (G, 9), dev)
    if order is not None:
        require(order, "order", I32, (T,), dev)
    if (slot_rec is None) != (pos_count is None) or (slot_rec is not None and order is None):
        raise ValueError("slot_rec and pos_count go together, and need order")
    if slot_rec is not None:
        _aligned16(require(slot_rec, "slot_rec", F32, (T, K, 12), dev), "slot_rec")
        require(pos_count, "pos_count", I32, (T,), dev)
    if advance is not None:
        require(advance, "advance", I32, (4,), dev)
    call("tts_assign_bins_counted", ptr(proj), ptr(keep), G, H, W, S, R, K, span, ptr(idx),
         ptr(valid), ptr(count), ptr(ncand), ptr(inv), ptr(order), ptr(slot_rec), ptr(pos_count),
         ptr(advance), b1, b2, ptr(workspace), workspace.numel(), stream())
    return idx, valid, count, ncand


# ---------------------------------------------------------------------------------- splat --
def _bins_check(idx, valid, H, W, S, dev):
    T = (H // S) * (W // S)
    if idx.dim() != 2 or idx.shape[0] != T:
        raise ValueError(f"idx must be [T={T},K], got {tuple(idx.shape)}")
    K = idx.shape[1]
    if valid.dtype == torch.bool:
        valid = valid.view(U8)
    require(idx, "idx", I32, (T, K), dev)
    require(valid, "valid", U8, (T, K), dev)
    return T, K, valid


def theta_gather(proj, idx, valid, H, W, S, k, theta=None, col=None, oc=None):
    dev = proj.device
    _aligned16(require(proj, "proj", F32, (proj.shape[0], 12)), "proj")
    T, K, valid = _bins_check(idx, valid, H, W, S, dev)
    theta = torch.empty(T, 6, K, device=dev, dtype=F32) if theta is None else theta
    col = torch.empty(T, K, 3, device=dev, dtype=F32) if col is None else col
    oc = torch.empty(T, K, device=dev, dtype=F32) if oc is None else oc
    require(theta, "theta", F32, (T, 6, K), dev)
    require(col, "col", F32, (T, K, 3), dev)
    require(oc, "oc", F32, (T, K), dev)
    call("tts_theta_u_gathered", ptr(proj), ptr(idx), ptr(valid), H, W, S, K, float(k),
         ptr(theta), ptr(col), ptr(oc), stream())
    return theta, col, oc


def tile_order(count, K, order=None):
    """Tile ids by kept count, heaviest first (scheduling order for the splat kernels)."""
    T = count.shape[0]
    require(count, "count", I32, (T,))
    order = torch.empty(T, device=count.device, dtype=I32) if order is None else order
    require(order, "order", I32, (T,), count.device)
    call("tts_tile_order", ptr(count), T, K, ptr(order), stream())
    return order


def splat_fwd(proj, idx, valid, bg, H, W, S, k, image=None, den=None, order=None):
    dev = proj.device
    _aligned16(require(proj, "proj", F32, (proj.shape[0], 12)), "proj")
    T, K, valid = _bins_check(idx, valid, H, W, S, dev)
    require(bg, "bg", F32, (4,), dev)
    image = torch.empty(H, W, 3, device=dev, dtype=F32) if image is None else image
    den = torch.empty(H, W, device=dev, dtype=F32) if den is None else den
    require(image, "image", F32, (H, W, 3), dev)
    require(den, "den", F32, (H, W), dev)
    if order is not None:
        require(order, "order", I32, (T,), dev)
    call("tts_splat_fwd", ptr(proj), ptr(idx), ptr(valid), ptr(order), H, W, S, K, float(k),
         ptr(bg), ptr(image), ptr(den), stream())
    return image, den


def _rec_check(slot_rec, pos_count, order, H, W, S, dev):
    if S != 16 or H % S or W % S:
        raise ValueError(f"the slot-record splat kernels take 16x16 tiles dividing {H}x{W}")
    T = (H // S) * (W // S)
    if slot_rec.dim() != 3 or slot_rec.shape[0] != T or slot_rec.shape[2] != 12:
        raise ValueError(f"slot_rec must be [T={T},K,12], got {tuple(slot_rec.shape)}")
    K = slot_rec.shape[1]
    _aligned16(require(slot_rec, "slot_rec", F32, (T, K, 12), dev), "slot_rec")
    require(pos_count, "pos_count", I32, (T,), dev)
    require(order, "order", I32, (T,), dev)
    return T, K


def splat_fwd_rec(slot_rec, pos_count, order, bg, H, W, S, k, image=None, den=None,
                  write_den=True):
    """splat_fwd on the slot records of geom_fwd_assign_bins (S = 16): the same image and den.
    write_den=False: a render only -- den (which only the backward reads) is not written."""
    dev = slot_rec.device
    T, K = _rec_check(slot_rec, pos_count, order, H, W, S, dev)
    require(bg, "bg", F32, (4,), dev)
    image = torch.empty(H, W, 3, device=dev, dtype=F32) if image is None else image
    require(image, "image", F32, (H, W, 3), dev)
    if write_den:
        den = torch.empty(H, W, device=dev, dtype=F32) if den is None else den
        require(den, "den", F32, (H, W), dev)
    else:
        den = None
    call("tts_splat_fwd_rec", ptr(slot_rec), ptr(pos_count), ptr(order), H, W, S, K, float(k),
         ptr(bg), ptr(image), ptr(den), stream())
    return image, den


def splat_fwd_mx_rec(slot_rec, pos_count, order, bg, H, W, S, k, image=None, den=None,
                     bf16=False, write_den=True):
    """splat_fwd_mx on the slot records of geom_fwd_assign_bins: the same image and den
    (write_den=False: den not written)."""
    dev = slot_rec.device
    T, K = _rec_check(slot_rec, pos_count, order, H, W, S, dev)
    require(bg, "bg", F32, (4,), dev)
    image = torch.empty(H, W, 3, device=dev, dtype=F32) if image is None else image
    require(image, "image", F32, (H, W, 3), dev)
    if write_den:
        den = torch.empty(H, W, device=dev, dtype=F32) if den is None else den
        require(den, "den", F32, (H, W), dev)
    else:
        den = None
    call("tts_splat_fwd_mx_rec", ptr(slot_rec), ptr(pos_count), ptr(order), H, W, S, K,
         float(k), ptr(bg), ptr(image), ptr(den), int(bool(bf16)), stream())
    return image, den


def splat_fwd_mx(proj, idx, valid, bg, H, W, S, k, image=None, den=None, order=None, bf16=False):
    """Matrix-core splat forward (S = 16): fp32-level accuracy, or the bf16 render variant."""
    dev = proj.device
    _aligned16(require(proj, "proj", F32, (proj.shape[0], 12)), "proj")
    T, K, valid = _bins_check(idx, valid, H, W, S, dev)
    require(bg, "bg", F32, (4,), dev)
    image = torch.empty(H, W, 3, device=dev, dtype=F32) if image is None else image
    den = torch.empty(H, W, device=dev, dtype=F32) if den is None else den
    require(image, "image", F32, (H, W, 3), dev)
    require(den, "den", F32, (H, W), dev)
    if order is not None:
        require(order, "order", I32, (T,), dev)
    call("tts_splat_fwd_mx", ptr(proj), ptr(idx), ptr(valid), ptr(order), H, W, S, K, float(k),
         ptr(bg), ptr(image), ptr(den), int(bool(bf16)), stream())
    return image, den


def splat_bwd(proj, idx, valid, bg, H, W, S, k, image, den, gimage, gslot=None, gwb=None,
              order=None):
    """Per-slot gradients gslot[T,K,9] (valid slots written); gwb[T] gets per-tile dL/dw_b."""
    dev = proj.device
    G = proj.shape[0]
    _aligned16(require(proj, "proj", F32, (G, 12)), "proj")
    T, K, valid = _bins_check(idx, valid, H, W, S, dev)
    require(bg, "bg", F32, (4,), dev)
    require(image, "image", F32, (H, W, 3), dev)
    require(den, "den", F32, (H, W), dev)
    require(gimage, "gimage", F32, (H, W, 3), dev)
    gslot = torch.zeros(T, K, 9, device=dev, dtype=F32) if gslot is None else gslot
    require(gslot, "gslot", F32, (T, K, 9), dev)
    if gwb is not None:
        require(gwb, "gwb", F32, (T,), dev)
    if order is not None:
        require(order, "order", I32, (T,), dev)
    call("tts_splat_bwd", ptr(proj), ptr(idx), ptr(valid), ptr(order), H, W, S, K, float(k),
         ptr(bg), ptr(image), ptr(den), ptr(gimage), ptr(gslot), ptr(gwb), stream())
    return gslot


def splat_bwd_rec(slot_rec, pos_count, order, bg, H, W, S, k, image, den, gimage, gslot=None,
                  gwb=None):
    """splat_bwd on the slot records of geom_fwd_assign_bins (S = 16): the same gslot."""
    dev = slot_rec.device
    T, K = _rec_check(slot_rec, pos_count, order, H, W, S, dev)
    require(bg, "bg", F32, (4,), dev)
    require(image, "image", F32, (H, W, 3), dev)
    require(den, "den", F32, (H, W), dev)
    require(gimage, "gimage", F32, (H, W, 3), dev)
    gslot = torch.zeros(T, K, 9, device=dev, dtype=F32) if gslot is None else gslot
    require(gslot, "gslot", F32, (T, K, 9), dev)
    if gwb is not None:
        require(gwb, "gwb", F32, (T,), dev)
    call("tts_splat_bwd_rec", ptr(slot_rec), ptr(pos_count), ptr(order), H, W, S, K, float(k),
         ptr(bg), ptr(image), ptr(den), ptr(gimage), ptr(gslot), ptr(gwb), stream())
    return gslot


def slot_reduce(gslot, inv, grad9=None):
    """grad9[G,9] = per-gaussian sum of its slots' gradients (through the inverse table)."""
    G = inv.shape[0]
    require(inv, "inv", I32, (G, 9))
    if gslot.dim() != 3 or gslot.shape[2] != 9:
        raise ValueError("gslot must be [T,K,9]")
    require(gslot, "gslot", F32, tuple(gslot.shape), inv.device)
    grad9 = torch.empty(G, 9, device=inv.device, dtype=F32) if grad9 is None else grad9
    require(grad9, "grad9", F32, (G, 9), inv.device)
    call("tts_slot_reduce", ptr(gslot), ptr(inv), G, ptr(grad9), stream())
    return grad9


def slot_scatter(gslot, idx, valid, G, grad9=None):
    """grad9[G,9] += gradients of every valid slot (float atomics; bins without inv)."""
    T, K = idx.shape
    if valid.dtype == torch.bool:
        valid = valid.view(U8)
    require(idx, "idx", I32, (T, K))
    require(valid, "valid", U8, (T, K), idx.device)
    require(gslot, "gslot", F32, (T, K, 9), idx.device)
    grad9 = torch.zeros(G, 9, device=idx.device, dtype=F32) if grad9 is None else grad9
    require(grad9, "grad9", F32, (G, 9), idx.device)
    call("tts_slot_scatter", ptr(gslot), ptr(idx), ptr(valid), T, K, ptr(grad9), stream())
    return grad9


def _theta_operands(theta, col, oc, H, W, S):
    """Checked operand triple; fp32 or bf16 (all three the same): returns (T, K, suffix)."""
    dev = theta.device
    T = (H // S) * (W // S)
    K = theta.shape[-1]
    dt = theta.dtype
    if dt not in (F32, torch.bfloat16):
        raise ValueError(f"theta must be float32 or bfloat16, got {dt}")
    require(theta, "theta", dt, (T, 6, K))
    require(col, "col", dt, (T, K, 3), dev)
    require(oc, "oc", dt, (T, K), dev)
    return T, K, ("_bf16" if dt == torch.bfloat16 else "")


def splat_fwd_theta(theta, col, oc, bg, H, W, S, image=None, den=None):
    """Splat forward from pre-gathered operands theta[T,6,K], col[T,K,3], oc[T,K]: fp32, or
    bf16 (the reference's operand upload, tools/m4_train_binned.py:42-43; fp32 arithmetic)."""
    dev = theta.device
    T, K, sfx = _theta_operands(theta, col, oc, H, W, S)
    require(bg, "bg", F32, (4,), dev)
    image = torch.empty(H, W, 3, device=dev, dtype=F32) if image is None else image
    den = torch.empty(H, W, device=dev, dtype=F32) if den is None else den
    call("tts_splat_fwd_theta" + sfx, ptr(theta), ptr(col), ptr(oc), H, W, S, K, ptr(bg),
         ptr(image), ptr(den), stream())
    return image, den


def splat_bwd_theta(theta, col, oc, bg, H, W, S, image, den, gimage, gwb=None):
    """Per-slot gtheta, gcol, goc (fp32, whatever the operand type); gwb[T] (optional) gets
    per-tile dL/dw_b partials."""
    dev = theta.device
    T, K, sfx = _theta_operands(theta, col, oc, H, W, S)
    require(bg, "bg", F32, (4,), dev)
    require(image, "image", F32, (H, W, 3), dev)
    require(den, "den", F32, (H, W), dev)
    require(gimage, "gimage", F32, (H, W, 3), dev)
    if gwb is not None:
        require(gwb, "gwb", F32, (T,), dev)
    gtheta = torch.empty(theta.shape, device=dev, dtype=F32)
    gcol = torch.empty(col.shape, device=dev, dtype=F32)
    goc = torch.empty(oc.shape, device=dev, dtype=F32)
    call("tts_splat_bwd_theta" + sfx, ptr(theta), ptr(col), ptr(oc), H, W, S, K, ptr(bg),
         ptr(image), ptr(den), ptr(gimage), ptr(gtheta), ptr(gcol), ptr(goc), ptr(gwb), stream())
    return gtheta, gcol, goc


# ----------------------------------------------------------------------------------- loss --
def loss_workspace(H, W, device):
    n = _lib.load().tts_loss_workspace_bytes(H, W)
    if n == 0:
        raise ValueError(f"image {H}x{W} is smaller than the 11x11 SSIM window")
    return torch.empty(n // 4, device=device, dtype=F32)


def loss_partials_count(H, W):
    ns = ctypes.c_int(0)
    n = _lib.load().tts_loss_partials_count(H, W, ctypes.byref(ns))
    return n, ns.value


def loss_grad(image, target, lam=0.2, gimage=None, partials=None, workspace=None):
    H, W = image.shape[0], image.shape[1]
    dev = image.device
    require(image, "image", F32, (H, W, 3))
    require(target, "target", F32, (H, W, 3), dev)
    gimage = torch.empty_like(image) if gimage is None else gimage
    require(gimage, "gimage", F32, (H, W, 3), dev)
    if partials is not None:
        require(partials, "partials", F32, (loss_partials_count(H, W)[0],), dev)
    workspace = loss_workspace(H, W, dev) if workspace is None else workspace
    require(workspace, "workspace", F32)
    call("tts_loss_grad", ptr(image), ptr(target), H, W, float(lam), ptr(gimage), ptr(partials),
         ptr(workspace), workspace.numel() * 4, stream())
    return gimage


def loss_stats_numel(H, W):
    """fp32 elements of one target's statistics buffer (loss_stats)."""
    n = _lib.load().tts_loss_stats_bytes(H, W)
    if n == 0:
        raise ValueError(f"image {H}x{W} is smaller than the 11x11 SSIM window")
    return n // 4


def loss_stats(target, stats=None):
    """The target's SSIM statistics (mu_y, s_y per channel on the valid map, then the target
    channel-planar), computed whenever the target changes and read by loss_grad_stats."""
    H, W = target.shape[0], target.shape[1]
    require(target, "target", F32, (H, W, 3))
    n = _lib.load().tts_loss_stats_bytes(H, W)
    if n == 0:
        raise ValueError(f"image {H}x{W} is smaller than the 11x11 SSIM window")
    stats = torch.empty(n // 4, device=target.device, dtype=F32) if stats is None else stats
    require(stats, "stats", F32, (n // 4,), target.device)
    call("tts_loss_target_stats", ptr(target), H, W, ptr(stats), stream())
    return stats


def rgba_premult(rgba):
    """[H,W,4] straight RGBA (spike's load_blender(keep_alpha=True)) -> [H,W,4] fp32
    (alpha r, alpha g, alpha b, 1 - alpha): the premultiplied colour and transmittance the
    random-background target is composited from (tools/resident_traced.py:184-185)."""
    rgba = torch.as_tensor(rgba, dtype=F32)
    if rgba.dim() != 3 or rgba.shape[2] != 4:
        raise ValueError(f"rgba must be [H,W,4], got {tuple(rgba.shape)}")
    a = rgba[..., 3:4]
    return torch.cat([rgba[..., :3] * a, 1.0 - a], dim=-1).contiguous()


def composite_random_bg(rgba_pm, step, view, seed, bg, target=None):
    """Draw this step's background (Philox, keyed by the device step count, `view` and `seed`)
    into bg[1..3] and composite target[H,W,3] = premult + (1 - alpha) * bg."""
    H, W = rgba_pm.shape[0], rgba_pm.shape[1]
    dev = rgba_pm.device
    _aligned16(require(rgba_pm, "rgba_pm", F32, (H, W, 4)), "rgba_pm")
    require(step, "step", I32, (4,), dev)
    require(bg, "bg", F32, (4,), dev)
    target = torch.empty(H, W, 3, device=dev, dtype=F32) if target is None else target
    require(target, "target", F32, (H, W, 3), dev)
    call("tts_composite_random_bg", ptr(rgba_pm), H, W, ptr(step), int(view),
         int(seed) & 0xFFFFFFFF, ptr(bg), ptr(target), stream())
    return target


def loss_grad_stats(image, target, stats, lam=0.2, gimage=None, partials=None):
    """loss_grad with the target's statistics from loss_stats: one kernel."""
    H, W = image.shape[0], image.shape[1]
    dev = image.device
    require(image, "image", F32, (H, W, 3))
    require(target, "target", F32, (H, W, 3), dev)
    require(stats, "stats", F32, (_lib.load().tts_loss_stats_bytes(H, W) // 4,), dev)
    gimage = torch.empty_like(image) if gimage is None else gimage
    require(gimage, "gimage", F32, (H, W, 3), dev)
    if partials is not None:
        require(partials, "partials", F32, (loss_partials_count(H, W)[0],), dev)
    call("tts_loss_grad_stats", ptr(image), ptr(target), ptr(stats), H, W, float(lam),
         ptr(gimage), ptr(partials), stream())
    return gimage


def loss_from_partials(partials, H, W, lam=0.2):
    """Loss value from the partial sums written by loss_grad (a device scalar)."""
    _, ns = loss_partials_count(H, W)
    s_sum = partials[:ns].double().sum()
    l1_sum = partials[ns:].double().sum()
    n = 3.0 * H * W
    n_s = 3.0 * (H - 10) * (W - 10)
    return ((1.0 - lam) * l1_sum / n + lam * (1.0 - s_sum / n_s)).float()


# ----------------------------------------------------------------------------------- adam --
def adam_state(device):
    """Step block: int32 step counter + the two fp32 bias-correction factors (4 words)."""
    return torch.zeros(4, device=device, dtype=I32)


def adam_advance(step, b1=BETA1, b2=BETA2):
    require(step, "step", I32, (4,))
    call("tts_adam_advance", ptr(step), b1, b2, stream())


def adam(params, m, v, grad, lr, step, b1=BETA1, b2=BETA2, eps=EPS):
    G = params.shape[0]
    dev = params.device
    for t, n in ((params, "params"), (m, "m"), (v, "v"), (grad, "grad")):
        require(t, n, F32, (G, 14), dev)
    require(lr, "lr", F32, (14,), dev)
    require(step, "step", I32, (4,), dev)
    call("tts_adam", ptr(params), ptr(m), ptr(v), ptr(grad), ptr(lr), G, ptr(step), b1, b2, eps,
         stream())


def adam_flat(params, m, v, grad, lr1, step, b1=BETA1, b2=BETA2, eps=EPS):
    """Adam over any contiguous fp32 block with one learning rate lr1[1] (device scalar)."""
    dev = params.device
    for t, n in ((params, "params"), (m, "m"), (v, "v"), (grad, "grad")):
        require(t, n, F32, tuple(params.shape), dev)
    require(lr1, "lr1", F32, (1,), dev)
    require(step, "step", I32, (4,), dev)
    call("tts_adam_flat", ptr(params), ptr(m), ptr(v), ptr(grad), ptr(lr1), params.numel(),
         ptr(step), b1, b2, eps, stream())


def geom_bwd_accum(params, camera, gslot, inv, gacc, scale=1.0, near=NEAR, blur=BLUR,
                   sh_rest=None, sh_degree=0, gacc_sh=None, depth_bt=None, gacc_depth=None):
    """gacc[G,14] += scale * dL/dparams for one view (slot gradients gathered through inv);
    with sh_degree > 0 also gacc_sh[15,3,G] += scale * dL/dsh_rest, with depth_bt also
    gacc_depth[G,2] += scale * dL/d(beta, tau)."""
    G = params.shape[0]
    dev = params.device
    require(params, "params", F32, (G, 14))
    require(camera, "camera", F32, (16,), dev)
    require(gslot, "gslot", F32, None, dev)
    require(inv, "inv", I32, (G, 9), dev)
    require(gacc, "gacc", F32, (G, 14), dev)
    _sh_check(sh_rest, sh_degree, G, dev)
    _dw_check(depth_bt, dev)
    if sh_degree > 0 or depth_bt is not None:
        if sh_degree > 0:
            require(gacc_sh, "gacc_sh", F32, (SH_REST, 3, G), dev)
        if depth_bt is not None:
            require(gacc_depth, "gacc_depth", F32, (G, 2), dev)
        call("tts_geom_bwd_accum_ex", ptr(params), ptr(sh_rest), int(sh_degree), ptr(depth_bt), G,
             ptr(camera), near, blur, ptr(gslot), ptr(inv), float(scale), ptr(gacc),
             ptr(gacc_sh), ptr(gacc_depth), stream())
        return gacc
    call("tts_geom_bwd_accum", ptr(params), G, ptr(camera), near, blur, ptr(gslot), ptr(inv),
         float(scale), ptr(gacc), stream())
    return gacc


def geom_bwd_adam(params, camera, gslot, inv, m, v, lr, step, near=NEAR, blur=BLUR, gparams=None,
                  b1=BETA1, b2=BETA2, eps=EPS, sh_rest=None, sh_m=None, sh_v=None, lr_sh=None,
                  sh_degree=0, lambda_o=0.0, lambda_s=0.0, noise_lr=0.0, seed=0, depth_bt=None,
                  gdepth=None):
    """Slot gradients (gathered through inv) -> geometry backward -> Adam, in one kernel.
    With sh_degree > 0 the rest coefficients sh_rest (moments sh_m, sh_v, all [15,3,G]) take
    the same Adam step at learning rate lr_sh[1] (device scalar).  lambda_o / lambda_s add the
    MCMC regulariser's gradient; noise_lr > 0 applies the SGLD step to the updated means
    (Philox draws keyed by seed and the device step number).  depth_bt: the depth weight, each
    gaussian's dL/d(beta, tau) into gdepth [G,2] (then depth_weight_adam)."""
    G = params.shape[0]
    dev = params.device
    for t, n in ((params, "params"), (m, "m"), (v, "v")):
        require(t, n, F32, (G, 14), dev)
    require(camera, "camera", F32, (16,), dev)
    require(inv, "inv", I32, (G, 9), dev)
    if gslot.dim() != 3 or gslot.shape[2] != 9:
        raise ValueError("gslot must be [T,K,9]")
    require(gslot, "gslot", F32, tuple(gslot.shape), dev)
    require(lr, "lr", F32, (14,), dev)
    require(step, "step", I32, (4,), dev)
    if gparams is not None:
        require(gparams, "gparams", F32, (G, 14), dev)
    _sh_check(sh_rest, sh_degree, G, dev)
    if min(lambda_o, lambda_s, noise_lr) < 0:
        raise ValueError("lambda_o, lambda_s and noise_lr must be >= 0")
    if sh_degree > 0:
        require(sh_m, "sh_m", F32, (SH_REST, 3, G), dev)
        require(sh_v, "sh_v", F32, (SH_REST, 3, G), dev)
        require(lr_sh, "lr_sh", F32, (1,), dev)
    _dw_check(depth_bt, dev)
    if gdepth is not None:
        require(gdepth, "gdepth", F32, (G, 2), dev)
    if sh_degree > 0 or lambda_o or lambda_s or noise_lr or depth_bt is not None:
        call("tts_geom_bwd_adam_ex", ptr(params), ptr(sh_rest), ptr(sh_m), ptr(sh_v),
             int(sh_degree), ptr(depth_bt), ptr(gdepth), G, ptr(camera), near, blur, ptr(gslot),
             ptr(inv), ptr(gparams), ptr(m), ptr(v), ptr(lr), ptr(lr_sh), ptr(step), b1, b2, eps,
             float(lambda_o), float(lambda_s), float(noise_lr), int(seed) & 0xFFFFFFFF, stream())
        return
    call("tts_geom_bwd_adam", ptr(params), G, ptr(camera), near, blur, ptr(gslot), ptr(inv),
         ptr(gparams), ptr(m), ptr(v), ptr(lr), ptr(step), b1, b2, eps, stream())


def depth_weight_workspace(G, device):
    n = _lib.load().tts_depth_weight_workspace_bytes(G)
    return torch.empty(max(n, 1), device=device, dtype=U8)


def depth_weight_adam(gdepth, depth_bt, bt_state, lr1, step, workspace=None, b1=BETA1, b2=BETA2,
                      eps=EPS):
    """Sum gdepth [G,2] over the gaussians and take one Adam step on depth_bt = (beta, tau)
    (state (m_beta, m_tau, v_beta, v_tau), learning rate lr1[1])."""
    G = gdepth.shape[0]
    dev = gdepth.device
    require(gdepth, "gdepth", F32, (G, 2))
    require(depth_bt, "depth_bt", F32, (2,), dev)
    require(bt_state, "bt_state", F32, (4,), dev)
    require(lr1, "lr1", F32, (1,), dev)
    require(step, "step", I32, (4,), dev)
    ws = depth_weight_workspace(G, dev) if workspace is None else workspace
    require(ws, "workspace", U8, None, dev)
    call("tts_depth_weight_adam", ptr(gdepth), G, ptr(depth_bt), ptr(bt_state), ptr(lr1),
         ptr(step), b1, b2, eps, ptr(ws), ws.numel(), stream())


# ----------------------------------------------------------------------------- MCMC --
def mcmc_reg_grad(params, grad, lambda_o, lambda_s):
    """grad[G,14] += gradient of the MCMC regulariser (spike/mcmc.py:18-22)."""
    G = params.shape[0]
    dev = params.device
    require(params, "params", F32, (G, 14))
    require(grad, "grad", F32, (G, 14), dev)
    call("tts_mcmc_reg_grad", ptr(params), G, float(lambda_o), float(lambda_s), ptr(grad),
         stream())


def sgld_noise(params, lr, noise_lr, step, seed=0):
    """SGLD step on the means (spike/mcmc.py:25-34), noise scale noise_lr * lr[0]."""
    G = params.shape[0]
    dev = params.device
    require(params, "params", F32, (G, 14))
    require(lr, "lr", F32, (14,), dev)
    require(step, "step", I32, (4,), dev)
    call("tts_sgld_noise", ptr(params), G, ptr(lr), float(noise_lr), int(seed) & 0xFFFFFFFF,
         ptr(step), stream())


def relocate_workspace(G, device):
    n = _lib.load().tts_relocate_workspace_bytes(G)
    return torch.empty(max(n, 1), device=device, dtype=U8)


def relocate(params, m, v, step, dead_thr=0.005, offset=0.005, seed=0, workspace=None,
             moved=None, sh_rest=None, sh_m=None, sh_v=None):
    """MCMC relocation of dead slots onto live gaussians (spike/mcmc.py:41-93), on the device.
    Returns the device int32 [1] holding the number of relocated slots."""
    G = params.shape[0]
    dev = params.device
    for t, n in ((params, "params"), (m, "m"), (v, "v")):
        require(t, n, F32, (G, 14), dev)
    require(step, "step", I32, (4,), dev)
    if sh_rest is not None:
        for t, n in ((sh_rest, "sh_rest"), (sh_m, "sh_m"), (sh_v, "sh_v")):
            require(t, n, F32, (SH_REST, 3, G), dev)
    ws = relocate_workspace(G, dev) if workspace is None else workspace
    require(ws, "workspace", U8, None, dev)
    moved = torch.zeros(1, device=dev, dtype=I32) if moved is None else moved
    require(moved, "moved", I32, (1,), dev)
    call("tts_relocate", ptr(params), ptr(m), ptr(v), ptr(sh_rest), ptr(sh_m), ptr(sh_v), G,
         float(dead_thr), float(offset), int(seed) & 0xFFFFFFFF, ptr(step), ptr(moved), ptr(ws),
         ws.numel(), stream())
    return moved


def zero_(buf):
    require(buf, "buf", F32)
    call("tts_zero", ptr(buf), buf.numel(), stream())
    return buf


# ---------------------------------------------------------------------------------- dense --
def dense_workspace(G, P, device):
    n = _lib.load().tts_dense_workspace_bytes(G, P)
    return torch.empty(max(n, 1), device=device, dtype=U8)


def render_dense(proj, H, W, k, bg, image=None, den=None):
    """Dense arm-A render of every projected gaussian onto an H x W image (any H, W)."""
    G = proj.shape[0]
    dev = proj.device
    _aligned16(require(proj, "proj", F32, (G, 12)), "proj")
    require(bg, "bg", F32, (4,), dev)
    image = torch.empty(H, W, 3, device=dev, dtype=F32) if image is None else image
    den = torch.empty(H, W, device=dev, dtype=F32) if den is None else den
    require(image, "image", F32, (H, W, 3), dev)
    require(den, "den", F32, (H, W), dev)
    call("tts_render_dense", ptr(proj), G, H, W, float(k), ptr(bg), ptr(image), ptr(den),
         stream())
    return image, den


def render_dense_bwd(proj, H, W, k, bg, image, den, gimage, grad9=None, gwb=None, workspace=None):
    """Returns grad9 [G,9] (conic, mean, col_o, o_col gradients) and gwb [1]."""
    G = proj.shape[0]
    dev = proj.device
    _aligned16(require(proj, "proj", F32, (G, 12)), "proj")
    require(bg, "bg", F32, (4,), dev)
    require(image, "image", F32, (H, W, 3), dev)
    require(den, "den", F32, (H, W), dev)
    require(gimage, "gimage", F32, (H, W, 3), dev)
    grad9 = torch.empty(G, 9, device=dev, dtype=F32) if grad9 is None else grad9
    gwb = torch.empty(1, device=dev, dtype=F32) if gwb is None else gwb
    require(grad9, "grad9", F32, (G, 9), dev)
    require(gwb, "gwb", F32, (1,), dev)
    workspace = dense_workspace(G, H * W, dev) if workspace is None else workspace
    call("tts_render_dense_bwd", ptr(proj), G, H, W, float(k), ptr(bg), ptr(image), ptr(den),
         ptr(gimage), ptr(grad9), ptr(gwb), ptr(workspace), workspace.numel(), stream())
    return grad9, gwb


ARM_CODES = {"A": 0, "SZ": 1, "RV": 2}


def render_dense_arm(proj, H, W, k, bg, arm, softz_beta=None, image=None, den=None, aux=None):
    """Dense render with a per-pixel occlusion arm ("A", "SZ" soft-Z, "RV" revealage;
    spike/arms.py).  Returns image, den, aux [H,W,4] (the per-pixel state the backward reads).
    softz_beta: device scalar [1] (SZ)."""
    G = proj.shape[0]
    dev = proj.device
    code = ARM_CODES[arm]
    _aligned16(require(proj, "proj", F32, (G, 12)), "proj")
    require(bg, "bg", F32, (4,), dev)
    if arm == "SZ":
        require(softz_beta, "softz_beta", F32, (1,), dev)
    image = torch.empty(H, W, 3, device=dev, dtype=F32) if image is None else image
    den = torch.empty(H, W, device=dev, dtype=F32) if den is None else den
    aux = torch.zeros(H, W, 4, device=dev, dtype=F32) if aux is None else aux
    require(image, "image", F32, (H, W, 3), dev)
    require(den, "den", F32, (H, W), dev)
    require(aux, "aux", F32, (H, W, 4), dev)
    call("tts_render_dense_arm", ptr(proj), G, H, W, float(k), ptr(bg), code, ptr(softz_beta),
         ptr(image), ptr(den), ptr(aux), stream())
    return image, den, aux


def render_dense_arm_bwd(proj, H, W, k, bg, arm, image, den, aux, gimage, softz_beta=None,
                         workspace=None):
    """Backward of render_dense_arm: grad [G,9] (or [G,10] for SZ, column 9 = each gaussian's
    dL/dsoftz_beta) and gwb [1]."""
    G = proj.shape[0]
    dev = proj.device
    code = ARM_CODES[arm]
    _aligned16(require(proj, "proj", F32, (G, 12)), "proj")
    require(bg, "bg", F32, (4,), dev)
    for t, n, sh in ((image, "image", (H, W, 3)), (den, "den", (H, W)), (aux, "aux", (H, W, 4)),
                     (gimage, "gimage", (H, W, 3))):
        require(t, n, F32, sh, dev)
    if arm == "SZ":
        require(softz_beta, "softz_beta", F32, (1,), dev)
    nc = 10 if arm == "SZ" else 9
    grad = torch.empty(G, nc, device=dev, dtype=F32)
    gwb = torch.empty(1, device=dev, dtype=F32)
    workspace = dense_workspace(G, H * W, dev) if workspace is None else workspace
    call("tts_render_dense_arm_bwd", ptr(proj), G, H, W, float(k), ptr(bg), code,
         ptr(softz_beta), ptr(image), ptr(den), ptr(aux), ptr(gimage), ptr(grad), ptr(gwb),
         ptr(workspace), workspace.numel(), stream())
    return grad, gwb


def _wsr_operands(theta, o, color, keep, phi):
    G, P = theta.shape[0], phi.shape[0]
    dev = theta.device
    require(theta, "theta", F32, (G, 6))
    require(o, "o", F32, (G,), dev)
    require(color, "color", F32, (G, 3), dev)
    require(phi, "phi", F32, (P, 6), dev)
    if keep is not None:
        if keep.dtype == torch.bool:
            keep = keep.view(U8)
        require(keep, "keep", U8, (G,), dev)
    return G, P, dev, keep


def wsr_dense(theta, o, color, keep, phi, bg, C=None, den=None):
    """C [P,3] = WSR of w = o*keep*max(phi@theta^T, 0)^2; also returns den [P]."""
    G, P, dev, keep = _wsr_operands(theta, o, color, keep, phi)
    require(bg, "bg", F32, (4,), dev)
    C = torch.empty(P, 3, device=dev, dtype=F32) if C is None else C
    den = torch.empty(P, device=dev, dtype=F32) if den is None else den
    require(C, "C", F32, (P, 3), dev)
    require(den, "den", F32, (P,), dev)
    call("tts_wsr_dense", ptr(theta), ptr(o), ptr(color), ptr(keep), ptr(phi), G, P, ptr(bg),
         ptr(C), ptr(den), stream())
    return C, den


def wsr_dense_bwd(theta, o, color, keep, phi, bg, C, den, gC, workspace=None):
    """Returns (gtheta [G,6], go [G], gcolor [G,3], gwb [1]) as views of one [G,10] buffer."""
    G, P, dev, keep = _wsr_operands(theta, o, color, keep, phi)
    require(bg, "bg", F32, (4,), dev)
    require(C, "C", F32, (P, 3), dev)
    require(den, "den", F32, (P,), dev)
    require(gC, "gC", F32, (P, 3), dev)
    g10 = torch.empty(G, 10, device=dev, dtype=F32)
    gwb = torch.empty(1, device=dev, dtype=F32)
    workspace = dense_workspace(G, P, dev) if workspace is None else workspace
    call("tts_wsr_dense_bwd", ptr(theta), ptr(o), ptr(color), ptr(keep), ptr(phi), G, P,
         ptr(bg), ptr(C), ptr(den), ptr(gC), ptr(g10), ptr(gwb), ptr(workspace),
         workspace.numel(), stream())
    return g10[:, 0:6], g10[:, 6], g10[:, 7:10], gwb
