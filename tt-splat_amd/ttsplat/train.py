"""The overfit loop under its reference names: spike/train.py:9-41.

`fit(model, cameras, gt_images, arm, iters, lambda_ssim, lr, k, blur_eps, near, log_every,
sh_degree)` minimises the mean photometric loss over all views per iteration (full batch), as
the reference does, with every op on the HIP path: dense render (tts_render_dense + geometry),
loss (tts_loss_grad), their backward kernels, and Adam (tts_adam) with the reference's
per-group learning rates.  The trained parameters are written back into `model`.
"""
import torch

from . import kernels
from .binned import params_of
from .loss import loss_fn, psnr
from .render import _check_arm, render

F32 = torch.float32

# spike/train.py:9-12
DEFAULT_LR = {
    "means": 5e-3, "scales": 5e-3, "quats": 1e-3, "opacity": 5e-2,
    "opacity_sh": 5e-2, "color": 1e-2, "wb": 1e-2, "depth": 1e-2,
}

# columns of the [G,14] block per Adam group (spike/model.py:82-95 group names)
_GROUP_COLS = (("means", 0, 3), ("quats", 3, 7), ("scales", 7, 10), ("color", 10, 13),
               ("opacity", 13, 14))


class _Fitted:
    """The trainable state fit() works on: the [G,14] block and w_b_raw as leaves."""

    def __init__(self, model):
        P = params_of(model).detach().float().contiguous().clone()
        if not P.is_cuda:
            raise ValueError("fit() needs the model on a GPU")
        self.params = P
        self.w_b_raw = torch.as_tensor(model.w_b_raw, dtype=F32).detach().to(P.device).reshape(())
        self.c_b = torch.as_tensor(model.c_b, dtype=F32).detach().to(P.device)
        # arm B's global depth-weight scalars (spike/model.py:48-49)
        self.depth_beta = torch.as_tensor(getattr(model, "depth_beta", 1.0),
                                          dtype=F32).detach().to(P.device).reshape(())
        self.depth_tau = torch.as_tensor(getattr(model, "depth_tau", 3.0),
                                         dtype=F32).detach().to(P.device).reshape(())
        self.softz_beta = torch.as_tensor(getattr(model, "softz_beta", 4.0),
                                          dtype=F32).detach().to(P.device).reshape(())
        rest = getattr(model, "color_rest", None)   # SH rest coefficients [G,15,3] or None
        self.color_rest = (None if rest is None
                           else rest.detach().to(P.device, F32).contiguous().clone())


def _write_back(model, st):
    with torch.no_grad():
        P = st.params
        if isinstance(getattr(model, "params", None), torch.Tensor) and model.params.shape == P.shape:
            model.params.copy_(P)
        else:
            model.means3d.copy_(P[:, 0:3])
            model.quats.copy_(P[:, 3:7])
            model.log_scales.copy_(P[:, 7:10])
            model.color_dc.copy_(P[:, 10:13])
            model.opacity_raw.copy_(P[:, 13].reshape(model.opacity_raw.shape))
        if st.color_rest is not None and torch.is_tensor(getattr(model, "color_rest", None)):
            model.color_rest.copy_(st.color_rest.reshape(model.color_rest.shape))
        if torch.is_tensor(model.w_b_raw):
            model.w_b_raw.copy_(st.w_b_raw.reshape(model.w_b_raw.shape))
        else:
            model.w_b_raw = float(st.w_b_raw)
        for name in ("depth_beta", "depth_tau", "softz_beta"):
            cur = getattr(model, name, None)
            if torch.is_tensor(cur):
                cur.copy_(getattr(st, name).reshape(cur.shape))


def fit(model, cameras, gt_images, arm, iters=800, lambda_ssim=0.2, lr=None, k=4.0, blur_eps=0.3,
        near=0.2, log_every=0, sh_degree=0):
    """Returns the per-iteration mean loss history (list of floats)."""
    _check_arm(arm, sh_degree)
    lr = {**DEFAULT_LR, **(lr or {})}
    st = _Fitted(model)
    dev = st.params.device
    G = st.params.shape[0]
    lrv = torch.zeros(14, dtype=F32)
    for name, a, b in _GROUP_COLS:
        lrv[a:b] = float(lr[name])
    lrv = lrv.to(dev)
    lrw = torch.zeros(14, dtype=F32)
    lrw[0] = float(lr["wb"])
    lrw[1:4] = float(lr["depth"])
    lrw = lrw.to(dev)
    # Adam state: [G,14] moments, plus w_b_raw (column 0) and, for arm B, depth_beta and
    # depth_tau (columns 1, 2), for arm SZ softz_beta (column 3), carried in a one-row block
    m, v = torch.zeros(G, 14, device=dev, dtype=F32), torch.zeros(G, 14, device=dev, dtype=F32)
    wrow = torch.zeros(1, 14, device=dev, dtype=F32)
    mw, vw = torch.zeros_like(wrow), torch.zeros_like(wrow)
    step = kernels.adam_state(dev)
    gts = [g.to(dev).float().contiguous() for g in gt_images]
    # view-dependent colour: the rest coefficients take Adam at lr color_rest (spike/model.py:91)
    use_sh = int(sh_degree) > 0 and st.color_rest is not None
    if use_sh:
        mr, vr = torch.zeros_like(st.color_rest), torch.zeros_like(st.color_rest)
        lr_rest = torch.tensor([float(lr.get("color_rest", lr["color"] / 20.0))], dtype=F32,
                               device=dev)

    class _View:                     # the duck-typed model render() reads
        pass

    history = []
    for it in range(iters):
        Pl = st.params.clone().requires_grad_(True)
        wl = st.w_b_raw.clone().requires_grad_(True)
        view = _View()
        view.params, view.w_b_raw, view.c_b = Pl, wl, st.c_b
        leaves = [Pl, wl]
        if arm == "B":
            view.depth_beta = st.depth_beta.clone().requires_grad_(True)
            view.depth_tau = st.depth_tau.clone().requires_grad_(True)
            leaves += [view.depth_beta, view.depth_tau]
        if arm == "SZ":
            view.softz_beta = st.softz_beta.clone().requires_grad_(True)
            leaves += [view.softz_beta]
        if use_sh:
            view.color_rest = st.color_rest.clone().requires_grad_(True)
            leaves += [view.color_rest]
        total = 0.0
        for cam, gt in zip(cameras, gts):
            img = render(view, cam, arm, k=k, blur_eps=blur_eps, near=near, sh_degree=sh_degree)
            total = total + loss_fn(img, gt, lambda_ssim)
        total = total / len(cameras)
        grads = torch.autograd.grad(total, leaves)
        kernels.adam_advance(step)
        kernels.adam(st.params, m, v, grads[0].contiguous(), lrv, step)
        if use_sh:
            kernels.adam_flat(st.color_rest, mr, vr, grads[-1].contiguous(), lr_rest, step)
        wrow[0, 0] = st.w_b_raw
        gwrow = torch.zeros_like(wrow)
        gwrow[0, 0] = grads[1]
        if arm == "B":
            wrow[0, 1], wrow[0, 2] = st.depth_beta, st.depth_tau
            gwrow[0, 1], gwrow[0, 2] = grads[2], grads[3]
        if arm == "SZ":
            wrow[0, 3] = st.softz_beta
            gwrow[0, 3] = grads[2]
        kernels.adam(wrow, mw, vw, gwrow, lrw, step)
        st.w_b_raw = wrow[0, 0].clone()
        if arm == "B":
            st.depth_beta, st.depth_tau = wrow[0, 1].clone(), wrow[0, 2].clone()
        if arm == "SZ":
            st.softz_beta = wrow[0, 3].clone()
        history.append(float(total.detach()))
        if log_every and (it % log_every == 0 or it == iters - 1):
            print(f"    iter {it:4d}  loss {history[-1]:.5f}")
    _write_back(model, st)
    return history


@torch.no_grad()
def eval_psnr(model, cameras, gt_images, arm, **kw):
    """Mean PSNR over the given views (spike/train.py:36-41)."""
    vals = [float(psnr(render(model, cam, arm, **kw), gt.to(params_of(model).device)))
            for cam, gt in zip(cameras, gt_images)]
    return sum(vals) / len(vals)
