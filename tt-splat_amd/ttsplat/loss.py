"""Photometric loss (1-l)*L1 + l*(1-SSIM) on the GPU (spike/metrics.py:26-28).

`loss_fn(pred, gt, lambda_ssim)` keeps the reference signature and is differentiable w.r.t.
pred: the forward runs the fused loss-gradient kernels once and keeps dL/dpred for backward.
"""
import torch

from . import kernels


class _PhotometricLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pred, gt, lam):
        H, W = pred.shape[0], pred.shape[1]
        x = pred.detach().float().contiguous()
        y = gt.detach().float().contiguous()
        n, _ = kernels.loss_partials_count(H, W)
        partials = torch.empty(n, device=x.device, dtype=torch.float32)
        g = kernels.loss_grad(x, y, lam, partials=partials)
        ctx.save_for_backward(g)
        return kernels.loss_from_partials(partials, H, W, lam)

    @staticmethod
    def backward(ctx, gout):
        (g,) = ctx.saved_tensors
        return g * gout, None, None


def loss_fn(pred, gt, lambda_ssim=0.2):
    """(1-l)*mean|pred-gt| + l*(1-SSIM(clamp(pred), clamp(gt))), 11-tap window, sigma 1.5."""
    return _PhotometricLoss.apply(pred, gt, float(lambda_ssim))


def psnr(pred, gt):
    """spike/metrics.py:10-12."""
    mse = (pred.clamp(0.0, 1.0) - gt.clamp(0.0, 1.0)).pow(2).mean()
    return -10.0 * torch.log10(mse.clamp(min=1e-12))
