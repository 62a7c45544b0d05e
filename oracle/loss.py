"""Oracle: photometric training loss (1-lambda)*L1 + lambda*(1-SSIM) and its gradient.

Test infrastructure only (see oracle/__init__.py).

Restates spike/metrics.py:6-28 (`loss_fn`): L1 on the raw prediction, SSIM on images clamped to
[0,1] (`_nchw`, :7) with data_range 1, an 11-tap gaussian window of sigma 1.5 applied as a
separable VALID convolution (H then W), C1 = (0.01)^2, C2 = (0.03)^2, mean over every channel
and output pixel.  The SSIM itself is the published algorithm of pytorch_msssim==1.0.0
(Dockerfile:47; call site spike/metrics.py:19), which is not installed here; its map is
    S = ((2 mu_x mu_y + C1)(2 s_xy + C2)) / ((mu_x^2 + mu_y^2 + C1)(s_x + s_y + C2))
with s_x = f(x*x) - mu_x^2, s_xy = f(x*y) - mu_x mu_y, as also restated by the reference in
tools/loss_manual.py:56-73.  The gradient is torch autograd of this forward (the reference's
manual gradient, tools/loss_manual.py:76-103, was validated against the same autograd).
"""
import torch
import torch.nn.functional as F

C1 = 0.01 ** 2
C2 = 0.03 ** 2
WIN = 11
SIGMA = 1.5
LAMBDA = 0.2


def gauss_1d(win=WIN, sigma=SIGMA, dtype=torch.float64):
    """Normalised 1-D gaussian taps centred on win//2 (tools/loss_manual.py:26-29)."""
    c = torch.arange(win, dtype=torch.float64) - win // 2
    g = torch.exp(-(c * c) / (2.0 * sigma * sigma))
    return (g / g.sum()).to(dtype)


def window_size(H, W, win=WIN):
    """Window actually used for an H x W image (spike/metrics.py:14-18): min(win, H, W), made
    odd by subtracting one, at least 3."""
    w = min(win, H, W)
    if w % 2 == 0:
        w -= 1
    return max(w, 3)


def gaussian_filter(x, g):
    """Separable valid filter of x[C,H,W]: along H, then along W."""
    C = x.shape[0]
    w = g.to(x.dtype)
    t = F.conv2d(x[None], w.view(1, 1, -1, 1).expand(C, 1, -1, 1), groups=C)
    t = F.conv2d(t, w.view(1, 1, 1, -1).expand(C, 1, 1, -1), groups=C)
    return t[0]


def ssim_map(x, y, g):
    """SSIM map [C,Hout,Wout] of CHW images (no clamp here)."""
    fx, fy = gaussian_filter(x, g), gaussian_filter(y, g)
    sx = gaussian_filter(x * x, g) - fx * fx
    sy = gaussian_filter(y * y, g) - fy * fy
    sxy = gaussian_filter(x * y, g) - fx * fy
    return ((2 * fx * fy + C1) * (2 * sxy + C2)) / ((fx * fx + fy * fy + C1) * (sx + sy + C2))


def loss_fn(pred, gt, lambda_ssim=LAMBDA):
    """(1-l)*mean|pred-gt| + l*(1 - mean SSIM(clamp(pred), clamp(gt))) on [H,W,3] images
    (spike/metrics.py:26-28)."""
    g = gauss_1d(window_size(pred.shape[0], pred.shape[1]), SIGMA, pred.dtype)
    l1 = (pred - gt).abs().mean()
    x = pred.clamp(0.0, 1.0).permute(2, 0, 1)
    y = gt.clamp(0.0, 1.0).permute(2, 0, 1)
    s = ssim_map(x, y, g).mean()
    return (1.0 - lambda_ssim) * l1 + lambda_ssim * (1.0 - s)


def loss_and_grad(pred, gt, lambda_ssim=LAMBDA):
    """(loss, dL/dpred[H,W,3]) by autograd of `loss_fn`."""
    x = pred.detach().clone().requires_grad_(True)
    loss = loss_fn(x, gt.detach(), lambda_ssim)
    loss.backward()
    return loss.detach(), x.grad


def band_matrix(n_in, g):
    """[n_out, n_in] valid-convolution band matrix (tools/loss_manual.py:32-39)."""
    win = g.numel()
    M = torch.zeros(n_in - win + 1, n_in, dtype=g.dtype)
    for o in range(n_in - win + 1):
        M[o, o:o + win] = g
    return M
