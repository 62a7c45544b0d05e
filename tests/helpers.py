"""Shared test inputs: seeded configurations, oracle camera dicts, comparison metrics."""
import torch

from ttsplat import scenes
from ttsplat.camera import Camera


def cam_dict(cam: Camera):
    return cam.as_dict()


def anisotropic(cam: Camera, ratio=1.13, px=0.46, py=0.53):
    """The same pose with fx = ratio * fy and the principal point off the image centre (at
    px * W, py * H), as COLMAP's PINHOLE / OPENCV models give (spike/data.py:127-150)."""
    return Camera(cam.R_v, cam.t_v, ratio * cam.fy, cam.fy, px * cam.W, py * cam.H, cam.H, cam.W)


def rel_l2(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp(min=1e-30))


def max_abs(a, b):
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max())


def update_error_ok(p_gpu, p0, ref, rtol=1e-4):
    """|(p - p0) - (ref - p0)| <= rtol |ref - p0| + 2 ulp(p) per entry: the update, not the
    parameter, is compared (updates ~ lr << |p|), with the fp32 rounding of p itself allowed."""
    pf = p_gpu.detach().cpu().float()
    ulp = (torch.nextafter(pf, torch.full_like(pf, float("inf"))) - pf).double()
    du = pf.double() - p0.double()
    dref = ref.double() - p0.double()
    bad = (du - dref).abs() > rtol * dref.abs() + 2.0 * ulp
    return int(bad.sum())


def config_inputs(name, seed=0, cam_index=0, G=None, aniso=False):
    """(config, params[G,14] CPU, camera) for a named configuration (G optionally reduced;
    aniso: the camera with fx = 1.13 fy and an off-centre principal point)."""
    cfg = scenes.CONFIGS[name]
    if G is not None:
        cfg = scenes.Config(**{**cfg.__dict__, "G": G, "span": cfg.span})
    P = cfg.params(seed)
    cam = cfg.cameras()[cam_index]
    return cfg, P, (anisotropic(cam) if aniso else cam)


def bins_equal_report(idx_a, valid_a, idx_b, valid_b):
    """Number of tiles whose (idx, valid) rows differ."""
    ia, va = idx_a.cpu().long(), valid_a.cpu().bool()
    ib, vb = idx_b.cpu().long(), valid_b.cpu().bool()
    diff = (ia != ib).any(1) | (va != vb).any(1)
    return int(diff.sum()), torch.nonzero(diff).flatten()


def oracle_render_chunked(P, cam, tmap, bins, k, R=None, dtype=torch.float64, chunk=512,
                          w_b_raw=-3.0, proj=None):
    """The oracle's binned render (tools/bh_views.py:65-71 on _operands) over tile chunks, so
    full-size frames fit in memory: returns img [H,W,3], den [H,W] and, with R [H,W,3],
    dL/dP [G,14] of L = sum(img * R) -- autograd of the same restated forward, accumulated chunk
    by chunk through leaf copies of the per-gaussian geometry outputs, then pushed through the
    geometry once.  Each chunk's slot range is trimmed to its last valid slot (exact: invalid
    slots have theta = 0, so w = 0).  proj (optional): dict of per-gaussian geometry outputs to
    use instead of computing them from P (then no dL/dP)."""
    from oracle import geometry as ogeo
    from oracle import splat as osplat
    names = ("mu2d", "conic", "color_o", "o_col")
    grad = R is not None and proj is None
    if proj is None:
        Pg = P.detach().to(dtype).clone().requires_grad_(grad)
        camd = {n: (v.to(dtype) if torch.is_tensor(v) else v) for n, v in cam.items()}
        pr = ogeo.project_params(Pg, camd)
    else:
        pr = {n: proj[n].to(dtype) for n in names}
    leaves = {n: pr[n].detach().clone().requires_grad_(R is not None) for n in names}
    idx, valid = bins[0].cpu().long(), bins[1].cpu().bool()
    T, K = idx.shape
    SS = tmap.S * tmap.S
    Phi = tmap.Phi.to(dtype)
    origins = tmap.origins.to(dtype)
    w_b = torch.nn.functional.softplus(torch.tensor(w_b_raw, dtype=dtype))
    c_b = torch.ones(3, dtype=dtype)
    Rt = None if R is None else R.reshape(-1, 3)[tmap.gidx].reshape(T, SS, 3).to(dtype)
    last = (valid.long() * torch.arange(1, K + 1)).amax(1)
    perm = torch.argsort(last, descending=True)
    C_all = torch.zeros(T, SS, 3, dtype=dtype)
    den_all = torch.zeros(T, SS, dtype=dtype)
    for c0 in range(0, T, chunk):
        tl = perm[c0:c0 + chunk]
        kc = max(int(last[tl].max()), 1)
        ii, vv = idx[tl, :kc], valid[tl, :kc]
        vf = vv.to(dtype)
        th = osplat.theta_u_gathered(leaves["conic"][ii], leaves["mu2d"][ii], origins[tl], k)
        th = th * vf[:, None, :]
        col = leaves["color_o"][ii] * vf[..., None]
        oc = leaves["o_col"][ii][..., None] * vf[..., None]
        C, den = osplat.splat_tiles(th, col, oc, Phi, w_b, c_b)
        C_all[tl] = C.detach()
        den_all[tl] = den.detach()
        if R is not None:
            (C * Rt[tl]).sum().backward()
    img = osplat.tiles_to_image(C_all, tmap)
    den = osplat.tiles_to_image(den_all[..., None], tmap)[..., 0]
    if R is None:
        return img, den
    lg = {n: (leaves[n].grad if leaves[n].grad is not None else torch.zeros_like(leaves[n]))
          for n in names}
    if not grad:
        return img, den, lg
    torch.autograd.backward([pr[n] for n in names], [lg[n] for n in names])
    return img, den, Pg.grad.detach()
