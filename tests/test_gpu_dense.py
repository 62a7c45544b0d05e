"""GPU dense render (spike/render.py:14-49, arm "A"), wsr_polysplat (spike/backward.py:11-63)
and fit() (spike/train.py:15-39) vs the oracle.

Images within 1e-4 max-abs; gradients within 1e-3 relative L2 of torch autograd through the
oracle's dense formulas (the same ones spike/render.py composes).
"""
import pytest
import torch

from helpers import cam_dict, config_inputs, max_abs, rel_l2
from oracle import geometry as ogeo
from oracle import loss as oloss
from oracle import splat as osplat
from ttsplat import backward as tback
from ttsplat import render as trender
from ttsplat import train as ttrain
from ttsplat.model import GaussianModel

pytestmark = pytest.mark.gpu

GROUPS = {"means": slice(0, 3), "quats": slice(3, 7), "scales": slice(7, 10),
          "color": slice(10, 13), "opacity": slice(13, 14)}


def oracle_dense(P, wb_raw, cam, k):
    """spike/render.py:14-49 arm A from the oracle's pieces, w_b_raw a differentiable leaf."""
    pr = ogeo.project_params(P, cam, 0.3, 0.2)
    px, py = ogeo.pixel_grid(cam["H"], cam["W"], dtype=P.dtype)
    Q = osplat.quad_form(px, py, pr["mu2d"], pr["conic"])
    w_geo = osplat.poly_splat_wgeo(Q, k, pr["keep"])
    color = ogeo.color_from_dc(P[:, 10:13])
    o = torch.sigmoid(P[:, 13])
    w_b = torch.nn.functional.softplus(wb_raw)
    img = osplat.wsr(o[None, :] * w_geo, color, w_b, torch.ones(3, dtype=P.dtype))
    return img.reshape(cam["H"], cam["W"], 3)


@pytest.mark.parametrize("name,k,G", [("c1_ref", 4.0, None), ("c1", 9.0, None),
                                      ("c1_ref", 4.0, 257)])
def test_render_dense_forward_and_grads(name, k, G):
    cfg, P, cam = config_inputs(name, G=G)
    print(f"[dense] {name} G={P.shape[0]} k={k}", flush=True)
    model = GaussianModel(P.cuda())
    model.params.requires_grad_(True)
    model.w_b_raw.requires_grad_(True)
    img = trender.render(model, cam, "A", k=k)
    R = torch.randn(cam.H, cam.W, 3, generator=torch.Generator().manual_seed(5))
    (img * R.cuda()).sum().backward()

    Pr = P.clone().requires_grad_(True)
    wr = torch.tensor(-3.0, requires_grad=True)
    ref = oracle_dense(Pr, wr, cam_dict(cam), k)
    err = max_abs(img, ref)
    print(f"[dense] {name} max|err| {err:.2e}")
    assert err <= 1e-4
    (ref * R).sum().backward()
    for gname, sl in GROUPS.items():
        e = rel_l2(model.params.grad[:, sl], Pr.grad[:, sl])
        print(f"[dense] {name} d{gname}: rel L2 {e:.2e}")
        assert e <= 1e-3, gname
    gw, gwr = float(model.w_b_raw.grad), float(wr.grad)
    assert abs(gw - gwr) <= 1e-3 * abs(gwr) + 1e-5


def test_render_dense_any_size_and_empty():
    """H, W need not be tile multiples; G = 0 gives the background."""
    cfg, P, cam0 = config_inputs("c1_ref", G=50)
    from ttsplat.camera import pinhole
    cam = pinhole(37, 53, (0.0, 0.0, 3.0))
    model = GaussianModel(P.cuda())
    img = trender.render(model, cam, "A")
    ref = oracle_dense(P, torch.tensor(-3.0), cam_dict(cam), 4.0)
    assert max_abs(img, ref) <= 1e-4
    empty = GaussianModel(torch.zeros(0, 14, device="cuda"))
    assert torch.allclose(trender.render(empty, cam, "A"), torch.ones(37, 53, 3, device="cuda"))


def test_render_dense_is_deterministic():
    cfg, P, cam = config_inputs("c1_ref")
    grads = []
    for _ in range(2):
        model = GaussianModel(P.cuda())
        model.params.requires_grad_(True)
        trender.render(model, cam, "A").square().sum().backward()
        grads.append(model.params.grad.clone())
    assert torch.equal(grads[0], grads[1])


@pytest.mark.parametrize("with_keep", [False, True])
def test_wsr_polysplat_matches_reference_autograd(with_keep):
    """A 32x32 pixel grid in coordinates centred on the grid (the tile-local fold of
    spike/forward.py:47-60: theta's terms stay O(100), so fp32 keeps u to ~1e-5), a few hundred
    gaussians, several pixel bands in the backward."""
    cfg, P, cam0 = config_inputs("c1_ref", G=300)
    from ttsplat.camera import pinhole
    cam = cam_dict(pinhole(32, 32, (0.0, 0.0, 3.0)))
    pr = ogeo.project_params(P, cam, 0.3, 0.2)
    _, th = osplat.theta_from_conic(pr["conic"], pr["mu2d"] - 16.0, 4.0)
    px, py = ogeo.pixel_grid(32, 32)
    Phi = osplat.phi(px - 16.0, py - 16.0)
    g = torch.Generator().manual_seed(11)
    o = torch.rand(300, generator=g) * 0.9 + 0.05
    color = torch.rand(300, 3, generator=g)
    keep = (torch.rand(300, generator=g) > 0.2) if with_keep else None
    cb = torch.ones(3)

    th_d = th.cuda().requires_grad_(True)
    o_d = o.cuda().requires_grad_(True)
    c_d = color.cuda().requires_grad_(True)
    wb_d = torch.tensor(0.05, device="cuda", requires_grad=True)
    C = tback.wsr_polysplat(th_d, o_d, c_d, wb_d, Phi.cuda(), cb.cuda(),
                            None if keep is None else keep.cuda())
    R = torch.randn(C.shape, generator=g)
    (C * R.cuda()).sum().backward()

    leaves = [t.double().requires_grad_(True) for t in (th, o, color)]
    wb = torch.tensor(0.05, dtype=torch.float64, requires_grad=True)
    ref = osplat.wsr_polysplat_ref(leaves[0], leaves[1], leaves[2], wb, Phi.double(), cb.double(),
                                   None if keep is None else keep.double())
    assert max_abs(C, ref) <= 1e-4
    (ref * R.double()).sum().backward()
    for mine, theirs, n in ((th_d, leaves[0], "theta"), (o_d, leaves[1], "o"),
                            (c_d, leaves[2], "color")):
        e = rel_l2(mine.grad, theirs.grad)
        print(f"[wsr] keep={with_keep} d{n}: rel L2 {e:.2e}")
        assert e <= 1e-3, n
    assert abs(float(wb_d.grad) - float(wb.grad)) <= 1e-3 * abs(float(wb.grad)) + 1e-6
    # the package's plain-tensor formula agrees with the kernel
    ref2 = tback.wsr_polysplat_ref(th.cuda(), o.cuda(), color.cuda(), 0.05, Phi.cuda(), cb.cuda(),
                                   None if keep is None else keep.cuda().float())
    assert max_abs(C, ref2) <= 1e-4


def _fit_setup(G=200, ncam=2):
    cfg, P, _ = config_inputs("c1_ref", G=G)
    cams = cfg.cameras()[:ncam]
    _, Pt, _ = config_inputs("c1_ref", seed=1, G=G)
    with torch.no_grad():
        gts = [trender.render(GaussianModel(Pt.cuda()), c, "A") for c in cams]
    return P, cams, gts


def test_fit_first_step_is_adam_on_the_mean_loss():
    """fit(): history[0] is the oracle's mean loss; one iteration equals torch.optim.Adam with the
    reference's per-group learning rates applied to the HIP gradient of that mean loss."""
    P, cams, gts = _fit_setup()
    # oracle loss at the initial parameters
    tot = sum(float(oloss.loss_fn(oracle_dense(P, torch.tensor(-3.0), cam_dict(c), 4.0), g.cpu()))
              for c, g in zip(cams, gts)) / len(cams)
    # HIP gradient of the mean loss (what fit's first iteration must use)
    Pl = P.cuda().requires_grad_(True)
    wl = torch.tensor(-3.0, device="cuda", requires_grad=True)

    class V:
        pass
    v = V()
    v.params, v.w_b_raw, v.c_b = Pl, wl, torch.ones(3, device="cuda")
    from ttsplat.loss import loss_fn
    total = sum(loss_fn(trender.render(v, c, "A"), g) for c, g in zip(cams, gts)) / len(cams)
    gP, gw = torch.autograd.grad(total, (Pl, wl))

    model = GaussianModel(P.cuda())
    hist = ttrain.fit(model, cams, gts, "A", iters=1)
    assert abs(hist[0] - tot) <= 1e-5 * abs(tot) + 1e-6

    lr = ttrain.DEFAULT_LR
    groups = (("means", 0, 3), ("quats", 3, 7), ("scales", 7, 10), ("color", 10, 13),
              ("opacity", 13, 14))
    cols = {n: P[:, a:b].clone().cuda().requires_grad_(True) for n, a, b in groups}
    wb = torch.tensor(-3.0, device="cuda", requires_grad=True)
    opt = torch.optim.Adam([{"params": [cols[n]], "lr": lr[n]} for n, _, _ in groups] +
                           [{"params": [wb], "lr": lr["wb"]}], foreach=False)
    for n, a, b in groups:
        cols[n].grad = gP[:, a:b].contiguous()
    wb.grad = gw.reshape(())
    opt.step()
    expect = torch.cat([cols[n].detach() for n, _, _ in groups], 1)
    assert max_abs(model.params, expect) <= 1e-6
    assert abs(float(model.w_b_raw) - float(wb.detach())) <= 1e-6


def test_fit_reduces_loss_and_eval_psnr():
    P, cams, gts = _fit_setup(G=300, ncam=2)
    model = GaussianModel(P.cuda())
    p0 = ttrain.eval_psnr(model, cams, gts, "A")
    hist = ttrain.fit(model, cams, gts, "A", iters=40)
    p1 = ttrain.eval_psnr(model, cams, gts, "A")
    print(f"[fit] loss {hist[0]:.4f} -> {hist[-1]:.4f}, psnr {p0:.2f} -> {p1:.2f}")
    assert hist[-1] < 0.8 * hist[0]
    assert p1 > p0


@pytest.mark.parametrize("arm,deg", [("A", 1), ("A", 3), ("B", 2), ("SZ", 3), ("RV", 3)])
def test_render_dense_view_dependent_colour(arm, deg):
    """spike/render.py with sh_degree > 0 (:23-25): SH colour in the direction means - centre,
    its gradient reaching the means through that direction, rest coefficients trained."""
    cfg, P, cam = config_inputs("c1_ref", G=600)
    g = torch.Generator().manual_seed(deg)
    rest = torch.randn(P.shape[0], 15, 3, generator=g) * 0.3
    print(f"[dense-sh] arm {arm} degree {deg}", flush=True)
    model = GaussianModel(P.cuda(), color_rest=rest.cuda())
    model.params.requires_grad_(True)
    model.color_rest.requires_grad_(True)
    img = trender.render(model, cam, arm, k=4.0, sh_degree=deg)
    R = torch.randn(cam.H, cam.W, 3, generator=torch.Generator().manual_seed(7))
    (img * R.cuda()).sum().backward()
    Pr = P.double().clone().requires_grad_(True)
    rr = rest.double().clone().requires_grad_(True)
    camd = {n: (v.double() if torch.is_tensor(v) else v) for n, v in cam_dict(cam).items()}
    kw = dict(k=4.0, rest=rr, sh_degree=deg)
    if arm == "B":
        kw["depth_bt"] = torch.tensor([1.0, 3.0], dtype=torch.float64)
    if arm == "SZ":
        kw["softz_beta"] = torch.tensor(4.0, dtype=torch.float64)
    ref = osplat.render_dense(Pr, camd, arm="A" if arm == "B" else arm, **kw)
    err = max_abs(img, ref)
    assert err <= 1e-4, err
    (ref * R.double()).sum().backward()
    for gname, sl in GROUPS.items():
        e = rel_l2(model.params.grad[:, sl], Pr.grad[:, sl])
        print(f"[dense-sh] {arm} deg {deg} d{gname}: rel L2 {e:.2e}", flush=True)
        assert e <= 1e-3, gname
    n = (deg + 1) ** 2 - 1
    assert rel_l2(model.color_rest.grad[:, :n], rr.grad[:, :n]) <= 1e-3
    if n < 15:       # rows beyond the degree take no gradient
        assert float(model.color_rest.grad[:, n:].abs().max()) == 0.0


def test_fit_with_view_dependent_colour():
    """fit(..., sh_degree=2): the rest coefficients train (Adam at lr color / 20, spike/model.py:91)
    and the loss falls; one step equals Adam on the oracle's gradient."""
    cfg, P, cam = config_inputs("c1_ref", G=400)
    rest = torch.zeros(P.shape[0], 15, 3)
    tgt_model = GaussianModel(cfg.params(seed=1)[:400].cuda(),
                              color_rest=torch.randn(400, 15, 3, generator=torch.Generator()
                                                     .manual_seed(3)).cuda() * 0.2)
    with torch.no_grad():
        tgt = trender.render(tgt_model, cam, "A", sh_degree=2)
    model = GaussianModel(P.cuda(), color_rest=rest.cuda())
    hist = ttrain.fit(model, [cam], [tgt], "A", iters=1, sh_degree=2)
    # oracle: one Adam step (first step: p -= lr * sign(g)) on the rest block
    rr = rest.double().clone().requires_grad_(True)
    camd = {n: (v.double() if torch.is_tensor(v) else v) for n, v in cam_dict(cam).items()}
    ref = osplat.render_dense(P.double(), camd, k=4.0, rest=rr, sh_degree=2)
    oloss.loss_fn(ref, tgt.cpu().double()).backward()
    lr_rest = ttrain.DEFAULT_LR["color"] / 20.0
    step = model.color_rest.cpu().double() - rest.double()
    exp = -lr_rest * rr.grad / (rr.grad.abs() + 1e-8)      # Adam's first step, eps = 1e-8
    big = rr.grad.abs() > 1e-5
    assert int(big.sum()) > 100
    assert torch.allclose(step[big], exp[big], rtol=1e-3, atol=1e-9)
    hist += ttrain.fit(model, [cam], [tgt], "A", iters=30, sh_degree=2)
    assert hist[-1] < 0.9 * hist[0]
