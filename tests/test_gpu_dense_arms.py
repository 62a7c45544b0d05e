"""The per-pixel occlusion arms of the dense render on the GPU vs the oracle (spike/arms.py:50-83):
soft-Z (two passes per pixel, a pixel pre-pass in the backward for the gradient through z*) and
revealage.  Images within 1e-4, gradients within 1e-3 relative L2 of autograd through the
oracle's restatement; fit() trains each arm."""
import pytest
import torch

from helpers import cam_dict, config_inputs, max_abs, rel_l2
from oracle import splat as osplat
from ttsplat import render as trender
from ttsplat import train as ttrain
from ttsplat.model import GaussianModel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("arm", ["SZ", "RV"])
@pytest.mark.parametrize("G", [None, 300])
def test_dense_arm_forward_and_grads(arm, G):
    cfg, P, cam = config_inputs("c1_ref", G=G)
    model = GaussianModel(P.cuda(), softz_beta=3.0)
    model.params.requires_grad_(True)
    model.w_b_raw.requires_grad_(True)
    model.softz_beta.requires_grad_(True)
    img = trender.render(model, cam, arm)
    R = torch.randn(cam.H, cam.W, 3, generator=torch.Generator().manual_seed(7))
    (img * R.cuda()).sum().backward()
    Pr = P.double().clone().requires_grad_(True)
    wr = torch.tensor(-3.0, dtype=torch.float64, requires_grad=True)
    sz = torch.tensor(3.0, dtype=torch.float64, requires_grad=True)
    ref = osplat.render_dense(Pr, cam_dict(cam), w_b_raw=wr, arm=arm, softz_beta=sz)
    err = max_abs(img, ref)
    print(f"[{arm}] G={P.shape[0]} max|err| {err:.2e}", flush=True)
    assert err <= 1e-4
    (ref * R.double()).sum().backward()
    for sl in (slice(0, 3), slice(3, 7), slice(7, 10), slice(10, 13), slice(13, 14)):
        e = rel_l2(model.params.grad[:, sl], Pr.grad[:, sl])
        print(f"[{arm}] grad {sl}: {e:.2e}", flush=True)
        assert e <= 1e-3, sl
    if arm == "SZ":
        gw, gwr = float(model.w_b_raw.grad), float(wr.grad)
        assert abs(gw - gwr) <= 1e-3 * abs(gwr) + 1e-5
        gs, gsr = float(model.softz_beta.grad), float(sz.grad)
        assert abs(gs - gsr) <= 1e-3 * abs(gsr) + 1e-6
    else:
        assert float(model.w_b_raw.grad) == 0.0            # revealage has no w_b


def test_revealage_clamps_near_opaque_splats():
    """Revealage clamps each alpha o w_geo at 1 - 1e-4 before log1p (spike/arms.py:71-83): with
    near-opaque, wide splats many pixels have o w_geo above 0.99, where the clamp decides the
    transmittance; image and gradients still follow the oracle."""
    import math
    from oracle import geometry as ogeo
    cfg, P, cam = config_inputs("c1_ref", G=300)
    P = P.clone()
    # twice as wide, still anisotropic (an isotropic covariance leaves the rotation without a
    # gradient); opacity 0.9995, where fp32 still resolves 1 - o to 1e-4 for the opacity gradient
    P[:, 7:10] += math.log(2.0)
    P[:, 13] = math.log(0.9995 / 0.0005)
    camd = cam_dict(cam)
    pr = ogeo.project_params(P.double(), camd)
    px, py = ogeo.pixel_grid(cam.H, cam.W, dtype=torch.float64)
    wg = osplat.poly_splat_wgeo(osplat.quad_form(px, py, pr["mu2d"], pr["conic"]), 4.0,
                                pr["keep"])
    alpha = torch.sigmoid(P[:, 13].double())[None, :] * wg
    n_hi = int((alpha > 0.99).any(dim=1).sum())
    print(f"[RV-opaque] pixels with an alpha above 0.99: {n_hi}", flush=True)
    assert n_hi >= 50
    model = GaussianModel(P.cuda())
    model.params.requires_grad_(True)
    img = trender.render(model, cam, "RV")
    R = torch.randn(cam.H, cam.W, 3, generator=torch.Generator().manual_seed(9))
    (img * R.cuda()).sum().backward()
    Pr = P.double().clone().requires_grad_(True)
    ref = osplat.render_dense(Pr, camd, arm="RV")
    err = max_abs(img, ref)
    print(f"[RV-opaque] max|err| {err:.2e}", flush=True)
    assert err <= 1e-4
    (ref * R.double()).sum().backward()
    for sl in (slice(0, 3), slice(3, 7), slice(7, 10), slice(10, 13), slice(13, 14)):
        e = rel_l2(model.params.grad[:, sl], Pr.grad[:, sl])
        print(f"[RV-opaque] grad {sl}: {e:.2e}", flush=True)
        assert e <= 1e-3, sl


@pytest.mark.parametrize("arm", ["SZ", "RV"])
def test_fit_trains_the_arm(arm):
    from ttsplat import scenes
    from ttsplat.camera import pinhole
    cfg, P, _ = config_inputs("c1_ref", G=300)
    cams = [pinhole(64, 64, e) for e in scenes.orbit_eyes(2)]
    gt = GaussianModel(cfg.params(seed=1)[:300].cuda(), softz_beta=6.0)
    with torch.no_grad():
        gts = [trender.render(gt, c, arm) for c in cams]
    model = GaussianModel(P.cuda())
    hist = ttrain.fit(model, cams, gts, arm, iters=40)
    print(f"[fit {arm}] {hist[0]:.4f} -> {hist[-1]:.4f}", flush=True)
    assert hist[-1] < 0.8 * hist[0]
    if arm == "SZ":
        assert abs(float(model.softz_beta) - 4.0) > 1e-3
