"""Host-side logic (CPU): seeded workloads, camera blocks, model layout, tile maps, the bench's
one-GPU contract."""
import math
import os
import sys

import torch

from ttsplat import scenes
from ttsplat.camera import Camera, look_at_opencv, pinhole


def test_params_are_seeded_and_in_range():
    a = scenes.make_params(5000, seed=0)
    b = scenes.make_params(5000, seed=0)
    c = scenes.make_params(5000, seed=1)
    assert torch.equal(a, b) and not torch.equal(a, c)
    assert a.shape == (5000, 14)
    assert float(a[:, 0:3].abs().max()) <= 1.0
    s = a[:, 7:10].exp()
    assert float(s.min()) >= 0.01 - 1e-6 and float(s.max()) <= 0.1 + 1e-6
    assert torch.allclose(a[:, 3:7].norm(dim=1), torch.ones(5000), atol=1e-5)
    o = torch.sigmoid(a[:, 13])
    assert float(o.min()) >= 0.05 - 1e-5 and float(o.max()) <= 0.95 + 1e-5
    rgb = 0.5 + scenes.C0 * a[:, 10:13]
    assert float(rgb.min()) >= -1e-6 and float(rgb.max()) <= 1 + 1e-6


def test_clustered_means():
    p = scenes.make_params(20000, seed=0, means="clustered")
    m = p[:, 0:3]
    assert float(m.abs().max()) < 2.0 + 6 * 0.2
    # 20 clusters: most points lie within 3 sigma of some centre in a k-means sense -> the
    # spread is much larger than one cluster's but far from uniform
    assert 0.5 < float(m.std(0).mean()) < 2.0


def test_configs_match_tile_counts():
    assert scenes.CONFIGS["c4"].W == 1264 and scenes.CONFIGS["c4"].H == 832
    for name, T in (("c1_ref", 64), ("c1", 16), ("c3", 2500), ("c4", 4108), ("c5", 8040)):
        c = scenes.CONFIGS[name]
        assert (c.H // c.S) * (c.W // c.S) == T, name
    assert scenes.CONFIGS["c1"].span == 8192 and scenes.CONFIGS["c4"].span == 2048


def test_orbit_cameras():
    eyes = scenes.orbit_eyes(8)
    assert len(eyes) == 8 and eyes == scenes.orbit_eyes(8)
    for e in eyes:
        assert abs(math.sqrt(sum(v * v for v in e)) - 3.0) < 1e-5
        assert abs(e[1]) / 3.0 <= 0.95


def test_camera_block_and_fov():
    cam = pinhole(832, 1264, (0.0, 0.0, 3.0))
    blk = cam.host_block()
    assert blk.shape == (16,)
    assert abs(float(blk[12]) - 0.5 * 1264 / math.tan(math.radians(25))) < 1e-3
    assert float(blk[14]) == 632.0 and float(blk[15]) == 416.0
    R, t = look_at_opencv((1.0, 2.0, 3.0))
    c = Camera(R, t, 1, 1, 0, 0, 16, 16)
    assert torch.allclose(c.center, torch.tensor([1.0, 2.0, 3.0]), atol=1e-5)


def test_model_views():
    from ttsplat.model import GaussianModel
    P = scenes.make_params(10, seed=3)
    m = GaussianModel(P)
    assert torch.equal(m.means3d, P[:, 0:3]) and torch.equal(m.opacity_raw, P[:, 13])
    assert m.G == 10


def test_render_rejects_arms_off_the_hip_path():
    import pytest
    from ttsplat import render, train
    for arm in ("C0", "C", "D"):
        with pytest.raises(NotImplementedError):
            render.render(None, None, arm)
    assert render.ARMS == ("A", "B", "SZ", "RV")
    with pytest.raises(ValueError):             # SH degree outside [0, 3]
        render.render(None, None, "A", sh_degree=4)
    assert train.DEFAULT_LR["means"] == 5e-3 and train.DEFAULT_LR["wb"] == 1e-2


def test_tensor_helpers_refuse_cpu_tensors():
    import pytest
    from ttsplat import forward, geometry
    x = torch.zeros(4)
    with pytest.raises(ValueError):
        forward.phi(x, x)
    with pytest.raises(ValueError):
        geometry.quat_to_rotmat(torch.zeros(2, 4))


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 (or a multi-rank launch) exits with status 2
    and says so, before touching a device."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for extra, env in ((["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})):
        r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), *extra],
                           capture_output=True, text=True, timeout=120,
                           env={**os.environ, **env})
        assert r.returncode == 2, r.stderr
        assert "exactly one GPU" in r.stderr
