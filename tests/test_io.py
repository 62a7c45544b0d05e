"""Scene IO on the CPU: the .ply writer/reader (the reference's 17-property layout and the
standard one with f_rest_*), the NeRF-synthetic and COLMAP loaders on synthetic files written
here, the OpenGL->OpenCV pose conversion (spike/tests/test_camera.py and
spike/tests/test_data.py restated), and the point-cloud initialisation."""
import json
import math
import os
import struct

import numpy as np
import pytest
import torch
from PIL import Image

from ttsplat import camera, io, model

D = torch.float64


def _params(G, seed=0):
    g = torch.Generator().manual_seed(seed)
    P = torch.randn(G, 14, generator=g)
    P[:, 3:7] = P[:, 3:7] / P[:, 3:7].norm(dim=1, keepdim=True)
    return P


def test_ply_round_trip_reference_layout(tmp_path):
    P = _params(1000)
    P[:, 3:7] *= 3.0                                      # stored normalised
    path = tmp_path / "g.ply"
    assert io.save_ply(path, P) == 1000
    raw = open(path, "rb").read()
    header, body = raw.split(b"end_header\n", 1)
    props = [ln.split()[-1].decode() for ln in header.split(b"\n") if ln.startswith(b"property")]
    assert props == io.PLY_FIELDS                          # spike/plyio.py:15-16 field order
    assert b"format binary_little_endian 1.0" in header and b"element vertex 1000" in header
    assert len(body) == 1000 * 17 * 4
    Q, rest = io.read_ply(path)
    assert rest is None
    Pn = P.clone()
    Pn[:, 3:7] = P[:, 3:7] / P[:, 3:7].norm(dim=1, keepdim=True)
    assert torch.allclose(Q, Pn, atol=1e-6)
    assert torch.equal(Q[:, [0, 1, 2, 7, 8, 9, 10, 11, 12, 13]],
                       P[:, [0, 1, 2, 7, 8, 9, 10, 11, 12, 13]])


def test_ply_with_sh_rest(tmp_path):
    P = _params(50)
    rest = torch.randn(50, 15, 3, generator=torch.Generator().manual_seed(1))
    path = tmp_path / "g.ply"
    io.save_ply(path, P, color_rest=rest)
    Q, r = io.read_ply(path)
    assert torch.equal(r, rest)
    # inria order: f_rest_{c*15 + l}
    rec = np.frombuffer(open(path, "rb").read().split(b"end_header\n", 1)[1], dtype="<f4")
    rec = rec.reshape(50, 17 + 45)
    assert rec[7, 17 + 2 * 15 + 4] == float(rest[7, 4, 2])


def test_ply_reads_other_property_orders(tmp_path):
    P = _params(20)
    fields = ["opacity", "x", "y", "z", "red"] + [f"rot_{i}" for i in range(4)] + \
        [f"scale_{i}" for i in range(3)] + [f"f_dc_{i}" for i in range(3)]
    cols = {"x": P[:, 0], "y": P[:, 1], "z": P[:, 2], "opacity": P[:, 13]}
    cols.update({f"rot_{i}": P[:, 3 + i] for i in range(4)})
    cols.update({f"scale_{i}": P[:, 7 + i] for i in range(3)})
    cols.update({f"f_dc_{i}": P[:, 10 + i] for i in range(3)})
    dt = np.dtype([(f, "<f4") if f != "red" else (f, "u1") for f in fields])
    arr = np.zeros(20, dtype=dt)
    for f in fields:
        arr[f] = 7 if f == "red" else cols[f].numpy()
    hdr = "ply\nformat binary_little_endian 1.0\nelement vertex 20\n" + "".join(
        f"property {'uchar' if f == 'red' else 'float'} {f}\n" for f in fields) + "end_header\n"
    path = tmp_path / "o.ply"
    open(path, "wb").write(hdr.encode() + arr.tobytes())
    Q, _ = io.read_ply(path)
    assert torch.equal(Q, P)


def test_camera_conversion():
    c2w = torch.eye(4, dtype=D)
    R_v, t_v = camera.opengl_c2w_to_opencv_w2c(c2w)
    pix, z = camera.project_point(torch.tensor([0.0, 0.0, -5.0], dtype=D), R_v, t_v, 100.0,
                                  100.0, 64.0, 64.0)
    assert z > 0 and torch.allclose(pix, torch.tensor([64.0, 64.0], dtype=D))
    pix2, _ = camera.project_point(torch.tensor([1.0, 0.0, -5.0], dtype=D), R_v, t_v, 100.0,
                                   100.0, 64.0, 64.0)
    assert abs(float(pix2[0]) - (100.0 / 5.0 + 64.0)) < 1e-9
    _, zb = camera.project_point(torch.tensor([0.0, 0.0, 5.0], dtype=D), R_v, t_v, 100.0, 100.0,
                                 64.0, 64.0)
    assert zb < 0
    c2w[2, 3] = 4.0
    R_v, t_v = camera.opengl_c2w_to_opencv_w2c(c2w)
    _, z = camera.project_point(torch.zeros(3, dtype=D), R_v, t_v, 100.0, 100.0, 64.0, 64.0)
    assert abs(float(z) - 4.0) < 1e-9
    th = 0.5
    c2w = torch.eye(4, dtype=D)
    c2w[:3, :3] = torch.tensor([[math.cos(th), 0, math.sin(th)], [0, 1, 0],
                                [-math.sin(th), 0, math.cos(th)]], dtype=D)
    c2w[:3, 3] = torch.tensor([1.0, 2.0, 3.0], dtype=D)
    R_v, _ = camera.opengl_c2w_to_opencv_w2c(c2w)
    assert torch.allclose(R_v @ R_v.T, torch.eye(3, dtype=D)) and abs(float(torch.det(R_v)) - 1) < 1e-9


def _fake_blender(root, angle_x=0.6911112070083618):
    os.makedirs(os.path.join(root, "train"), exist_ok=True)
    px = np.zeros((8, 8, 4), dtype=np.uint8)
    px[:, :] = (10, 20, 30, 255)
    px[0, 0] = (255, 0, 0, 255)
    px[0, 1] = (0, 255, 0, 0)
    px[1, 0] = (0, 0, 255, 128)
    for name in ("r_0", "r_1"):
        Image.fromarray(px, mode="RGBA").save(os.path.join(root, "train", f"{name}.png"))
    c2w1 = torch.eye(4)
    c2w1[2, 3] = 4.0
    meta = {"camera_angle_x": angle_x,
            "frames": [{"file_path": "./train/r_0", "transform_matrix": torch.eye(4).tolist()},
                       {"file_path": "./train/r_1", "transform_matrix": c2w1.tolist()}]}
    with open(os.path.join(root, "transforms_train.json"), "w") as f:
        json.dump(meta, f)
    return angle_x


def test_blender_loader(tmp_path):
    angle_x = _fake_blender(str(tmp_path))
    cams, imgs = io.load_blender(str(tmp_path), "train", res=8)
    assert len(cams) == 2 and imgs[0].shape == (8, 8, 3)
    assert torch.allclose(imgs[0][0, 0], torch.tensor([1.0, 0.0, 0.0]), atol=2e-2)
    assert torch.allclose(imgs[0][0, 1], torch.tensor([1.0, 1.0, 1.0]), atol=2e-2)
    b = imgs[0][1, 0]
    assert b[2] > 0.95 and abs(float(b[0]) - 128 / 255) < 3e-2
    assert torch.allclose(cams[0].R_v, torch.diag(torch.tensor([1.0, -1.0, -1.0])))
    assert abs(cams[0].fx - 0.5 * 8 / math.tan(0.5 * angle_x)) < 1e-5
    assert cams[0].H == 8 and cams[0].W == 8
    assert torch.allclose(cams[1].center, torch.tensor([0.0, 0.0, 4.0]), atol=1e-6)
    rgba = io.load_blender(str(tmp_path), "train", res=8, keep_alpha=True)[1][0]
    assert rgba.shape == (8, 8, 4) and abs(float(rgba[0, 1, 3])) < 1e-6
    assert io.select_indices(10, stride=3, n=2) == [0, 3]
    assert io.select_indices(10, indices=[2, 5]) == [2, 5]
    assert io.intrinsics_from_fov(0.6911112070083618, 800, 800)[2:] == (400.0, 400.0)


def _fake_colmap(root):
    sp = os.path.join(root, "sparse", "0")
    os.makedirs(sp)
    os.makedirs(os.path.join(root, "images"))
    with open(os.path.join(sp, "cameras.bin"), "wb") as f:
        f.write(struct.pack("<Q", 2))
        f.write(struct.pack("<iiQQ", 1, 0, 40, 30) + struct.pack("<3d", 50.0, 20.0, 15.0))
        f.write(struct.pack("<iiQQ", 2, 1, 40, 30) + struct.pack("<4d", 60.0, 61.0, 19.0, 14.0))
    qs = [(1.0, 0.0, 0.0, 0.0), (math.cos(0.3), 0.0, math.sin(0.3), 0.0)]
    ts = [(0.0, 0.0, 4.0), (0.5, -0.2, 3.0)]
    with open(os.path.join(sp, "images.bin"), "wb") as f:
        f.write(struct.pack("<Q", 2))
        for i, (name, q, t, cid) in enumerate([("b.png", qs[1], ts[1], 2),
                                               ("a.png", qs[0], ts[0], 1)]):
            f.write(struct.pack("<i", i + 1) + struct.pack("<4d", *q) + struct.pack("<3d", *t))
            f.write(struct.pack("<i", cid) + name.encode() + b"\x00")
            f.write(struct.pack("<Q", 3) + struct.pack("<ddq", 1.0, 2.0, -1) * 3)
    for name, c in (("a.png", (200, 10, 10)), ("b.png", (10, 200, 10))):
        Image.fromarray(np.full((30, 40, 3), c, dtype=np.uint8)).save(
            os.path.join(root, "images", name))
    pts = [((0.1, 0.2, 0.3), (255, 0, 128), 2), ((-1.0, 0.5, 2.0), (0, 64, 255), 0),
           ((3.0, -2.0, 1.0), (10, 20, 30), 5)]
    with open(os.path.join(sp, "points3D.bin"), "wb") as f:
        f.write(struct.pack("<Q", len(pts)))
        for k, (xyz, rgb, tl) in enumerate(pts):
            f.write(struct.pack("<Q", k) + struct.pack("<3d", *xyz) + struct.pack("<3B", *rgb))
            f.write(struct.pack("<d", 0.5) + struct.pack("<Q", tl) + struct.pack("<ii", 1, 2) * tl)
    return qs, ts, pts


def test_colmap_loader(tmp_path):
    qs, ts, pts = _fake_colmap(str(tmp_path))
    cams, imgs = io.load_colmap(str(tmp_path))
    assert len(cams) == 2                                  # sorted by name: a.png, b.png
    assert torch.allclose(imgs[0][0, 0], torch.tensor([200, 10, 10]) / 255.0)
    assert (cams[0].fx, cams[0].fy, cams[0].cx, cams[0].cy) == (50.0, 50.0, 20.0, 15.0)
    assert (cams[1].fx, cams[1].fy, cams[1].cx, cams[1].cy) == (60.0, 61.0, 19.0, 14.0)
    assert torch.allclose(cams[0].R_v, torch.eye(3)) and torch.allclose(cams[0].t_v,
                                                                          torch.tensor(ts[0]))
    R1 = cams[1].R_v.double()
    a = 0.6                                                # rotation by 2*0.3 about y
    assert torch.allclose(R1, torch.tensor([[math.cos(a), 0, math.sin(a)], [0, 1, 0],
                                            [-math.sin(a), 0, math.cos(a)]], dtype=D), atol=1e-6)
    cams2, imgs2 = io.load_colmap(str(tmp_path), downscale=2)
    assert imgs2[0].shape == (15, 20, 3) and cams2[1].fx == 30.0 and cams2[1].cy == 7.0
    xyz, rgb = io.load_colmap_points(str(tmp_path))
    assert np.allclose(xyz, [p[0] for p in pts]) and np.allclose(rgb * 255, [p[1] for p in pts])
    xyz2, _ = io.load_colmap_points(str(tmp_path), max_pts=2)
    assert xyz2.shape == (2, 3)


def test_init_from_points():
    g = torch.Generator().manual_seed(3)
    xyz = torch.rand(500, 3, generator=g)
    rgb = torch.rand(500, 3, generator=g)
    P = model.init_from_points(xyz, rgb, 300, seed=1)
    assert P.shape == (300, 14)
    # every mean is one of the points, colour the inverse DC SH of its colour
    eq = (P[:, None, 0:3] == xyz[None]).all(-1)            # [300, 500] exact matches
    assert bool(eq.any(1).all())
    j = eq.float().argmax(1)
    assert torch.allclose(P[:, 10:13] * model.C0 + 0.5, rgb[j], atol=1e-6)
    assert bool((P[:, 7:10] == P[0, 7]).all())
    sub_nn = torch.cdist(P[:, 0:3], P[:, 0:3]).fill_diagonal_(float("inf")).min(1).values
    assert abs(float(P[0, 7]) - math.log(float(sub_nn.median()))) < 1e-5   # all 300 sampled
    Q = model.init_from_points(xyz[:100], rgb[:100], 300, seed=1)        # padded with jitter
    assert torch.equal(Q[:100, 0:3], xyz[:100])
    assert torch.equal(model.init_from_points(xyz, rgb, 300, seed=1), P)
