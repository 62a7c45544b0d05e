"""On-disk formats for real scenes: the 3DGS .ply writer/reader and the NeRF-synthetic
("blender") and COLMAP loaders (spike/plyio.py:20-40, tools/bh_views.py:30-47,
spike/data.py:20-171).

Host-side parsers: they return CPU tensors (cameras as ttsplat.camera.Camera, images [H,W,3]
fp32 in [0, 1]) which TrainStep moves to the device once.  The binary COLMAP files are parsed
with numpy record views of each fixed-size field group instead of per-field struct calls.

.ply layout (binary_little_endian, one float32 per property, the standard inria/gsplat names):
  x y z  nx ny nz  f_dc_0..2  opacity (logit)  scale_0..2 (log)  rot_0..3 (w x y z, normalised)
then, when SH rest coefficients are written, f_rest_0..44 in the inria order
(f_rest_{c*15 + l} = rest coefficient l of channel c).  The reference writes the first 17
properties only (DC colour); read_ply reads either, and any property order, by name.
"""
import json
import math
import os
import struct

import numpy as np
import torch

from .camera import Camera, opengl_c2w_to_opencv_w2c

PLY_FIELDS = (["x", "y", "z", "nx", "ny", "nz", "f_dc_0", "f_dc_1", "f_dc_2", "opacity"]
              + [f"scale_{i}" for i in range(3)] + [f"rot_{i}" for i in range(4)])
REST_FIELDS = [f"f_rest_{i}" for i in range(45)]


# ------------------------------------------------------------------------------ .ply --
def _params_of(model):
    """[G,14] parameter block of a ttsplat GaussianModel, a spike model, or a tensor."""
    if isinstance(model, torch.Tensor):
        return model.detach().float().cpu()
    if hasattr(model, "params"):
        return model.params.detach().float().cpu()
    return torch.cat([model.means3d.detach().reshape(-1, 3), model.quats.detach().reshape(-1, 4),
                      model.log_scales.detach().reshape(-1, 3),
                      model.color_dc.detach().reshape(-1, 3),
                      model.opacity_raw.detach().reshape(-1, 1)], dim=1).float().cpu()


def save_ply(path, model, color_rest=None):
    """Write a gaussian set ([G,14] params, a GaussianModel or a spike model) as a 3DGS .ply
    (spike/plyio.py:20-40: zero normals, logit opacity, log scales, normalised quaternion).
    color_rest [G,15,3] (or the model's color_rest when present and non-zero) adds f_rest_*.
    Returns the number of gaussians."""
    P = _params_of(model)
    n = P.shape[0]
    if color_rest is None and not isinstance(model, torch.Tensor):
        cr = getattr(model, "color_rest", None)
        if cr is not None and bool((cr != 0).any()):
            color_rest = cr
    q = P[:, 3:7]
    q = q / q.norm(dim=-1, keepdim=True).clamp(min=1e-12)
    cols = [P[:, 0:3], torch.zeros(n, 3), P[:, 10:13], P[:, 13:14], P[:, 7:10], q]
    fields = list(PLY_FIELDS)
    if color_rest is not None:
        rest = torch.as_tensor(color_rest).detach().float().cpu().reshape(n, 15, 3)
        cols.append(rest.transpose(1, 2).reshape(n, 45))       # f_rest_{c*15 + l}
        fields += REST_FIELDS
    data = torch.cat(cols, dim=1).numpy().astype("<f4")
    header = ("ply\nformat binary_little_endian 1.0\n"
              f"element vertex {n}\n"
              + "".join(f"property float {f}\n" for f in fields)
              + "end_header\n")
    with open(path, "wb") as fh:
        fh.write(header.encode("ascii"))
        fh.write(data.tobytes())
    return n


_PLY_TYPES = {"float": "<f4", "float32": "<f4", "double": "<f8", "float64": "<f8",
              "uchar": "u1", "uint8": "u1", "char": "i1", "int8": "i1", "short": "<i2",
              "int16": "<i2", "ushort": "<u2", "uint16": "<u2", "int": "<i4", "int32": "<i4",
              "uint": "<u4", "uint32": "<u4"}


def read_ply(path):
    """Read a binary little-endian 3DGS .ply (this writer's, the reference's 17-property
    layout, or a standard file with extra properties).  Returns (params [G,14] fp32,
    color_rest [G,15,3] or None).  Quaternions are returned as stored."""
    with open(path, "rb") as fh:
        if fh.readline().strip() != b"ply":
            raise ValueError(f"{path}: not a .ply file")
        n, props, in_vertex = None, [], False
        while True:
            line = fh.readline()
            if not line:
                raise ValueError(f"{path}: header has no end_header")
            tok = line.split()
            if not tok:
                continue
            if tok[0] == b"format" and tok[1] != b"binary_little_endian":
                raise ValueError(f"{path}: only binary_little_endian is supported")
            if tok[0] == b"element":
                in_vertex = tok[1] == b"vertex"
                if in_vertex:
                    n = int(tok[2])
            elif tok[0] == b"property" and in_vertex:
                if tok[1] == b"list":
                    raise ValueError(f"{path}: list properties in the vertex element")
                props.append((tok[2].decode(), _PLY_TYPES[tok[1].decode()]))
            elif tok[0] == b"end_header":
                break
        if n is None:
            raise ValueError(f"{path}: no vertex element")
        rec = np.frombuffer(fh.read(), dtype=np.dtype(props), count=n)
    names = {p for p, _ in props}
    missing = [f for f in PLY_FIELDS if f not in names and f not in ("nx", "ny", "nz")]
    if missing:
        raise ValueError(f"{path}: missing properties {missing}")

    def col(*fs):
        return np.stack([rec[f].astype(np.float32) for f in fs], axis=1)

    P = np.concatenate([col("x", "y", "z"), col("rot_0", "rot_1", "rot_2", "rot_3"),
                        col("scale_0", "scale_1", "scale_2"),
                        col("f_dc_0", "f_dc_1", "f_dc_2"), col("opacity")], axis=1)
    rest = None
    if all(f in names for f in REST_FIELDS):
        rest = torch.from_numpy(col(*REST_FIELDS).reshape(n, 3, 15).transpose(0, 2, 1).copy())
    return torch.from_numpy(np.ascontiguousarray(P)), rest


# ---------------------------------------------------------------------- NeRF-synthetic --
def intrinsics_from_fov(camera_angle_x, W, H):
    """Square-pixel pinhole intrinsics from the horizontal field of view (spike/data.py:20-23)."""
    fx = 0.5 * W / math.tan(0.5 * camera_angle_x)
    return fx, fx, W / 2.0, H / 2.0


def composite_over_white(rgba):
    """[..., 4] straight RGBA in [0, 1] -> [..., 3] over a white background."""
    rgb, a = rgba[..., :3], rgba[..., 3:4]
    return rgb * a + (1.0 - a)


def select_indices(n_frames, indices=None, stride=None, n=None):
    """Explicit indices, or every `stride`-th frame, capped at `n` (spike/data.py:40-45)."""
    if indices is not None:
        return list(indices)
    idx = list(range(0, n_frames, stride)) if stride else list(range(n_frames))
    return idx[:n] if n is not None else idx


def _load_rgba(path, size=None):
    from PIL import Image
    img = Image.open(path).convert("RGBA")
    if size is not None and (img.width, img.height) != size:
        img = img.resize(size, Image.BILINEAR)
    return torch.from_numpy(np.asarray(img, dtype=np.float32) / 255.0)


def load_blender(root, split="train", res=200, indices=None, stride=None, n=None,
                 keep_alpha=False):
    """NeRF-synthetic split (transforms_{split}.json + RGBA PNGs) -> (cameras, images)
    (spike/data.py:48-76): poses converted OpenGL c2w -> OpenCV w2c, frames resized to res x res
    (None keeps the file size), composited over white unless keep_alpha."""
    with open(os.path.join(root, f"transforms_{split}.json")) as f:
        meta = json.load(f)
    frames = meta["frames"]
    cameras, images = [], []
    for i in select_indices(len(frames), indices, stride, n):
        fr = frames[i]
        R_v, t_v = opengl_c2w_to_opencv_w2c(
            torch.tensor(fr["transform_matrix"], dtype=torch.float64))
        fp = fr["file_path"]
        png = os.path.normpath(os.path.join(root, fp if fp.endswith(".png") else fp + ".png"))
        rgba = _load_rgba(png, None if res is None else (res, res))
        img = rgba if keep_alpha else composite_over_white(rgba)
        H, W = img.shape[0], img.shape[1]
        fx, fy, cx, cy = intrinsics_from_fov(meta["camera_angle_x"], W, H)
        cameras.append(Camera(R_v, t_v, fx, fy, cx, cy, H, W))
        images.append(img.contiguous())
    return cameras, images


# ----------------------------------------------------------------------------- COLMAP --
# Parameter counts of COLMAP's camera models (SIMPLE_PINHOLE, PINHOLE, SIMPLE_RADIAL, RADIAL,
# OPENCV, OPENCV_FISHEYE, FULL_OPENCV, FOV, SIMPLE_RADIAL_FISHEYE, RADIAL_FISHEYE,
# THIN_PRISM_FISHEYE); the models with a single focal length store f, cx, cy first.
COLMAP_NPARAMS = {0: 3, 1: 4, 2: 4, 3: 5, 4: 8, 5: 8, 6: 12, 7: 5, 8: 4, 9: 5, 10: 12}
COLMAP_SINGLE_F = {0, 2, 3, 8, 9}


def qvec_to_rotmat(q):
    """COLMAP quaternion (w, x, y, z) -> world->camera rotation [3,3] float64."""
    w, x, y, z = q
    return np.array([
        [1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
        [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
        [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]], dtype=np.float64)


def read_colmap_cameras(path):
    """cameras.bin -> {camera_id: (fx, fy, cx, cy, W, H)} (spike/data.py:92-107)."""
    buf = open(path, "rb").read()
    (n,), off, cams = struct.unpack_from("<Q", buf, 0), 8, {}
    for _ in range(n):
        cid, model, W, H = struct.unpack_from("<iiQQ", buf, off)
        off += 24
        if model not in COLMAP_NPARAMS:
            raise ValueError(f"{path}: unknown COLMAP camera model {model}")
        k = COLMAP_NPARAMS[model]
        p = np.frombuffer(buf, dtype="<f8", count=k, offset=off)
        off += 8 * k
        if model in COLMAP_SINGLE_F:
            fx = fy = p[0]
            cx, cy = p[1], p[2]
        else:
            fx, fy, cx, cy = p[0], p[1], p[2], p[3]
        cams[cid] = (float(fx), float(fy), float(cx), float(cy), int(W), int(H))
    return cams


def read_colmap_images(path):
    """images.bin -> [(qvec[4], tvec[3], camera_id, name)] (spike/data.py:110-130)."""
    buf = open(path, "rb").read()
    (n,), off, out = struct.unpack_from("<Q", buf, 0), 8, []
    for _ in range(n):
        off += 4                                                     # image_id
        qt = np.frombuffer(buf, dtype="<f8", count=7, offset=off)
        off += 56
        (cid,) = struct.unpack_from("<i", buf, off)
        off += 4
        end = buf.index(b"\x00", off)
        name = buf[off:end].decode()
        off = end + 1
        (npts,) = struct.unpack_from("<Q", buf, off)
        off += 8 + 24 * npts                                         # skip the 2-D points
        out.append((qt[:4].copy(), qt[4:].copy(), cid, name))
    return out


def load_colmap(root, downscale=1, n=None, stride=None):
    """COLMAP scene (root/sparse/0/{cameras,images}.bin + root/images) -> (cameras, images)
    (spike/data.py:133-156): views sorted by file name, optional integer downscale of the
    images and intrinsics, COLMAP's world->camera pose used as is."""
    from PIL import Image
    sp = os.path.join(root, "sparse", "0")
    cams = read_colmap_cameras(os.path.join(sp, "cameras.bin"))
    metas = sorted(read_colmap_images(os.path.join(sp, "images.bin")), key=lambda r: r[3])
    cameras, images = [], []
    for i in select_indices(len(metas), None, stride, n):
        q, t, cid, name = metas[i]
        fx, fy, cx, cy, W, H = cams[cid]
        im = Image.open(os.path.join(root, "images", name)).convert("RGB")
        if downscale > 1:
            W, H = W // downscale, H // downscale
            im = im.resize((W, H), Image.BILINEAR)
            s = 1.0 / downscale
            fx, fy, cx, cy = fx * s, fy * s, cx * s, cy * s
        images.append(torch.from_numpy(np.asarray(im, dtype=np.float32) / 255.0))
        cameras.append(Camera(torch.from_numpy(qvec_to_rotmat(q)), torch.from_numpy(t),
                              fx, fy, cx, cy, H, W))
    return cameras, images


def load_colmap_points(root, max_pts=None):
    """sparse/0/points3D.bin -> (xyz [N,3] fp32, rgb [N,3] in [0, 1]) for initialisation
    (spike/data.py:159-171; subsampled with numpy's default_rng(0) when above max_pts)."""
    buf = open(os.path.join(root, "sparse", "0", "points3D.bin"), "rb").read()
    (n,), off = struct.unpack_from("<Q", buf, 0), 8
    rec = np.dtype([("id", "<u8"), ("xyz", "<f8", 3), ("rgb", "u1", 3), ("err", "<f8"),
                    ("tlen", "<u8")])
    xyz = np.empty((n, 3), dtype=np.float32)
    rgb = np.empty((n, 3), dtype=np.float32)
    for i in range(n):
        r = np.frombuffer(buf, dtype=rec, count=1, offset=off)[0]
        xyz[i] = r["xyz"]
        rgb[i] = r["rgb"]
        off += rec.itemsize + 8 * int(r["tlen"])                     # skip the track
    rgb /= 255.0
    if max_pts and n > max_pts:
        sel = np.random.default_rng(0).choice(n, max_pts, replace=False)
        xyz, rgb = xyz[sel], rgb[sel]
    return xyz, rgb
