"""Pinhole cameras in the OpenCV convention (spike/camera.py:14-70).

`Camera` keeps the reference's fields (R_v, t_v, fx, fy, cx, cy, H, W).  `device_block()`
packs them into the 16-float camera block the HIP kernels read
(R_v row-major, t_v, fx, fy, cx, cy).
"""
import math

import torch


class Camera:
    """An OpenCV pinhole camera: world->camera R_v[3,3], t_v[3], intrinsics, image size."""

    __slots__ = ("R_v", "t_v", "fx", "fy", "cx", "cy", "H", "W", "_block")

    def __init__(self, R_v, t_v, fx, fy, cx, cy, H, W):
        self.R_v = torch.as_tensor(R_v, dtype=torch.float32).cpu()
        self.t_v = torch.as_tensor(t_v, dtype=torch.float32).cpu()
        self.fx, self.fy, self.cx, self.cy = float(fx), float(fy), float(cx), float(cy)
        self.H, self.W = int(H), int(W)
        self._block = {}

    @property
    def center(self):
        return -self.R_v.T @ self.t_v

    def host_block(self):
        return torch.cat([self.R_v.reshape(-1), self.t_v.reshape(-1),
                          torch.tensor([self.fx, self.fy, self.cx, self.cy])]).float()

    def device_block(self, device="cuda"):
        """[16] fp32 camera block on `device` (cached per device)."""
        key = str(torch.device(device))
        if key not in self._block:
            self._block[key] = self.host_block().to(device)
        return self._block[key]

    def as_dict(self):
        return dict(R_v=self.R_v, t_v=self.t_v, fx=self.fx, fy=self.fy, cx=self.cx, cy=self.cy,
                    H=self.H, W=self.W)


def opengl_c2w_to_opencv_w2c(c2w):
    """OpenGL camera-to-world [4,4] (camera looks down -z, +y up; NeRF-synthetic's
    transform_matrix) -> OpenCV world-to-camera (R_v[3,3], t_v[3]) (spike/camera.py:16-24):
    R_v = (R_c diag(1,-1,-1))^T, t_v = -R_v cam_pos.  Computed in the input's dtype."""
    c2w = torch.as_tensor(c2w)
    R_c, cam_pos = c2w[:3, :3], c2w[:3, 3]
    flip = torch.diag(torch.tensor([1.0, -1.0, -1.0], dtype=c2w.dtype))
    R_v = (R_c @ flip).transpose(-1, -2)
    return R_v, -R_v @ cam_pos


def project_point(p_world, R_v, t_v, fx, fy, cx, cy):
    """Pixel and depth of one world point (spike/camera.py:27-33); z > 0 is in front."""
    p_cam = R_v @ p_world + t_v
    z = p_cam[2]
    return torch.stack([fx * p_cam[0] / z + cx, fy * p_cam[1] / z + cy]), z


def look_at_opencv(eye, target=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0)):
    """World->camera (R_v, t_v) for a camera at `eye` looking at `target` (spike/camera.py:51-63)."""
    eye = torch.as_tensor(eye, dtype=torch.float32)
    fwd = torch.as_tensor(target, dtype=torch.float32) - eye
    fwd = fwd / fwd.norm()
    right = torch.linalg.cross(torch.as_tensor(up, dtype=torch.float32), fwd)
    right = right / right.norm()
    down = torch.linalg.cross(fwd, right)
    R_v = torch.stack([right, down, fwd], dim=0)
    return R_v, -(R_v @ eye)


def pinhole(H, W, eye, fov_deg=50.0, target=(0.0, 0.0, 0.0)):
    """Camera at `eye` looking at `target` with horizontal field of view `fov_deg`
    (fx = fy = 0.5*W/tan(fov/2), principal point at the image centre)."""
    R_v, t_v = look_at_opencv(eye, target)
    f = 0.5 * W / math.tan(math.radians(fov_deg) / 2.0)
    return Camera(R_v, t_v, f, f, W / 2.0, H / 2.0, H, W)
