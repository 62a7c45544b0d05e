"""GPU-resident gaussian set in the [G,14] layout of the device trainer.

The reference model (spike/model.py:16-95) keeps separate tensors; the device trainer keeps the
14 per-gaussian columns mx,my,mz, qw,qx,qy,qz, lx,ly,lz, cr,cg,cb, op in one block
(tools/resident_traced.py:91, :233-235).  `GaussianModel` holds that block and exposes the
reference attribute names as views, so code written against spike.model reads it unchanged.
"""
import torch

PN = ("mx", "my", "mz", "qw", "qx", "qy", "qz", "lx", "ly", "lz", "cr", "cg", "cb", "op")


class GaussianModel:
    def __init__(self, params, w_b_raw=-3.0, c_b=(1.0, 1.0, 1.0)):
        if params.dim() != 2 or params.shape[1] != 14:
            raise ValueError(f"params must be [G,14], got {tuple(params.shape)}")
        self.params = params.float().contiguous()
        dev = self.params.device
        self.w_b_raw = torch.tensor(float(w_b_raw), device=dev)
        self.c_b = torch.as_tensor(c_b, dtype=torch.float32, device=dev)

    @classmethod
    def from_reference(cls, model, device="cuda"):
        """Pack a spike-style model (separate tensors) into the [G,14] block."""
        P = torch.cat([model.means3d.detach(), model.quats.detach(), model.log_scales.detach(),
                       model.color_dc.detach(), model.opacity_raw.detach().reshape(-1, 1)], 1)
        return cls(P.to(device), float(model.w_b_raw), model.c_b.detach().cpu())

    @property
    def G(self):
        return self.params.shape[0]

    @property
    def means3d(self):
        return self.params[:, 0:3]

    @property
    def quats(self):
        return self.params[:, 3:7]

    @property
    def log_scales(self):
        return self.params[:, 7:10]

    @property
    def color_dc(self):
        return self.params[:, 10:13]

    @property
    def opacity_raw(self):
        return self.params[:, 13]
