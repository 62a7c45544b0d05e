"""ttsplat -- the poly-splat / WSR binned 3DGS hot path on MI355X (gfx950).

Host side in Python on PyTorch-ROCm (device memory and streams); every op is a hand-written
HIP kernel in libttsplat.so, called through its C ABI (include/ttsplat.h).  No CPU fallback.

Entry points mirror the reference's:
  ttsplat.binned   TileMap, assign_bins, theta_u_gathered, _operands, DevRenderBinned,
                   render_binned_device, K_POLY        (tools/m4_train_binned.py)
  ttsplat.render   render (dense arm A)                (spike/render.py)
  ttsplat.backward wsr_polysplat, WSRPolySplatHot      (spike/backward.py)
  ttsplat.train    fit, eval_psnr, DEFAULT_LR          (spike/train.py)
  ttsplat.forward / ttsplat.geometry  the reference's tensor helpers (spike/forward.py,
                   spike/geometry.py) and project_params (one HIP kernel)
  ttsplat.loss     loss_fn, psnr                       (spike/metrics.py)
  ttsplat.step     TrainStep: the graph-captured training step (tools/resident_traced.py)
  ttsplat.camera   Camera, look_at_opencv              (spike/camera.py)
  ttsplat.model    GaussianModel in the [G,14] layout  (spike/model.py, resident_traced.py:91)
  ttsplat.scenes   the seeded benchmark configurations
  ttsplat.kernels  typed wrappers over every C entry point
"""
from . import camera, kernels, model, scenes  # noqa: F401

__all__ = ["camera", "kernels", "model", "scenes"]
