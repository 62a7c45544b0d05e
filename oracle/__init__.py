"""CPU oracle for the poly-splat / WSR binned 3DGS hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this package: only
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, and
only as the checker (or, for the CPU baseline, as the timed CPU restatement).  The product
path runs on the HIP library and fails loudly when that library is missing.

The oracle restates the reference algorithm in PyTorch-CPU (fp32 by default, fp64 on
request).  Every function cites the reference file:line it follows (paths relative to the
reference checkout).  Gradients are NOT restated by hand: they are torch autograd of the
restated forward, which is what the reference's own manual backward chain was validated
against (tools/geom_bwd.py:173-194, tools/operands_manual.py:118-144,
tools/loss_manual.py:131-147, spike/tests/test_backward.py:36-48).

Modules
  geometry  quat->R, covariance, EWA projection, activations        (spike/geometry.py, spike/forward.py)
  binning   TileMap, assign_bins (reference torch-default order and the stable order)
                                                                    (tools/m4_train_binned.py:60-127)
  splat     theta maps, dense arm-A render, binned render            (spike/forward.py, spike/arms.py,
                                                                     tools/m4_train_binned.py:130-212,
                                                                     tools/bh_views.py:65-71)
  loss      0.8*L1 + 0.2*(1-SSIM), 11-tap gaussian window            (spike/metrics.py, tools/loss_manual.py)
  adam      Adam recurrence                                          (tools/resident_traced.py:478-490)
  pipeline  one binned training step composed from the above         (tools/resident_traced.py:667-744)

Pinning status (how each part is checked, see tests/test_oracle_*.py):
  geometry  reference KATs spike/tests/test_geometry_analytic.py (isotropic conic, depth x4,
            near cull) + manual-chain identities; off-axis EWA against the autograd Jacobian of
            the pinhole map and scipy rotations; the depth weight against its closed form and
            the closed-form gradients of tools/m8_depthweight_oracle.py:7-12.  pinned
  binning   brute force on tiny inputs; invariants; golden fixtures written by the reference's
            own assign_bins (tests/golden/).                                   pinned
  splat     reference KATs spike/tests/test_transform.py, test_toy_1g.py, test_tile_local.py,
            test_backward.py (gradcheck), dense==binned when every splat fits its stencil.
                                                                               pinned
  loss      closed forms (x==y -> SSIM 1, L1 0; constant images; y = a x + b), the window taps
            against exp(-c^2/4.5)/sum, the map against directly summed 2-D window moments, the
            mean over 3 Hout Wout on a non-square image, gradcheck, the banded-matrix form of
            tools/loss_manual.py.  The pytorch_msssim==1.0.0 call in spike/metrics.py:19
            is absent here, so agreement with THAT library's numerics is parity unpinned.
  adam      torch.optim.Adam (present here).                                   pinned
"""
