"""Oracle: Adam over the [G,14] parameter block with a per-column learning rate.

Test infrastructure only (see oracle/__init__.py).

Restates the fused device Adam of tools/resident_traced.py:478-490 (B1, B2, EPS at :92):
    m <- b1 m + (1-b1) g ;  v <- b2 v + (1-b2) g^2
    p <- p - (lr/bc1) * m / (sqrt(v)/sqrt(bc2) + eps),   bc_i = 1 - b_i^t
which is torch.optim.Adam's update (spike/train.py:19), used here as the cross-check.
"""
import math

import torch

B1, B2, EPS = 0.9, 0.999, 1e-8


def adam_step(p, m, v, g, lr, t, b1=B1, b2=B2, eps=EPS):
    """One in-place Adam step at step number t (1-based).  lr broadcasts over rows ([14])."""
    bc1, bc2 = 1.0 - b1 ** t, 1.0 - b2 ** t
    m.mul_(b1).add_((1.0 - b1) * g)
    v.mul_(b2).add_((1.0 - b2) * g * g)
    p.sub_((lr / bc1) * m / (v.sqrt() / math.sqrt(bc2) + eps))
    return p, m, v


def torch_adam_reference(p0, grads, lr, b1=B1, b2=B2, eps=EPS):
    """Run torch.optim.Adam on a copy of p0 (one param group per column) over a list of grads."""
    cols = [p0[:, j].clone().requires_grad_(True) for j in range(p0.shape[1])]
    opt = torch.optim.Adam([{"params": [c], "lr": float(lr[j])} for j, c in enumerate(cols)],
                           betas=(b1, b2), eps=eps, foreach=False)
    for g in grads:
        for j, c in enumerate(cols):
            c.grad = g[:, j].clone()
        opt.step()
    return torch.stack([c.detach() for c in cols], dim=1)
