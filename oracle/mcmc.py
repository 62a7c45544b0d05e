"""Oracle: fixed-count MCMC density control on the [G,14] parameter block.

Test infrastructure only (see oracle/__init__.py).

Restates
  spike/mcmc.py:13-15   op_sigmoid(x, k=100, x0=0.995): the near-dead gate
  spike/mcmc.py:18-22   reg_loss = lambda_o mean(sigmoid(op)) + lambda_s mean(exp(log_scales));
                        its gradient as the device step adds it before Adam
                        (tools/resident_traced.py:732-738)
  spike/mcmc.py:25-34   add_sgld_noise: means += (R(q) diag(s) eps) * op_sigmoid(1-o) * noise_lr*lr
  spike/mcmc.py:41-77   relocate: dead = o < thr (ascending index), one live target per dead slot
                        sampled with probability o / sum(o) (with replacement), target opacity
                        split o_t / (n_t + 1) clamped to [1e-6, 1-1e-6], the dead slot copies the
                        target (means + offset * N(0, 1)) with the split opacity
  spike/mcmc.py:80-93   reset_adam_state: Adam moments of the touched slots (dead and targets)
                        zeroed

The random draws are inputs here (eps, the per-dead uniforms and offsets): the device draws
them from Philox (oracle/rng.py), and the tests hand the same numbers to these functions.
"""
import torch

from . import geometry


def op_sigmoid(x, k=100.0, x0=0.995):
    return torch.sigmoid(k * (x - x0))


def reg_loss(P, lambda_o, lambda_s):
    o = torch.sigmoid(P[:, 13])
    s = torch.exp(P[:, 7:10])
    return lambda_o * o.abs().mean() + lambda_s * s.abs().mean()


def reg_grad(P, lambda_o, lambda_s):
    """d reg_loss / dP [G,14]."""
    Pg = P.detach().clone().requires_grad_(True)
    reg_loss(Pg, lambda_o, lambda_s).backward()
    return Pg.grad.detach()


def sgld_noise(P, lr_means, noise_lr, eps):
    """The noise add_sgld_noise adds to the means for standard normals eps [G,3]."""
    o = torch.sigmoid(P[:, 13])
    s = torch.exp(P[:, 7:10])
    R = geometry.quat_to_rotmat(P[:, 3:7])
    L = R * s[:, None, :]
    w = op_sigmoid(1.0 - o) * (noise_lr * lr_means)
    return torch.einsum("gij,gj->gi", L, eps) * w[:, None]


def _logit(p):
    return torch.log(p / (1.0 - p))


def classify(P, dead_thr):
    o = torch.sigmoid(P[:, 13])
    dead = torch.where(o < dead_thr)[0]
    alive = torch.where(o >= dead_thr)[0]
    return o, dead, alive


def pick_targets(o, alive, u):
    """Inverse-CDF multinomial over the live gaussians in ascending index order: for each
    uniform u in (0, 1), the first live j whose inclusive opacity prefix sum exceeds u * total."""
    w = o[alive].double()
    cdf = torch.cumsum(w, 0)
    x = u.double() * cdf[-1]
    j = torch.searchsorted(cdf, x, right=True).clamp(max=alive.numel() - 1)
    return alive[j]


def relocate(P, m, v, dead, targets, offsets, rest=None, rest_m=None, rest_v=None):
    """In place on P [G,14] (+ SH rest [G,15,3]); dead slots in ascending order, one target and
    one offset [3] per dead slot.  Returns the touched indices (dead and targets)."""
    if dead.numel() == 0:
        return dead
    o = torch.sigmoid(P[:, 13])
    uniq, counts = torch.unique(targets, return_counts=True)
    n_at = torch.zeros(P.shape[0], dtype=torch.long)
    n_at[uniq] = counts + 1
    new_o = (o / n_at.clamp(min=1).to(o.dtype)).clamp(1e-6, 1 - 1e-6)
    new_op = _logit(new_o)
    src = P[targets].clone()
    P[dead] = src
    P[dead, 0:3] = src[:, 0:3] + offsets.to(P.dtype)
    P[dead, 13] = new_op[targets]
    P[uniq, 13] = new_op[uniq]
    if rest is not None:
        rest[dead] = rest[targets].clone()
    touched = torch.unique(torch.cat([dead, uniq]))
    for t in (m, v, rest_m, rest_v):
        if t is not None:
            t[touched] = 0
    return touched
