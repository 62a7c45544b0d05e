"""Oracle: the counter-based random numbers of the device MCMC kernels.

Test infrastructure only (see oracle/__init__.py).

Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
SC'11): 10 rounds of two 32x32->64 multiplies (multipliers 0xD2511F53, 0xCD9E8D57) over a
128-bit counter, the 64-bit key bumped by the Weyl constants (0x9E3779B9, 0xBB67AE85) between
rounds.  The reference draws its MCMC noise from torch's host generator
(spike/mcmc.py:26-34,46-64); a device kernel cannot reproduce that stream, so the device uses
Philox with counter (index, step, stream tag, 0) and key (seed, 0), and this file restates
it with integer arithmetic (bit-exact) so the tests can feed the oracle the same draws.

Conversions (the device's):
  uniform(x) = (x >> 8) * 2^-24 + 2^-25            in (0, 1), 24 bits
  normal pair from (x0, x1): r = sqrt(-2 ln u0), (r cos 2 pi u1, r sin 2 pi u1)   (Box-Muller)

Pinned by tests/test_oracle_mcmc.py: the Philox4x32-10 known-answer vectors of the Random123
distribution, the uniform grid's symmetry about 1/2 and its ends, and the moments of the derived
normals.  The counter word layout (index, step, tag, 0) and the Box-Muller output order are
this library's own conventions, not the reference's (it draws from torch's host generator): no
CPU fact fixes them, and the device parity tests (tests/test_gpu_mcmc.py) hold the device to
this file on them.
"""
import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK = 0xFFFFFFFF

# stream tags (counter word 2) of the device kernels
TAG_SGLD = 1           # SGLD noise on the means
TAG_RELOC_PICK = 2     # relocation: which live gaussian a dead slot copies
TAG_RELOC_OFFSET = 3   # relocation: the position offset of the copy
TAG_BG = 4             # random training background of a view


def philox4x32_10(ctr, key):
    """ctr: uint64 array [..., 4] of 32-bit words; key: [..., 2].  Returns uint64 [..., 4]."""
    c = [np.asarray(ctr[..., i], dtype=np.uint64) & MASK for i in range(4)]
    k0 = np.asarray(key[..., 0], dtype=np.uint64) & MASK
    k1 = np.asarray(key[..., 1], dtype=np.uint64) & MASK
    for r in range(10):
        if r:
            k0 = (k0 + W0) & MASK
            k1 = (k1 + W1) & MASK
        p0 = np.uint64(M0) * c[0]
        p1 = np.uint64(M1) * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return np.stack(c, axis=-1)


def draws(index, step, tag, seed):
    """The 4 words of Philox for counters (index, step, tag, 0), key (seed, 0); index an
    int array."""
    index = np.asarray(index, dtype=np.uint64)
    z = np.zeros_like(index)
    ctr = np.stack([index, z + np.uint64(step & MASK), z + np.uint64(tag), z], axis=-1)
    key = np.stack([z + np.uint64(seed & MASK), z], axis=-1)
    return philox4x32_10(ctr, key)


def uniform(x):
    return (np.asarray(x, dtype=np.uint64) >> np.uint64(8)).astype(np.float64) * 2.0 ** -24 \
        + 2.0 ** -25


def normals3(index, step, tag, seed):
    """Three standard normals per index (two Box-Muller pairs, the fourth value unused)."""
    w = draws(index, step, tag, seed)
    u = uniform(w)
    r0 = np.sqrt(-2.0 * np.log(u[..., 0]))
    r1 = np.sqrt(-2.0 * np.log(u[..., 2]))
    a0 = 2.0 * np.pi * u[..., 1]
    a1 = 2.0 * np.pi * u[..., 3]
    return np.stack([r0 * np.cos(a0), r0 * np.sin(a0), r1 * np.cos(a1)], axis=-1)


def uniform1(index, step, tag, seed):
    """One uniform in (0, 1) per index (word 0)."""
    return uniform(draws(index, step, tag, seed)[..., 0])


def random_bg(view, step, seed):
    """The background colour a random-background training step draws for `view` after `step`
    completed steps: words 0..2 of Philox (view, step, TAG_BG, 0; key (seed, 0)) as uniforms in
    (0, 1), rounded to fp32 (the reference draws torch.rand(3) on the host,
    tools/resident_traced.py:672)."""
    w = draws(np.array([view]), step, TAG_BG, seed)[0]
    return uniform(w[:3]).astype(np.float32)
