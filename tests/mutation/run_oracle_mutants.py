"""Mutation check of the oracle (CPU): plant one mistake at a time in a copy of the repository and
run the CPU test suite on that copy.  Every mistake marked "fails" must make at least one test
fail; "convention" marks a choice of this library's own that only the device parity tests fix
(the Philox counter layout and Box-Muller output order), "no-op" an edit that changes no result
(a flip of the symmetric SSIM window, a one-ulp change of a constant).  The working tree is never
modified.  Not collected by pytest (a full run is ~100 suite runs): run it by hand.

Usage: python tests/mutation/run_oracle_mutants.py [-j WORKERS] [-k SUBSTRING]
Exit status 1 if a mistake marked "fails" passes every test.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
COPY = ("oracle", "tests", "tt-splat_amd", "include", "bench.py", "__graft_entry__.py")

# (file, text, replacement, expected): one mistake each
MUTANTS = [
    ('oracle/splat.py',
     'tq = torch.stack([a, c, 2 * b,',
     'tq = torch.stack([a, c, b,', 'fails'),
    ('oracle/splat.py',
     '-2 * (b * mx + c * my),',
     '-2 * (b * my + c * mx),', 'fails'),
    ('oracle/splat.py',
     'tu = tq * (-1.0 / k)',
     'tu = tq * (1.0 / k)', 'fails'),
    ('oracle/splat.py',
     'torch.stack([px * px, py * py, px * py, px, py, torch.ones_like(px)], dim=-1)',
     'torch.stack([px * px, py * py, px * px, px, py, torch.ones_like(px)], dim=-1)', 'fails'),
    ('oracle/splat.py',
     'w = (1.0 - Q / k).clamp(min=0.0) ** 2',
     'w = (1.0 - Q / k).clamp(min=0.0)', 'fails'),
    ('oracle/splat.py',
     'return (W @ color + w_b * c_b[None, :]) / (W.sum(dim=1, keepdim=True) + w_b)',
     'return (W @ color + w_b * c_b[None, :]) / (W.sum(dim=1, keepdim=True))', 'fails'),
    ('oracle/loss.py',
     'C1 = 0.01 ** 2',
     'C1 = 0.02 ** 2', 'fails'),
    ('oracle/loss.py',
     'SIGMA = 1.5',
     'SIGMA = 1.4', 'fails'),
    ('oracle/loss.py',
     'return (1.0 - lambda_ssim) * l1 + lambda_ssim * (1.0 - s)',
     'return lambda_ssim * l1 + (1.0 - lambda_ssim) * (1.0 - s)', 'fails'),
    ('oracle/loss.py',
     'return ((2 * fx * fy + C1) * (2 * sxy + C2)) / ((fx * fx + fy * fy + C1) * (sx + sy + C2))',
     'return ((2 * fx * fy + C1) * (2 * sxy + C2)) / ((fx * fx + fy * fy + C1) * (sx + sy + C1))', 'fails'),
    ('oracle/binning.py',
     '    cx = ((tiles % tmap.ntx).float() + 0.5) * S',
     '    cx = ((tiles % tmap.ntx).float() + 0.0) * S', 'fails'),
    ('oracle/binning.py',
     '    return (dx * dx + dy * dy).long().clamp(0, span - 1)',
     '    return (dx * dx + dy * dy).long().clamp(0, span - 2)', 'fails'),
    ('oracle/binning.py',
     '    gx = (mu2d[:, 0] / S).floor().long().clamp(0, tmap.ntx - 1)',
     '    gx = (mu2d[:, 0] / S).round().long().clamp(0, tmap.ntx - 1)', 'fails'),
    ('oracle/adam.py',
     '    bc1, bc2 = 1.0 - b1 ** t, 1.0 - b2 ** t',
     '    bc1, bc2 = 1.0 - b1 ** (t + 1), 1.0 - b2 ** t', 'fails'),
    ('oracle/adam.py',
     '    p.sub_((lr / bc1) * m / (v.sqrt() / math.sqrt(bc2) + eps))',
     '    p.sub_((lr / bc1) * m / (v.sqrt() / math.sqrt(bc2) + 10 * eps))', 'fails'),
    ('oracle/adam.py',
     '    v.mul_(b2).add_((1.0 - b2) * g * g)',
     '    v.mul_(b2).add_((1.0 - b2) * g.abs())', 'fails'),
    ('oracle/geometry.py',
     '    mu2d = torch.stack([fx * xc / z + cx, fy * yc / z + cy], dim=-1)',
     '    mu2d = torch.stack([fx * xc / z + cx, fx * yc / z + cy], dim=-1)', 'fails'),
    ('oracle/geometry.py',
     '    s11 = S2[:, 1, 1] + blur_eps',
     '    s11 = S2[:, 1, 1] + 0.5 * blur_eps', 'fails'),
    ('oracle/geometry.py',
     '    conic = torch.stack([s11 / det, -s01 / det, s00 / det], dim=-1)',
     '    conic = torch.stack([s11 / det, s01 / det, s00 / det], dim=-1)', 'fails'),
    ('oracle/geometry.py',
     'torch.stack([zero, fy / z, -fy * yc / zz], -1)',
     'torch.stack([zero, fy / z, -fy * xc / zz], -1)', 'fails'),
    ('oracle/binning.py',
     '            j += 1\n',
     '            j += 2\n', 'fails'),
    ('oracle/binning.py',
     '    for dy in range(-R, R + 1):\n        for dx in range(-R, R + 1):\n            tx, ty = gx + dx',
     '    for dx in range(-R, R + 1):\n        for dy in range(-R, R + 1):\n            tx, ty = gx + dx', 'fails'),
    ('oracle/binning.py',
     '    keepm = rank < K\n',
     '    keepm = rank <= K - 2\n', 'fails'),
    ('oracle/binning.py',
     '    key = tiles * span + quantised_dist2(mu2d, tiles, gs, tmap, span)\n    order',
     '    key = tiles * (span - 1) + quantised_dist2(mu2d, tiles, gs, tmap, span)\n    order', 'fails'),
    ('oracle/binning.py',
     '            j = (dy + R) * (2 * R + 1) + (dx + R)',
     '            j = (dx + R) * (2 * R + 1) + (dy + R)', 'fails'),
    ('oracle/binning.py',
     '            q = min(max(int(d2), 0), span - 1)',
     '            q = min(max(int(round(d2)), 0), span - 1)', 'fails'),
    ('oracle/binning.py',
     '        lx = (p % S).to(dtype) + 0.5',
     '        lx = (p % S).to(dtype) + 0.0', 'fails'),
    ('oracle/binning.py',
     '        self.Phi = torch.stack([lx * lx, ly * ly, lx * ly, lx, ly, torch.ones_like(lx)], dim=-1)',
     '        self.Phi = torch.stack([lx * lx, ly * ly, lx * ly, ly, lx, torch.ones_like(lx)], dim=-1)', 'fails'),
    ('oracle/mcmc.py',
     '    n_at[uniq] = counts + 1',
     '    n_at[uniq] = counts', 'fails'),
    ('oracle/mcmc.py',
     '    new_o = (o / n_at.clamp(min=1).to(o.dtype)).clamp(1e-6, 1 - 1e-6)',
     '    new_o = (o / n_at.clamp(min=1).to(o.dtype)).clamp(1e-3, 1 - 1e-6)', 'fails'),
    ('oracle/mcmc.py',
     '    j = torch.searchsorted(cdf, x, right=True)',
     '    j = torch.searchsorted(cdf, x, right=False)', 'fails'),
    ('oracle/mcmc.py',
     '    return lambda_o * o.abs().mean() + lambda_s * s.abs().mean()',
     '    return lambda_o * o.abs().mean() + lambda_s * s.abs().sum() / P.shape[0]', 'fails'),
    ('oracle/mcmc.py',
     '    w = op_sigmoid(1.0 - o) * (noise_lr * lr_means)',
     '    w = op_sigmoid(o) * (noise_lr * lr_means)', 'fails'),
    ('oracle/mcmc.py',
     '    L = R * s[:, None, :]',
     '    L = R * s[:, :, None]', 'fails'),
    ('oracle/mcmc.py',
     '    touched = torch.unique(torch.cat([dead, uniq]))',
     '    touched = dead', 'fails'),
    ('oracle/mcmc.py',
     '    P[dead, 0:3] = src[:, 0:3] + offsets.to(P.dtype)',
     '    P[dead, 0:3] = src[:, 0:3] - offsets.to(P.dtype)', 'fails'),
    ('oracle/mcmc.py',
     '    dead = torch.where(o < dead_thr)[0]',
     '    dead = torch.where(o <= dead_thr)[0]', 'fails'),
    ('oracle/mcmc.py',
     'def op_sigmoid(x, k=100.0, x0=0.995):',
     'def op_sigmoid(x, k=100.0, x0=0.99):', 'fails'),
    ('oracle/sh.py',
     '        b += [-C1 * y, C1 * z, -C1 * x]',
     '        b += [C1 * y, C1 * z, -C1 * x]', 'fails'),
    ('oracle/sh.py',
     'C3[3] * z * (2 * zz - 3 * xx - 3 * yy)',
     'C3[3] * z * (2 * zz - 3 * xx - 2 * yy)', 'fails'),
    ('oracle/sh.py',
     '    return -(R_v.transpose(-1, -2) @ t_v)',
     '    return -(R_v @ t_v)', 'fails'),
    ('oracle/sh.py',
     '    return (r + 0.5).clamp(min=0.0)',
     '    return (r + 0.5).clamp(0.0, 1.0)', 'fails'),
    ('oracle/sh.py',
     '    dirs = (means3d - camera_center(R_v, t_v)[None, :]).detach()',
     '    dirs = (means3d - camera_center(R_v, t_v)[None, :])', 'fails'),
    ('oracle/rng.py',
     'W0, W1 = 0x9E3779B9, 0xBB67AE85',
     'W0, W1 = 0x9E3779B9, 0xBB67AE84', 'fails'),
    ('oracle/rng.py',
     '        + 2.0 ** -25',
     '        + 2.0 ** -24', 'fails'),
    ('oracle/rng.py',
     '    return np.stack([r0 * np.cos(a0), r0 * np.sin(a0), r1 * np.cos(a1)], axis=-1)',
     '    return np.stack([r0 * np.sin(a0), r0 * np.cos(a0), r1 * np.cos(a1)], axis=-1)', 'convention'),
    ('oracle/rng.py',
     '    r1 = np.sqrt(-2.0 * np.log(u[..., 2]))',
     '    r1 = np.sqrt(-2.0 * np.log(u[..., 3]))', 'fails'),
    ('oracle/rng.py',
     '    ctr = np.stack([index, z + np.uint64(step & MASK), z + np.uint64(tag), z], axis=-1)',
     '    ctr = np.stack([index, z + np.uint64(tag), z + np.uint64(step & MASK), z], axis=-1)', 'convention'),
    ('oracle/rng.py',
     '    return uniform(w[:3]).astype(np.float32)',
     '    return uniform(w[1:4]).astype(np.float32)', 'fails'),
    ('oracle/splat.py',
     '    Q0 = a * mx * mx + 2.0 * b * mx * my + c * my * my',
     '    Q0 = a * mx * mx + b * mx * my + c * my * my', 'fails'),
    ('oracle/splat.py',
     '                      2.0 * (a * mx + b * my) * ik, 2.0 * (b * mx + c * my) * ik,',
     '                      2.0 * (a * mx + b * my) * ik, 2.0 * (b * my + c * mx) * ik,', 'fails'),
    ('oracle/splat.py',
     '    h = torch.sigmoid(-softz_beta * (z[None, :] - zstar))',
     '    h = torch.sigmoid(softz_beta * (z[None, :] - zstar))', 'fails'),
    ('oracle/splat.py',
     '    a = W.clamp(0.0, 1.0 - 1e-4)',
     '    a = W.clamp(0.0, 1.0 - 1e-2)', 'fails'),
    ('oracle/splat.py',
     '    return C_avg * (1.0 - R) + c_b[None, :] * R',
     '    return C_avg * R + c_b[None, :] * (1.0 - R)', 'fails'),
    ('oracle/splat.py',
     '    den = w @ oc + w_b\n',
     '    den = w @ oc + 2 * w_b\n', 'fails'),
    ('oracle/splat.py',
     '    theta = theta * valid[:, None, :].to(P.dtype)\n',
     '', 'fails'),
    ('oracle/geometry.py',
     '    return (0.5 + C0 * color_dc).clamp(min=0.0)',
     '    return (0.5 + C0 * color_dc).clamp(0.0, 1.0)', 'fails'),
    ('oracle/geometry.py',
     '        keo = keo * torch.sigmoid(depth_bt[0] * (depth_bt[1] - z))',
     '        keo = keo * torch.sigmoid(depth_bt[0] * (z - depth_bt[1]))', 'fails'),
    ('oracle/geometry.py',
     '        z = depth if depth_zgrad else depth.detach()',
     '        z = depth', 'fails'),
    ('oracle/pipeline.py',
     '        adam.adam_step(P, m, v, g, lr, t)',
     '        adam.adam_step(P, m, v, g, lr, t + 1)', 'fails'),
    ('oracle/loss.py',
     '    if w % 2 == 0:\n        w -= 1',
     '    if w % 2 == 0:\n        w += 1', 'fails'),
    ('oracle/loss.py',
     '    return max(w, 3)',
     '    return max(w, 1)', 'fails'),
    ('oracle/loss.py',
     '    x = pred.clamp(0.0, 1.0).permute(2, 0, 1)',
     '    x = pred.permute(2, 0, 1)', 'fails'),
    ('oracle/loss.py',
     '    l1 = (pred - gt).abs().mean()',
     '    l1 = (pred.clamp(0.0, 1.0) - gt).abs().mean()', 'fails'),
    ('oracle/loss.py',
     '    sx = gaussian_filter(x * x, g) - fx * fx',
     '    sx = gaussian_filter(x * x, g) - fx * fy', 'fails'),
    ('oracle/loss.py',
     '    t = F.conv2d(t, w.view(1, 1, 1, -1).expand(C, 1, 1, -1), groups=C)',
     '    t = F.conv2d(t, w.flip(0).view(1, 1, 1, -1).expand(C, 1, 1, -1), groups=C)', 'no-op'),
    ('oracle/loss.py',
     '        M[o, o:o + win] = g',
     '        M[o, o:o + win] = g.flip(0)', 'no-op'),
    ('oracle/loss.py',
     '    c = torch.arange(win, dtype=torch.float64) - win // 2',
     '    c = torch.arange(win, dtype=torch.float64) - win // 2 + 0.5', 'fails'),
    ('oracle/loss.py',
     '    y = gt.clamp(0.0, 1.0).permute(2, 0, 1)',
     '    y = gt.permute(2, 0, 1)', 'fails'),
    ('oracle/geometry.py',
     '    keep = depth > near',
     '    keep = depth >= near', 'fails'),
    ('oracle/geometry.py',
     '    z = depth.clamp(min=near)',
     '    z = depth.clamp(min=1e-6)', 'fails'),
    ('oracle/geometry.py',
     '    S_cam = R_v @ cov_w @ R_v.T',
     '    S_cam = R_v.T @ cov_w @ R_v', 'fails'),
    ('oracle/geometry.py',
     '    mu_cam = means3d @ R_v.T + t_v',
     '    mu_cam = means3d @ R_v + t_v', 'fails'),
    ('oracle/geometry.py',
     '    det = (s00 * s11 - s01 * s01).clamp(min=1e-12)',
     '    det = (s00 * s11 + s01 * s01).clamp(min=1e-12)', 'fails'),
    ('oracle/geometry.py',
     '    q = q / q.norm(dim=-1, keepdim=True).clamp(min=1e-12)',
     '    q = q', 'fails'),
    ('oracle/geometry.py',
     '        (2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)),',
     '        (2 * (x * y - w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)),', 'fails'),
    ('oracle/geometry.py',
     '    return (R * (scales * scales)[..., None, :]) @ R.transpose(-1, -2)',
     '    return (R * scales[..., None, :]) @ R.transpose(-1, -2)', 'fails'),
    ('oracle/geometry.py',
     '    right = torch.linalg.cross(torch.as_tensor(up, dtype=dtype), fwd)',
     '    right = torch.linalg.cross(fwd, torch.as_tensor(up, dtype=dtype))', 'fails'),
    ('oracle/geometry.py',
     '    return cols + 0.5, rows + 0.5',
     '    return cols, rows', 'fails'),
    ('oracle/geometry.py',
     '    f = 0.5 * W / math.tan(math.radians(fov_deg) / 2.0)',
     '    f = 0.5 * H / math.tan(math.radians(fov_deg) / 2.0)', 'fails'),
    ('oracle/geometry.py',
     '    keo = keep.to(dt) * torch.sigmoid(op)',
     '    keo = torch.sigmoid(op)', 'fails'),
    ('oracle/splat.py',
     '    return a * dx * dx + 2 * b * dx * dy + c * dy * dy',
     '    return a * dx * dx + b * dx * dy + c * dy * dy', 'fails'),
    ('oracle/splat.py',
     '        w = w * keep[None, :].to(w.dtype)',
     '        w = w', 'fails'),
    ('oracle/splat.py',
     '    w = torch.relu(torch.einsum("pf,tfg->tpg", Phi, theta)) ** 2',
     '    w = torch.einsum("pf,tfg->tpg", Phi, theta) ** 2', 'fails'),
    ('oracle/splat.py',
     '    img = img.index_copy(0, tmap.gidx, C.reshape(-1, C.shape[-1]))',
     '    img = C.reshape(-1, C.shape[-1]).clone()', 'fails'),
    ('oracle/splat.py',
     '    mx = mu_t[..., 0] - origins[:, None, 0]',
     '    mx = mu_t[..., 0] - origins[:, None, 1]', 'fails'),
    ('oracle/splat.py',
     '    zstar = (W0 @ z[:, None]) / den0',
     '    zstar = (W0 @ z[:, None]) / W0.shape[1]', 'fails'),
    ('oracle/splat.py',
     '    R = torch.exp(torch.log1p(-a).sum(dim=1, keepdim=True))',
     '    R = torch.exp(torch.log1p(-a).mean(dim=1, keepdim=True))', 'fails'),
    ('oracle/splat.py',
     '    C_avg = (W @ color) / den',
     '    C_avg = (W @ color) / (den + 1.0)', 'fails'),
    ('oracle/splat.py',
     '    col = pr["color_o"][idx] * vf',
     '    col = pr["color_o"][idx]', 'fails'),
    ('oracle/sh.py',
     'C0 = 0.28209479177387814',
     'C0 = 0.2820947917738781', 'no-op'),
    ('oracle/sh.py',
     'C2[2] * (2.0 * zz - xx - yy)',
     'C2[2] * (2.0 * zz - xx + yy)', 'fails'),
    ('oracle/sh.py',
     'C3[6] * x * (xx - 3 * yy)',
     'C3[6] * x * (3 * xx - yy)', 'fails'),
    ('oracle/sh.py',
     '    d = dirs / dirs.norm(dim=-1, keepdim=True).clamp(min=1e-12)',
     '    d = dirs', 'fails'),
    ('oracle/sh.py',
     '    coeffs = torch.cat([color_dc[:, None, :], color_rest], dim=1)\n    return eval_sh_color',
     '    coeffs = torch.cat([color_rest[:, :1], color_dc[:, None, :], color_rest[:, 1:]], dim=1)\n    return eval_sh_color', 'fails'),
    ('oracle/adam.py',
     '    m.mul_(b1).add_((1.0 - b1) * g)',
     '    m.mul_(b1).add_(g)', 'fails'),
]


def make_copy(dst):
    for name in COPY:
        src = os.path.join(ROOT, name)
        if os.path.isdir(src):
            shutil.copytree(src, os.path.join(dst, name),
                            ignore=shutil.ignore_patterns("__pycache__", "_build", "mutation"))
        else:
            shutil.copy2(src, os.path.join(dst, name))


def suite_passes(copy_dir):
    """The CPU suite on a copy (test_citations.py needs the git checkout, and checks only the
    citations' line numbers)."""
    env = dict(os.environ, OMP_NUM_THREADS="2")
    r = subprocess.run([sys.executable, "-m", "pytest", "tests", "-x", "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider", "--ignore=tests/test_citations.py"],
                       cwd=copy_dir, env=env, capture_output=True, text=True, timeout=900)
    return r.returncode == 0


def run_one(copy_dir, mutant):
    path, old, new, _ = mutant
    target = os.path.join(copy_dir, path)
    original = open(target).read()
    if original.count(old) != 1:
        return "not found"
    open(target, "w").write(original.replace(old, new))
    try:
        return "passes" if suite_passes(copy_dir) else "fails"
    finally:
        open(target, "w").write(original)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=4, help="parallel workers (one repository copy each)")
    ap.add_argument("-k", default="", help="only mutants whose file or text contains this")
    args = ap.parse_args()
    todo = [m for m in MUTANTS if args.k in m[0] or args.k in m[1]]
    with tempfile.TemporaryDirectory() as tmp:
        copies = []
        for w in range(max(1, args.j)):
            d = os.path.join(tmp, f"w{w}")
            os.makedirs(d)
            make_copy(d)
            copies.append(d)
        if not suite_passes(copies[0]):
            sys.exit("the CPU suite fails on an unmodified copy: fix that first")
        chunks = [todo[w::len(copies)] for w in range(len(copies))]

        def worker(w):
            return [(m, run_one(copies[w], m)) for m in chunks[w]]

        with cf.ThreadPoolExecutor(len(copies)) as ex:
            results = [r for part in ex.map(worker, range(len(copies))) for r in part]
    bad = 0
    for (path, old, _, expected), got in results:
        ok = got == "fails" if expected == "fails" else got in ("fails", "passes")
        bad += not ok
        flag = "" if ok else "   <-- not caught"
        print(f"{got:9s} {expected:10s} {path}: {old.strip()[:70]}{flag}")
    n_fail = sum(1 for _, got in results if got == "fails")
    print(f"{n_fail} of {len(results)} mistakes fail a test; {bad} expected to fail did not")
    sys.exit(1 if bad else 0)


if __name__ == "__main__":
    main()
