"""TEST INFRASTRUCTURE ONLY -- dense Torch references (fp32 by default).

Restates, from the reference's maths, the dense renderers its own tests and
benchmark compare against (every splat evaluated at every pixel, gradients by
autograd):

  dense_reference(early_stop=False)
      benchmarks/benchmark_full_matrix.py:128-152 (``torch_direct``) and
      variants/v8/tests/reference_check.py:15-50
  dense_reference(early_stop=True)
      variants/v8/tests/reference_check.py:53-104 (``saturating_reference``):
      a splat only contributes while T > transmittance_threshold, which is
      the kernels' early stop
  project_pinhole_reference
      variants/v9_project3d_train/torch_gsplat_bridge_v9_project3d_train/
      rasterize.py:288-358

Used by tests/ and bench.py's cpu_baseline leg only.
"""
from __future__ import annotations

import torch


def dense_reference(means2d, conics, colors, opacities, depths, height, width, *, background=(0.0, 0.0, 0.0),
                    alpha_threshold=1.0 / 255.0, max_alpha=0.99, early_stop=False, transmittance_threshold=1e-4,
                    x0=0, y0=0):
    """[G,..] -> [H,W,3] or [B,G,..] -> [B,H,W,3].  Output pixel (y, x) of image b is pixel
    (y0 + y, x0 + x) of a larger image, centre (x0 + x + 0.5, y0 + y + 0.5): x0 / y0 are ints or
    int sequences of length B (one crop origin per image), and a crop is evaluated exactly as in
    the whole image.  The images of the batch are evaluated together, each with the same
    operations in the same order as alone."""
    squeeze = means2d.ndim == 2
    if squeeze:
        means2d, conics, colors, opacities, depths = (t.unsqueeze(0) for t in
                                                      (means2d, conics, colors, opacities, depths))
    dt, dev = means2d.dtype, means2d.device
    Bn = means2d.shape[0]
    bg = torch.tensor(background, dtype=dt, device=dev)
    ox = torch.as_tensor(x0, dtype=dt, device=dev).reshape(-1, 1, 1)
    oy = torch.as_tensor(y0, dtype=dt, device=dev).reshape(-1, 1, 1)
    ys = torch.arange(height, dtype=dt, device=dev).reshape(1, -1, 1)
    xs = torch.arange(width, dtype=dt, device=dev).reshape(1, 1, -1)
    # integer-valued floats below 2^24: (origin + index) + 0.5 is exact
    yy = ((ys + oy) + 0.5).expand(-1, height, width)
    xx = ((xs + ox) + 0.5).expand(-1, height, width)
    perm = torch.argsort(depths.detach(), dim=1, stable=True)

    def gather(t):
        if t.ndim == 2:
            return torch.gather(t, 1, perm)
        return torch.gather(t, 1, perm[..., None].expand(-1, -1, t.shape[-1]))

    m, q, c, o = gather(means2d), gather(conics), gather(colors), gather(opacities)
    out = torch.zeros(Bn, height, width, 3, dtype=dt, device=dev)
    T = torch.ones(Bn, height, width, dtype=dt, device=dev)
    for i in range(m.shape[1]):
        dx = xx - m[:, i, 0, None, None]
        dy = yy - m[:, i, 1, None, None]
        power = -0.5 * (q[:, i, 0, None, None] * dx * dx + 2.0 * q[:, i, 1, None, None] * dx * dy
                        + q[:, i, 2, None, None] * dy * dy)
        alpha = torch.clamp(o[:, i, None, None] * torch.exp(power), max=max_alpha)
        keep = (power <= 0.0) & (alpha >= alpha_threshold)
        if early_stop:
            keep = keep & (T > transmittance_threshold)
        alpha = torch.where(keep, alpha, torch.zeros_like(alpha))
        out = out + (T * alpha)[..., None] * c[:, i, None, None, :]
        T = T * (1.0 - alpha)
    out = out + T[..., None] * bg
    return out[0] if squeeze else out


def quat_to_rotmat(quats):
    """Rotation matrix of an (r,i,j,k) quaternion, not normalised."""
    r, i, j, k = quats.unbind(-1)
    R = torch.stack([
        1 - 2 * (j * j + k * k), 2 * (i * j - r * k), 2 * (i * k + r * j),
        2 * (i * j + r * k), 1 - 2 * (i * i + k * k), 2 * (j * k - r * i),
        2 * (i * k - r * j), 2 * (j * k + r * i), 1 - 2 * (i * i + j * j),
    ], dim=-1)
    return R.reshape(*quats.shape[:-1], 3, 3)


def project_pinhole_reference(means3d, scales, quats, opacities, camera_to_world, camera_params, near_plane=1e-4):
    """Batched [B,G,..] pinhole projection; returns (means2d, conics, opacities, depths)."""
    R = quat_to_rotmat(quats)
    M = R * scales[..., None, :]
    cov3d = M @ M.transpose(-1, -2)
    Rcw = camera_to_world[:, :3, :3]
    t = camera_to_world[:, :3, 3]
    xc = (means3d - t[:, None, :]) @ Rcw
    covc = Rcw.transpose(1, 2).unsqueeze(1) @ cov3d @ Rcw.unsqueeze(1)
    x, y, z = xc[..., 0], xc[..., 1], xc[..., 2]
    front = z > near_plane
    zs = torch.where(front, torch.clamp(z, min=near_plane), torch.ones_like(z))
    xp = torch.where(front, x, torch.zeros_like(x))
    yp = torch.where(front, y, torch.zeros_like(y))
    fx, fy, cx, cy = (camera_params[:, i:i + 1] for i in range(4))
    zero = torch.zeros_like(zs)
    J = torch.stack([
        torch.stack([fx / zs, zero, -(fx * xp) / (zs * zs)], dim=-1),
        torch.stack([zero, fy / zs, -(fy * yp) / (zs * zs)], dim=-1),
    ], dim=-2)
    cov2d = J @ covc @ J.transpose(-1, -2)
    c00 = cov2d[..., 0, 0] + 0.3
    c01 = cov2d[..., 0, 1]
    c11 = cov2d[..., 1, 1] + 0.3
    det = torch.clamp(c00 * c11 - c01 * c01, min=1e-6)
    conics = torch.stack([c11 / det, -c01 / det, c00 / det], dim=-1)
    means2d = torch.stack([(fx * xp) / zs + cx, (fy * yp) / zs + cy], dim=-1)
    opac = torch.where(front, opacities, torch.zeros_like(opacities))
    return means2d, conics, opac, z
