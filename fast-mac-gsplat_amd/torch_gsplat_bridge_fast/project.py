"""Pinhole projection of 3D Gaussians (reference: variants/v9_project3d_train/
torch_gsplat_bridge_v9_project3d_train/rasterize.py).

  project_pinhole_gaussians    v9 rasterize.py:544-572
  rasterize_pinhole_gaussians  v9 rasterize.py:958-1003

means3d [G,3]|[B,G,3], scales (linear) same shape, quats [..,4] = (r,i,j,k)
(used as given, not normalised), opacities [G]|[G,1]|[B,G]|[B,G,1];
fx, fy, cx, cy are Python scalars or tensors with 1 or B values;
camera_to_world is None (identity), [4,4] or [B,4,4], row-major, with the
camera axes as the columns of its rotation block.  Gradients flow to
means3d, scales, quats, opacities and (when they require grad) the camera
tensors.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib, _ops
from .rasterize import RasterConfig, _rasterize_batched, _runtime_validate


def _normalize_3d_inputs(means3d, scales, quats, opacities):
    if opacities.ndim >= 1 and opacities.shape[-1:] == (1,):
        opacities = opacities.squeeze(-1)
    if means3d.ndim == 2:
        return means3d.unsqueeze(0), scales.unsqueeze(0), quats.unsqueeze(0), opacities.unsqueeze(0), False
    if means3d.ndim != 3:
        raise ValueError("means3d must have shape [G,3] or [B,G,3]")
    return means3d, scales, quats, opacities, True


def _check_3d_inputs(means3d, scales, quats, opacities) -> None:
    """Checks with the reference's messages (v9 rasterize.py:217-240)."""
    tensors = {"means3d": means3d, "scales": scales, "quats": quats, "opacities": opacities}
    if len({t.device for t in tensors.values()}) != 1:
        raise ValueError("means3d/scales/quats/opacities must be on the same device")
    if means3d.device.type != "cuda":
        raise ValueError("HIP projection inputs must be ROCm device tensors (device type 'cuda')")
    for name, t in tensors.items():
        if t.dtype != torch.float32:
            raise ValueError(f"{name} must be float32")
    if means3d.ndim not in (2, 3) or means3d.shape[-1] != 3:
        raise ValueError("means3d must have shape [G,3] or [B,G,3]")
    if scales.shape != means3d.shape:
        raise ValueError("scales must match means3d shape")
    if quats.shape[:-1] != means3d.shape[:-1] or quats.shape[-1] != 4:
        raise ValueError("quats must have shape [G,4] or [B,G,4]")
    op_shape = opacities.shape[:-1] if opacities.ndim >= 1 and opacities.shape[-1:] == (1,) else opacities.shape
    if op_shape != means3d.shape[:-1]:
        raise ValueError("opacities must have shape [G], [G,1], [B,G], or [B,G,1]")
    if means3d.shape[-2] == 0:
        raise ValueError("at least one Gaussian is required (G >= 1)")


def _normalize_colors(colors, batch_size, gaussians, was_batched):
    if colors.ndim == 2:
        colors_b = colors.unsqueeze(0)
    elif colors.ndim == 3:
        colors_b = colors
    else:
        raise ValueError("colors must have shape [G,3] or [B,G,3]")
    if colors_b.shape != (batch_size, gaussians, 3):
        expected = "[B,G,3]" if was_batched else "[G,3]"
        raise ValueError(f"colors must match Gaussian shape {expected}; got {tuple(colors.shape)}")
    return colors_b


def _camera_scalar_batch(value, batch_size, device, dtype, name):
    if torch.is_tensor(value):
        value = value.to(device=device, dtype=dtype)
        if value.ndim == 0:
            return value.expand(batch_size)
        if value.numel() == batch_size:
            return value.reshape(batch_size)
        raise ValueError(f"{name} must be scalar or have {batch_size} values")
    return torch.full((batch_size,), float(value), device=device, dtype=dtype)


def _camera_to_world_batch(camera_to_world, batch_size, device, dtype):
    if camera_to_world is None:
        return torch.eye(4, device=device, dtype=dtype).unsqueeze(0).expand(batch_size, -1, -1).contiguous()
    camera_to_world = camera_to_world.to(device=device, dtype=dtype)
    if camera_to_world.shape == (4, 4):
        return camera_to_world.unsqueeze(0).expand(batch_size, -1, -1).contiguous()
    if camera_to_world.shape == (batch_size, 4, 4):
        return camera_to_world.contiguous()
    raise ValueError(f"camera_to_world must be [4,4] or [{batch_size},4,4]")


class _ProjectPinholeGaussians(torch.autograd.Function):
    """Autograd wrapper (reference _ProjectPinholeGaussiansV9Project3DTrain, v9 rasterize.py:371-481)."""

    @staticmethod
    def forward(ctx, means3d_b, scales_b, quats_b, opacities_b, c2w_b, camera_params, near_plane: float):
        B, G = means3d_b.shape[:2]
        meta = _lib.make_project_meta(B, G, near_plane)
        flat = (means3d_b.detach().reshape(-1, 3).contiguous(), scales_b.detach().reshape(-1, 3).contiguous(),
                quats_b.detach().reshape(-1, 4).contiguous(), opacities_b.detach().reshape(-1).contiguous(),
                c2w_b.detach().contiguous(), camera_params.detach().contiguous())
        m2, cq, op, dp = _ops.project_forward(meta, *flat)
        ctx.save_for_backward(*flat)
        ctx.meta = meta
        ctx.shape = (B, G)
        return m2.view(B, G, 2), cq.view(B, G, 3), op.view(B, G), dp.view(B, G)

    @staticmethod
    def backward(ctx, g_m2, g_cq, g_op, g_dp):
        means3d, scales, quats, opacities, c2w, cam = ctx.saved_tensors
        B, G = ctx.shape
        if not any(ctx.needs_input_grad[:6]):
            return (None,) * 7
        dev = means3d.device

        def z(g, shape):
            return torch.zeros(shape, dtype=torch.float32, device=dev) if g is None else g.reshape(shape).contiguous()

        # a depth gradient of None (the rasterizer's) is zero: the C ABI takes a null pointer for it
        g_dp = None if g_dp is None else g_dp.reshape(B * G).contiguous()
        grads = _ops.project_backward(ctx.meta, z(g_m2, (B * G, 2)), z(g_cq, (B * G, 3)), z(g_op, (B * G,)),
                                      g_dp, means3d, scales, quats, opacities, c2w, cam)
        gm3, gs, gq, go, gc2w, gcam = grads
        out = [gm3.view(B, G, 3), gs.view(B, G, 3), gq.view(B, G, 4), go.view(B, G), gc2w, gcam]
        for i, need in enumerate(ctx.needs_input_grad[:6]):
            if not need:
                out[i] = None
        return (*out, None)


_scalar_cams: dict = {}


def _camera_params(fx, fy, cx, cy, B, dev, dt):
    """[B,4] (fx, fy, cx, cy).  For Python numbers the device tensor is kept per value and device
    (at most 64 entries), so a training loop with fixed intrinsics builds it once; it is only read."""
    if not any(torch.is_tensor(v) for v in (fx, fy, cx, cy)):
        key = (float(fx), float(fy), float(cx), float(cy), B, str(dev), dt)
        t = _scalar_cams.get(key)
        if t is None:
            if len(_scalar_cams) >= 64:
                _scalar_cams.clear()
            t = _scalar_cams[key] = torch.tensor([[key[0], key[1], key[2], key[3]]] * B, dtype=dt).to(dev)
        return t
    return torch.stack([
        _camera_scalar_batch(fx, B, dev, dt, "fx"),
        _camera_scalar_batch(fy, B, dev, dt, "fy"),
        _camera_scalar_batch(cx, B, dev, dt, "cx"),
        _camera_scalar_batch(cy, B, dev, dt, "cy"),
    ], dim=1).contiguous()


def _project_pinhole_gaussians_batched(means3d_b, scales_b, quats_b, opacities_b, fx, fy, cx, cy, camera_to_world,
                                       near_plane):
    B = means3d_b.shape[0]
    dev, dt = means3d_b.device, means3d_b.dtype
    camera_params = _camera_params(fx, fy, cx, cy, B, dev, dt)
    c2w_b = _camera_to_world_batch(camera_to_world, B, dev, dt)
    return _ProjectPinholeGaussians.apply(means3d_b, scales_b, quats_b, opacities_b, c2w_b, camera_params,
                                          float(near_plane))


def project_pinhole_gaussians(means3d: Tensor, scales: Tensor, quats: Tensor, opacities: Tensor, fx, fy, cx, cy,
                              camera_to_world=None, near_plane: float = 1e-4):
    """Returns (means2d, conics, projected_opacities, depths)."""
    _check_3d_inputs(means3d, scales, quats, opacities)
    m_b, s_b, q_b, o_b, was_batched = _normalize_3d_inputs(means3d, scales, quats, opacities)
    out = _project_pinhole_gaussians_batched(m_b.contiguous(), s_b.contiguous(), q_b.contiguous(), o_b.contiguous(),
                                             fx, fy, cx, cy, camera_to_world, near_plane)
    if was_batched:
        return out
    return tuple(t[0] for t in out)


def rasterize_pinhole_gaussians(means3d: Tensor, scales: Tensor, quats: Tensor, opacities: Tensor, colors: Tensor,
                                fx, fy, cx, cy, camera_to_world=None, near_plane: float = 1e-4,
                                config: RasterConfig | None = None) -> Tensor:
    if config is None:
        raise ValueError("config is required")
    _check_3d_inputs(means3d, scales, quats, opacities)
    m_b, s_b, q_b, o_b, was_batched = _normalize_3d_inputs(means3d, scales, quats, opacities)
    B, G = m_b.shape[:2]
    colors_b = _normalize_colors(colors, B, G, was_batched)
    if colors_b.device != m_b.device:
        raise ValueError("colors must be on the same device as means3d")
    if colors_b.dtype != torch.float32:
        raise ValueError("colors must be float32")
    _runtime_validate(config)
    means2d, conics, opac, depths = _project_pinhole_gaussians_batched(
        m_b.contiguous(), s_b.contiguous(), q_b.contiguous(), o_b.contiguous(), fx, fy, cx, cy, camera_to_world,
        near_plane)
    out = _rasterize_batched(means2d, conics, colors_b.contiguous(), opac, depths, config, depth_grad=False)
    return out if was_batched else out[0]
