"""torch.library operators over the C ABI: the op-level boundary.

The reference registers its kernels as operators of the namespace
gsplat_metal_v8 (variants/v8/csrc/bindings.cpp:200-222: bin,
render_fast_forward_state / _eval, render_fast_backward_saved) and of
gsplat_metal_v9_project3d_train (variants/v9_project3d_train/csrc/
bindings.cpp:175-176: project_pinhole_forward / _backward).  The same roles
are registered here as torch.ops.gsplat_hip.*, each with a fake (meta)
implementation so that FakeTensor tracing and torch.compile can see through
them.  The static render parameters the reference passes as meta tensors
(MetaI32 / MetaF32) are plain scalar arguments here:

  bin(means2d, conics, colors, opacities, depths, height, width, batch,
      alpha_threshold, transmittance_threshold, background)
      -> (tile_counts, tile_offsets, binned_ids, packed, perm)
  render_forward(packed, tile_offsets, binned_ids, height, width, batch,
      gaussians_per_batch, alpha_threshold, transmittance_threshold,
      background, save_state) -> (image, final_T, last, tile_stop, workspace)
  render_backward(grad_image, packed, tile_offsets, binned_ids, final_T,
      last, tile_stop, workspace, height, width, batch, gaussians_per_batch,
      alpha_threshold, transmittance_threshold, background)
      -> (g_means2d, g_conics, g_colors, g_opacities)
  project_forward(means3d, scales, quats, opacities, camera_to_world,
      camera_params, near_plane) -> (means2d, conics, opacities, depths)
  project_backward(g_means2d, g_conics, g_opacities, g_depths, means3d,
      scales, quats, opacities, camera_to_world, camera_params, near_plane)
      -> (g_means3d, g_scales, g_quats, g_opacities, g_camera_to_world,
          g_camera_params)

Inputs are flat [B*G, ...] float32 ROCm tensors in the original splat order
(bin computes the stable depth order itself; perm is that order), the
gradients come back in the original order and shaped [B, G, ...].  binned_ids
has a data-dependent length (the pair count N), which the fake
implementation expresses as an unbacked size.  Without the state
(save_state=False, the eval path) render_forward returns empty final_T,
last, tile_stop and workspace tensors.  Every op raises RuntimeError with the
C ABI's message on failure, like the reference's TORCH_CHECK.
"""
from __future__ import annotations

from typing import List, Tuple

import torch
from torch import Tensor

from . import _lib, _ops

_NS = "gsplat_hip"


def _meta(height, width, batch, gpb, alpha_threshold, transmittance_threshold, background):
    return _lib.make_raster_meta(height, width, batch, gpb, alpha_threshold, transmittance_threshold,
                                 tuple(background), 1e-8, 0.99)


def _tiles(height: int, width: int, batch: int) -> int:
    return batch * ((height + 15) // 16) * ((width + 15) // 16)


@torch.library.custom_op(f"{_NS}::bin", mutates_args=())
def bin(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor, depths: Tensor, height: int,
        width: int, batch: int, alpha_threshold: float, transmittance_threshold: float,
        background: List[float]) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """gsplat_metal_v8::bin (bindings.cpp:201) plus the stable depth order and record packing."""
    gpb = means2d.shape[0] // batch
    meta = _meta(height, width, batch, gpb, alpha_threshold, transmittance_threshold, background)
    st = _ops.bin_gaussians(meta, means2d.contiguous(), conics.contiguous(), colors.contiguous(),
                            opacities.contiguous(), depths.contiguous())
    return st.tile_counts, st.tile_offsets, st.binned_ids.clone(), st.packed, st.perm


@bin.register_fake
def _(means2d, conics, colors, opacities, depths, height, width, batch, alpha_threshold,
      transmittance_threshold, background):
    T = _tiles(height, width, batch)
    n = torch.library.get_ctx().new_dynamic_size()
    i32 = dict(dtype=torch.int32, device=means2d.device)
    BG = means2d.shape[0]
    return (means2d.new_empty((T,), **i32), means2d.new_empty((T + 1,), **i32), means2d.new_empty((n,), **i32),
            means2d.new_empty((BG, _lib.RECORD_FLOATS)), means2d.new_empty((BG,), **i32))


@torch.library.custom_op(f"{_NS}::render_forward", mutates_args=())
def render_forward(packed: Tensor, tile_offsets: Tensor, binned_ids: Tensor, height: int, width: int, batch: int,
                   gaussians_per_batch: int, alpha_threshold: float, transmittance_threshold: float,
                   background: List[float], save_state: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """render_fast_forward_state / render_fast_forward_eval (bindings.cpp:202-203)."""
    meta = _meta(height, width, batch, gaussians_per_batch, alpha_threshold, transmittance_threshold, background)
    st = _ops.BinState(None, packed, None, tile_offsets, binned_ids, binned_ids.numel())
    img, final_T, last, tile_stop, ws = _ops.render_forward(meta, st, save_state=save_state)
    if not save_state:
        dev = packed.device
        final_T = torch.empty((0,), device=dev)
        last = torch.empty((0,), dtype=torch.int32, device=dev)
        tile_stop = torch.empty((0,), dtype=torch.int32, device=dev)
        ws = torch.empty((0,), dtype=torch.uint8, device=dev)
    return img, final_T, last, tile_stop, ws


@render_forward.register_fake
def _(packed, tile_offsets, binned_ids, height, width, batch, gaussians_per_batch, alpha_threshold,
      transmittance_threshold, background, save_state):
    dev = packed.device
    img = packed.new_empty((batch, height, width, 3))
    if not save_state:
        return (img, packed.new_empty((0,)), packed.new_empty((0,), dtype=torch.int32),
                packed.new_empty((0,), dtype=torch.int32), packed.new_empty((0,), dtype=torch.uint8))
    meta = _meta(height, width, batch, gaussians_per_batch, alpha_threshold, transmittance_threshold, background)
    ws_bytes = _lib.lib().gsplat_hip_render_workspace_bytes(meta, binned_ids.shape[0]) \
        if isinstance(binned_ids.shape[0], int) else torch.library.get_ctx().new_dynamic_size()
    return (img, packed.new_empty((batch, height, width)),
            packed.new_empty((batch, height, width), dtype=torch.int32),
            packed.new_empty((tile_offsets.shape[0] - 1,), dtype=torch.int32),
            torch.empty((ws_bytes,), dtype=torch.uint8, device=dev))


@torch.library.custom_op(f"{_NS}::render_backward", mutates_args=())
def render_backward(grad_image: Tensor, packed: Tensor, tile_offsets: Tensor, binned_ids: Tensor, final_T: Tensor,
                    last: Tensor, tile_stop: Tensor, workspace: Tensor, height: int, width: int, batch: int,
                    gaussians_per_batch: int, alpha_threshold: float, transmittance_threshold: float,
                    background: List[float]) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """render_fast_backward_saved (bindings.cpp:204) plus the unsort: gradients in original order."""
    meta = _meta(height, width, batch, gaussians_per_batch, alpha_threshold, transmittance_threshold, background)
    st = _ops.BinState(None, packed, None, tile_offsets, binned_ids, binned_ids.numel())
    ws = workspace if workspace.numel() > 0 else None
    return tuple(_ops.render_backward(meta, st, final_T, last, tile_stop, grad_image, ws))


@render_backward.register_fake
def _(grad_image, packed, tile_offsets, binned_ids, final_T, last, tile_stop, workspace, height, width, batch,
      gaussians_per_batch, alpha_threshold, transmittance_threshold, background):
    B, G = batch, gaussians_per_batch
    return (packed.new_empty((B, G, 2)), packed.new_empty((B, G, 3)), packed.new_empty((B, G, 3)),
            packed.new_empty((B, G)))


@torch.library.custom_op(f"{_NS}::project_forward", mutates_args=())
def project_forward(means3d: Tensor, scales: Tensor, quats: Tensor, opacities: Tensor, camera_to_world: Tensor,
                    camera_params: Tensor, near_plane: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """project_pinhole_forward (variants/v9_project3d_train/csrc/bindings.cpp:175)."""
    B = camera_to_world.shape[0]
    meta = _lib.make_project_meta(B, means3d.shape[0] // B, near_plane)
    return _ops.project_forward(meta, means3d.contiguous(), scales.contiguous(), quats.contiguous(),
                                opacities.contiguous(), camera_to_world.contiguous(), camera_params.contiguous())


@project_forward.register_fake
def _(means3d, scales, quats, opacities, camera_to_world, camera_params, near_plane):
    n = means3d.shape[0]
    return (means3d.new_empty((n, 2)), means3d.new_empty((n, 3)), means3d.new_empty((n,)),
            means3d.new_empty((n,)))


@torch.library.custom_op(f"{_NS}::project_backward", mutates_args=())
def project_backward(g_means2d: Tensor, g_conics: Tensor, g_opacities: Tensor, g_depths: Tensor, means3d: Tensor,
                     scales: Tensor, quats: Tensor, opacities: Tensor, camera_to_world: Tensor,
                     camera_params: Tensor, near_plane: float
                     ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """project_pinhole_backward (variants/v9_project3d_train/csrc/bindings.cpp:176)."""
    B = camera_to_world.shape[0]
    meta = _lib.make_project_meta(B, means3d.shape[0] // B, near_plane)
    return _ops.project_backward(meta, *(t.contiguous() for t in (g_means2d, g_conics, g_opacities, g_depths,
                                                                    means3d, scales, quats, opacities,
                                                                    camera_to_world, camera_params)))


@project_backward.register_fake
def _(g_means2d, g_conics, g_opacities, g_depths, means3d, scales, quats, opacities, camera_to_world,
      camera_params, near_plane):
    n, B = means3d.shape[0], camera_to_world.shape[0]
    return (means3d.new_empty((n, 3)), means3d.new_empty((n, 3)), means3d.new_empty((n, 4)),
            means3d.new_empty((n,)), means3d.new_empty((B, 4, 4)), means3d.new_empty((B, 4)))
