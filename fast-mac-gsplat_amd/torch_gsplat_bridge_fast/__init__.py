"""MI355X (gfx950) differentiable Gaussian-splat rasterizer.

Drop-in for the reference package of the same name, exposing its batched
projected-2D API plus the pinhole projection front end.
"""
from .rasterize import (
    ProjectedGaussianRasterizer,
    RasterConfig,
    RuntimeShaderConfig,
    get_runtime_shader_config,
    profile_projected_gaussians,
    rasterize_projected_gaussians,
)
from .project import project_pinhole_gaussians, rasterize_pinhole_gaussians
from . import ops  # noqa: F401  (registers torch.ops.gsplat_hip.*)
from . import v8_ops  # noqa: F401  (registers the reference's torch.ops.gsplat_metal_v8.*)

__all__ = [
    "RasterConfig",
    "RuntimeShaderConfig",
    "ProjectedGaussianRasterizer",
    "rasterize_projected_gaussians",
    "profile_projected_gaussians",
    "get_runtime_shader_config",
    "project_pinhole_gaussians",
    "rasterize_pinhole_gaussians",
]
