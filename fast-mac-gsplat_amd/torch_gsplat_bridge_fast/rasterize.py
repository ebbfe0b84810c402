"""Batched differentiable rasterizer for projected 2D Gaussian splats.

Public API of the reference's batched path (variants/v8/torch_gsplat_bridge_v8/
rasterize.py), backed by the HIP kernels of libgsplat_hip.so:

  RasterConfig                    v8 rasterize.py:64-82
  rasterize_projected_gaussians   v8 rasterize.py:843-857
  profile_projected_gaussians     v8 rasterize.py:860-1014
  ProjectedGaussianRasterizer     v8 rasterize.py:1017-1023

Inputs are [G,...] or [B,G,...] contiguous float32 tensors on a ROCm device:
means2d [..,2] pixel centres, conics [..,3] = (a, b, c) with
power = -0.5*(a dx^2 + 2 b dx dy + c dy^2), colors [..,3], opacities [..],
depths [..] (only ordered; their gradient is zero).  Output is [H,W,3] or
[B,H,W,3].

Semantics that differ from the reference only in mechanism (results are the
same):
  * Tiles of any length are composited by the main kernels (the reference
    falls back to a host-sorted overflow path above max_fast_pairs).
    ``enable_overflow_fallback=False`` still raises "Tile overflow detected"
    when a tile holds more than ``max_fast_pairs`` pairs.
  * ``use_active_tiles``, ``active_policy``, ``sort_active_tiles_by_count``,
    ``stop_count_mode`` and ``stop_count_dense_threshold`` are validated like
    the reference but do not change the computation: empty tiles cost one
    early-exiting wavefront, and backward always uses exact per-pixel stop
    state saved by forward.  profile_projected_gaussians reports the
    reference's active-tile decision and its stop counts (0 for tiles above
    max_fast_pairs).  ``max_pairs_per_launch`` splits training batches
    into launches of at most that many tile pairs, as the reference does.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any, Dict, List, Tuple

import torch
from torch import Tensor

from . import _lib, _ops


@dataclass(frozen=True)
class RuntimeShaderConfig:
    """Compiled compositor parameters (reference fields, v8 rasterize.py:17-23):
    tile_size (pixels per tile side), threads (lanes of a tile's workgroup),
    chunk_size (splats staged per batch), fast_cap (the max_fast_pairs
    bound) and simdgroups (hardware execution groups per tile workgroup:
    64-lane wavefronts here)."""
    tile_size: int
    threads: int
    chunk_size: int
    fast_cap: int
    simdgroups: int


def _env_int(name: str, default: int) -> int:
    raw = os.environ.get(name)
    if raw is None or raw == "":
        return int(default)
    return int(raw)


def get_runtime_shader_config() -> RuntimeShaderConfig:
    """Compiled kernel parameters (reference: v8 rasterize.py:33-53), with the
    reference's environment variables and checks.

    The HIP kernels are built for 16x16 tiles walked by one 64-lane wavefront
    (threads = 64, simdgroups = 1 wavefront) and 64-splat LDS batches;
    GSP_TILE_SIZE other than 16 and GSP_CHUNK other than 64 are rejected.
    GSP_FAST_CAP bounds ``max_fast_pairs`` as in the reference."""
    tile_size = _env_int("GSP_TILE_SIZE", 16)
    chunk_size = _env_int("GSP_CHUNK", 64)
    fast_cap = _env_int("GSP_FAST_CAP", 2048)
    if tile_size not in (8, 16, 32):
        raise ValueError(f"GSP_TILE_SIZE must be one of 8, 16, 32; got {tile_size}")
    if tile_size != _lib.TILE_SIZE:
        raise ValueError(f"GSP_TILE_SIZE={tile_size} is not supported: the HIP kernels are built for 16x16 tiles")
    if chunk_size <= 0:
        raise ValueError("GSP_CHUNK must be positive")
    if chunk_size != 64:
        raise ValueError(f"GSP_CHUNK={chunk_size} is not supported: the HIP kernels stage 64-splat batches")
    if fast_cap <= 0:
        raise ValueError("GSP_FAST_CAP must be positive")
    return RuntimeShaderConfig(tile_size=tile_size, threads=64, chunk_size=chunk_size, fast_cap=fast_cap,
                               simdgroups=1)


@dataclass(frozen=True)
class RasterConfig:
    height: int
    width: int
    tile_size: int = 16
    max_fast_pairs: int = 2048
    alpha_threshold: float = 1.0 / 255.0
    transmittance_threshold: float = 1e-4
    background: Tuple[float, float, float] = (0.0, 0.0, 0.0)
    enable_overflow_fallback: bool = True
    batch_strategy: str = "auto"  # auto | flatten | serial
    batch_launch_limit_tiles: int = 262144
    batch_launch_limit_gaussians: int = 262144
    use_active_tiles: bool = False
    active_policy: str = "off"  # off | on | auto
    sort_active_tiles_by_count: bool = True
    stop_count_mode: str = "adaptive"  # always | never | adaptive
    stop_count_dense_threshold: int = 64
    max_pairs_per_launch: int = 0


_EPS = 1e-8
_MAX_ALPHA = 0.99


_validated: dict = {}


def _runtime_validate(config: RasterConfig) -> RuntimeShaderConfig:
    """Same checks and messages as v8 rasterize.py:85-107.  A config that passed once with the same
    environment is not checked again (RasterConfig is frozen)."""
    env = (os.environ.get("GSP_TILE_SIZE"), os.environ.get("GSP_CHUNK"), os.environ.get("GSP_FAST_CAP"))
    key = (config, env)
    try:
        rt = _validated.get(key)
    except TypeError:   # a field that is not hashable (e.g. a list background): no cache
        return _runtime_validate_uncached(config)
    if rt is not None:
        return rt
    rt = _runtime_validate_uncached(config)
    if len(_validated) > 256:
        _validated.clear()
    _validated[key] = rt
    return rt


def _runtime_validate_uncached(config: RasterConfig) -> RuntimeShaderConfig:
    rt = get_runtime_shader_config()
    if config.tile_size != rt.tile_size:
        raise ValueError(
            f"RasterConfig.tile_size={config.tile_size} does not match runtime shader tile size {rt.tile_size}. "
            "Set GSP_TILE_SIZE before importing/running the extension, or adjust RasterConfig."
        )
    if config.max_fast_pairs > rt.fast_cap:
        raise ValueError(
            f"RasterConfig.max_fast_pairs={config.max_fast_pairs} exceeds compiled fast cap {rt.fast_cap}. "
            "Lower the runtime cap or set GSP_FAST_CAP before import."
        )
    if config.height <= 0 or config.width <= 0:
        raise ValueError("RasterConfig.height and width must be positive")
    if config.batch_strategy not in ("auto", "flatten", "serial"):
        raise ValueError("batch_strategy must be one of: auto, flatten, serial")
    if config.active_policy not in ("off", "on", "auto"):
        raise ValueError("active_policy must be one of: off, on, auto")
    if config.stop_count_mode not in ("always", "never", "adaptive"):
        raise ValueError("stop_count_mode must be one of: always, never, adaptive")
    if config.stop_count_dense_threshold <= 0:
        raise ValueError("stop_count_dense_threshold must be positive")
    if config.max_pairs_per_launch < 0:
        raise ValueError("max_pairs_per_launch must be non-negative")
    if len(config.background) != 3:
        raise ValueError("background must have 3 components")
    return rt


def _effective_active_policy(config: RasterConfig) -> str:
    if config.active_policy == "off" and config.use_active_tiles:
        return "on"
    return config.active_policy


def _resolve_active_tile_use(policy: str, active_fraction: float, overflow_tiles: int, max_pairs: int,
                             max_fast_pairs: int) -> bool:
    """The reference's choice between its active-tile and its fast kernels for one launch
    (v8 rasterize.py:401-424): "on" / "off" as given; "auto" takes the active-tile kernels for
    sparse images (under 10% of the tiles occupied), when a tile overflows max_fast_pairs or one
    holds more than twice that, and never when over 75% of the tiles are occupied with no
    overflow.  Here both kernel sets are one compositor; the choice is reported only."""
    if policy == "off":
        return False
    if policy == "on":
        return True
    if active_fraction > 0.75 and overflow_tiles == 0:
        return False
    return active_fraction < 0.10 or overflow_tiles > 0 or max_pairs > 2 * max_fast_pairs


_metas: dict = {}


def _meta(config: RasterConfig, batch_size: int, gaussians_per_batch: int) -> _lib.RasterMeta:
    """The C-ABI meta struct, built once per (config, B, G): it is only read by the calls."""
    key = (config, batch_size, gaussians_per_batch)
    try:
        m = _metas.get(key)
    except TypeError:   # a field that is not hashable (e.g. a list background): no cache
        key, m = None, None
    if m is None:
        m = _lib.make_raster_meta(
            config.height, config.width, batch_size, gaussians_per_batch, config.alpha_threshold,
            config.transmittance_threshold, config.background, _EPS, _MAX_ALPHA)
        if key is not None:
            if len(_metas) > 256:
                _metas.clear()
            _metas[key] = m
    return m


def _normalize_inputs(means2d, conics, colors, opacities, depths):
    if means2d.ndim == 2:
        return (means2d.unsqueeze(0), conics.unsqueeze(0), colors.unsqueeze(0), opacities.unsqueeze(0),
                depths.unsqueeze(0), False)
    if means2d.ndim != 3:
        raise ValueError("means2d must have shape [G,2] or [B,G,2]")
    return means2d, conics, colors, opacities, depths, True


def _check_inputs(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor, depths: Tensor) -> None:
    """Shape/dtype/device checks with the reference's messages (v8 rasterize.py:197-226)."""
    if means2d.ndim not in (2, 3):
        raise ValueError("means2d must have shape [G,2] or [B,G,2]")
    if conics.ndim != means2d.ndim or colors.ndim != means2d.ndim:
        raise ValueError("conics/colors rank must match means2d rank")
    if opacities.ndim != means2d.ndim - 1 or depths.ndim != means2d.ndim - 1:
        raise ValueError("opacities/depths rank must be one less than means2d rank")
    if means2d.shape[-1] != 2:
        raise ValueError("means2d must have last dim = 2")
    if conics.shape[-1] != 3:
        raise ValueError("conics must have last dim = 3")
    if colors.shape[-1] != 3:
        raise ValueError("colors must have last dim = 3")
    if means2d.shape[:-1] != conics.shape[:-1] or means2d.shape[:-1] != colors.shape[:-1]:
        raise ValueError("means2d/conics/colors batch/G dimensions must match")
    if means2d.shape[:-1] != opacities.shape or means2d.shape[:-1] != depths.shape:
        raise ValueError("means2d/opacities/depths batch/G dimensions must match")
    for name, t in (("means2d", means2d), ("conics", conics), ("colors", colors), ("opacities", opacities),
                    ("depths", depths)):
        if t.device != means2d.device:
            raise ValueError(f"{name} must be on the same device as means2d")
        if t.dtype != torch.float32:
            raise ValueError(f"{name} must be float32")
    if means2d.device.type != "cuda":
        raise ValueError("HIP fast path requires ROCm device tensors (device type 'cuda')")
    if means2d.shape[-2] == 0:
        raise ValueError("at least one Gaussian is required (G >= 1)")


def _should_use_training_path(means2d, conics, colors, opacities) -> bool:
    if not torch.is_grad_enabled():
        return False
    return bool(means2d.requires_grad or conics.requires_grad or colors.requires_grad or opacities.requires_grad)


def _choose_batch_chunk_size(config: RasterConfig, batch_size: int, gaussians_per_batch: int,
                             tiles_per_image: int) -> int:
    """Reference batch chunking (v8 rasterize.py:324-331)."""
    if config.batch_strategy == "flatten":
        return batch_size
    if config.batch_strategy == "serial":
        return 1
    by_tiles = max(1, config.batch_launch_limit_tiles // max(tiles_per_image, 1))
    by_gaussians = max(1, config.batch_launch_limit_gaussians // max(gaussians_per_batch, 1))
    return max(1, min(batch_size, by_tiles, by_gaussians))


def _flat(means2d_b, conics_b, colors_b, opacities_b, depths_b):
    B, G = means2d_b.shape[:2]
    return (means2d_b.reshape(B * G, 2).contiguous(), conics_b.reshape(B * G, 3).contiguous(),
            colors_b.reshape(B * G, 3).contiguous(), opacities_b.reshape(B * G).contiguous(),
            depths_b.reshape(B * G).contiguous())


def _check_overflow(config: RasterConfig, st: _ops.BinState) -> None:
    if config.enable_overflow_fallback or st.tile_counts.numel() == 0:
        return
    if bool((st.tile_counts > int(config.max_fast_pairs)).any().item()):
        raise RuntimeError(
            f"Tile overflow detected with max_fast_pairs={config.max_fast_pairs}. "
            "Enable overflow fallback or increase the runtime cap."
        )


class _RasterizeProjectedGaussians(torch.autograd.Function):
    """Training path (reference _RasterizeProjectedGaussiansV8, v8 rasterize.py:444-681).

    Forward saves the compact binning state plus per-pixel final transmittance
    and last-composited index; backward writes gradients straight into the
    original splat order, so no unsort is needed."""

    @staticmethod
    def forward(ctx, means2d_b, conics_b, colors_b, opacities_b, depths_b, config: RasterConfig,
                depth_grad: bool = True):
        B, G = means2d_b.shape[:2]
        meta = _meta(config, B, G)
        flat = _flat(means2d_b.detach(), conics_b.detach(), colors_b.detach(), opacities_b.detach(),
                     depths_b.detach())
        # the first backward's outputs, allocated before the host waits on the binning
        ctx.grad_bufs = _ops.gradient_buffers(B, G, means2d_b.device)
        st, (img, final_T, last, tile_stop, ws) = _ops.bin_and_render(meta, flat, save_state=True)
        _check_overflow(config, st)
        ctx.save_for_backward(st.packed, st.tile_offsets, st.pairs, final_T, last, tile_stop, ws)
        # the binning's status is read before the backward (by then the GPU is done with it)
        ctx.check_status = st.check_status
        ctx.meta = meta
        ctx.shape = (B, G)
        ctx.depth_shape = depths_b.shape
        ctx.depth_grad = depth_grad
        return img

    @staticmethod
    def backward(ctx, grad_out):
        packed, tile_offsets, pairs, final_T, last, tile_stop, ws = ctx.saved_tensors
        ctx.check_status()
        st = _ops.BinState(None, packed, None, tile_offsets, pairs, pairs.numel())
        bufs, ctx.grad_bufs = ctx.grad_bufs, None   # a second backward (retain_graph) allocates anew
        g_m, g_q, g_c, g_o = _ops.render_backward(ctx.meta, st, final_T, last, tile_stop, grad_out, ws, out=bufs)
        need = ctx.needs_input_grad
        # The depth gradient is zero (the reference returns zeros, v8 rasterize.py:680).  For depths
        # computed by the projection (depth_grad False) it is returned as None, which autograd
        # propagates as zero without a zero-filled tensor.
        g_depth = (torch.zeros(ctx.depth_shape, dtype=torch.float32, device=grad_out.device)
                   if need[4] and ctx.depth_grad else None)
        return (g_m if need[0] else None,
                g_q if need[1] else None,
                g_c if need[2] else None,
                g_o if need[3] else None,
                g_depth, None, None)


def _rasterize_chunk_eval(means2d_b, conics_b, colors_b, opacities_b, depths_b, config: RasterConfig) -> Tensor:
    """Eval path (reference v8 rasterize.py:684-786): no saved state."""
    B, G = means2d_b.shape[:2]
    meta = _meta(config, B, G)
    st, out = _ops.bin_and_render(meta, _flat(means2d_b, conics_b, colors_b, opacities_b, depths_b),
                                  save_state=False)
    _check_overflow(config, st)
    st.check_status()
    return out[0]


def _choose_batch_slices(means2d_b, conics_b, colors_b, opacities_b, depths_b, config: RasterConfig, *,
                         train_mode: bool, tiles_per_image: int) -> List[Tuple[int, int]]:
    """Batch slices per launch (reference _choose_batch_slices, v8 rasterize.py:339-391): contiguous
    chunks of _choose_batch_chunk_size images; in training with batch_strategy "auto" and a positive
    max_pairs_per_launch, each chunk is binned and split greedily so that a launch holds at most that
    many tile pairs (a single image above the budget still gets its own launch)."""
    B, G = means2d_b.shape[:2]
    chunk_b = _choose_batch_chunk_size(config, B, G, tiles_per_image)
    base = [(b0, min(B, b0 + chunk_b)) for b0 in range(0, B, chunk_b)]
    if not train_mode or config.batch_strategy != "auto" or config.max_pairs_per_launch <= 0 or B <= 1:
        return base
    return _split_by_pair_budget(means2d_b, conics_b, colors_b, opacities_b, depths_b, config, base,
                                 tiles_per_image)


@torch.no_grad()
def _split_by_pair_budget(means2d_b, conics_b, colors_b, opacities_b, depths_b, config: RasterConfig,
                          base: List[Tuple[int, int]], tiles_per_image: int) -> List[Tuple[int, int]]:
    G = means2d_b.shape[1]
    budget = int(config.max_pairs_per_launch)
    out: List[Tuple[int, int]] = []
    for b0, b1 in base:
        st = _ops.bin_gaussians(_meta(config, b1 - b0, G),
                                *_flat(means2d_b[b0:b1], conics_b[b0:b1], colors_b[b0:b1], opacities_b[b0:b1],
                                       depths_b[b0:b1]))
        per_image = st.tile_counts.view(b1 - b0, tiles_per_image).sum(dim=1).tolist()
        cur, cur_pairs = b0, 0
        for off, pairs in enumerate(per_image):
            b = b0 + off
            if b > cur and cur_pairs + int(pairs) > budget:
                out.append((cur, b))
                cur, cur_pairs = b, 0
            cur_pairs += int(pairs)
        if cur < b1:
            out.append((cur, b1))
    return out


def _rasterize_batched(means2d_b, conics_b, colors_b, opacities_b, depths_b, config: RasterConfig,
                       depth_grad: bool = True) -> Tensor:
    """depth_grad False: depths are an intermediate result whose (zero) gradient need not be
    materialised."""
    B, G = means2d_b.shape[:2]
    tiles_per_image = ((config.height + 15) // 16) * ((config.width + 15) // 16)
    train_mode = _should_use_training_path(means2d_b, conics_b, colors_b, opacities_b)
    slices = _choose_batch_slices(means2d_b, conics_b, colors_b, opacities_b, depths_b, config,
                                  train_mode=train_mode, tiles_per_image=tiles_per_image)
    outs = []
    for b0, b1 in slices:
        if b0 == 0 and b1 == B:
            # one chunk: no slice views (their backward would zero-fill and copy every gradient)
            args = (means2d_b, conics_b, colors_b, opacities_b, depths_b)
        else:
            args = (means2d_b[b0:b1], conics_b[b0:b1], colors_b[b0:b1], opacities_b[b0:b1], depths_b[b0:b1])
        if train_mode:
            outs.append(_RasterizeProjectedGaussians.apply(*args, config, depth_grad))
        else:
            with torch.no_grad():
                outs.append(_rasterize_chunk_eval(*args, config))
    return torch.cat(outs, dim=0) if len(outs) > 1 else outs[0]


def rasterize_projected_gaussians(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor,
                                  depths: Tensor, config: RasterConfig) -> Tensor:
    _check_inputs(means2d, conics, colors, opacities, depths)
    means2d_b, conics_b, colors_b, opacities_b, depths_b, was_batched = _normalize_inputs(
        means2d, conics, colors, opacities, depths)
    _runtime_validate(config)
    out = _rasterize_batched(means2d_b, conics_b, colors_b, opacities_b, depths_b, config)
    return out if was_batched else out[0]


@torch.no_grad()
def profile_projected_gaussians(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor,
                                depths: Tensor, config: RasterConfig, *, run_forward: bool = False,
                                return_image: bool = False) -> Dict[str, Any]:
    """Tile statistics with the reference's keys and meaning (v8 rasterize.py:860-1014).  The stop
    count statistics are those of the reference's fast kernels: a tile above max_fast_pairs (left
    to the reference's overflow path) or without pairs counts as 0 (gsplat_v8_kernels.metal:
    423-431); resolved_use_active_tiles / resolved_active_chunks report the reference's policy
    decision per launch."""
    _check_inputs(means2d, conics, colors, opacities, depths)
    means2d_b, conics_b, colors_b, opacities_b, depths_b, was_batched = _normalize_inputs(
        means2d, conics, colors, opacities, depths)
    B, G = means2d_b.shape[:2]
    _runtime_validate(config)
    tiles_per_image = ((config.height + 15) // 16) * ((config.width + 15) // 16)
    chunk_b = _choose_batch_chunk_size(config, B, G, tiles_per_image)
    slices = _choose_batch_slices(means2d_b, conics_b, colors_b, opacities_b, depths_b, config,
                                  train_mode=True, tiles_per_image=tiles_per_image)
    mfp = int(config.max_fast_pairs)
    counts_all, stops_all, images, chunk_rows = [], [], [], []
    for b0, b1 in slices:
        args = _flat(means2d_b[b0:b1], conics_b[b0:b1], colors_b[b0:b1], opacities_b[b0:b1], depths_b[b0:b1])
        meta = _meta(config, b1 - b0, G)
        st = _ops.bin_gaussians(meta, *args)
        cnt = st.tile_counts
        counts_all.append(cnt)
        # per launch: occupied fraction, overflowing tiles, largest tile (the policy's inputs)
        chunk_rows.append(torch.stack([(cnt > 0).sum().to(torch.float32) / max(cnt.numel(), 1),
                                       (cnt > mfp).sum().to(torch.float32), cnt.max().to(torch.float32)]))
        if run_forward or return_image:
            img, _, _, tile_stop, _ = _ops.render_forward(meta, st, save_state=True)
            # the reference's fast kernels report 0 for the tiles they leave to the overflow path
            stops_all.append(torch.where(cnt <= mfp, tile_stop, torch.zeros_like(tile_stop)))
            if return_image:
                images.append(img)
    # The statistics are reduced on the device; one small vector comes back.
    counts = torch.cat(counts_all).to(torch.float32)
    n = counts.numel()
    occupied = counts > 0
    fast = occupied & (counts <= mfp)
    dense = counts >= int(config.stop_count_dense_threshold)
    if n:
        vec = torch.cat([torch.stack([counts.sum(), counts.mean(), torch.quantile(counts, 0.95), counts.max(),
                                      (counts > mfp).sum().to(torch.float32),
                                      fast.sum().to(torch.float32), occupied.sum().to(torch.float32),
                                      (fast & dense).sum().to(torch.float32)])]
                        + chunk_rows).tolist()
    else:
        vec = [0.0] * 8
    policy = _effective_active_policy(config)
    resolved = [_resolve_active_tile_use(policy, vec[8 + 3 * k], int(vec[9 + 3 * k]), int(vec[10 + 3 * k]), mfp)
                for k in range(len(chunk_rows))] if n else [False for _ in slices]
    stats: Dict[str, Any] = {
        "batch_size": int(B),
        "gaussians_per_batch": int(G),
        "height": int(config.height),
        "width": int(config.width),
        "tile_size": int(config.tile_size),
        "tiles": int(n),
        "total_pairs": int(vec[0]),
        "mean_pairs_per_tile": float(vec[1]),
        "p95_pairs_per_tile": float(vec[2]),
        "max_pairs_per_tile": int(vec[3]),
        "overflow_tile_count": int(vec[4]),
        "active_tile_count": int(vec[5]),
        "active_tile_fraction": float(vec[6] / max(n, 1)),
        "dense_active_tile_count": int(vec[7]),
        "chosen_batch_chunk": int(chunk_b),
        "chosen_batch_chunks": [int(b1 - b0) for b0, b1 in slices],
        "max_pairs_per_launch": int(config.max_pairs_per_launch),
        "active_policy": policy,
        "resolved_use_active_tiles": bool(any(resolved)),
        "resolved_active_chunks": [bool(x) for x in resolved],
        "stop_count_mode": config.stop_count_mode,
    }
    if stops_all and n:
        stop = torch.cat(stops_all).to(torch.float32)
        ratio = torch.where(counts > 0, stop / torch.clamp(counts, min=1.0), torch.zeros_like(stop))
        sv = torch.stack([stop.mean(), torch.quantile(stop, 0.95), stop.max(), ratio.mean(),
                          torch.quantile(ratio, 0.95)]).tolist()
        stats.update({
            "mean_stop_count": float(sv[0]),
            "p95_stop_count": float(sv[1]),
            "max_stop_count": int(sv[2]),
            "mean_stop_ratio": float(sv[3]),
            "p95_stop_ratio": float(sv[4]),
        })
    if return_image:
        out = torch.cat(images, dim=0) if len(images) > 1 else images[0]
        return {"image": out if was_batched else out[0], "stats": stats}
    return stats


class ProjectedGaussianRasterizer(torch.nn.Module):
    def __init__(self, config: RasterConfig):
        super().__init__()
        self.config = config

    def forward(self, means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor, depths: Tensor) -> Tensor:
        return rasterize_projected_gaussians(means2d, conics, colors, opacities, depths, self.config)
