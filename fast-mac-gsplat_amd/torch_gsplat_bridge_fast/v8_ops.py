"""The reference's operator namespace, torch.ops.gsplat_metal_v8.*, over the C ABI.

variants/v8/csrc/bindings.cpp:200-210 defines nine operators, and
variants/v8/torch_gsplat_bridge_v8/rasterize.py calls every one of them (bin :368, :477, :705;
render_fast_forward_state :514, render_active_forward_state :498, render_overflow_forward :541,
:757; render_fast_backward_saved :637, render_active_backward_saved :620,
render_overflow_backward :655; render_fast_forward_eval :738, render_active_forward_eval :723).
This module registers the same names with the same schemas (argument names, order, the in-place
binned_ids of the state forwards) for ROCm tensors, so that the reference's Python -- its
autograd Function, eval path and batch splitting -- runs unchanged on the HIP kernels.  The meta
tensors are read as the reference's ParsedMeta reads them (variants/v8/csrc/shared/common.h:
9-62, packed by v8 rasterize.py:129-173): host int32 [H, W, tiles_y, tiles_x, tile_size, B*G, T,
max_fast_pairs, B, G, tiles_per_image, stop_count_mode, stop_count_dense_threshold, 0] and host
float32 [alpha_threshold, transmittance_threshold, bg_r, bg_g, bg_b, eps, max_alpha]; the device
copies (meta_i32, meta_f32) are accepted and not read.

Per operator, what the reference's kernels (variants/v8/csrc/metal/gsplat_v8_kernels.metal)
compute, which is what is returned here:
  bin                         (tile_counts [T], tile_offsets [T+1], binned_ids [N]) of the
                              depth-sorted flat inputs; binned ids are flat indices into them.
                              Inside a tile the ids come out ascending (depth order); the
                              reference's come in atomic-cursor order and its compositors sort
                              them.
  render_fast_forward_eval /  the image; tiles with no pair or more than max_fast_pairs are
  render_fast_forward_state   background with stop count 0 (:351-358, :423-431), left to the
                              overflow operators.  The state forward also returns the per-tile
                              stop counts and sorts each such tile's ids in binned_ids in place.
  render_fast_backward_saved  the gradients of the tiles with 0 < count <= max_fast_pairs
                              (:504), in the order of the flat inputs; the forward is replayed
                              for its per-pixel state, as the reference's backward replays it
                              (:511-540).
  render_active_forward_* /   the same over the listed active tiles only (:613-885); every other
  render_active_backward_saved tile is background with stop count 0.
  render_overflow_forward     [To, 16, 16, 3] images of the listed tiles, background outside the
                              image (:887-946); the caller scatters them into a clone of the
                              fast image (v8 rasterize.py:554).
  render_overflow_backward    the listed tiles' gradients for grad_tiles [To, 16, 16, 3]
                              (:948-1081), which the caller adds to the fast ones (:671-674).
Each operator runs the HIP compositors over the tile ranges it covers (the other ranges empty),
so the fast and overflow parts add up to the whole image and gradient.  Images agree bit for bit
with gsplat_hip_render_forward over all tiles; gradients agree up to float summation order.
Errors raise RuntimeError with the reference's messages where it has one (TORCH_CHECK).

The state and the segment records that the HIP backward reads are not part of the reference's
operator signatures, so each backward here replays the forward; the package's own autograd path
(rasterize_projected_gaussians) keeps them and does not.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch
from torch import Tensor

from . import _lib, _ops

NAMESPACE = "gsplat_metal_v8"
TILE = _lib.TILE_SIZE


# The reference's operator schemas (variants/v8/csrc/bindings.cpp:201-209), argument list and
# results; the interface a drop-in has to keep.
_M = "Tensor means2d, Tensor conics, Tensor colors, Tensor opacities, Tensor meta_i32, Tensor meta_f32, " \
     "Tensor meta_host_i32, Tensor meta_host_f32"
SCHEMAS = {
    "bin": f"({_M}) -> (Tensor, Tensor, Tensor)",
    "render_fast_forward_eval": f"({_M}, Tensor tile_counts, Tensor tile_offsets, Tensor binned_ids) -> Tensor",
    "render_fast_forward_state":
        f"({_M}, Tensor(a!) binned_ids, Tensor tile_counts, Tensor tile_offsets) -> (Tensor, Tensor)",
    "render_fast_backward_saved":
        f"(Tensor grad_out, {_M}, Tensor tile_counts, Tensor tile_offsets, Tensor binned_ids, "
        "Tensor tile_stop_counts) -> (Tensor, Tensor, Tensor, Tensor)",
    "render_active_forward_eval":
        f"({_M}, Tensor active_tile_ids, Tensor tile_counts, Tensor tile_offsets, Tensor binned_ids) -> Tensor",
    "render_active_forward_state":
        f"({_M}, Tensor(a!) binned_ids, Tensor active_tile_ids, Tensor tile_counts, Tensor tile_offsets) "
        "-> (Tensor, Tensor)",
    "render_active_backward_saved":
        f"(Tensor grad_out, {_M}, Tensor active_tile_ids, Tensor tile_counts, Tensor tile_offsets, "
        "Tensor binned_ids, Tensor tile_stop_counts) -> (Tensor, Tensor, Tensor, Tensor)",
    "render_overflow_forward":
        f"({_M}, Tensor overflow_tile_ids, Tensor overflow_tile_offsets, Tensor overflow_sorted_ids) -> Tensor",
    "render_overflow_backward":
        f"(Tensor grad_tiles, {_M}, Tensor overflow_tile_ids, Tensor overflow_tile_offsets, "
        "Tensor overflow_sorted_ids) -> (Tensor, Tensor, Tensor, Tensor)",
}


@dataclass
class V8Meta:
    raster: _lib.RasterMeta
    height: int
    width: int
    tiles_y: int
    tiles_x: int
    tile_count: int
    max_fast_pairs: int
    batch: int
    gaussians_per_batch: int
    tiles_per_image: int


def parse_meta(meta_host_i32: Tensor, meta_host_f32: Tensor, n_splats: int) -> V8Meta:
    """ParsedMeta (common.h:9-62) plus the checks of the reference's bin (gsplat_metal.mm:149-157)."""
    if meta_host_i32.device.type != "cpu":
        raise RuntimeError("host meta_i32 must be on CPU")
    if meta_host_f32.device.type != "cpu":
        raise RuntimeError("host meta_f32 must be on CPU")
    if meta_host_i32.dtype != torch.int32 or meta_host_i32.numel() < 14:
        raise RuntimeError("host meta_i32 must be int32 with 14 entries")
    if meta_host_f32.dtype != torch.float32 or meta_host_f32.numel() < 7:
        raise RuntimeError("host meta_f32 must be float32 with 7 entries")
    i = [int(v) for v in meta_host_i32.reshape(-1).tolist()]
    f = [float(v) for v in meta_host_f32.reshape(-1).tolist()]
    H, W, tiles_y, tiles_x, tile_size, gaussians, tile_count, max_fast, B, G, tpi = i[:11]
    from .rasterize import get_runtime_shader_config
    sc = get_runtime_shader_config()
    if tile_size != sc.tile_size:
        raise RuntimeError(f"meta.tile_size must match shader tile size {sc.tile_size}")
    if max_fast > sc.fast_cap:
        raise RuntimeError(f"meta.max_fast_pairs exceeds shader compile-time cap {sc.fast_cap}")
    if B <= 0:
        raise RuntimeError("meta.batch_size must be positive")
    if G <= 0:
        raise RuntimeError("meta.gaussians_per_batch must be positive")
    if tpi != tiles_y * tiles_x:
        raise RuntimeError("meta.tiles_per_image mismatch")
    if gaussians != n_splats:
        raise RuntimeError("flattened Gaussian count mismatch")
    if (tiles_y != (H + TILE - 1) // TILE or tiles_x != (W + TILE - 1) // TILE or tile_count != B * tpi
            or gaussians != B * G):
        raise RuntimeError("meta: tiles_y/tiles_x/tile_count/gaussians disagree with height, width, batch "
                           "and gaussians_per_batch")
    raster = _lib.make_raster_meta(H, W, B, G, f[0], f[1], (f[2], f[3], f[4]), f[5], f[6])
    return V8Meta(raster, H, W, tiles_y, tiles_x, tile_count, max_fast, B, G, tpi)


def _check_inputs(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor) -> None:
    """check_inputs of the reference host (gsplat_metal.mm:104-121), for ROCm tensors."""
    for name, t in (("means2d", means2d), ("conics", conics), ("colors", colors), ("opacities", opacities)):
        if t.device.type != "cuda":
            raise RuntimeError(f"{name} must be on the GPU (ROCm)")
        if t.dtype != torch.float32:
            raise RuntimeError(f"{name} must be float32")
    if not (means2d.dim() == 2 and means2d.shape[1] == 2):
        raise RuntimeError("means2d must be [BG,2]")
    if not (conics.dim() == 2 and conics.shape[1] == 3):
        raise RuntimeError("conics must be [BG,3]")
    if not (colors.dim() == 2 and colors.shape[1] == 3):
        raise RuntimeError("colors must be [BG,3]")
    if opacities.dim() != 1:
        raise RuntimeError("opacities must be [BG]")
    n = means2d.shape[0]
    if not (conics.shape[0] == n and colors.shape[0] == n and opacities.shape[0] == n):
        raise RuntimeError("All inputs must agree on flattened BG")


def _check_aux_i32(t: Tensor, name: str, device: torch.device) -> None:
    if t.device != device:
        raise RuntimeError(f"{name} must be on the GPU (ROCm)")
    if t.dtype != torch.int32:
        raise RuntimeError(f"{name} must be int32")
    if t.dim() != 1:
        raise RuntimeError(f"{name} must be one-dimensional")


def _packed(meta: V8Meta, means2d, conics, colors, opacities) -> Tensor:
    """The HIP compositors' records of the flat (depth-sorted) inputs, in their order."""
    n = means2d.shape[0]
    m, q, c, o = (t.contiguous() for t in (means2d, conics, colors, opacities))
    packed = torch.empty((n, _lib.RECORD_FLOATS), dtype=torch.float32, device=means2d.device)
    _lib.check(_lib.lib().gsplat_hip_pack_records(meta.raster, _lib.ptr(m), _lib.ptr(q), _lib.ptr(c), _lib.ptr(o),
                                                  _lib.ptr(packed), _lib.stream_of(means2d)),
               "gsplat_hip_pack_records")
    return packed


@dataclass
class _Ranges:
    """A binning over the tiles an operator covers: tile_offsets [T+1], ids grouped by tile in
    ascending tile order and ascending inside each tile, and where those ids sit in the caller's
    id buffer (positions, for the in-place write-back)."""
    tile_offsets: Tensor
    ids: Tensor
    positions: Tensor
    changed: bool


def _ranges(T: int, tiles: Tensor, starts: Tensor, counts: Tensor, ids: Tensor, n_splats: int,
            what: str) -> _Ranges:
    """tiles: int64 [k] distinct tile ids; tile tiles[j] holds ids[starts[j] : starts[j] + counts[j]].
    Every index is checked on the host before anything reads through it."""
    dev = ids.device
    k = tiles.numel()
    if k:
        lo_t, hi_t = int(tiles.min()), int(tiles.max())
        if lo_t < 0 or hi_t >= T:
            raise RuntimeError(f"{what}: tile id out of range [0, {T})")
        if int(starts.min()) < 0 or int(counts.min()) < 0 or int((starts + counts).max()) > ids.numel():
            raise RuntimeError(f"{what}: tile range outside binned ids ({ids.numel()} entries)")
        if torch.unique(tiles).numel() != k:
            raise RuntimeError(f"{what}: a tile is listed twice")
        order = torch.argsort(tiles)
        tiles, starts, counts = tiles[order], starts[order], counts[order]
    total = int(counts.sum()) if k else 0
    per_tile = torch.zeros(T, dtype=torch.int64, device=dev)
    if k:
        per_tile[tiles] = counts
    offsets = torch.zeros(T + 1, dtype=torch.int64, device=dev)
    offsets[1:] = torch.cumsum(per_tile, 0)
    if total >= 2 ** 31:
        raise RuntimeError(f"{what}: too many pairs")
    offsets = offsets.to(torch.int32)
    if total == 0:
        z = torch.zeros(1, dtype=torch.int32, device=dev)
        return _Ranges(offsets, z, z[:0].long(), False)
    excl = torch.cumsum(counts, 0) - counts
    pos = torch.repeat_interleave(starts - excl, counts, output_size=total) + torch.arange(total, device=dev)
    got = ids[pos].to(torch.int64)
    if int(got.min()) < 0 or int(got.max()) >= n_splats:
        raise RuntimeError(f"{what}: binned id out of range [0, {n_splats})")
    # depth order inside each tile = ascending flat index (the reference's per-tile sort)
    tile_of = torch.repeat_interleave(tiles, counts, output_size=total)
    key = (tile_of << 32) | got
    changed = bool((key[1:] <= key[:-1]).any()) if total > 1 else False
    if changed:
        key = torch.sort(key).values
    return _Ranges(offsets, (key & 0xFFFFFFFF).to(torch.int32).contiguous(), pos, changed)


def _fast_ranges(meta: V8Meta, tile_counts: Tensor, tile_offsets: Tensor, binned_ids: Tensor,
                 select: Tensor, what: str) -> _Ranges:
    """The ranges of the tiles in `select` (bool [T]) with 0 < count <= max_fast_pairs."""
    T = meta.tile_count
    if tile_counts.numel() != T or tile_offsets.numel() < T:
        raise RuntimeError(f"{what}: tile_counts must be [T] and tile_offsets [T+1] (T = {T})")
    counts = tile_counts.to(torch.int64)
    keep = select & (counts > 0) & (counts <= meta.max_fast_pairs)
    tiles = torch.nonzero(keep).flatten()
    return _ranges(T, tiles, tile_offsets[:T].to(torch.int64)[tiles], counts[tiles], binned_ids,
                   meta.batch * meta.gaussians_per_batch, what)


def _overflow_ranges(meta: V8Meta, tile_ids: Tensor, seg_offsets: Tensor, seg_ids: Tensor, what: str) -> _Ranges:
    k = tile_ids.numel()
    if seg_offsets.numel() != k + 1:
        raise RuntimeError(f"{what}: overflow_tile_offsets must have one more entry than overflow_tile_ids")
    so = seg_offsets.to(torch.int64)
    return _ranges(meta.tile_count, tile_ids.to(torch.int64), so[:-1], so[1:] - so[:-1], seg_ids,
                   meta.batch * meta.gaussians_per_batch, what)


def _forward(meta: V8Meta, packed: Tensor, r: _Ranges, save_state: bool):
    st = _ops.BinState(None, packed, None, r.tile_offsets, r.ids, r.ids.numel())
    return _ops.render_forward(meta.raster, st, save_state=save_state), st


def _backward(meta: V8Meta, packed: Tensor, r: _Ranges, grad_img: Tensor):
    """Forward replay for the state, then the backward; gradients flat, in the inputs' order."""
    (img, final_T, last, tile_stop, ws), st = _forward(meta, packed, r, True)
    g_m, g_q, g_c, g_o = _ops.render_backward(meta.raster, st, final_T, last, tile_stop, grad_img, ws)
    n = meta.batch * meta.gaussians_per_batch
    return g_m.reshape(n, 2), g_q.reshape(n, 3), g_c.reshape(n, 3), g_o.reshape(n)


def _check_grad_image(meta: V8Meta, g: Tensor, device) -> Tensor:
    if g.device != device or g.dtype != torch.float32:
        raise RuntimeError("grad_out must be float32 on the GPU (ROCm)")
    if tuple(g.shape) != (meta.batch, meta.height, meta.width, 3):
        raise RuntimeError(f"grad_out must be [B,H,W,3] = {(meta.batch, meta.height, meta.width, 3)}")
    return g.contiguous()


def _tile_pixels(meta: V8Meta, tile_ids: Tensor):
    """For [To] tile ids: (batch, y, x) int64 [To,16,16] of each tile pixel and whether it lies in
    the image."""
    dev = tile_ids.device
    t = tile_ids.to(torch.int64)
    b = t // meta.tiles_per_image
    lt = t % meta.tiles_per_image
    y0 = (lt // meta.tiles_x) * TILE
    x0 = (lt % meta.tiles_x) * TILE
    r = torch.arange(TILE, device=dev)
    y = y0[:, None, None] + r[None, :, None]
    x = x0[:, None, None] + r[None, None, :]
    y, x = torch.broadcast_tensors(y, x)
    bb = b[:, None, None].expand_as(y)
    valid = (y < meta.height) & (x < meta.width)
    return bb, y, x, valid


def _register():
    """Defines the nine operators (once per process).  The fake (meta) implementations give
    FakeTensor tracing the output shapes; sizes that only the host meta holds (B, H, W, T) and the
    pair count N are unbacked sizes there."""

    @torch.library.custom_op(f"{NAMESPACE}::bin", mutates_args=(),
                             schema=SCHEMAS["bin"])
    def bin(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor, meta_i32: Tensor,
            meta_f32: Tensor, meta_host_i32: Tensor, meta_host_f32: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
        _check_inputs(means2d, conics, colors, opacities)
        meta = parse_meta(meta_host_i32, meta_host_f32, means2d.shape[0])
        # equal depths: the stable depth order is the inputs' own order (they are depth-sorted)
        depths = torch.zeros(means2d.shape[0], dtype=torch.float32, device=means2d.device)
        st = _ops.bin_gaussians(meta.raster, means2d.contiguous(), conics.contiguous(), colors.contiguous(),
                                opacities.contiguous(), depths)
        return st.tile_counts.contiguous(), st.tile_offsets.clone(), st.binned_ids.clone()

    @bin.register_fake
    def _(means2d, conics, colors, opacities, meta_i32, meta_f32, meta_host_i32, meta_host_f32):
        ctx = torch.library.get_ctx()
        T, n = ctx.new_dynamic_size(), ctx.new_dynamic_size()
        return (means2d.new_empty((T,), dtype=torch.int32), means2d.new_empty((T + 1,), dtype=torch.int32),
                means2d.new_empty((n,), dtype=torch.int32))

    def _fast_eval(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32, tile_counts, tile_offsets,
                   binned_ids, select, what, check=None):
        """Validates everything (check(meta): an operator's own checks), then the tile ranges it
        covers and the records."""
        _check_inputs(means2d, conics, colors, opacities)
        meta = parse_meta(meta_host_i32, meta_host_f32, means2d.shape[0])
        dev = means2d.device
        for name, t in (("tile_counts", tile_counts), ("tile_offsets", tile_offsets), ("binned_ids", binned_ids)):
            _check_aux_i32(t, name, dev)
        if check is not None:
            check(meta)
        r = _fast_ranges(meta, tile_counts, tile_offsets, binned_ids, select(meta, dev), what)
        return meta, r, _packed(meta, means2d, conics, colors, opacities)

    def _all_tiles(meta, dev):
        return torch.ones(meta.tile_count, dtype=torch.bool, device=dev)

    def _active(ids):
        def sel(meta, dev):
            _check_aux_i32(ids, "active_tile_ids", dev)
            a = ids.to(torch.int64)
            if a.numel() and (int(a.min()) < 0 or int(a.max()) >= meta.tile_count):
                raise RuntimeError("active_tile_ids out of range")
            s = torch.zeros(meta.tile_count, dtype=torch.bool, device=dev)
            s[a] = True
            return s
        return sel

    @torch.library.custom_op(f"{NAMESPACE}::render_fast_forward_eval", mutates_args=(),
                             schema=SCHEMAS["render_fast_forward_eval"])
    def render_fast_forward_eval(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor,
                                 meta_i32: Tensor, meta_f32: Tensor, meta_host_i32: Tensor, meta_host_f32: Tensor,
                                 tile_counts: Tensor, tile_offsets: Tensor, binned_ids: Tensor) -> Tensor:
        meta, r, packed = _fast_eval(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32,
                                     tile_counts, tile_offsets, binned_ids, _all_tiles, "render_fast_forward_eval")
        (img, *_), _ = _forward(meta, packed, r, False)
        return img

    @torch.library.custom_op(f"{NAMESPACE}::render_active_forward_eval", mutates_args=(),
                             schema=SCHEMAS["render_active_forward_eval"])
    def render_active_forward_eval(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor,
                                   meta_i32: Tensor, meta_f32: Tensor, meta_host_i32: Tensor,
                                   meta_host_f32: Tensor, active_tile_ids: Tensor, tile_counts: Tensor,
                                   tile_offsets: Tensor, binned_ids: Tensor) -> Tensor:
        meta, r, packed = _fast_eval(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32,
                                     tile_counts, tile_offsets, binned_ids, _active(active_tile_ids),
                                     "render_active_forward_eval")
        (img, *_), _ = _forward(meta, packed, r, False)
        return img

    def _state_forward(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32, binned_ids,
                       tile_counts, tile_offsets, select, what):
        meta, r, packed = _fast_eval(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32,
                                     tile_counts, tile_offsets, binned_ids, select, what)
        if r.changed:
            # the reference writes each rendered tile's sorted ids back (gsplat_v8_kernels.metal:442)
            binned_ids.index_copy_(0, r.positions, r.ids)
        (img, _, _, tile_stop, _), _ = _forward(meta, packed, r, True)
        return img, tile_stop

    @torch.library.custom_op(f"{NAMESPACE}::render_fast_forward_state", mutates_args=("binned_ids",),
                             schema=SCHEMAS["render_fast_forward_state"])
    def render_fast_forward_state(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor,
                                  meta_i32: Tensor, meta_f32: Tensor, meta_host_i32: Tensor, meta_host_f32: Tensor,
                                  binned_ids: Tensor, tile_counts: Tensor,
                                  tile_offsets: Tensor) -> Tuple[Tensor, Tensor]:
        return _state_forward(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32, binned_ids,
                              tile_counts, tile_offsets, _all_tiles, "render_fast_forward_state")

    @torch.library.custom_op(f"{NAMESPACE}::render_active_forward_state", mutates_args=("binned_ids",),
                             schema=SCHEMAS["render_active_forward_state"])
    def render_active_forward_state(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor,
                                    meta_i32: Tensor, meta_f32: Tensor, meta_host_i32: Tensor,
                                    meta_host_f32: Tensor, binned_ids: Tensor, active_tile_ids: Tensor,
                                    tile_counts: Tensor, tile_offsets: Tensor) -> Tuple[Tensor, Tensor]:
        return _state_forward(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32, binned_ids,
                              tile_counts, tile_offsets, _active(active_tile_ids), "render_active_forward_state")

    def _saved_backward(grad_out, means2d, conics, colors, opacities, meta_host_i32, meta_host_f32, tile_counts,
                        tile_offsets, binned_ids, tile_stop_counts, select, what):
        grad = []

        def check(meta):
            _check_aux_i32(tile_stop_counts, "tile_stop_counts", means2d.device)
            grad.append(_check_grad_image(meta, grad_out, means2d.device))

        meta, r, packed = _fast_eval(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32,
                                     tile_counts, tile_offsets, binned_ids, select, what, check)
        return _backward(meta, packed, r, grad[0])

    @torch.library.custom_op(f"{NAMESPACE}::render_fast_backward_saved", mutates_args=(),
                             schema=SCHEMAS["render_fast_backward_saved"])
    def render_fast_backward_saved(grad_out: Tensor, means2d: Tensor, conics: Tensor, colors: Tensor,
                                   opacities: Tensor, meta_i32: Tensor, meta_f32: Tensor, meta_host_i32: Tensor,
                                   meta_host_f32: Tensor, tile_counts: Tensor, tile_offsets: Tensor,
                                   binned_ids: Tensor, tile_stop_counts: Tensor
                                   ) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
        return _saved_backward(grad_out, means2d, conics, colors, opacities, meta_host_i32, meta_host_f32,
                               tile_counts, tile_offsets, binned_ids, tile_stop_counts, _all_tiles,
                               "render_fast_backward_saved")

    @torch.library.custom_op(f"{NAMESPACE}::render_active_backward_saved", mutates_args=(),
                             schema=SCHEMAS["render_active_backward_saved"])
    def render_active_backward_saved(grad_out: Tensor, means2d: Tensor, conics: Tensor, colors: Tensor,
                                     opacities: Tensor, meta_i32: Tensor, meta_f32: Tensor, meta_host_i32: Tensor,
                                     meta_host_f32: Tensor, active_tile_ids: Tensor, tile_counts: Tensor,
                                     tile_offsets: Tensor, binned_ids: Tensor, tile_stop_counts: Tensor
                                     ) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
        return _saved_backward(grad_out, means2d, conics, colors, opacities, meta_host_i32, meta_host_f32,
                               tile_counts, tile_offsets, binned_ids, tile_stop_counts, _active(active_tile_ids),
                               "render_active_backward_saved")

    def _overflow_setup(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32, tile_ids, seg_offsets,
                        seg_ids, what, grad_tiles=None):
        _check_inputs(means2d, conics, colors, opacities)
        meta = parse_meta(meta_host_i32, meta_host_f32, means2d.shape[0])
        dev = means2d.device
        for name, t in (("overflow_tile_ids", tile_ids), ("overflow_tile_offsets", seg_offsets),
                        ("overflow_sorted_ids", seg_ids)):
            _check_aux_i32(t, name, dev)
        k = tile_ids.numel()
        if grad_tiles is not None and (grad_tiles.device != dev or grad_tiles.dtype != torch.float32
                                       or tuple(grad_tiles.shape) != (k, TILE, TILE, 3)):
            raise RuntimeError(f"grad_tiles must be float32 [{k},{TILE},{TILE},3] on the GPU (ROCm)")
        r = _overflow_ranges(meta, tile_ids, seg_offsets, seg_ids, what)
        return meta, r, _packed(meta, means2d, conics, colors, opacities)

    @torch.library.custom_op(f"{NAMESPACE}::render_overflow_forward", mutates_args=(),
                             schema=SCHEMAS["render_overflow_forward"])
    def render_overflow_forward(means2d: Tensor, conics: Tensor, colors: Tensor, opacities: Tensor,
                                meta_i32: Tensor, meta_f32: Tensor, meta_host_i32: Tensor, meta_host_f32: Tensor,
                                overflow_tile_ids: Tensor, overflow_tile_offsets: Tensor,
                                overflow_sorted_ids: Tensor) -> Tensor:
        meta, r, packed = _overflow_setup(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32,
                                          overflow_tile_ids, overflow_tile_offsets, overflow_sorted_ids,
                                          "render_overflow_forward")
        (img, *_), _ = _forward(meta, packed, r, False)
        b, y, x, valid = _tile_pixels(meta, overflow_tile_ids)
        tiles = img[b, y.clamp(max=meta.height - 1), x.clamp(max=meta.width - 1)]
        bg = torch.tensor(list(meta.raster.background), dtype=torch.float32, device=img.device)
        return torch.where(valid[..., None], tiles, bg).contiguous()

    @torch.library.custom_op(f"{NAMESPACE}::render_overflow_backward", mutates_args=(),
                             schema=SCHEMAS["render_overflow_backward"])
    def render_overflow_backward(grad_tiles: Tensor, means2d: Tensor, conics: Tensor, colors: Tensor,
                                 opacities: Tensor, meta_i32: Tensor, meta_f32: Tensor, meta_host_i32: Tensor,
                                 meta_host_f32: Tensor, overflow_tile_ids: Tensor, overflow_tile_offsets: Tensor,
                                 overflow_sorted_ids: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
        meta, r, packed = _overflow_setup(means2d, conics, colors, opacities, meta_host_i32, meta_host_f32,
                                          overflow_tile_ids, overflow_tile_offsets, overflow_sorted_ids,
                                          "render_overflow_backward", grad_tiles)
        grad = torch.zeros((meta.batch, meta.height, meta.width, 3), dtype=torch.float32, device=means2d.device)
        b, y, x, valid = _tile_pixels(meta, overflow_tile_ids)
        grad[b[valid], y[valid], x[valid]] = grad_tiles[valid]
        return _backward(meta, packed, r, grad)

    def _img_fake(means2d, meta_host_i32):
        ctx = torch.library.get_ctx()
        return means2d.new_empty((ctx.new_dynamic_size(), ctx.new_dynamic_size(), ctx.new_dynamic_size(), 3))

    def _grads_fake(means2d, conics, colors, opacities):
        return (torch.empty_like(means2d), torch.empty_like(conics), torch.empty_like(colors),
                torch.empty_like(opacities))

    @render_fast_forward_eval.register_fake
    def _(means2d, conics, colors, opacities, meta_i32, meta_f32, meta_host_i32, meta_host_f32, *rest):
        return _img_fake(means2d, meta_host_i32)

    @render_active_forward_eval.register_fake
    def _(means2d, conics, colors, opacities, meta_i32, meta_f32, meta_host_i32, meta_host_f32, *rest):
        return _img_fake(means2d, meta_host_i32)

    @render_fast_forward_state.register_fake
    def _(means2d, conics, colors, opacities, meta_i32, meta_f32, meta_host_i32, meta_host_f32, binned_ids,
          tile_counts, tile_offsets):
        return _img_fake(means2d, meta_host_i32), tile_counts.new_empty(tile_counts.shape)

    @render_active_forward_state.register_fake
    def _(means2d, conics, colors, opacities, meta_i32, meta_f32, meta_host_i32, meta_host_f32, binned_ids,
          active_tile_ids, tile_counts, tile_offsets):
        return _img_fake(means2d, meta_host_i32), tile_counts.new_empty(tile_counts.shape)

    @render_fast_backward_saved.register_fake
    def _(grad_out, means2d, conics, colors, opacities, *rest):
        return _grads_fake(means2d, conics, colors, opacities)

    @render_active_backward_saved.register_fake
    def _(grad_out, means2d, conics, colors, opacities, *rest):
        return _grads_fake(means2d, conics, colors, opacities)

    @render_overflow_forward.register_fake
    def _(means2d, conics, colors, opacities, meta_i32, meta_f32, meta_host_i32, meta_host_f32, tile_ids, *rest):
        return means2d.new_empty((tile_ids.shape[0], TILE, TILE, 3))

    @render_overflow_backward.register_fake
    def _(grad_tiles, means2d, conics, colors, opacities, *rest):
        return _grads_fake(means2d, conics, colors, opacities)


def registered() -> bool:
    """Whether this process has the namespace's operators (ours or another library's)."""
    try:
        torch.ops.gsplat_metal_v8.bin.default  # noqa: B018
        return True
    except (AttributeError, RuntimeError):
        return False


if not registered():
    _register()
