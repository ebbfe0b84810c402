"""CPU checks of the reference's operator namespace, torch.ops.gsplat_metal_v8.* (v8_ops.py).

The nine operators that variants/v8/csrc/bindings.cpp:201-209 defines are registered with the
argument names, order, in-place binned_ids and result counts that the reference's Python calls
them with (v8 rasterize.py:368-757); their fake implementations trace under FakeTensorMode; the
meta tensors are parsed as ParsedMeta does and malformed ones raise the reference's messages;
CPU inputs are rejected before anything runs."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.symbolic_shapes import ShapeEnv

import torch_gsplat_bridge_fast  # noqa: F401  (registers the operators)
from torch_gsplat_bridge_fast import v8_ops

META = ["means2d", "conics", "colors", "opacities", "meta_i32", "meta_f32", "meta_host_i32", "meta_host_f32"]
# name -> (argument names in order, the argument written in place or None, number of results)
SPEC = {
    "bin": (META, None, 3),
    "render_fast_forward_eval": (META + ["tile_counts", "tile_offsets", "binned_ids"], None, 1),
    "render_fast_forward_state": (META + ["binned_ids", "tile_counts", "tile_offsets"], "binned_ids", 2),
    "render_fast_backward_saved": (["grad_out"] + META + ["tile_counts", "tile_offsets", "binned_ids",
                                                         "tile_stop_counts"], None, 4),
    "render_active_forward_eval": (META + ["active_tile_ids", "tile_counts", "tile_offsets", "binned_ids"], None, 1),
    "render_active_forward_state": (META + ["binned_ids", "active_tile_ids", "tile_counts", "tile_offsets"],
                                    "binned_ids", 2),
    "render_active_backward_saved": (["grad_out"] + META + ["active_tile_ids", "tile_counts", "tile_offsets",
                                                           "binned_ids", "tile_stop_counts"], None, 4),
    "render_overflow_forward": (META + ["overflow_tile_ids", "overflow_tile_offsets", "overflow_sorted_ids"],
                                None, 1),
    "render_overflow_backward": (["grad_tiles"] + META + ["overflow_tile_ids", "overflow_tile_offsets",
                                                         "overflow_sorted_ids"], None, 4),
}


def _ref_meta(H=40, W=70, B=2, G=100, max_fast=2048, bg=(0.0, 0.0, 0.0)):
    ty, tx = (H + 15) // 16, (W + 15) // 16
    hi = torch.tensor([H, W, ty, tx, 16, B * G, B * ty * tx, max_fast, B, G, ty * tx, 0, 64, 0], dtype=torch.int32)
    hf = torch.tensor([1 / 255, 1e-4, *bg, 1e-8, 0.99], dtype=torch.float32)
    return hi, hf


def test_schemas_are_the_references():
    for name, (args, mutated, n_out) in SPEC.items():
        schema = getattr(torch.ops.gsplat_metal_v8, name).default._schema
        assert schema.name == f"gsplat_metal_v8::{name}"
        assert [a.name for a in schema.arguments] == args, name
        assert all(str(a.type) == "Tensor" for a in schema.arguments)
        written = [a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write]
        assert written == ([mutated] if mutated else []), name
        assert len(schema.returns) == n_out and all(str(r.type) == "Tensor" for r in schema.returns), name
    assert "Tensor(a!) binned_ids" in str(torch.ops.gsplat_metal_v8.render_fast_forward_state.default._schema)


def test_parse_meta_reads_the_reference_layout():
    hi, hf = _ref_meta(H=37, W=53, B=3, G=77, max_fast=300, bg=(0.1, 0.2, 0.3))
    m = v8_ops.parse_meta(hi, hf, 3 * 77)
    assert (m.height, m.width, m.batch, m.gaussians_per_batch, m.max_fast_pairs) == (37, 53, 3, 77, 300)
    assert (m.tiles_y, m.tiles_x, m.tiles_per_image, m.tile_count) == (3, 4, 12, 36)
    r = m.raster
    assert (r.height, r.width, r.batch, r.gaussians_per_batch, r.tile_size) == (37, 53, 3, 77, 16)
    assert abs(r.alpha_threshold - 1 / 255) < 1e-9 and abs(r.background[2] - 0.3) < 1e-7
    assert abs(r.max_alpha - 0.99) < 1e-7 and abs(r.eps - 1e-8) < 1e-15


@pytest.mark.parametrize("index,value,msg", [
    (4, 8, "meta.tile_size must match shader tile size 16"),
    (7, 4096, "meta.max_fast_pairs exceeds shader compile-time cap 2048"),
    (8, 0, "meta.batch_size must be positive"),
    (9, 0, "meta.gaussians_per_batch must be positive"),
    (10, 99, "meta.tiles_per_image mismatch"),
    (5, 7, "flattened Gaussian count mismatch"),
    (6, 1000, "disagree"),
])
def test_parse_meta_errors(index, value, msg):
    hi, hf = _ref_meta()
    hi[index] = value
    with pytest.raises(RuntimeError, match=msg):
        v8_ops.parse_meta(hi, hf, 200)


def test_host_meta_must_be_on_the_cpu_and_inputs_on_the_gpu():
    hi, hf = _ref_meta()
    with pytest.raises(RuntimeError, match="host meta_i32 must be on CPU"):
        v8_ops.parse_meta(hi.to("meta"), hf, 200)
    f = lambda *s: torch.zeros(*s)  # noqa: E731
    with pytest.raises(RuntimeError, match="means2d must be on the GPU"):
        torch.ops.gsplat_metal_v8.bin(f(200, 2), f(200, 3), f(200, 3), f(200), hi, hf, hi, hf)
    with pytest.raises(RuntimeError, match="must be on the GPU"):
        torch.ops.gsplat_metal_v8.render_fast_forward_eval(f(200, 2), f(200, 3), f(200, 3), f(200), hi, hf, hi, hf,
                                                           hi, hi, hi)


def test_fake_implementations_shapes():
    B, G = 2, 100
    with FakeTensorMode(shape_env=ShapeEnv()):
        f = lambda *s, **kw: torch.empty(*s, device="cuda", **kw)  # noqa: E731
        m2, q, c, o = f(B * G, 2), f(B * G, 3), f(B * G, 3), f(B * G)
        hi, hf = torch.empty(14, dtype=torch.int32), torch.empty(7)
        mi, mf = f(14, dtype=torch.int32), f(7)
        ops = torch.ops.gsplat_metal_v8
        counts, offsets, ids = ops.bin(m2, q, c, o, mi, mf, hi, hf)
        assert counts.dtype == offsets.dtype == ids.dtype == torch.int32
        assert not isinstance(ids.shape[0], int)            # the data-dependent pair count
        counts, offsets, ids = f(30, dtype=torch.int32), f(31, dtype=torch.int32), f(500, dtype=torch.int32)
        img, stop = ops.render_fast_forward_state(m2, q, c, o, mi, mf, hi, hf, ids, counts, offsets)
        assert img.dim() == 4 and img.shape[3] == 3 and stop.shape == (30,) and stop.dtype == torch.int32
        ev = ops.render_fast_forward_eval(m2, q, c, o, mi, mf, hi, hf, counts, offsets, ids)
        assert ev.dim() == 4
        act = f(7, dtype=torch.int32)
        img, stop = ops.render_active_forward_state(m2, q, c, o, mi, mf, hi, hf, ids, act, counts, offsets)
        assert stop.shape == (30,)
        g = ops.render_fast_backward_saved(img, m2, q, c, o, mi, mf, hi, hf, counts, offsets, ids, stop)
        assert [t.shape for t in g] == [(B * G, 2), (B * G, 3), (B * G, 3), (B * G,)]
        g = ops.render_active_backward_saved(img, m2, q, c, o, mi, mf, hi, hf, act, counts, offsets, ids, stop)
        assert [t.shape for t in g] == [(B * G, 2), (B * G, 3), (B * G, 3), (B * G,)]
        ov = f(5, dtype=torch.int32)
        tiles = ops.render_overflow_forward(m2, q, c, o, mi, mf, hi, hf, ov, f(6, dtype=torch.int32), ids)
        assert tiles.shape == (5, 16, 16, 3)
        g = ops.render_overflow_backward(tiles, m2, q, c, o, mi, mf, hi, hf, ov, f(6, dtype=torch.int32), ids)
        assert [t.shape for t in g] == [(B * G, 2), (B * G, 3), (B * G, 3), (B * G,)]
