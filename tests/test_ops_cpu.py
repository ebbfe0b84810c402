"""CPU checks of the torch.library boundary (torch.ops.gsplat_hip.*): the
operators are registered with the expected schemas, and their fake
implementations give the output shapes and dtypes of the real ones under
FakeTensor tracing (no GPU needed), including the data-dependent pair count
of bin as an unbacked size."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.symbolic_shapes import ShapeEnv

import torch_gsplat_bridge_fast  # noqa: F401  (registers the operators)
from torch_gsplat_bridge_fast import RuntimeShaderConfig, get_runtime_shader_config

OPS = ("bin", "render_forward", "render_backward", "project_forward", "project_backward")


def test_operators_registered():
    for name in OPS:
        schema = str(getattr(torch.ops.gsplat_hip, name).default._schema)
        assert schema.startswith(f"gsplat_hip::{name}(")
    assert "float[] background" in str(torch.ops.gsplat_hip.bin.default._schema)


def test_runtime_shader_config_matches_reference_fields(monkeypatch):
    rt = get_runtime_shader_config()
    assert isinstance(rt, RuntimeShaderConfig)
    assert (rt.tile_size, rt.threads, rt.chunk_size, rt.simdgroups) == (16, 64, 64, 1)
    monkeypatch.setenv("GSP_CHUNK", "0")
    with pytest.raises(ValueError, match="GSP_CHUNK must be positive"):
        get_runtime_shader_config()
    monkeypatch.setenv("GSP_CHUNK", "32")
    with pytest.raises(ValueError, match="64-splat"):
        get_runtime_shader_config()


def test_fake_implementations_shapes():
    B, G, H, W = 2, 100, 40, 70
    T = B * 3 * 5
    with FakeTensorMode(shape_env=ShapeEnv()):
        f = lambda *s, **kw: torch.empty(*s, **kw)  # noqa: E731
        m2, q, c, o, d = f(B * G, 2), f(B * G, 3), f(B * G, 3), f(B * G), f(B * G)
        counts, offsets, ids, packed, perm = torch.ops.gsplat_hip.bin(m2, q, c, o, d, H, W, B, 1 / 255, 1e-4,
                                                                      [0.0, 0.0, 0.0])
        assert counts.shape == (T,) and offsets.shape == (T + 1,) and counts.dtype == torch.int32
        assert packed.shape == (B * G, 16) and perm.shape == (B * G,) and ids.dtype == torch.int32
        assert not isinstance(ids.shape[0], int)          # data-dependent pair count
        ids = f(500, dtype=torch.int32)
        img, fT, last, stop, ws = torch.ops.gsplat_hip.render_forward(packed, offsets, ids, H, W, B, G, 1 / 255,
                                                                      1e-4, [0.0, 0.0, 0.0], True)
        assert img.shape == (B, H, W, 3) and fT.shape == (B, H, W) and last.dtype == torch.int32
        assert stop.shape == (T,) and ws.dtype == torch.uint8 and ws.shape[0] > 0
        ev = torch.ops.gsplat_hip.render_forward(packed, offsets, ids, H, W, B, G, 1 / 255, 1e-4, [0.0, 0.0, 0.0],
                                                 False)
        assert ev[0].shape == (B, H, W, 3) and all(t.numel() == 0 for t in ev[1:])
        gm, gq, gc, go = torch.ops.gsplat_hip.render_backward(img, packed, offsets, ids, fT, last, stop, ws, H, W,
                                                              B, G, 1 / 255, 1e-4, [0.0, 0.0, 0.0])
        assert (gm.shape, gq.shape, gc.shape, go.shape) == ((B, G, 2), (B, G, 3), (B, G, 3), (B, G))
        m3, s3, q4, o1 = f(B * G, 3), f(B * G, 3), f(B * G, 4), f(B * G)
        c2w, cam = f(B, 4, 4), f(B, 4)
        out = torch.ops.gsplat_hip.project_forward(m3, s3, q4, o1, c2w, cam, 1e-4)
        assert [t.shape for t in out] == [(B * G, 2), (B * G, 3), (B * G,), (B * G,)]
        g = torch.ops.gsplat_hip.project_backward(*out, m3, s3, q4, o1, c2w, cam, 1e-4)
        assert [t.shape for t in g] == [(B * G, 3), (B * G, 3), (B * G, 4), (B * G,), (B, 4, 4), (B, 4)]
