"""CPU checks of the Python API's host logic: input validation (same errors
as the reference's rasterize.py:85-107 and :197-226), config handling,
batching helpers, scene generators and bench.py's contract for --gpus."""
import os
import subprocess
import sys

import pytest
import torch

from torch_gsplat_bridge_fast import (RasterConfig, profile_projected_gaussians, project_pinhole_gaussians,
                                      rasterize_pinhole_gaussians, rasterize_projected_gaussians)
from torch_gsplat_bridge_fast import rasterize as R
from torch_gsplat_bridge_fast.scenes import CONFIGS, make_scene_2d, make_scene_3d

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _inputs(B=None, G=8, device="cpu", dtype=torch.float32):
    shape = (G,) if B is None else (B, G)
    return (torch.zeros(*shape, 2, dtype=dtype, device=device), torch.ones(*shape, 3, dtype=dtype, device=device),
            torch.zeros(*shape, 3, dtype=dtype, device=device), torch.ones(*shape, dtype=dtype, device=device),
            torch.zeros(*shape, dtype=dtype, device=device))


def test_cpu_tensors_rejected():
    with pytest.raises(ValueError, match="ROCm device"):
        rasterize_projected_gaussians(*_inputs(), RasterConfig(16, 16))


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: (a[0].unsqueeze(0).unsqueeze(0),) + a[1:], "must have shape"),
    (lambda a: (a[0], a[1][..., :2]) + a[2:], "conics must have last dim = 3"),
    (lambda a: (a[0][..., :1],) + a[1:], "means2d must have last dim = 2"),
    (lambda a: a[:2] + (a[2][..., :2],) + a[3:], "colors must have last dim = 3"),
    (lambda a: a[:3] + (a[3][:4],) + a[4:], "opacities/depths batch/G dimensions must match"),
    (lambda a: a[:3] + (a[3].double(),) + a[4:], "opacities must be float32"),
    (lambda a: a[:4] + (a[4].unsqueeze(-1),), "rank must be one less"),
])
def test_input_validation_messages(mutate, msg):
    with pytest.raises(ValueError, match=msg):
        rasterize_projected_gaussians(*mutate(_inputs()), RasterConfig(16, 16))


@pytest.mark.parametrize("kw,msg", [
    (dict(tile_size=8), "tile_size=8 does not match"),
    (dict(max_fast_pairs=4096), "exceeds compiled fast cap"),
    (dict(batch_strategy="x"), "batch_strategy"),
    (dict(active_policy="x"), "active_policy"),
    (dict(stop_count_mode="x"), "stop_count_mode"),
    (dict(stop_count_dense_threshold=0), "stop_count_dense_threshold"),
    (dict(max_pairs_per_launch=-1), "max_pairs_per_launch"),
])
def test_config_validation(kw, msg):
    with pytest.raises(ValueError, match=msg):
        R._runtime_validate(RasterConfig(16, 16, **kw))


def test_env_tile_size(monkeypatch):
    monkeypatch.setenv("GSP_TILE_SIZE", "32")
    with pytest.raises(ValueError, match="not supported"):
        R.get_runtime_shader_config()
    monkeypatch.setenv("GSP_TILE_SIZE", "7")
    with pytest.raises(ValueError, match="one of 8, 16, 32"):
        R.get_runtime_shader_config()
    monkeypatch.setenv("GSP_TILE_SIZE", "16")
    monkeypatch.setenv("GSP_FAST_CAP", "4096")
    assert R.get_runtime_shader_config().fast_cap == 4096
    R._runtime_validate(RasterConfig(16, 16, max_fast_pairs=4096))


def test_batch_chunking_matches_reference_rule():
    cfg = RasterConfig(4096, 4096)
    tpi = 256 * 256
    assert R._choose_batch_chunk_size(cfg, 1, 65536, tpi) == 1
    assert R._choose_batch_chunk_size(cfg, 8, 65536, tpi) == 4
    assert R._choose_batch_chunk_size(RasterConfig(64, 64, batch_strategy="serial"), 8, 10, 16) == 1
    assert R._choose_batch_chunk_size(RasterConfig(64, 64, batch_strategy="flatten"), 8, 10, 16) == 8


def test_active_policy_alias():
    assert R._effective_active_policy(RasterConfig(16, 16, use_active_tiles=True)) == "on"
    assert R._effective_active_policy(RasterConfig(16, 16, active_policy="auto")) == "auto"


def test_profile_and_projection_validate_on_cpu():
    with pytest.raises(ValueError):
        profile_projected_gaussians(*_inputs(), RasterConfig(16, 16))
    m3 = torch.zeros(5, 3)
    with pytest.raises(ValueError, match="ROCm device"):
        project_pinhole_gaussians(m3, torch.ones(5, 3), torch.ones(5, 4), torch.ones(5), 1.0, 1.0, 0.0, 0.0)
    with pytest.raises(ValueError, match="config is required"):
        rasterize_pinhole_gaussians(m3, torch.ones(5, 3), torch.ones(5, 4), torch.ones(5), torch.ones(5, 3), 1, 1, 0, 0)


def test_scenes_deterministic_and_shaped():
    a = make_scene_2d(0, seed=0)
    b = make_scene_2d(0, seed=0)
    for k in ("means2d", "conics", "colors", "opacities", "depths"):
        assert torch.equal(a[k], b[k])
    assert a["means2d"].shape == (1, 512, 2) and a["conics"].dtype == torch.float32
    c3 = make_scene_2d(3, seed=0, G=1000)
    assert c3["means2d"].shape == (4, 1000, 2) and (c3["H"], c3["W"]) == (512, 1024)
    # conics are symmetric positive definite
    q = a["conics"][0]
    assert bool(((q[:, 0] * q[:, 2] - q[:, 1] ** 2) > 0).all())
    s3 = make_scene_3d(seed=0, G=1000)
    assert s3["means3d"].shape == (1, 1000, 3)
    assert torch.allclose(s3["quats"].norm(dim=-1), torch.ones(1, 1000), atol=1e-6)
    assert set(CONFIGS) == {0, 1, 2, 3, 4}


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_pair_capacity_is_clamped_to_the_sort_limit(monkeypatch):
    """A capacity remembered for a shape never exceeds the pair sort's limit
    when the count itself fits (a larger one would make every later call of
    the shape fail); counts above the limit keep their headroom (and fail
    loudly in the sort)."""
    from torch_gsplat_bridge_fast import _ops

    monkeypatch.setattr(_ops, "MAX_PAIRS", 1000)
    assert _ops._headroom(10) == 10 + 2 + 4096 if 10 + 2 + 4096 <= 1000 else _ops._headroom(10) == 1000
    assert _ops._headroom(900) == 1000
    assert _ops._headroom(1000) == 1000
    assert _ops._headroom(1001) == 1001 + 250 + 4096
    monkeypatch.setattr(_ops, "MAX_PAIRS", 1 << 29)
    n = 429_493_500                         # 1.25 n + 4096 > 2^29 >= n
    assert _ops._headroom(n) == 1 << 29
    assert _ops._headroom(1000) == 1000 + 250 + 4096


class _DoneEvent:
    def synchronize(self):
        pass


def test_binning_status_word_raises():
    """check_status turns a set status word into RuntimeError (and a zero one
    into nothing); it waits on the status event first."""
    import torch

    from torch_gsplat_bridge_fast import _ops

    def state(word):
        host = torch.tensor([[123, word]], dtype=torch.int32)
        t = torch.zeros(1)
        return _ops.BinState(None, t, None, t, t, 1, host, _DoneEvent(), None, None, (0, 0), host, (0, 1),
                             _DoneEvent())

    state(0).check_status()
    with pytest.raises(RuntimeError, match="look-back wait gave up"):
        state(1).check_status()
    with pytest.raises(RuntimeError, match="device status"):
        state(4).check_status()
    assert state(0).n_pairs == 123
