"""GPU: the allocation-free projection backward
(gsplat_hip_project_backward_noalloc) against gsplat_hip_project_backward,
both called through the C ABI on the same inputs.  They run the same
kernels in the same order (no atomics), so every output must be bit
identical.  Two calls in a row, the second with a smaller input (the static
scratch keeps the first call's partial sums, which the second must not
read), then the first shape again; a problem beyond the scratch is refused
with an error before anything is launched."""
import numpy as np
import pytest
import torch

from torch_gsplat_bridge_fast import _lib
from torch_gsplat_bridge_fast.scenes import make_scene_3d

pytestmark = pytest.mark.gpu


def _inputs(B, G, seed, dev):
    per = [make_scene_3d(seed + b, G=G) for b in range(B)]
    cat = {k: torch.cat([p[k] for p in per]).reshape(B * G, -1).squeeze(-1).contiguous().to(dev)
           for k in ("means3d", "scales", "quats", "opacities")}
    c2w = torch.eye(4).repeat(B, 1, 1)
    c2w[:, 2, 3] = -15.0 - torch.arange(B, dtype=torch.float32)
    cam = torch.tensor([[900.0, 880.0, 256.0, 240.0]]).repeat(B, 1)
    g = torch.Generator().manual_seed(seed)
    cot = [torch.randn(B * G, 2, generator=g), torch.randn(B * G, 3, generator=g) * 1e3,
           torch.randn(B * G, generator=g), torch.randn(B * G, generator=g)]
    return cat, c2w.contiguous().to(dev), cam.contiguous().to(dev), [c.contiguous().to(dev) for c in cot]


def _outputs(B, G, dev):
    return [torch.full(s, float("nan"), device=dev) for s in
            ((B * G, 3), (B * G, 3), (B * G, 4), (B * G,), (B, 4, 4), (B, 4))]


def _run(B, G, seed, dev):
    L = _lib.lib()
    meta = _lib.make_project_meta(B, G, 1e-4)
    x, c2w, cam, cot = _inputs(B, G, seed, dev)
    args = [_lib.ptr(t) for t in cot] + [_lib.ptr(x[k]) for k in ("means3d", "scales", "quats", "opacities")] + \
           [_lib.ptr(c2w), _lib.ptr(cam)]
    ref = _outputs(B, G, dev)
    wsb = L.gsplat_hip_project_backward_workspace_bytes(meta)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    stream = _lib.stream_of(ws)
    _lib.check(L.gsplat_hip_project_backward(meta, *args, *[_lib.ptr(t) for t in ref], _lib.ptr(ws), wsb, stream),
               "gsplat_hip_project_backward")
    got = _outputs(B, G, dev)
    _lib.check(L.gsplat_hip_project_backward_noalloc(meta, *args, *[_lib.ptr(t) for t in got], stream),
               "gsplat_hip_project_backward_noalloc")
    torch.cuda.synchronize()
    for name, a, b in zip(("means3d", "scales", "quats", "opacities", "camera_to_world", "camera_params"), got, ref):
        assert torch.equal(a, b), name
    return ref


def test_noalloc_matches_workspace_entry_point(gpu):
    print("noalloc: B=2 G=300000", flush=True)
    first = _run(2, 300_000, 1, gpu)
    print("noalloc: B=1 G=5000 (smaller, right after)", flush=True)
    _run(1, 5_000, 2, gpu)
    print("noalloc: B=2 G=300000 again", flush=True)
    again = _run(2, 300_000, 1, gpu)
    for a, b in zip(first, again):
        assert torch.equal(a, b)


def test_noalloc_rejects_problems_beyond_its_scratch(gpu):
    L = _lib.lib()
    limit = _lib.PROJECT_NOALLOC_SCRATCH_BYTES // 64          # B * ceil(G / 256)
    meta = _lib.make_project_meta(1, limit * 256 + 1, 1e-4)
    dummy = torch.zeros(16, device=gpu)
    p = _lib.ptr(dummy)
    rc = L.gsplat_hip_project_backward_noalloc(meta, *([p] * 16), _lib.stream_of(dummy))
    assert rc == 1
    assert b"exceeds the static scratch" in L.gsplat_hip_last_error()
    # the largest accepted size at the limit needs exactly the whole scratch
    assert L.gsplat_hip_project_backward_workspace_bytes(_lib.make_project_meta(1, limit * 256, 1e-4)) == \
        _lib.PROJECT_NOALLOC_SCRATCH_BYTES
