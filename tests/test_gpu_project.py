"""GPU parity of the pinhole projection (project_pinhole_gaussians) and of the
full 3D path (rasterize_pinhole_gaussians).

Checker: oracle/dense_reference.project_pinhole_reference, the restatement of
the reference's projection (v9 rasterize.py:288-358), evaluated in float64 on
the CPU, with torch autograd for the VJP.  It is pinned on the CPU by closed
forms, fp64 gradcheck and the golden projection cases (tests/test_oracle_cpu.py).

Tolerances: means2d and depths rtol 1e-5 / atol 1e-4 px; projected opacity
exact; conics compared after dividing each splat's three entries by that
splat's largest |entry| (the inverse of the 2D covariance loses about
cond(cov2d) * 2^-24 relative to its largest entry in float32), rtol 1e-4 /
atol 1e-4.  Gradients rtol 1e-3 with atol 1e-5 times the tensor's largest
magnitude (float atomics reorder the per-camera sums).  The full 3D path is
compared with the dense Torch reference on the reference projection at the
image bar (rtol 1e-4 / atol 1e-5) and the gradient bar above.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle.dense_reference import dense_reference, project_pinhole_reference
from torch_gsplat_bridge_fast import RasterConfig, project_pinhole_gaussians, rasterize_pinhole_gaussians
from torch_gsplat_bridge_fast.scenes import make_scene_3d

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _rotation(seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(4, generator=g, dtype=torch.float64)
    q = q / q.norm()
    r, i, j, k = q.tolist()
    return torch.tensor([
        [1 - 2 * (j * j + k * k), 2 * (i * j - k * r), 2 * (i * k + j * r)],
        [2 * (i * j + k * r), 1 - 2 * (i * i + k * k), 2 * (j * k - i * r)],
        [2 * (i * k - j * r), 2 * (j * k + i * r), 1 - 2 * (i * i + j * j)],
    ], dtype=torch.float64)


def _scene(B, G, seed=0):
    """B cameras looking at a [-5,5]^3 cloud from about 15 units away; a few
    splats of every batch sit behind the camera."""
    per = [make_scene_3d(seed + b, G=G) for b in range(B)]
    m = torch.cat([p["means3d"] for p in per]).double()
    s = torch.cat([p["scales"] for p in per]).double()
    q = torch.cat([p["quats"] for p in per]).double()
    o = torch.cat([p["opacities"] for p in per]).double()
    c2w = torch.eye(4, dtype=torch.float64).repeat(B, 1, 1)
    for b in range(B):
        R = _rotation(100 + b) if b > 0 else torch.eye(3, dtype=torch.float64)
        c2w[b, :3, :3] = R
        c2w[b, :3, 3] = -15.0 * R[:, 2]        # camera on its own -z axis, 15 from the origin
        # splats behind the camera: 2 units behind its centre along its view axis
        m[b, :8] = c2w[b, :3, 3] - 2.0 * R[:, 2] + 0.1 * torch.arange(8, dtype=torch.float64)[:, None]
    cam = torch.tensor([[900.0, 880.0, 256.0, 240.0]], dtype=torch.float64).repeat(B, 1)
    cam[:, 0] += 25.0 * torch.arange(B)
    return m, s, q, o, c2w, cam


def _gpu_project(m, s, q, o, c2w, cam, near=1e-4, grads=False):
    dev = torch.device("cuda:0")
    ts = [t.float().to(dev).requires_grad_(grads) for t in (m, s, q, o)]
    c2w_d = c2w.float().to(dev).requires_grad_(grads)
    cam_d = cam.float().to(dev)
    fx, fy, cx, cy = (cam_d[:, i].clone().requires_grad_(grads) for i in range(4))
    out = project_pinhole_gaussians(*ts, fx, fy, cx, cy, camera_to_world=c2w_d, near_plane=near)
    return out, ts + [c2w_d, fx, fy, cx, cy]


def _conic_close(got, ref):
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    scale = np.maximum(np.abs(r).max(axis=-1, keepdims=True), 1e-30)
    np.testing.assert_allclose(g / scale, r / scale, rtol=1e-4, atol=1e-4, err_msg="conics")


def _grad_close(got, ref, name, rtol=1e-3, atol_rel=1e-5):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64).reshape(got.shape)
    atol = atol_rel * max(1.0, float(np.abs(ref).max()))
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=atol, err_msg=name)


@pytest.mark.parametrize("B,G", [(1, 4096), (2, 1500)])
def test_projection_forward_matches_reference(gpu, B, G):
    m, s, q, o, c2w, cam = _scene(B, G)
    print(f"projection forward B={B} G={G}", flush=True)
    (m2, cq, op, dp), _ = _gpu_project(m, s, q, o, c2w, cam)
    torch.cuda.synchronize()
    rm2, rcq, rop, rdp = project_pinhole_reference(m, s, q, o, c2w, cam)
    np.testing.assert_allclose(m2.detach().cpu().numpy(), rm2.numpy(), rtol=1e-5, atol=1e-4, err_msg="means2d")
    np.testing.assert_allclose(dp.detach().cpu().numpy(), rdp.numpy(), rtol=1e-5, atol=1e-4, err_msg="depths")
    np.testing.assert_array_equal(op.detach().cpu().numpy(), rop.float().numpy(), err_msg="opacities")
    _conic_close(cq.detach().cpu().numpy(), rcq.numpy())
    # behind-camera splats: opacity 0, centred at the principal point
    assert float(op[:, :8].abs().max()) == 0.0
    np.testing.assert_allclose(m2[:, :8].detach().cpu().numpy(),
                               cam[:, None, 2:4].expand(B, 8, 2).numpy(), rtol=0, atol=1e-4)


@pytest.mark.parametrize("B,G", [(1, 2048), (2, 700)])
def test_projection_backward_matches_reference(gpu, B, G):
    m, s, q, o, c2w, cam = _scene(B, G, seed=3)
    print(f"projection backward B={B} G={G}", flush=True)
    gen = torch.Generator().manual_seed(7)
    w = [torch.randn(B, G, 2, generator=gen, dtype=torch.float64),
         torch.randn(B, G, 3, generator=gen, dtype=torch.float64) * 1e3,
         torch.randn(B, G, generator=gen, dtype=torch.float64),
         torch.randn(B, G, generator=gen, dtype=torch.float64)]
    out, leaves = _gpu_project(m, s, q, o, c2w, cam, grads=True)
    loss = sum((t * wi.float().to(t.device)).sum() for t, wi in zip(out, w))
    loss.backward()
    torch.cuda.synchronize()
    ref_leaves = [t.clone().requires_grad_(True) for t in (m, s, q, o, c2w, cam)]
    rout = project_pinhole_reference(*ref_leaves)
    sum((t * wi).sum() for t, wi in zip(rout, w)).backward()
    names = ("means3d", "scales", "quats", "opacities", "camera_to_world")
    for name, got, ref in zip(names, leaves[:5], ref_leaves[:5]):
        _grad_close(got.grad.cpu().numpy(), ref.grad.numpy(), name)
    cam_grad = torch.stack([t.grad.cpu() for t in leaves[5:9]], dim=1)
    _grad_close(cam_grad.numpy(), ref_leaves[5].grad.numpy(), "camera_params")


def test_projection_golden_cases(gpu):
    with open(os.path.join(GOLDEN, "projection_cases.json")) as f:
        pc = json.load(f)
    i = {k: torch.tensor(v, dtype=torch.float64) for k, v in pc["inputs"].items()}
    (m2, cq, op, dp), _ = _gpu_project(i["means3d"], i["scales"], i["quats"], i["opacities"],
                                       i["camera_to_world"], i["camera_params"], near=pc["near_plane"])
    torch.cuda.synchronize()
    ref = {k: np.array(v) for k, v in pc["outputs"].items()}
    np.testing.assert_allclose(m2.detach().cpu().numpy(), ref["means2d"], rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(dp.detach().cpu().numpy(), ref["depths"], rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(op.detach().cpu().numpy(), ref["opacities_out"].astype(np.float32))
    _conic_close(cq.detach().cpu().numpy(), ref["conics"])


def test_rasterize_pinhole_end_to_end(gpu):
    """Full 3D path (project + bin + composite, forward and backward) against
    the reference projection followed by the dense Torch reference, in fp32 on
    the CPU, 128x128, G=256, loss = sum(img * w)."""
    H = W = 128
    G = 256
    sc = make_scene_3d(11, G=G, H=H, W=W, adversarial_fraction=0.0)
    f = 180.0
    c2w = torch.eye(4)
    c2w[2, 3] = -15.0
    cam = torch.tensor([[f, f, W / 2.0, H / 2.0]])
    w = torch.rand(1, H, W, 3, generator=torch.Generator().manual_seed(5))
    keys = ("means3d", "scales", "quats", "opacities")
    # reference: CPU fp32 autograd through projection + dense compositing
    r_leaves = [sc[k].clone().requires_grad_(True) for k in keys]
    rm2, rcq, rop, rdp = project_pinhole_reference(*r_leaves, c2w.unsqueeze(0), cam)
    rimg = dense_reference(rm2, rcq, sc["colors"], rop, rdp, H, W, early_stop=True)
    (rimg * w).sum().backward()
    # GPU
    dev = torch.device("cuda:0")
    leaves = [sc[k].to(dev).clone().requires_grad_(True) for k in keys]
    img = rasterize_pinhole_gaussians(*leaves, sc["colors"].to(dev), f, f, W / 2.0, H / 2.0,
                                      camera_to_world=c2w.to(dev), config=RasterConfig(height=H, width=W))
    (img * w.to(dev)).sum().backward()
    torch.cuda.synchronize()
    assert float(img.detach().abs().max()) > 0.05       # the scene is visible
    np.testing.assert_allclose(img.detach().cpu().numpy(), rimg.detach().numpy(), rtol=1e-4, atol=1e-5)
    for name, g, r in zip(keys, leaves, r_leaves):
        _grad_close(g.grad.cpu().numpy(), r.grad.numpy(), name)
