"""GPU parity of the pinhole projection (project_pinhole_gaussians) and of the
full 3D path (rasterize_pinhole_gaussians), up to config 4's full workload.

Checker: the projection and its VJP evaluated in float64 with a first-order
float32 running error bound (oracle/projection_bounds.py), whose values are
pinned on the CPU against float64 autograd through
oracle/dense_reference.project_pinhole_reference (itself pinned by closed
forms, fp64 gradcheck and the golden projection cases).

Bars: projected values |got - ref| <= 1e-7 |ref| + 2 err (err: the running
bound); projected opacity exact; gradients |got - ref| <= 1e-5 + 1e-3 |ref|
+ 2 err, per entry.  For the full 3D path the reference gradients are the
VJP of the tile oracle's 2D gradients (computed at the GPU's projected
values), and err also carries the 2D gradients' own allowance
(oracle/parity.py) through the VJP.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import parity
from oracle import projection_bounds as PB
from oracle import tile_oracle as TO
from oracle.dense_reference import dense_reference
from torch_gsplat_bridge_fast import (RasterConfig, project_pinhole_gaussians, rasterize_pinhole_gaussians,
                                      rasterize_projected_gaussians)
from torch_gsplat_bridge_fast import _lib, _ops
from torch_gsplat_bridge_fast.scenes import make_scene_3d

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
KEYS2 = ("means2d", "conics", "colors", "opacities", "depths")
KEYS3 = ("means3d", "scales", "quats", "opacities")


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


def _np(t):
    return t.detach().cpu().double().numpy()


def _check_forward(out, m, s_, q, o, c2w, cam, near=1e-4):
    """GPU projected values against the running-error forward."""
    m2, cq, op, dp = out
    B, G = m.shape[:2]
    fw = PB.project_forward(_np(m), _np(s_), _np(q), _np(o), _np(c2w), _np(cam), near)
    assert not fw["ambiguous"].any()
    PB.assert_close(_np(m2).reshape(B * G, 2), fw["means2d"], "means2d", rtol=1e-7, atol=1e-30)
    PB.assert_close(_np(cq).reshape(B * G, 3), fw["conics"], "conics", rtol=1e-7, atol=1e-30)
    PB.assert_close(_np(dp).reshape(B * G), fw["depths"], "depths", rtol=1e-7, atol=1e-30)
    np.testing.assert_array_equal(_np(op).reshape(-1), fw["opacities"].v, err_msg="opacities")


@pytest.mark.parametrize("B,G", [(1, 4096), (2, 1500)])
def test_projection_forward_matches_reference(gpu, B, G):
    m, s, q, o, c2w, cam = _scene(B, G)
    print(f"projection forward B={B} G={G}", flush=True)
    (m2, cq, op, dp), _ = _gpu_project(m, s, q, o, c2w, cam)
    torch.cuda.synchronize()
    _check_forward((m2, cq, op, dp), *(t.float() for t in (m, s, q, o, c2w, cam)))
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
    inp = [_np(t.float()) for t in (m, s, q, o, c2w, cam)]
    r = PB.project_vjp(*inp, *(_np(wi.float()) for wi in w))
    assert not r["ambiguous"].any()
    for key, leaf in zip(KEYS3, leaves[:4]):
        PB.assert_close(_np(leaf.grad).reshape(B * G, -1), r[key], key)
    PB.assert_close(_np(leaves[4].grad).reshape(B, 16), r["camera_to_world"], "camera_to_world")
    cam_grad = torch.stack([t.grad.cpu() for t in leaves[5:9]], dim=1)
    PB.assert_close(cam_grad.double().numpy(), r["camera_params"], "camera_params")


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
    cg, cr = cq.detach().cpu().double().numpy(), np.asarray(ref["conics"])
    scale = np.abs(cr).max(axis=-1, keepdims=True)
    np.testing.assert_allclose(cg / scale, cr / scale, rtol=1e-5, atol=1e-6)


def three_d_parity(m3, s3, q3, o3, colors, c2w, cam, H, W, w, img, g3d, g_colors, label, near=1e-4):
    """The full 3D path of one GPU run (img, g3d = gradients of means3d /
    scales / quats / opacities, g_colors) against the oracle:
      1. the GPU's projected values against the running-error forward;
      2. binning of those values bit-exact against the tile oracle;
      3. image at every pixel and the 2D gradients (a separate GPU run of
         rasterize_projected_gaussians on the projected values) at the
         raster bar; colour gradients of the 3D run at the same bar;
      4. 3D gradients against the VJP of the oracle's 2D gradients, with the
         2D allowance carried through it.
    Tensors are CPU float32 [B,G,..]; c2w [B,4,4]; cam [B,4]."""
    dev = torch.device("cuda:0")
    B, G = m3.shape[:2]
    with torch.no_grad():
        proj = project_pinhole_gaussians(m3.to(dev), s3.to(dev), q3.to(dev), o3.to(dev), cam[:, 0].to(dev),
                                         cam[:, 1].to(dev), cam[:, 2].to(dev), cam[:, 3].to(dev),
                                         camera_to_world=c2w.to(dev), near_plane=near)
    print(f"{label}: projection forward", flush=True)
    _check_forward(proj, m3, s3, q3, o3, c2w, cam, near)
    sc2 = {"means2d": proj[0].cpu(), "conics": proj[1].cpu(), "colors": colors, "opacities": proj[2].cpu(),
           "depths": proj[3].cpu()}
    # 2. binning
    print(f"{label}: binning", flush=True)
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    flat = [p.reshape(B * G, -1).squeeze(-1).contiguous() for p in (proj[0], proj[1], colors.to(dev), proj[2],
                                                                      proj[3])]
    st = _ops.bin_gaussians(meta, *flat)
    ometa = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(sc2[k].numpy() for k in KEYS2), B, G)
    bins = TO.bin_scene(ometa, s)
    np.testing.assert_array_equal(st.perm.cpu().numpy(), bins.perm, err_msg="depth order")
    np.testing.assert_array_equal(st.tile_offsets.cpu().numpy(), bins.tile_offsets, err_msg="tile ranges")
    assert st.n_pairs == bins.binned_ids.size
    np.testing.assert_array_equal(st.binned_ids.cpu().numpy(), bins.binned_ids, err_msg="sorted pair ids")
    print(f"{label}: {bins.binned_ids.size} pairs bit-exact", flush=True)
    # 3. image and 2D gradients
    _, _, last, _, _ = _ops.render_forward(meta, st, save_state=True)
    del st
    force, (oimg, _, _, _), rep = parity.gpu_decisions(ometa, s, bins, last.cpu().numpy())
    parity.check_image(np.asarray(img), oimg, label)
    w_np = np.asarray(w, dtype=np.float32).reshape(B, H, W, 3)
    ograds, bounds = TO.render_backward(ometa, s, bins, w_np, force_last=force, with_bounds=True)
    leaves2 = [sc2[k].to(dev).requires_grad_(k != "depths") for k in KEYS2]
    img2 = rasterize_projected_gaussians(*leaves2, RasterConfig(height=H, width=W))
    (img2 * torch.as_tensor(w_np).to(dev)).sum().backward()
    assert torch.equal(img2.detach().cpu(), torch.as_tensor(np.asarray(img)))
    tiles = parity.tiles_per_splat(bins, B, G)
    g2 = [leaves2[i].grad.cpu().numpy() for i in range(4)]
    grep = parity.check_grads(g2, ograds, bounds, tiles, f"{label} 2D")
    parity.check_grads([g2[0], g2[1], np.asarray(g_colors), g2[3]], ograds, bounds, tiles, f"{label} colors")
    print(f"{label}: image and 2D gradients at the bar ({rep}); 2D error / allowance "
          + ", ".join(f"{k} {v['max_over_allowance']:.3g}" for k, v in grep.items()), flush=True)
    # 4. 3D gradients through the VJP
    ref9 = np.concatenate([np.asarray(g, np.float64).reshape(B * G, -1) for g in ograds], axis=1)
    allow = parity.grad_allowance(ref9, bounds, tiles)
    g_err = {"means2d": allow[:, 0:2], "conics": allow[:, 2:5], "opacities": allow[:, 8]}
    r = PB.project_vjp(*(t.double().numpy() for t in (m3, s3, q3, o3, c2w, cam)),
                       ograds[0].reshape(B, G, 2), ograds[1].reshape(B, G, 3), ograds[3].reshape(B, G),
                       np.zeros((B, G)), near, g_err=g_err)
    worst = {}
    for key, g in zip(KEYS3, g3d):
        worst[key] = PB.assert_close(np.asarray(g, np.float64).reshape(B * G, -1), r[key], f"{label} {key}")
    print(f"{label}: 3D gradients at the bar; error / allowance {worst}", flush=True)
    return bins


def test_rasterize_pinhole_end_to_end(gpu):
    """Full 3D path (project + bin + composite, forward and backward) at
    128x128, G=256: image against the dense Torch reference on the
    reference projection (fp32 on the CPU), and everything against the
    oracle (three_d_parity)."""
    from oracle.dense_reference import project_pinhole_reference

    H = W = 128
    G = 256
    sc = make_scene_3d(11, G=G, H=H, W=W, adversarial_fraction=0.0)
    f = 180.0
    c2w = torch.eye(4)
    c2w[2, 3] = -15.0
    cam = torch.tensor([[f, f, W / 2.0, H / 2.0]])
    w = torch.rand(1, H, W, 3, generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        rm2, rcq, rop, rdp = project_pinhole_reference(*(sc[k] for k in KEYS3), c2w.unsqueeze(0), cam)
        rimg = dense_reference(rm2, rcq, sc["colors"], rop, rdp, H, W, early_stop=True)
    dev = torch.device("cuda:0")
    leaves = [sc[k].to(dev).clone().requires_grad_(True) for k in KEYS3]
    colors = sc["colors"].to(dev).clone().requires_grad_(True)
    img = rasterize_pinhole_gaussians(*leaves, colors, f, f, W / 2.0, H / 2.0,
                                      camera_to_world=c2w.to(dev), config=RasterConfig(height=H, width=W))
    (img * w.to(dev)).sum().backward()
    torch.cuda.synchronize()
    assert float(img.detach().abs().max()) > 0.05       # the scene is visible
    parity.check_image(img.detach().cpu().numpy(), rimg.numpy(), "3D end to end vs dense")
    three_d_parity(*(sc[k] for k in KEYS3), sc["colors"], c2w.unsqueeze(0), cam, H, W, w.numpy(),
                   img.detach().cpu().numpy(), [t.grad.cpu().numpy() for t in leaves], colors.grad.cpu().numpy(),
                   "3D 128x128")


def test_config4_full_workload(gpu):
    """Config 4 at its full workload: 4096x4096, 2^20 3D splats (10% with 10x
    scales), pinhole camera at z = -15, forward and backward through
    rasterize_pinhole_gaussians, every check of three_d_parity (about 1.2e8
    tile pairs compared bit for bit)."""
    sc = make_scene_3d(0)
    H, W, G = sc["H"], sc["W"], sc["G"]
    print(f"config 4: {W}x{H} G={G}", flush=True)
    c2w = sc["camera_to_world"]
    cam = torch.tensor([[sc["fx"], sc["fy"], sc["cx"], sc["cy"]]])
    w = torch.rand(1, H, W, 3, generator=torch.Generator().manual_seed(44))
    dev = torch.device("cuda:0")
    leaves = [sc[k].to(dev).clone().requires_grad_(True) for k in KEYS3]
    colors = sc["colors"].to(dev).clone().requires_grad_(True)
    img = rasterize_pinhole_gaussians(*leaves, colors, sc["fx"], sc["fy"], sc["cx"], sc["cy"],
                                      camera_to_world=c2w.to(dev), config=RasterConfig(height=H, width=W))
    (img * w.to(dev)).sum().backward()
    torch.cuda.synchronize()
    print("config 4: GPU forward and backward done", flush=True)
    bins = three_d_parity(*(sc[k] for k in KEYS3), sc["colors"], c2w.unsqueeze(0), cam, H, W, w.numpy(),
                          img.detach().cpu().numpy(), [t.grad.cpu().numpy() for t in leaves],
                          colors.grad.cpu().numpy(), "config 4")
    assert bins.binned_ids.size > 100_000_000


def test_torch_ops_projection(gpu):
    """torch.ops.gsplat_hip.project_forward / project_backward (the roles of the
    reference's project_pinhole_forward / _backward ops) against the
    running-error reference, as the autograd path above."""
    B, G = 2, 900
    m, s, q, o, c2w, cam = (t.float() for t in _scene(B, G, seed=9))
    dev = torch.device("cuda:0")
    args = [t.reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for t in (m, s, q, o)] + \
        [c2w.contiguous().to(dev), cam.contiguous().to(dev)]
    out = torch.ops.gsplat_hip.project_forward(*args, 1e-4)
    _check_forward(tuple(t.reshape(B, G, -1).squeeze(-1) for t in out), m, s, q, o, c2w, cam)
    gen = torch.Generator().manual_seed(19)
    w = [torch.randn(B * G, 2, generator=gen), torch.randn(B * G, 3, generator=gen) * 1e3,
         torch.randn(B * G, generator=gen), torch.randn(B * G, generator=gen)]
    g = torch.ops.gsplat_hip.project_backward(*(x.to(dev) for x in w), *args, 1e-4)
    torch.cuda.synchronize()
    r = PB.project_vjp(*(_np(t) for t in (m, s, q, o, c2w, cam)), *(x.reshape(B, G, -1).squeeze(-1).double().numpy()
                                                                    for x in w))
    for key, got in zip(KEYS3, g[:4]):
        PB.assert_close(_np(got).reshape(B * G, -1), r[key], key)
    PB.assert_close(_np(g[4]).reshape(B, 16), r["camera_to_world"], "camera_to_world")
    PB.assert_close(_np(g[5]), r["camera_params"], "camera_params")
