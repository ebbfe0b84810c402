"""GPU parity: forward image and gradients of rasterize_projected_gaussians.

Checkers:
  * the CPU tile oracle (oracle/tile_oracle.c) at the full sizes of configs
    0-3 and on the edge-case scenes, every pixel and every splat: pixels
    whose stop decision lies in exp's last-ulp window are re-walked by the
    oracle with the GPU's stop count, accepted only inside that window
    (oracle/parity.py: gpu_decisions);
  * the dense Torch reference (oracle/dense_reference.py) -- the reference's
    own oracle -- on the reference's test cases and on config 0.
Bars (oracle/parity.py): image rtol 1e-4 / atol 1e-5; gradients
|got - ref| <= 1e-5 + 1e-3 |ref| + 2^-24 (4 chain + (16 + tiles) mag) + slack
per entry, the rounding allowance built from the oracle's per-entry sums of
cancellation-free contribution magnitudes.  The reference's own hand cases
keep its max-abs 1e-5 bar (loss = mean(img^2)).
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import parity
from oracle import tile_oracle as TO
from oracle.dense_reference import dense_reference
from torch_gsplat_bridge_fast import RasterConfig, rasterize_projected_gaussians
from torch_gsplat_bridge_fast.scenes import make_scene_2d

pytestmark = pytest.mark.gpu

KEYS = ("means2d", "conics", "colors", "opacities", "depths")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _run_gpu(sc, cfg, w=None, loss="sum_w"):
    dev = torch.device("cuda:0")
    ts = [sc[k].to(dev).clone().requires_grad_(k != "depths") for k in KEYS]
    img = rasterize_projected_gaussians(*ts, cfg)
    if loss == "sum_w":
        (img * w.to(dev)).sum().backward()
    else:
        img.square().mean().backward()
    torch.cuda.synchronize()
    return img.detach().cpu(), [t.grad.detach().cpu() if t.grad is not None else None for t in ts]


def _run_dense(sc, H, W, bg, w=None, loss="sum_w", early_stop=True):
    ts = [sc[k].clone().requires_grad_(k != "depths") for k in KEYS]
    img = dense_reference(*ts, H, W, background=bg, early_stop=early_stop)
    if loss == "sum_w":
        (img * w).sum().backward()
    else:
        img.square().mean().backward()
    return img.detach(), [t.grad for t in ts]


def _hand_case(B):
    with open(os.path.join(GOLDEN, "reference_hand_cases.json")) as f:
        hc = json.load(f)
    g = torch.Generator().manual_seed(0)
    colors = torch.rand(2, 4, 3, generator=g)
    sc = {
        "means2d": torch.tensor(hc["means2d"])[:B],
        "conics": torch.tensor(hc["conics"])[:B],
        "colors": colors[:B],
        "opacities": torch.tensor(hc["opacities"])[:B],
        "depths": torch.tensor(hc["depths"])[:B],
    }
    if B == 1:
        sc = {k: v[0] for k, v in sc.items()}
    return sc


@pytest.mark.parametrize("B", [1, 2])
def test_reference_hand_case(gpu, B):
    """variants/v8/tests/reference_check.py:118-177 (16x16, G=4), tolerance 1e-5 max-abs."""
    sc = _hand_case(B)
    cfg = RasterConfig(height=16, width=16, max_fast_pairs=128)
    img, grads = _run_gpu(sc, cfg, loss="mean_sq")
    ref, rgrads = _run_dense(sc, 16, 16, (0.0, 0.0, 0.0), loss="mean_sq", early_stop=False)
    assert float((img - ref).abs().max()) <= 1e-5
    for name, g, r in zip(KEYS[:4], grads, rgrads):
        assert float((g - r).abs().max()) <= 1e-5, name


def test_reference_saturated_case(gpu):
    """variants/v8/tests/reference_check.py:180-231: 32x32, G=64, white background, early stop."""
    with open(os.path.join(GOLDEN, "reference_saturated_case.json")) as f:
        sc = {k: torch.tensor(v) for k, v in json.load(f).items()}
    cfg = RasterConfig(height=32, width=32, background=(1.0, 1.0, 1.0), stop_count_mode="always")
    img, grads = _run_gpu(sc, cfg, loss="mean_sq")
    ref, rgrads = _run_dense(sc, 32, 32, (1.0, 1.0, 1.0), loss="mean_sq", early_stop=True)
    assert float((img - ref).abs().max()) <= 1e-5
    for name, g, r in zip(KEYS[:4], grads, rgrads):
        assert float((g - r).abs().max()) <= 1e-5, name


def test_config0_vs_dense_reference(gpu):
    """Config 0 (512x512, G=512) against the dense Torch reference (fp32 on
    the CPU): image at the image bar, gradients at the gradient bar with the
    rounding allowance of the tile oracle's bounds."""
    sc0 = make_scene_2d(0, seed=0)
    sc = {k: sc0[k][0] for k in KEYS}
    H, W = sc0["H"], sc0["W"]
    w = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(123))
    cfg = RasterConfig(height=H, width=W)
    img, grads = _run_gpu(sc, cfg, w)
    ref, rgrads = _run_dense(sc, H, W, (0.0, 0.0, 0.0), w, early_stop=True)
    parity.check_image(img.numpy(), ref.numpy(), "cfg0 dense")
    meta = TO.make_meta(H, W, 1, 512)
    s = TO.Scene(*(sc[k].numpy() for k in KEYS), 1, 512)
    bins = TO.bin_scene(meta, s)
    force, _, _ = parity.gpu_decisions(meta, s, bins, gpu_state(sc0, H, W, 1, 512, (0.0, 0.0, 0.0))[1])
    _, bounds = TO.render_backward(meta, s, bins, w.numpy()[None], force_last=force, with_bounds=True)
    rep = parity.check_grads([g.numpy() for g in grads[:4]], [r.numpy() for r in rgrads[:4]], bounds,
                             parity.tiles_per_splat(bins, 1, 512), "cfg0 dense")
    print("cfg0 vs dense:", rep, flush=True)


def gpu_state(sc, H, W, B, G, bg, cfg=None):
    """The GPU forward's per-pixel stop counts (render_forward with state) for
    the scene; the forward is deterministic, so they are those of any other
    GPU forward of the same inputs."""
    from torch_gsplat_bridge_fast import _lib, _ops

    cfg = cfg or RasterConfig(height=H, width=W, background=bg)
    meta = _lib.make_raster_meta(H, W, B, G, cfg.alpha_threshold, cfg.transmittance_threshold, bg)
    flat = [torch.as_tensor(sc[k]).reshape(B * G, -1).squeeze(-1).contiguous().cuda() for k in KEYS]
    st = _ops.bin_gaussians(meta, *flat)
    _, T, last, stop, _ = _ops.render_forward(meta, st, save_state=True)
    return T.cpu().numpy(), last.cpu().numpy(), stop.cpu().numpy(), st


def oracle_parity(sc, H, W, B, G, bg, w, img, grads, label, gpu_last=None):
    """Image and gradients of one GPU run against the tile oracle at every
    pixel and splat (the module docstring's bars).  Returns the oracle's
    (bins, tile_stop, force_last)."""
    if gpu_last is None:
        gpu_last = gpu_state(sc, H, W, B, G, bg)[1]
    meta = TO.make_meta(H, W, B, G, background=bg)
    s = TO.Scene(*(np.asarray(sc[k]) for k in KEYS), B, G)
    bins = TO.bin_scene(meta, s)
    force, (oimg, _, _, ostop), rep = parity.gpu_decisions(meta, s, bins, gpu_last)
    parity.check_image(np.asarray(img), oimg, label)
    ograds, bounds = TO.render_backward(meta, s, bins, np.asarray(w).reshape(B, H, W, 3), force_last=force,
                                        with_bounds=True)
    if grads is not None:
        grep = parity.check_grads([np.asarray(g) for g in grads], ograds, bounds,
                                  parity.tiles_per_splat(bins, B, G), label)
        print(f"{label}: {rep}; gradient error / allowance, / stated bar: "
              + ", ".join(f"{k} {v['max_over_allowance']:.3g} {v['max_over_stated_bar']:.3g}"
                          for k, v in grep.items()), flush=True)
    return bins, ostop, force


@pytest.mark.parametrize("cfg_id,kw,bg", [
    (0, {}, (0.0, 0.0, 0.0)),
    (0, dict(H=37, W=53, G=777), (0.3, 0.6, 0.9)),
    (1, {}, (0.0, 0.0, 0.0)),
    (2, {}, (0.0, 0.0, 0.0)),
    (3, {}, (1.0, 1.0, 1.0)),
])
def test_configs_vs_tile_oracle(gpu, cfg_id, kw, bg):
    sc = make_scene_2d(cfg_id, seed=0, **kw)
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    print(f"raster cfg{cfg_id} {W}x{H} B={B} G={G}", flush=True)
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(99))
    cfg = RasterConfig(height=H, width=W, background=bg)
    img, grads = _run_gpu({k: sc[k] for k in KEYS}, cfg, w)
    oracle_parity(sc, H, W, B, G, bg, w.numpy(), img.numpy(), [g.numpy() for g in grads[:4]], f"cfg{cfg_id}")


def test_state_outputs_match_oracle(gpu):
    """final_T, stop counts (local_stop) and tile stop counts saved by forward,
    at every pixel (ambiguous stops with the GPU's decision, see
    gpu_decisions)."""
    sc = make_scene_2d(1, seed=4, G=20000, H=300, W=500)
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    T, last, stop, _ = gpu_state(sc, H, W, B, G, (0.0, 0.0, 0.0))
    meta = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(sc[k].numpy() for k in KEYS), B, G)
    bins = TO.bin_scene(meta, s)
    _, (_, oT, olast, ostop), rep = parity.gpu_decisions(meta, s, bins, last)
    print("state outputs:", rep, flush=True)
    np.testing.assert_allclose(T, oT, rtol=1e-4, atol=1e-6)
    np.testing.assert_array_equal(last, olast)
    np.testing.assert_array_equal(stop, ostop)


def test_forward_rebins_when_pairs_exceed_capacity(gpu):
    """A pair capacity remembered from a smaller scene is detected after the forward has been
    enqueued; the forward bins and renders again, giving the same image and gradients."""
    from torch_gsplat_bridge_fast import _ops

    H, W, B, G = 200, 260, 1, 5000
    print(f"rebin {H}x{W} G={G}", flush=True)
    sc0 = make_scene_2d(1, seed=2, G=G, H=H, W=W)
    sc = {k: sc0[k].to(gpu) for k in KEYS}
    cfg = RasterConfig(height=H, width=W)
    wgt = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(3)).to(gpu)
    key = (0, B, G, H, W)
    _ops._capacity.pop(key, None)
    results = []
    for forced in (None, 100):
        if forced is not None:
            _ops._capacity[key] = forced
        with torch.no_grad():
            ev = rasterize_projected_gaussians(*[sc[k] for k in KEYS], cfg)
        if forced is not None:
            _ops._capacity[key] = forced
        leaves = [sc[k].clone().requires_grad_(k != "depths") for k in KEYS]
        img = rasterize_projected_gaussians(*leaves, cfg)
        (img * wgt).sum().backward()
        results.append((ev, img.detach(), [leaves[i].grad for i in range(4)]))
        assert _ops._capacity[key] > 100
    (ev0, img0, g0), (ev1, img1, g1) = results
    assert torch.equal(ev0, ev1) and torch.equal(img0, img1) and torch.equal(ev0, img0)
    for a, b in zip(g0, g1):
        # equal up to the order of the float atomics (cancellation makes single sums differ in the
        # fifth digit)
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-6)


def test_unbatched_matches_batched(gpu):
    sc0 = make_scene_2d(3, seed=5, G=3000, B=2, H=64, W=96)
    cfg = RasterConfig(height=64, width=96)
    with torch.no_grad():
        both = rasterize_projected_gaussians(*[sc0[k].to(gpu) for k in KEYS], cfg)
        for b in range(2):
            one = rasterize_projected_gaussians(*[sc0[k][b].to(gpu) for k in KEYS], cfg)
            assert one.shape == (64, 96, 3)
            assert torch.equal(one, both[b])


def test_overflow_disabled_raises(gpu):
    """variants/v5/tests/reference_check.py:217-235: max_fast_pairs=1 without fallback raises."""
    sc = _hand_case(1)
    cfg = RasterConfig(height=16, width=16, max_fast_pairs=1, enable_overflow_fallback=False)
    with pytest.raises(RuntimeError, match="Tile overflow detected"):
        with torch.no_grad():
            rasterize_projected_gaussians(*[sc[k].to(gpu) for k in KEYS], cfg)


def test_depth_gradient_is_zero(gpu):
    sc = _hand_case(1)
    ts = [sc[k].to(gpu).clone().requires_grad_(True) for k in KEYS]
    img = rasterize_projected_gaussians(*ts, RasterConfig(height=16, width=16))
    img.sum().backward()
    assert torch.count_nonzero(ts[4].grad) == 0


def test_backward_twice_with_retained_graph(gpu):
    """The forward allocates the first backward's gradient buffers ahead; a second backward of the
    same graph (retain_graph) writes fresh ones, so the leaves' .grad ends at twice one backward."""
    sc = make_scene_2d(1, seed=4, G=2000, H=96, W=128)
    H, W = sc["H"], sc["W"]
    print(f"retain_graph {W}x{H}", flush=True)
    leaves = [sc[k].to(gpu).requires_grad_(k != "depths") for k in KEYS]
    w = torch.rand((1, H, W, 3), generator=torch.Generator().manual_seed(3)).to(gpu)
    img = rasterize_projected_gaussians(*leaves, RasterConfig(height=H, width=W))
    img.backward(w, retain_graph=True)
    once = [t.grad.clone() for t in leaves[:4]]
    img.backward(w)
    for t, g in zip(leaves[:4], once):
        # (the two backwards add their atomics in different orders)
        torch.testing.assert_close(t.grad, 2 * g, rtol=1e-4, atol=1e-5 * float(g.abs().max()) + 1e-6)


def _faint_crowd(seed, B, G, H, W):
    """Many large, faint splats: every tile holds several hundred pairs and
    few pixels reach the early-stop threshold, so tile stops exceed 256."""
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, G, 2, generator=g) * torch.tensor([W, H], dtype=torch.float32)
    sig = 3.0 + 7.0 * torch.rand(B, G, 2, generator=g)
    th = torch.rand(B, G, generator=g) * np.pi
    c, s = torch.cos(th), torch.sin(th)
    ia, ib = 1.0 / sig[..., 0] ** 2, 1.0 / sig[..., 1] ** 2
    conics = torch.stack([c * c * ia + s * s * ib, c * s * (ia - ib), s * s * ia + c * c * ib], dim=-1)
    return {
        "means2d": m.contiguous(),
        "conics": conics.contiguous(),
        "colors": torch.rand(B, G, 3, generator=g),
        "opacities": 0.005 + 0.045 * torch.rand(B, G, generator=g),
        "depths": torch.rand(B, G, generator=g) * 10.0,
    }


def _backward_variants(meta, st, T, last, stop, w, ws):
    """The backward over one forward state: with the forward's workspace
    (segmented heavy tiles), without it (one wavefront per tile), and with
    the workspace again (it is read-only in the backward)."""
    from torch_gsplat_bridge_fast import _ops

    out = {"segmented": _ops.render_backward(meta, st, T, last, stop, w, ws),
           "one_wave": _ops.render_backward(meta, st, T, last, stop, w, None),
           "segmented_again": _ops.render_backward(meta, st, T, last, stop, w, ws)}
    torch.cuda.synchronize()
    return {k: [g.cpu().numpy() for g in v] for k, v in out.items()}


def _forward_without_workspace(meta, st):
    """render_forward with the state outputs and no workspace: every tile
    walked by one wavefront (no hand-off to the continuation kernel)."""
    from torch_gsplat_bridge_fast import _lib

    B, H, W = meta.batch, meta.height, meta.width
    dev = st.packed.device
    img = torch.empty((B, H, W, 3), device=dev)
    T = torch.empty((B, H, W), device=dev)
    last = torch.empty((B, H, W), dtype=torch.int32, device=dev)
    stop = torch.empty((st.num_tiles,), dtype=torch.int32, device=dev)
    L = _lib.lib()
    _lib.check(L.gsplat_hip_render_forward(meta, _lib.ptr(st.packed), _lib.ptr(st.tile_offsets),
                                           _lib.ptr(st.binned_ids), _lib.ptr(img), _lib.ptr(T), _lib.ptr(last),
                                           _lib.ptr(stop), st.n_pairs, None, 0, _lib.stream_of(img)),
               "gsplat_hip_render_forward")
    return img, T, last, stop


def _heavy_check(gpu, sc, B, G, H, W, w, label, min_stop):
    """Public-API run vs the oracle, then every compositor variant over the
    same binning vs the oracle: the forward with and without the
    continuation kernel and the eval forward (bit-identical images), and the
    segmented and one-wavefront backward (each at the gradient bar)."""
    from torch_gsplat_bridge_fast import _lib, _ops

    img, grads = _run_gpu(sc, RasterConfig(height=H, width=W), w)
    T, last, stop, st = gpu_state(sc, H, W, B, G, (0.0, 0.0, 0.0))
    bins, ostop, force = oracle_parity(sc, H, W, B, G, (0.0, 0.0, 0.0), w.numpy(), img.numpy(),
                                       [g.numpy() for g in grads[:4]], label, gpu_last=last)
    assert int(ostop.max()) > min_stop
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0, 0, 0))
    img_ws, T_ws, last_ws, stop_ws, ws = _ops.render_forward(meta, st, save_state=True)
    img1, T1, last1, stop1 = _forward_without_workspace(meta, st)
    img_eval = _ops.render_forward(meta, st, save_state=False)[0]
    torch.cuda.synchronize()
    assert torch.equal(img1, img_ws) and torch.equal(img_eval, img_ws)
    assert torch.equal(T1, T_ws) and torch.equal(last1, last_ws) and torch.equal(stop1, stop_ws)
    np.testing.assert_array_equal(stop_ws.cpu().numpy(), ostop)
    meta_o = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(np.asarray(sc[k]) for k in KEYS), B, G)
    ograds, bounds = TO.render_backward(meta_o, s, bins, w.numpy(), force_last=force, with_bounds=True)
    tiles = parity.tiles_per_splat(bins, B, G)
    for name, g in _backward_variants(meta, st, T_ws, last_ws, stop_ws, w.to(gpu), ws).items():
        parity.check_grads(g, ograds, bounds, tiles, f"{label} {name}")
    return ostop


def test_heavy_tiles_segmented_backward(gpu):
    """Tiles with up to ~970 composited splats: the forward continues them
    with four wavefronts after 128 splats and records 128-splat segments,
    which the backward walks in parallel, each started from the records.
    Every variant is checked against the tile oracle (_heavy_check)."""
    B, G, H, W = 2, 2500, 48, 80
    sc = _faint_crowd(21, B, G, H, W)
    print(f"heavy tiles {W}x{H} B={B} G={G}", flush=True)
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(8))
    ostop = _heavy_check(gpu, sc, B, G, H, W, w, "heavy", 3 * 256)
    assert int((ostop > 256).sum()) >= 20


def test_plain_and_general_batches(gpu):
    """The compositors drop the p <= 0 test and the max_alpha clamp/gate for a
    batch whose records are all well-conditioned (positive-definite conic
    with margin, opacity below max_alpha).  Here the left half of each image
    also holds records that need the general path -- hair-thin splats
    (sigma 0.02 x 20 px, conic too ill-conditioned for the shortcut) and a
    few with opacity 0.995, whose alpha the clamp limits -- so left-half tiles
    take the general path and right-half tiles the shortcut, in the
    one-wavefront and the continuation kernels (tiles of several hundred
    splats) and in the backward.  Every variant is checked against the tile
    oracle (_heavy_check)."""
    B, G, H, W = 2, 2500, 48, 80
    sc = _faint_crowd(33, B, G, H, W)
    g = torch.Generator().manual_seed(34)
    left = sc["means2d"][..., 0] < W / 2
    idx = torch.arange(G).expand(B, G)
    thin = left & (idx % 5 == 0)
    sc["conics"][thin] = torch.tensor([1.0 / 0.02 ** 2, 0.0, 1.0 / 20.0 ** 2])
    bright = left & (idx % 50 == 1)
    sc["opacities"][bright] = 0.995
    sc["opacities"][left & (idx % 50 == 2)] = 0.99 * (1.0 - 2.0 ** -21)  # just above the shortcut's bound
    sc["colors"] = torch.rand(B, G, 3, generator=g)
    print(f"plain/general batches {W}x{H} B={B} G={G} thin={int(thin.sum())} bright={int(bright.sum())}",
          flush=True)
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(35))
    ostop = _heavy_check(gpu, sc, B, G, H, W, w, "plain/general", 128)
    assert int((ostop > 128).sum()) >= 10  # the continuation kernel runs


def test_pair_budget_splits_training_launches(gpu):
    """max_pairs_per_launch (reference _choose_batch_slices, v8 rasterize.py:339-391):
    a budget below two images' pairs gives one launch per image.  Both the
    split and the single-launch run are checked against the tile oracle, and
    their images are identical."""
    from torch_gsplat_bridge_fast import profile_projected_gaussians

    B, G, H, W = 3, 3000, 96, 128
    sc0 = make_scene_2d(1, seed=7, G=G, B=B, H=H, W=W)
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(3))
    base = RasterConfig(height=H, width=W)
    with torch.no_grad():
        prof = profile_projected_gaussians(*[sc0[k].to(gpu) for k in KEYS], base)
    per_image = prof["total_pairs"] / B
    split = RasterConfig(height=H, width=W, max_pairs_per_launch=int(per_image * 1.2))
    img1, g1 = _run_gpu({k: sc0[k] for k in KEYS}, base, w)
    img2, g2 = _run_gpu({k: sc0[k] for k in KEYS}, split, w)
    assert torch.equal(img1, img2)
    last = gpu_state(sc0, H, W, B, G, (0.0, 0.0, 0.0))[1]
    for label, img, g in (("single launch", img1, g1), ("split launches", img2, g2)):
        oracle_parity(sc0, H, W, B, G, (0.0, 0.0, 0.0), w.numpy(), img.numpy(), [x.numpy() for x in g[:4]],
                      f"pair budget, {label}", gpu_last=last)
    with torch.no_grad():
        prof2 = profile_projected_gaussians(*[sc0[k].to(gpu) for k in KEYS], split)
    assert prof["chosen_batch_chunks"] == [3]
    assert prof2["chosen_batch_chunks"] == [1, 1, 1]


def test_eval_path_vs_tile_oracle(gpu):
    """The eval forward (no grad: render_forward without state, reference
    _rasterize_chunk_eval, v8 rasterize.py:684-786) against the oracle's image,
    and bit-identical to the training forward."""
    B, G, H, W = 2, 6000, 200, 260
    sc = make_scene_2d(3, seed=2, G=G, B=B, H=H, W=W)
    cfg = RasterConfig(height=H, width=W, background=(0.2, 0.1, 0.4))
    dev_in = [sc[k].to(gpu) for k in KEYS]
    with torch.no_grad():
        ev = rasterize_projected_gaussians(*dev_in, cfg)
    tr = rasterize_projected_gaussians(*[t.clone().requires_grad_(k != "depths") for k, t in zip(KEYS, dev_in)], cfg)
    assert torch.equal(ev, tr.detach())
    oracle_parity(sc, H, W, B, G, cfg.background, np.zeros((B, H, W, 3), np.float32), ev.cpu().numpy(), None,
                  "eval path")


@pytest.mark.parametrize("policy,strategy", [("auto", "serial"), ("off", "auto")])
def test_profile_statistics_match_oracle(gpu, policy, strategy):
    """profile_projected_gaussians (reference v8 rasterize.py:860-1014) reduces
    its statistics on the device; they equal the statistics of the tile
    oracle's tile counts and stop counts, with the reference's meaning: a tile
    above max_fast_pairs (the reference's overflow path) or without pairs has a
    stop count of 0 (gsplat_v8_kernels.metal:423-431), and
    resolved_active_chunks is the reference's policy decision per launch
    (v8 rasterize.py:401-424), here per image (serial launches) or for the
    whole batch."""
    from torch_gsplat_bridge_fast import profile_projected_gaussians

    B, G, H, W, mfp = 2, 4000, 128, 192, 300
    sc = make_scene_2d(3, seed=1, G=G, B=B, H=H, W=W)
    cfg = RasterConfig(height=H, width=W, max_fast_pairs=mfp, active_policy=policy, batch_strategy=strategy)
    with torch.no_grad():
        out = profile_projected_gaussians(*[sc[k].to(gpu) for k in KEYS], cfg, run_forward=True, return_image=True)
    st_ = out["stats"]
    meta = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(sc[k].numpy() for k in KEYS), B, G)
    bins = TO.bin_scene(meta, s)
    _, (oimg, _, _, ostop), _ = parity.gpu_decisions(meta, s, bins, gpu_state(sc, H, W, B, G, (0, 0, 0))[1])
    parity.check_image(out["image"].cpu().numpy(), oimg, "profile image")
    c = bins.tile_counts.astype(np.float64)
    assert (c > mfp).sum() > 0 and (ostop[c > mfp] > 0).all()      # overflow tiles with real stops
    stop = np.where(c <= mfp, ostop, 0).astype(np.float64)
    assert st_["tiles"] == c.size and st_["total_pairs"] == int(c.sum())
    assert st_["max_pairs_per_tile"] == int(c.max()) and st_["max_stop_count"] == int(stop.max())
    assert st_["overflow_tile_count"] == int((c > mfp).sum())
    assert st_["active_tile_count"] == int(((c > 0) & (c <= mfp)).sum())
    assert st_["dense_active_tile_count"] == int(((c > 0) & (c <= mfp) & (c >= 64)).sum())
    np.testing.assert_allclose(st_["active_tile_fraction"], (c > 0).mean(), rtol=1e-6)
    np.testing.assert_allclose(st_["mean_pairs_per_tile"], c.mean(), rtol=1e-5)
    np.testing.assert_allclose(st_["p95_pairs_per_tile"], np.quantile(c, 0.95), rtol=1e-5)
    np.testing.assert_allclose(st_["mean_stop_count"], stop.mean(), rtol=1e-5)
    np.testing.assert_allclose(st_["p95_stop_count"], np.quantile(stop, 0.95), rtol=1e-5)
    ratio = np.where(c > 0, stop / np.maximum(c, 1), 0)
    np.testing.assert_allclose(st_["mean_stop_ratio"], ratio.mean(), rtol=1e-5)
    np.testing.assert_allclose(st_["p95_stop_ratio"], np.quantile(ratio, 0.95), rtol=1e-5)
    # the reference's policy per launch, restated
    launches = [c[b * (c.size // B):(b + 1) * (c.size // B)] for b in range(B)] if strategy == "serial" else [c]
    want = []
    for lc in launches:
        frac, over, mx = (lc > 0).mean(), int((lc > mfp).sum()), int(lc.max())
        if policy == "off":
            want.append(False)
        elif frac > 0.75 and over == 0:
            want.append(False)
        else:
            want.append(bool(frac < 0.10 or over > 0 or mx > 2 * mfp))
    assert st_["resolved_active_chunks"] == want and st_["resolved_use_active_tiles"] == any(want)
    assert st_["chosen_batch_chunks"] == ([1] * B if strategy == "serial" else [B])
    if policy == "auto":
        assert any(want)


def test_recorded_trace_vs_tile_oracle(gpu, tmp_path):
    """Real-trace input (reference benchmark_mps.py:26-47): a seeded scene
    written with torch.save as [G,...] float64 tensors, read back by
    scenes.load_trace (weights_only) and rasterized through the public API,
    forward and backward, against the tile oracle."""
    from torch_gsplat_bridge_fast.scenes import load_trace

    H, W, G = 144, 200, 5000
    sc = make_scene_2d(1, seed=11, G=G, H=H, W=W)
    f = tmp_path / "trace.pt"
    torch.save({k: sc[k][0].double() for k in KEYS}, f)
    tr = load_trace(str(f), device=gpu)
    assert tr["means2d"].shape == (1, G, 2) and tr["means2d"].dtype == torch.float32
    leaves = [tr[k].clone().requires_grad_(k != "depths") for k in KEYS]
    cfg = RasterConfig(height=H, width=W)
    img = rasterize_projected_gaussians(*leaves, cfg)
    w = torch.rand(1, H, W, 3, generator=torch.Generator().manual_seed(12))
    (img * w.to(gpu)).sum().backward()
    host = {k: tr[k].cpu() for k in KEYS}
    oracle_parity(host, H, W, 1, G, (0.0, 0.0, 0.0), w.numpy(), img.detach().cpu().numpy(),
                  [t.grad.cpu().numpy() for t in leaves[:4]], "recorded trace")


def test_torch_ops_vs_tile_oracle(gpu):
    """The torch.library operators (torch.ops.gsplat_hip.bin / render_forward /
    render_backward, the roles of torch.ops.gsplat_metal_v8.bin /
    render_fast_forward_state / render_fast_backward_saved), composed as the
    reference's autograd function composes its ops: binning bit-exact, image
    and gradients at the bar against the tile oracle, and the eval forward
    bit-identical to the state forward."""
    B, G, H, W = 2, 5000, 96, 160
    bg = [0.2, 0.3, 0.4]
    sc = make_scene_2d(3, seed=6, G=G, B=B, H=H, W=W)
    flat = [sc[k].reshape(B * G, -1).squeeze(-1).contiguous().to(gpu) for k in KEYS]
    counts, offsets, ids, packed, perm = torch.ops.gsplat_hip.bin(*flat, H, W, B, 1.0 / 255.0, 1e-4, bg)
    bins = TO.bin_scene(TO.make_meta(H, W, B, G, background=bg), TO.Scene(*(sc[k].numpy() for k in KEYS), B, G))
    np.testing.assert_array_equal(perm.cpu().numpy(), bins.perm)
    np.testing.assert_array_equal(counts.cpu().numpy(), bins.tile_counts)
    np.testing.assert_array_equal(offsets.cpu().numpy(), bins.tile_offsets)
    np.testing.assert_array_equal(ids.cpu().numpy(), bins.binned_ids)
    img, fT, last, stop, ws = torch.ops.gsplat_hip.render_forward(packed, offsets, ids, H, W, B, G, 1.0 / 255.0,
                                                                  1e-4, bg, True)
    ev = torch.ops.gsplat_hip.render_forward(packed, offsets, ids, H, W, B, G, 1.0 / 255.0, 1e-4, bg, False)
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(17))
    grads = torch.ops.gsplat_hip.render_backward(w.to(gpu), packed, offsets, ids, fT, last, stop, ws, H, W, B, G,
                                                 1.0 / 255.0, 1e-4, bg)
    torch.cuda.synchronize()
    assert torch.equal(ev[0], img)
    oracle_parity(sc, H, W, B, G, tuple(bg), w.numpy(), img.cpu().numpy(), [g.cpu().numpy() for g in grads],
                  "torch.ops", gpu_last=last.cpu().numpy())


def _dust(seed, B, G, H, W):
    """Very small, faint splats: each is visible only near its centre, so every
    pixel stays alive through the whole tile list (hundreds of thousands of
    splats per tile are walked)."""
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, G, 2, generator=g) * torch.tensor([W, H], dtype=torch.float32)
    sig = 0.2 + 0.1 * torch.rand(B, G, generator=g)
    inv = 1.0 / sig ** 2
    return {"means2d": m, "conics": torch.stack([inv, torch.zeros_like(inv), inv], dim=-1),
            "colors": torch.rand(B, G, 3, generator=g),
            "opacities": 0.006 + 0.006 * torch.rand(B, G, generator=g),
            "depths": torch.rand(B, G, generator=g)}


def test_segment_records_overflow(gpu):
    """More 128-splat segments are walked than the workspace holds (T + 1024
    records for a 2x2-tile image): tiles that find the records full break
    their chain and are walked whole by the backward.  Checked against the
    oracle, with the overflow asserted from the workspace's slot counter."""
    from torch_gsplat_bridge_fast import _lib, _ops

    B, G, H, W = 1, 300_000, 32, 32
    sc = _dust(41, B, G, H, W)
    print(f"segment overflow {W}x{H} G={G}", flush=True)
    T, last, stop, st = gpu_state(sc, H, W, B, G, (0.0, 0.0, 0.0))
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0, 0, 0))
    img, T2, last2, stop2, ws = _ops.render_forward(meta, st, save_state=True)
    torch.cuda.synchronize()
    slots_used = int(ws[:4].view(torch.int32).item())
    max_slots = 4 + 1024
    assert slots_used > max_slots, slots_used          # the records ran out
    assert int(stop2.min().item()) > 128 * 300           # every tile walked far past one segment
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(42))
    grads = _ops.render_backward(meta, st, T2, last2, stop2, w.to(gpu), ws)
    torch.cuda.synchronize()
    oracle_parity(sc, H, W, B, G, (0.0, 0.0, 0.0), w.numpy(), img.cpu().numpy(), [g.cpu().numpy() for g in grads],
                  "segment overflow", gpu_last=last2.cpu().numpy())


def test_backward_with_another_n_pairs_ignores_records(gpu):
    """The compositor workspace's layout follows n_pairs: a backward given
    another n_pairs than its forward must not read the segment records (it
    walks every tile whole) and still meets the bar."""
    from torch_gsplat_bridge_fast import _lib, _ops

    B, G, H, W = 2, 2500, 48, 80
    sc = _faint_crowd(21, B, G, H, W)
    T, last, stop, st = gpu_state(sc, H, W, B, G, (0.0, 0.0, 0.0))
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0, 0, 0))
    L = _lib.lib()
    n1, n2 = st.capacity, st.capacity + 50_000
    assert L.gsplat_hip_render_workspace_bytes(meta, n2) > L.gsplat_hip_render_workspace_bytes(meta, n1)
    wsb = L.gsplat_hip_render_workspace_bytes(meta, n2)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    img = torch.empty((B, H, W, 3), device=gpu)
    T1, last1 = torch.empty((B, H, W), device=gpu), torch.empty((B, H, W), dtype=torch.int32, device=gpu)
    stop1 = torch.empty((st.num_tiles,), dtype=torch.int32, device=gpu)
    _lib.check(L.gsplat_hip_render_forward(meta, _lib.ptr(st.packed), _lib.ptr(st.tile_offsets), _lib.ptr(st.pairs),
                                           _lib.ptr(img), _lib.ptr(T1), _lib.ptr(last1), _lib.ptr(stop1), n1,
                                           _lib.ptr(ws), wsb, _lib.stream_of(img)), "forward")
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(8))
    out = [torch.empty(s, device=gpu) for s in ((B, G, 2), (B, G, 3), (B, G, 3), (B, G))]
    _lib.check(L.gsplat_hip_render_backward(meta, _lib.ptr(st.packed), _lib.ptr(st.tile_offsets), _lib.ptr(st.pairs),
                                            _lib.ptr(T1), _lib.ptr(last1), _lib.ptr(stop1), _lib.ptr(w.to(gpu)),
                                            *[_lib.ptr(t) for t in out], n2, _lib.ptr(ws), wsb,
                                            _lib.stream_of(img)), "backward")
    torch.cuda.synchronize()
    assert int(stop1.max().item()) > 256
    oracle_parity(sc, H, W, B, G, (0.0, 0.0, 0.0), w.numpy(), img.cpu().numpy(), [t.cpu().numpy() for t in out],
                  "backward with another n_pairs", gpu_last=last1.cpu().numpy())


def _tile_stack(n, seed, B=1, H=64, W=80, extra=60):
    """n tiny splats whose supports lie inside tile (1, 1) of every image
    (that tile's range holds exactly n pairs) plus `extra` small splats
    spread over the image's right part."""
    g = torch.Generator().manual_seed(seed)
    G = n + extra
    # the others lie right of pixel column 35, clear of tile (1, 1) (supports
    # reach 4.5 pixels from the centre)
    m = torch.rand(B, G, 2, generator=g) * torch.tensor([W - 44.0, H - 8.0]) + torch.tensor([40.0, 4.0])
    m[:, :n] = 23.5 + torch.rand(B, n, 2, generator=g)
    conics = torch.zeros(B, G, 3)
    conics[..., 0] = 4.0
    conics[..., 2] = 4.0
    conics[:, n:, 0] = 0.5
    conics[:, n:, 2] = 0.5
    return {
        "means2d": m.contiguous(),
        "conics": conics.contiguous(),
        "colors": torch.rand(B, G, 3, generator=g),
        "opacities": 0.1 + 0.5 * torch.rand(B, G, generator=g),
        "depths": torch.rand(B, G, generator=g) * 10.0,
    }


@pytest.mark.parametrize("kind", ["config1_small", "heavy", "stack128", "stack129"])
def test_one_call_bin_and_forward(gpu, kind):
    """With the shape's pair capacity known, bin_and_render bins and composites in one C-ABI call
    (gsplat_hip_bin_render_forward: the tile-range launch zeroes the forward's workspace words)
    and continues long tiles (gsplat_hip_render_forward_long) only when the binning reports a
    tile range longer than HANDOFF_PAIRS.  Checked: the flag against the tile counts (a range of
    exactly 128 pairs is not long, 129 is), binning, image and state bit-identical to the
    separate calls of the first binning of the shape (last where the pixel stopped: the one-call
    forward stores it only in such tiles), the eval forward's image, and image and gradients of the
    one-call forward's state, its other last entries zeroed, against the tile oracle."""
    from torch_gsplat_bridge_fast import _lib, _ops

    if kind == "config1_small":
        B, G, H, W = 2, 3000, 200, 264
        sc = make_scene_2d(1, seed=5, G=G, B=B, H=H, W=W)
    elif kind == "heavy":
        B, G, H, W = 2, 2500, 48, 80
        sc = _faint_crowd(21, B, G, H, W)
    else:
        n = 128 if kind == "stack128" else 129
        B, H, W = 2, 64, 80
        sc = _tile_stack(n, seed=n, B=B, H=H, W=W)
        G = sc["opacities"].shape[1]
    print(f"one-call binning + forward: {kind} B={B} G={G} {W}x{H}", flush=True)
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    flat = [torch.as_tensor(sc[k]).reshape(B * G, -1).squeeze(-1).contiguous().to(gpu) for k in KEYS]
    _ops._capacity.pop((0, B, G, H, W), None)
    st0, out0 = _ops.bin_and_render(meta, flat, save_state=True)   # first binning of the shape
    st1, out1 = _ops.bin_and_render(meta, flat, save_state=True)   # one call
    st2, out2 = _ops.bin_and_render(meta, flat, save_state=False)  # one call, eval forward
    assert st0._long_index is None and st1._long_index is not None and st2._long_index is not None
    st1.check_status()
    st2.check_status()
    counts = (st1.tile_offsets[1:] - st1.tile_offsets[:-1]).cpu().numpy()
    long_expected = bool(counts.max() > _lib.HANDOFF_PAIRS)
    assert st1.long_tiles == st2.long_tiles == long_expected
    if kind.startswith("stack"):
        assert int(counts.max()) == int(kind[5:])
    n = st0.n_pairs
    assert st1.n_pairs == n
    for a, b in [(st0.perm, st1.perm), (st0.packed, st1.packed), (st0.tile_offsets, st1.tile_offsets),
                 (st0.splat_offsets, st1.splat_offsets), (st0.pairs[:n], st1.pairs[:n])]:
        assert torch.equal(a, b)
    for i in (0, 1, 3):  # image, final_T, tile stops
        assert torch.equal(out0[i], out1[i])
    # the one-call forward stores last only in the tiles where a pixel stopped (T <= threshold)
    T = out1[1]
    stopped = ~(T > meta.transmittance_threshold)
    assert torch.equal(out0[2][stopped], out1[2][stopped])
    assert torch.equal(out2[0], out0[0])
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(3))
    img, _, last, stop, ws = out1
    # the backward must not read the other entries: zero them (a read would skip every splat there)
    last = torch.where(stopped, last, torch.zeros_like(last))
    grads = _ops.render_backward(meta, st1, T, last, stop, w.to(gpu), ws)
    torch.cuda.synchronize()
    oracle_parity(sc, H, W, B, G, (0.0, 0.0, 0.0), w.numpy(), img.cpu().numpy(),
                  [g.cpu().numpy() for g in grads], f"one call {kind}", gpu_last=out0[2].cpu().numpy())


def test_launch_trace_sees_every_kernel_of_a_step(gpu):
    """gsplat_hip_trace_launches (the benchmark's per-kernel breakdown): a traced forward +
    backward through the public API, after a first call that sizes the pair buffers, lists the
    kernels of the one-call path in launch order (the backward's from the autograd engine's
    thread too), each with a positive duration; tracing changes no result."""
    from torch_gsplat_bridge_fast import _ops

    H, W, G = 512, 512, 8000
    sc = make_scene_2d(2, seed=3, G=G, H=H, W=W)
    cfg = RasterConfig(height=H, width=W)
    w = torch.rand(1, H, W, 3, generator=torch.Generator().manual_seed(4)).to(gpu)

    def step():
        leaves = [sc[k].to(gpu).clone().requires_grad_(k != "depths") for k in KEYS]
        img = rasterize_projected_gaussians(*leaves, cfg)
        img.backward(w)
        return img.detach(), [t.grad for t in leaves[:4]]

    ref_img, ref_grads = step()
    trace = _ops.LaunchTrace(capacity=64)
    with trace:
        img, grads = step()
    names = [n for n, _ in trace.launches]
    print("traced launches:", trace.launches, flush=True)
    want = ["count_depth_runs_kernel", "rank_pack_kernel", "emit_kernel<true>", "rs_onesweep_kernel(keys)",
            "bucket_sort_kernel", "render_fwd_kernel", "render_bwd_kernel", "render_grads_unpack_kernel"]
    pos = [names.index(k) for k in want]
    assert pos == sorted(pos), names
    assert all(ms > 0 for _, ms in trace.launches)
    assert torch.equal(img, ref_img)
    for g, r in zip(grads, ref_grads):   # equal up to the order of the gradient atomics
        torch.testing.assert_close(g, r, rtol=1e-4, atol=1e-5 * float(r.abs().max()))
