"""CPU tests of the parallel oracle's backward, its error bounds and its
forced stop decisions (oracle/tile_oracle.c, oracle/parity.py).

  * The parallel backward (double sums, tile order) agrees with the serial
    restatement that sums float32 contributions in the reference kernels'
    pixel order, within the allowance of oracle/parity.py, on uniform,
    clustered and heavy-tile scenes: a genuine reordering of the same
    contributions stays inside the bar.
  * The allowance is not vacuous: a dropped pixel, a flipped sign and a
    0.3% scale error each fail it.
  * Results do not depend on the thread count.
  * Forced stop decisions: accepted inside the ambiguity window, flagged
    outside it.
"""
import os
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from oracle import parity
from oracle import tile_oracle as TO
from torch_gsplat_bridge_fast.scenes import make_scene_2d

KEYS = ("means2d", "conics", "colors", "opacities", "depths")


def _faint_crowd(seed, B, G, H, W):
    """Large faint splats: tiles keep hundreds of splats alive (long walks)."""
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, G, 2, generator=g) * torch.tensor([W, H], dtype=torch.float32)
    sig = 3.0 + 7.0 * torch.rand(B, G, 2, generator=g)
    th = torch.rand(B, G, generator=g) * np.pi
    c, s = torch.cos(th), torch.sin(th)
    ia, ib = 1.0 / sig[..., 0] ** 2, 1.0 / sig[..., 1] ** 2
    conics = torch.stack([c * c * ia + s * s * ib, c * s * (ia - ib), s * s * ia + c * c * ib], dim=-1)
    return {"means2d": m, "conics": conics, "colors": torch.rand(B, G, 3, generator=g),
            "opacities": 0.005 + 0.045 * torch.rand(B, G, generator=g),
            "depths": torch.rand(B, G, generator=g) * 10.0, "H": H, "W": W, "B": B, "G": G}


SCENES = {
    "cfg0": lambda: make_scene_2d(0, seed=0),
    "cfg1_sub": lambda: make_scene_2d(1, seed=4, G=20000, H=300, W=500),
    "cfg3_sub": lambda: make_scene_2d(3, seed=1, G=6000, B=2, H=128, W=192),
    "heavy": lambda: _faint_crowd(21, 2, 2500, 48, 80),
}


def _setup(sc, bg=(0.0, 0.0, 0.0), seed=99):
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    meta = TO.make_meta(H, W, B, G, background=bg)
    s = TO.Scene(*(np.asarray(sc[k]) for k in KEYS), B, G)
    bins = TO.bin_scene(meta, s)
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(seed)).numpy()
    return meta, s, bins, w


@pytest.mark.parametrize("name", sorted(SCENES))
def test_parallel_backward_matches_serial_within_bounds(name):
    sc = SCENES[name]()
    meta, s, bins, w = _setup(sc, bg=(0.3, 0.6, 0.9))
    serial = TO.render_backward_serial(meta, s, bins, w)
    got, bounds = TO.render_backward(meta, s, bins, w, with_bounds=True)
    tiles = parity.tiles_per_splat(bins, s.B, s.G)
    report = parity.check_grads(serial, got, bounds, tiles, name)
    print(name, report)
    # the bound terms are non-negative and the magnitudes dominate the values
    assert all((bounds[k] >= 0).all() for k in bounds)
    g9 = np.concatenate([np.asarray(x, np.float64).reshape(s.B * s.G, -1) for x in got], axis=1)
    assert np.all(np.abs(g9) <= bounds["mag"] * (1 + 1e-6) + 1e-30)


def test_bar_catches_planted_mistakes():
    sc = SCENES["cfg0"]()
    meta, s, bins, w = _setup(sc)
    ref, bounds = TO.render_backward(meta, s, bins, w, with_bounds=True)
    tiles = parity.tiles_per_splat(bins, s.B, s.G)
    parity.check_grads(ref, ref, bounds, tiles)
    # (a) one pixel's contributions dropped (the pixel with most visible splats)
    _, _, last, _ = TO.render_forward(meta, s, bins)
    b, y, x = np.unravel_index(np.argmax(last), last.shape)
    w2 = w.copy()
    w2[b, y, x] = 0.0
    dropped = TO.render_backward(meta, s, bins, w2)
    with pytest.raises(AssertionError):
        parity.check_grads(dropped, ref, bounds, tiles)
    # (b) the sign of one conic gradient flipped
    flipped = [g.copy() for g in ref]
    i = int(np.argmax(np.abs(ref[1][:, 1])))
    flipped[1][i, 1] = -flipped[1][i, 1]
    with pytest.raises(AssertionError):
        parity.check_grads(flipped, ref, bounds, tiles)
    # (c) the mean gradients 0.3% too large
    scaled = [g.copy() for g in ref]
    scaled[0] *= 1.003
    with pytest.raises(AssertionError):
        parity.check_grads(scaled, ref, bounds, tiles)


def test_results_do_not_depend_on_thread_count():
    sc = SCENES["cfg3_sub"]()
    n0 = TO.threads()
    outs = []
    try:
        for n in (1, 3, max(n0, 2)):
            TO.set_threads(n)
            meta, s, bins, w = _setup(sc)
            fwd = TO.render_forward(meta, s, bins, with_ambiguity=True)
            bwd, bounds = TO.render_backward(meta, s, bins, w, with_bounds=True)
            outs.append((bins, fwd, bwd, bounds))
    finally:
        TO.set_threads(n0)
    b0, f0, g0, k0 = outs[0]
    for b1, f1, g1, k1 in outs[1:]:
        for a, c in ((b0.perm, b1.perm), (b0.tile_counts, b1.tile_counts), (b0.binned_ids, b1.binned_ids)):
            np.testing.assert_array_equal(a, c)
        for a, c in zip(f0, f1):
            np.testing.assert_array_equal(a, c)
        for a, c in zip(g0, g1):
            np.testing.assert_array_equal(a, c)
        for k in k0:
            np.testing.assert_array_equal(k0[k], k1[k])


def _saturating_tile(n_layers):
    """One 16x16 tile covered by n_layers very wide splats of raw alpha 0.999
    (clamped to max_alpha = 0.99): T after two blends is (1 - 0.99)^2, within
    rounding of the 1e-4 threshold, so the stop there is ambiguous."""
    G = n_layers
    conics = np.tile(np.array([[1e-8, 0.0, 1e-8]], np.float32), (G, 1))
    means = np.full((G, 2), 8.0, np.float32)
    sc = TO.Scene(means, conics, np.full((G, 3), 0.5, np.float32), np.full(G, 0.999, np.float32),
                  np.arange(1, G + 1, dtype=np.float32), 1, G)
    meta = TO.make_meta(16, 16, 1, G)
    return meta, sc, TO.bin_scene(meta, sc)


def test_forced_stops_inside_and_outside_the_window():
    meta, s, bins = _saturating_tile(4)
    img, T, last, stop, amb = TO.render_forward(meta, s, bins, with_ambiguity=True)
    assert np.all(last == 2) and np.all((amb & TO.AMB_STOP) != 0)
    assert np.all((amb & TO.AMB_GATE) == 0)
    # the other valid decision: continue through the ambiguous stop, stop at the next blend
    f3 = np.full((1, 16, 16), 3, np.int32)
    img3, T3, last3, _, amb3 = TO.render_forward(meta, s, bins, with_ambiguity=True, force_last=f3)
    assert np.all((amb3 & TO.AMB_FORCED_BAD) == 0) and np.all(last3 == 3)
    np.testing.assert_allclose(T3, T * np.float32(0.01), rtol=1e-5)
    # stopping before T is near the threshold, or walking past a certain stop, is rejected
    for k in (1, 4):
        fk = np.full((1, 16, 16), k, np.int32)
        ambk = TO.render_forward(meta, s, bins, with_ambiguity=True, force_last=fk)[4]
        assert np.all((ambk & TO.AMB_FORCED_BAD) != 0), k
    # -1 leaves the decision to the oracle: identical to no forcing
    fm = np.full((1, 16, 16), -1, np.int32)
    outm = TO.render_forward(meta, s, bins, force_last=fm)
    for a, c in zip(outm, (img, T, last, stop)):
        np.testing.assert_array_equal(a, c)
    # the backward follows the forced walk: the third layer gets gradients
    w = np.ones((1, 16, 16, 3), np.float32)
    g_own = TO.render_backward(meta, s, bins, w)
    g_forced = TO.render_backward(meta, s, bins, w, force_last=f3)
    assert np.all(g_own[2][2:] == 0) and np.all(g_forced[2][2] > 0) and np.all(g_forced[2][3] == 0)


def test_gpu_decisions_helper_forces_only_ambiguous_pixels():
    meta, s, bins = _saturating_tile(4)
    _, _, last, _ = TO.render_forward(meta, s, bins)
    force, (img, T, flast, stop), rep = parity.gpu_decisions(meta, s, bins, last + 1, max_ambiguous_fraction=1.0)
    assert rep["forced_pixels"] == 256 and np.all(flast == 3)
    # a clear decision that differs is a failure, not a forced pixel
    meta1, s1, bins1 = _saturating_tile(1)
    _, _, last1, _ = TO.render_forward(meta1, s1, bins1)
    with pytest.raises(AssertionError):
        parity.gpu_decisions(meta1, s1, bins1, last1 + 1, max_ambiguous_fraction=1.0)


# ------------------------------------------- projection running-error bound
def test_running_error_arithmetic_bounds_float32():
    """RE's first-order bounds hold for float32 evaluations of sums,
    products and quotients of random operands (with cancellation)."""
    from oracle import projection_bounds as PB

    rng = np.random.default_rng(0)
    a, b, c, d = (rng.normal(size=10000).astype(np.float32) for _ in range(4))
    checks = (
        (lambda x, y, z, w: x * y - z * w, None),
        (lambda x, y, z, w: (x + y) / (z * z + 0.5) - w, None),
        (lambda x, y, z, w: ((x * y) * z + w) * (x - w), None),
    )
    for expr, _ in checks:
        got32 = expr(a, b, c, d)
        assert got32.dtype == np.float32
        re = expr(*(PB.RE(v) for v in (a, b, c, d)))
        assert np.all(np.abs(got32.astype(np.float64) - re.v) <= re.e * (1 + 1e-9) + 1e-300)
    # a long float32 sum: the running bound covers it
    x = rng.normal(size=5000).astype(np.float32)
    acc32, acc = np.float32(0.0), PB.RE(0.0)
    for v in x:
        acc32 = np.float32(acc32 + v)
        acc = acc + PB.RE(np.float64(v))
    assert abs(float(acc32) - float(acc.v)) <= float(acc.e)


def _proj_case(B, G, seed):
    from test_gpu_project import _scene

    m, s, q, o, c2w, cam = (t.float().double() for t in _scene(B, G, seed=seed))
    gen = torch.Generator().manual_seed(7)
    w = [torch.randn(B, G, 2, generator=gen, dtype=torch.float64),
         torch.randn(B, G, 3, generator=gen, dtype=torch.float64) * 1e3,
         torch.randn(B, G, generator=gen, dtype=torch.float64),
         torch.randn(B, G, generator=gen, dtype=torch.float64)]
    return (m, s, q, o, c2w, cam), [x.float().double() for x in w]


@pytest.mark.parametrize("B,G", [(1, 2048), (2, 700)])
def test_projection_running_error_vjp_matches_autograd(B, G):
    """The RE evaluation of the projection and its VJP equals float64
    autograd through project_pinhole_reference (values), a float32 autograd
    evaluation stays inside its error bound, and the bound rejects a 0.3%
    scale error and a flipped sign."""
    from oracle import projection_bounds as PB
    from oracle.dense_reference import project_pinhole_reference

    inp, w = _proj_case(B, G, 3)
    leaves = [t.clone().requires_grad_(True) for t in inp]
    out = project_pinhole_reference(*leaves)
    sum((t * wi).sum() for t, wi in zip(out, w)).backward()
    fw = PB.project_forward(*(t.numpy() for t in inp))
    r = PB.project_vjp(*(t.numpy() for t in inp), *(x.numpy() for x in w))
    assert not r["ambiguous"].any()
    for name, ref, k in (("means2d", out[0], 2), ("conics", out[1], 3)):
        v, _ = PB.stack(fw[name])
        np.testing.assert_allclose(v, ref.detach().numpy().reshape(-1, k), rtol=1e-12, atol=1e-12)
    keys = ("means3d", "scales", "quats", "opacities")
    for key, leaf in zip(keys, leaves[:4]):
        v, _ = PB.stack(r[key])
        np.testing.assert_allclose(v, leaf.grad.numpy().reshape(v.shape), rtol=1e-9, atol=1e-9)
    v, _ = PB.stack(r["camera_to_world"])
    np.testing.assert_allclose(v.reshape(B, 4, 4), leaves[4].grad.numpy(), rtol=1e-9, atol=1e-8)
    v, _ = PB.stack(r["camera_params"])
    np.testing.assert_allclose(v, leaves[5].grad.numpy(), rtol=1e-9, atol=1e-9)
    l32 = [t.float().clone().requires_grad_(True) for t in inp]
    out32 = project_pinhole_reference(*l32)
    sum((t * wi.float()).sum() for t, wi in zip(out32, w)).backward()
    for key, leaf in zip(keys, l32[:4]):
        PB.assert_close(leaf.grad.numpy(), r[key], key)
        bad = leaf.grad.numpy().reshape(B * G, -1).astype(np.float64) * 1.003
        with pytest.raises(AssertionError):
            PB.assert_close(bad, r[key], key)
    flipped = l32[0].grad.numpy().reshape(B * G, 3).astype(np.float64).copy()
    i = np.unravel_index(np.argmax(np.abs(flipped)), flipped.shape)
    flipped[i] = -flipped[i]
    with pytest.raises(AssertionError):
        PB.assert_close(flipped, r["means3d"], "means3d")
