"""CPU tests that pin the oracle (oracle/) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle fails it:
  * oracle_logf against libm in double precision (ulp bound) and its special
    values;
  * the binning predicate against brute force in double precision:
    completeness (every pixel-centre point with alpha >= threshold has its
    tile listed) and tightness (every listed tile really comes within the
    support ellipse), plus count/order invariants;
  * the depth order against numpy's stable argsort (ties, -0/+0, NaN, inf);
  * the dense Torch reference against closed forms and finite differences;
  * the C tile oracle against the dense Torch reference (image and gradients);
  * the committed golden fixtures (regression anchors).
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import parity
from oracle import tile_oracle as TO
from oracle.dense_reference import dense_reference, project_pinhole_reference
from torch_gsplat_bridge_fast.scenes import make_scene_2d

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
KEYS = ("means2d", "conics", "colors", "opacities", "depths")
THR = 1.0 / 255.0


def _ulp(x):
    return np.spacing(np.float32(x)).astype(np.float64)


# ----------------------------------------------------------------- logf
def test_logf_accuracy_against_libm():
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        10.0 ** rng.uniform(-8, 0, 20000),            # the predicate's range
        10.0 ** rng.uniform(-37, 37, 5000),
        np.array([1.0, 2.0, 0.5, np.sqrt(2), 1.0 / 255.0, 1e-8, 3e-39, 1e-45]),
    ]).astype(np.float32)
    worst = 0.0
    for x in xs:
        got = TO.logf(float(x))
        ref = math.log(float(x))
        err = abs(got - ref) / float(_ulp(ref if ref != 0 else 1.0))
        worst = max(worst, err)
    assert worst <= 4.0, worst
    assert TO.logf(1.0) == 0.0


def test_logf_special_values():
    assert math.isnan(TO.logf(float("nan")))
    assert TO.logf(0.0) == -math.inf
    assert math.isnan(TO.logf(-1.0))
    assert TO.logf(math.inf) == math.inf


# ----------------------------------------------------------------- plim
def test_plim_is_the_alpha_threshold_exponent():
    """o * 2^plim == alpha_threshold up to a few float ulps (closed form), so the
    compositor's p >= plim is the reference's o*exp(power) >= threshold."""
    rng = np.random.default_rng(5)
    thr = np.float32(THR)
    for o in np.concatenate([rng.uniform(0.004, 1.0, 2000), [1.0, 0.5, 0.99, float(thr)]]).astype(np.float32):
        p = TO.plim(float(o), float(thr), 0.99)
        exact = math.log2(float(thr) / float(o))
        assert abs(p - exact) <= 8 * abs(_ulp(exact)) + 1e-7, (o, p, exact)
        assert abs(float(o) * 2.0 ** p - float(thr)) <= 1e-6 * float(thr) + 1e-12
    # opacity exactly at the threshold: plim == 0, only p == 0 is visible
    assert TO.plim(float(thr), float(thr), 0.99) == 0.0


def test_opacity_log2_is_log2_of_the_opacity():
    """lo = log2(e)_f32 * ln(o) within a few float ulps of log2(o) (closed form), so 2^(p + lo) is
    o * 2^p; plim + lo is the exponent limit with lo folded in, log2(threshold) up to rounding."""
    rng = np.random.default_rng(6)
    thr = np.float32(THR)
    for o in np.concatenate([10.0 ** rng.uniform(-6, 0, 2000), [1.0, 0.5, 0.25, 0.99, float(thr)]]).astype(np.float32):
        lo = TO.opacity_log2(float(o))
        exact = math.log2(float(o))
        assert abs(lo - exact) <= 8 * abs(_ulp(exact if exact != 0 else 1.0)), (o, lo, exact)
        q = np.float32(TO.plim(float(o), float(thr), 0.99)) + np.float32(lo)
        assert abs(float(q) - math.log2(float(thr))) <= 1e-5, (o, q)
    assert TO.opacity_log2(1.0) == 0.0 and TO.opacity_log2(0.5) == -1.0
    assert TO.opacity_log2(0.0) == -math.inf
    assert math.isnan(TO.opacity_log2(-0.5)) and math.isnan(TO.opacity_log2(float("nan")))


def test_plim_special_cases():
    assert TO.plim(0.0, THR, 0.99) == math.inf            # nothing visible
    assert TO.plim(-0.5, THR, 0.99) == math.inf
    assert TO.plim(float("nan"), THR, 0.99) == math.inf
    assert TO.plim(0.5, 0.5, 0.4) == math.inf             # max_alpha < threshold
    assert TO.plim(0.5, 0.0, 0.99) == -math.inf           # every p <= 0 visible
    assert TO.plim(1e-45, THR, 0.99) > 100                # thr/o overflows: invisible
    # o far above thr: thr/o clamps at FLT_MIN, plim = log2(FLT_MIN) = -126
    assert abs(TO.plim(3e38, 1e-30, 0.99) + 126.0) < 1e-4


# ----------------------------------------------------------- depth order
def test_depth_order_matches_stable_argsort():
    rng = np.random.default_rng(1)
    B, G = 3, 500
    d = rng.integers(-3, 4, size=(B, G)).astype(np.float32)
    d[0, :5] = [0.0, -0.0, np.nan, np.inf, -np.inf]
    d[1, 10:20] = np.nan
    d[2] = rng.normal(size=G).astype(np.float32)
    perm = TO.depth_order(d, B, G).reshape(B, G)
    for b in range(B):
        np.testing.assert_array_equal(perm[b], np.argsort(d[b], kind="stable"))


# ------------------------------------------------------------- binning
def _splat_set(bins, G):
    """{orig index: set(tile)} from the oracle's tile lists (B=1)."""
    out = {}
    for t in range(bins.tile_counts.size):
        for gid in bins.binned_ids[bins.tile_offsets[t]:bins.tile_offsets[t + 1]]:
            out.setdefault(int(bins.perm[gid]), set()).add(t)
    return out


def _random_splats(rng, G, H, W, off=20):
    m = rng.uniform(-off, W + off, size=(G, 2))
    m[:, 1] = rng.uniform(-off, H + off, size=G)
    sig = rng.uniform(0.3, 9.0, size=(G, 2))
    th = rng.uniform(0, np.pi, size=G)
    c, s = np.cos(th), np.sin(th)
    ix, iy = 1 / sig[:, 0] ** 2, 1 / sig[:, 1] ** 2
    q = np.stack([c * c * ix + s * s * iy, c * s * (ix - iy), s * s * ix + c * c * iy], -1)
    o = rng.uniform(0.0, 1.0, size=G)
    return m.astype(np.float32), q.astype(np.float32), o.astype(np.float32)


def _q64(a, b, c, dx, dy):
    return a * dx * dx + 2 * b * dx * dy + c * dy * dy


@pytest.mark.parametrize("seed,H,W,G", [(0, 48, 64, 60), (1, 37, 29, 80), (2, 64, 64, 40)])
def test_binning_complete_and_tight(seed, H, W, G):
    rng = np.random.default_rng(seed)
    m, q, o = _random_splats(rng, G, H, W)
    col = rng.uniform(0, 1, (G, 3)).astype(np.float32)
    d = rng.uniform(0, 1, G).astype(np.float32)
    meta = TO.make_meta(H, W, 1, G)
    bins = TO.bin_scene(meta, TO.Scene(m, q, col, o, d, 1, G))
    sets = _splat_set(bins, G)
    tiles_x = (W + 15) // 16
    tiles_y = (H + 15) // 16
    for i in range(G):
        listed = sets.get(i, set())
        a, b, c = (float(v) for v in q[i])
        if o[i] <= THR:
            assert not listed
            continue
        tau = -2.0 * math.log(THR / float(o[i]))
        for ty in range(tiles_y):
            for tx in range(tiles_x):
                t = ty * tiles_x + tx
                # pixel-centre rectangle of the tile, sampled on a 1/8 px grid
                xs = np.arange(tx * 16 + 0.5, min(tx * 16 + 15, W - 1) + 0.5 + 1e-9, 0.125)
                ys = np.arange(ty * 16 + 0.5, min(ty * 16 + 15, H - 1) + 0.5 + 1e-9, 0.125)
                X, Y = np.meshgrid(xs, ys)
                qq = _q64(a, b, c, X - float(m[i, 0]), Y - float(m[i, 1]))
                qmin = float(qq.min())
                # completeness: a point clearly inside the support => listed
                if qmin < tau * (1.0 - 1e-5):
                    assert t in listed, (i, t, qmin, tau)
                # tightness: listed => the rectangle reaches the support
                # (grid error <= |grad q| * half-diagonal of a grid cell)
                if t in listed:
                    gx = 2 * (a * (X - m[i, 0]) + b * (Y - m[i, 1]))
                    gy = 2 * (b * (X - m[i, 0]) + c * (Y - m[i, 1]))
                    slack = float(np.sqrt(gx * gx + gy * gy).max()) * 0.0885
                    assert qmin <= tau * (1.0 + 1e-5) + slack, (i, t, qmin, tau)


def test_binning_isotropic_closed_form():
    """An isotropic splat centred on a tile corner, radius r = sqrt(tau)*sigma,
    touches exactly the tiles whose pixel-centre rectangles meet the disk."""
    H = W = 64
    sigma, o = 5.0, 0.9
    m = np.array([[32.0, 32.0]], np.float32)
    q = np.array([[1 / sigma ** 2, 0.0, 1 / sigma ** 2]], np.float32)
    meta = TO.make_meta(H, W, 1, 1)
    bins = TO.bin_scene(meta, TO.Scene(m, q, np.ones((1, 3)), np.array([o]), np.zeros(1), 1, 1))
    r = math.sqrt(-2 * math.log(THR / o)) * sigma
    expect = set()
    for ty in range(4):
        for tx in range(4):
            x0, x1 = tx * 16 + 0.5, tx * 16 + 15.5
            y0, y1 = ty * 16 + 0.5, ty * 16 + 15.5
            dx = max(x0 - 32, 0, 32 - x1)
            dy = max(y0 - 32, 0, 32 - y1)
            if dx * dx + dy * dy <= r * r:
                expect.add(ty * 4 + tx)
    got = {t for t in range(16) if bins.tile_counts[t] > 0}
    assert got == expect == {5, 6, 9, 10}


def test_binning_invariants_config0():
    sc = make_scene_2d(0, seed=3)
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    meta = TO.make_meta(H, W, B, G)
    bins = TO.bin_scene(meta, TO.Scene(*(sc[k].numpy() for k in KEYS), B, G))
    assert bins.tile_counts.sum() == bins.binned_ids.size == bins.tile_offsets[-1]
    np.testing.assert_array_equal(np.diff(bins.tile_offsets), bins.tile_counts)
    keys = bins.sorted_keys()
    assert np.all(keys[1:] > keys[:-1])           # sorted, no duplicate pairs


# ------------------------------------------------- dense reference (math)
def _one(m, q, c, o, d):
    t = lambda v: torch.tensor(v, dtype=torch.float64)  # noqa: E731
    return t(m), t(q), t(c), t(o), t(d)


def test_dense_single_splat_closed_form():
    # splat centred on pixel (3,2): power = 0 there, alpha = min(0.99, o)
    for o, expect_alpha in ((0.7, 0.7), (0.999, 0.99)):
        m, q, c, op, d = _one([[3.5, 2.5]], [[0.3, 0.05, 0.2]], [[0.2, 0.4, 0.8]], [o], [1.0])
        img = dense_reference(m, q, c, op, d, 5, 6, background=(0.1, 0.1, 0.1))
        exp = expect_alpha * np.array([0.2, 0.4, 0.8]) + (1 - expect_alpha) * 0.1
        np.testing.assert_allclose(img[2, 3].numpy(), exp, rtol=1e-12)
        # a pixel one step right: alpha = o * exp(-0.5 * a)
        a1 = min(0.99, o * math.exp(-0.5 * 0.3))
        np.testing.assert_allclose(img[2, 4].numpy(), a1 * np.array([0.2, 0.4, 0.8]) + (1 - a1) * 0.1, rtol=1e-12)


def test_dense_threshold_and_two_layers():
    # below 1/255 the splat is dropped entirely
    m, q, c, op, d = _one([[1.5, 1.5]], [[1.0, 0.0, 1.0]], [[1.0, 1.0, 1.0]], [0.003], [1.0])
    assert float(dense_reference(m, q, c, op, d, 3, 3).abs().max()) == 0.0
    # two coincident splats: C = a_front c_front + (1-a_front) a_back c_back;
    # the green splat (depth 1) is in front of the red one (depth 2)
    m, q, c, op, d = _one([[1.5, 1.5], [1.5, 1.5]], [[1, 0, 1], [1, 0, 1]], [[1, 0, 0], [0, 1, 0]],
                          [0.6, 0.5], [2.0, 1.0])
    img = dense_reference(m, q, c, op, d, 3, 3)
    np.testing.assert_allclose(img[1, 1].numpy(), [0.5 * 0.6, 0.5, 0.0], rtol=1e-12)


def test_dense_early_stop_semantics():
    # four layers of alpha 0.99 at one pixel (red, green, blue, white): T after
    # them is 1e-2, 1e-4 (+rounding, still > 1e-4), 1e-6; the early-stop
    # reference drops the fourth layer, the plain one composites it
    m, q, c, op, d = _one([[0.5, 0.5]] * 4, [[1, 0, 1]] * 4, [[1, 0, 0], [0, 1, 0], [0, 0, 1], [1, 1, 1]],
                          [0.99] * 4, [1.0, 2.0, 3.0, 4.0])
    full = dense_reference(m, q, c, op, d, 1, 1)[0, 0].numpy()
    stop = dense_reference(m, q, c, op, d, 1, 1, early_stop=True)[0, 0].numpy()
    w4 = 0.99 * 1e-6
    np.testing.assert_allclose(full, [0.99 + w4, 0.0099 + w4, 0.000099 + w4], rtol=1e-9)
    np.testing.assert_allclose(stop, [0.99, 0.0099, 0.000099], rtol=1e-9)


def test_dense_gradcheck():
    torch.manual_seed(0)
    m = torch.tensor([[2.3, 1.8], [3.1, 2.6], [1.2, 2.9]], dtype=torch.float64, requires_grad=True)
    q = torch.tensor([[0.4, 0.05, 0.3], [0.25, -0.04, 0.35], [0.5, 0.1, 0.45]], dtype=torch.float64,
                     requires_grad=True)
    c = torch.rand(3, 3, dtype=torch.float64, requires_grad=True)
    o = torch.tensor([0.6, 0.5, 0.7], dtype=torch.float64, requires_grad=True)
    d = torch.tensor([0.3, 0.1, 0.2], dtype=torch.float64)

    def f(m, q, c, o):
        return dense_reference(m, q, c, o, d, 4, 5, background=(0.2, 0.3, 0.4))

    assert torch.autograd.gradcheck(f, (m, q, c, o), eps=1e-6, atol=1e-6)


# ------------------------------------------- C oracle vs dense reference
@pytest.mark.parametrize("seed,H,W,G,bg", [(3, 64, 64, 64, (0, 0, 0)), (4, 48, 72, 100, (1, 1, 1)),
                                          (5, 37, 53, 40, (0.2, 0.5, 0.9)), (6, 128, 128, 400, (0.1, 0.2, 0.3))])
def test_tile_oracle_matches_dense_reference(seed, H, W, G, bg):
    sc = make_scene_2d(0, seed=seed, G=G, H=H, W=W)
    meta = TO.make_meta(H, W, 1, G, background=bg)
    s = TO.Scene(*(sc[k][0].numpy() for k in KEYS), 1, G)
    bins = TO.bin_scene(meta, s)
    img, T, last, stop = TO.render_forward(meta, s, bins)
    ts = [sc[k][0].clone().requires_grad_(k != "depths") for k in KEYS]
    ref = dense_reference(*ts, H, W, background=bg, early_stop=True)
    # pixels where the dense form's alpha test or early stop may decide otherwise (tile_oracle:
    # render_forward) weigh nothing in the loss, so that no gradient depends on them
    _, _, _, _, amb = TO.render_forward(meta, s, bins, with_ambiguity=True)
    flagged = (amb[0] & (TO.AMB_ALPHA | TO.AMB_STOP)) != 0
    assert flagged.mean() < 1e-3
    w = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(seed))
    w[torch.from_numpy(flagged)] = 0.0
    (ref * w).sum().backward()
    grads, bounds = TO.render_backward(meta, s, bins, w.numpy()[None], with_bounds=True)
    parity.check_image(img[0][~flagged], ref.detach().numpy()[~flagged], "oracle vs dense")
    # the gradient bar of the GPU tests, entry by entry: 1e-5 + 1e-3 |ref| plus the rounding
    # allowance (dense autograd sums each entry over every pixel in float32)
    dense = [t.grad.numpy() for t in ts[:4]]
    parity.check_grads(dense, grads, bounds, parity.tiles_per_splat(bins, 1, G), "dense vs oracle")
    # final T and last index are consistent with the image definition
    assert np.all((T >= 0) & (T <= 1))
    assert np.all(stop == np.array([last[0, ty * 16:(ty + 1) * 16, tx * 16:(tx + 1) * 16].max()
                                    for ty in range((H + 15) // 16) for tx in range((W + 15) // 16)]))


# ------------------------------------------------------ golden fixtures
def test_golden_config0_regression():
    g = np.load(os.path.join(GOLDEN, "config0_oracle.npz"))
    sc = make_scene_2d(0, seed=0)
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    meta = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(sc[k].numpy() for k in KEYS), B, G)
    bins = TO.bin_scene(meta, s)
    np.testing.assert_array_equal(bins.perm, g["perm"])
    np.testing.assert_array_equal(bins.tile_counts, g["tile_counts"])
    np.testing.assert_array_equal(bins.binned_ids, g["binned_ids"])
    img, T, last, stop = TO.render_forward(meta, s, bins)
    np.testing.assert_allclose(img[0, 200:264, 300:364], g["img_crop"], rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(stop, g["tile_stop"])
    w = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(123)).numpy()
    # the fixture holds the reference-order float32 sums (render_backward_serial)
    serial = TO.render_backward_serial(meta, s, bins, w[None])
    for name, v in zip(("g_means2d", "g_conics", "g_colors", "g_opacities"), serial):
        np.testing.assert_allclose(v, g[name], rtol=1e-6, atol=1e-6 * max(1.0, float(np.abs(g[name]).max())))
    # the parallel double-sum backward agrees with them within its own bounds
    got, bounds = TO.render_backward(meta, s, bins, w[None], with_bounds=True)
    fixture = [g[k] for k in ("g_means2d", "g_conics", "g_colors", "g_opacities")]
    parity.check_grads(fixture, got, bounds, parity.tiles_per_splat(bins, B, G), "config0 fixture")


def test_golden_reference_hand_case_values():
    """The fixture holds the reference test's literal inputs (reference_check.py:118-144)."""
    with open(os.path.join(GOLDEN, "reference_hand_cases.json")) as f:
        hc = json.load(f)
    assert np.array(hc["means2d"]).shape == (2, 4, 2)
    assert hc["opacities"][0] == [0.8, 0.6, 0.5, 0.7]
    assert hc["depths"][1] == [0.3, 0.1, 0.4, 0.2]


# ------------------------------------------------------------ projection
def test_projection_closed_form():
    z, s, f = 4.0, 0.2, 500.0
    t = lambda v: torch.tensor(v, dtype=torch.float64)  # noqa: E731
    means = t([[[0.0, 0.0, z], [0.0, 0.0, -2.0]]])
    scales = t([[[s, s, s], [s, s, s]]])
    quats = t([[[1.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0]]])
    opac = t([[0.8, 0.8]])
    c2w = torch.eye(4, dtype=torch.float64).unsqueeze(0)
    cam = t([[f, f, 320.0, 240.0]])
    m2, cq, op, dp = project_pinhole_reference(means, scales, quats, opac, c2w, cam)
    var = (f * s / z) ** 2 + 0.3
    np.testing.assert_allclose(m2[0, 0].numpy(), [320.0, 240.0])
    np.testing.assert_allclose(cq[0, 0].numpy(), [1 / var, 0.0, 1 / var], rtol=1e-12)
    assert float(dp[0, 0]) == z and float(op[0, 0]) == 0.8
    # behind the near plane: opacity 0, centred, depth kept
    np.testing.assert_allclose(m2[0, 1].numpy(), [320.0, 240.0])
    assert float(op[0, 1]) == 0.0 and float(dp[0, 1]) == -2.0


def test_projection_gradcheck():
    torch.manual_seed(1)
    means = torch.tensor([[[0.3, -0.2, 2.0], [1.0, 0.5, 6.0]]], dtype=torch.float64, requires_grad=True)
    scales = torch.tensor([[[0.1, 0.2, 0.05], [0.3, 0.25, 0.2]]], dtype=torch.float64, requires_grad=True)
    quats = torch.tensor([[[0.9, 0.1, -0.3, 0.2], [0.7, 0.2, 0.1, -0.4]]], dtype=torch.float64, requires_grad=True)
    opac = torch.tensor([[0.7, 0.4]], dtype=torch.float64, requires_grad=True)
    c2w = torch.eye(4, dtype=torch.float64).unsqueeze(0).clone()
    c2w[0, :3, 3] = torch.tensor([0.1, -0.05, -0.5], dtype=torch.float64)
    c2w.requires_grad_(True)
    cam = torch.tensor([[500.0, 480.0, 320.0, 240.0]], dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda *a: project_pinhole_reference(*a), (means, scales, quats, opac, c2w, cam),
                                    eps=1e-6, atol=1e-5, rtol=1e-4)


def test_golden_projection_regression():
    with open(os.path.join(GOLDEN, "projection_cases.json")) as f:
        pc = json.load(f)
    i = {k: torch.tensor(v, dtype=torch.float64) for k, v in pc["inputs"].items()}
    out = project_pinhole_reference(i["means3d"], i["scales"], i["quats"], i["opacities"], i["camera_to_world"],
                                    i["camera_params"], pc["near_plane"])
    for name, v in zip(("means2d", "conics", "opacities_out", "depths"), out):
        np.testing.assert_allclose(v.numpy(), np.array(pc["outputs"][name]), rtol=1e-12, atol=1e-12)


# ------------------------------------------------ stop counts (local_stop)
def _stop_scene(opacities, sigmas, means):
    """One 16x16 tile; splats in depth order with isotropic sigmas."""
    G = len(opacities)
    s2 = np.asarray(sigmas, dtype=np.float32) ** 2
    conics = np.stack([1.0 / s2, np.zeros(G, np.float32), 1.0 / s2], axis=1).astype(np.float32)
    meta = TO.make_meta(16, 16, 1, G)
    sc = TO.Scene(np.asarray(means, np.float32), conics, np.full((G, 3), 0.5, np.float32),
                  np.asarray(opacities, np.float32), np.arange(1, G + 1, dtype=np.float32), 1, G)
    bins = TO.bin_scene(meta, sc)
    assert int(bins.tile_counts[0]) == G
    return TO.render_forward(meta, sc, bins)


def test_stop_count_of_pixels_that_never_stop_is_the_list_length():
    """Reference tile_fast_forward_state (gsplat_v8_kernels.metal:455-467) sets
    local_stop = j + 1 for every splat a live pixel iterates, visible or not:
    two wide splats (alpha 0.9 each, T = 0.01 > 1e-4 after both) and a small one
    seen only near the tile's corner.  Every pixel iterates all three."""
    img, T, last, stop = _stop_scene([0.9, 0.9, 0.5], [1000.0, 1000.0, 1.0],
                                     [[8.0, 8.0], [8.0, 8.0], [1.5, 1.5]])
    assert np.all(T > 1e-4)
    assert np.all(last == 3) and int(stop[0]) == 3
    # the small splat is invisible at the far corner, so "last composited"
    # would have been 2 there
    assert abs(float(T[0, 15, 15]) - 0.01) < 1e-4


def test_stop_count_is_one_past_the_stopping_splat():
    """Five wide splats of alpha ~0.95: T = 0.05, 2.5e-3, 1.25e-4 (> 1e-4), then
    6.3e-6 <= 1e-4, so every pixel stops at the fourth (local_stop = 4 and the
    loop breaks, gsplat_v8_kernels.metal:467); the fifth is never iterated."""
    img, T, last, stop = _stop_scene([0.95] * 5, [1000.0] * 5, [[8.0, 8.0]] * 5)
    assert np.all((T > 5e-6) & (T < 7e-6))
    assert np.all(last == 4) and int(stop[0]) == 4
