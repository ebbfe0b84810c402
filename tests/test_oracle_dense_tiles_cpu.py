"""The tile oracle against the dense Torch form of the reference, per tile, on full-size scenes.

The oracle (and the HIP compositors, bit for bit) decide the alpha test in a base-2 form;
the reference decides min(max_alpha, o*exp(power)) >= alpha_threshold with power rounded
left to right (gsplat_v8_kernels.metal:121-139), which dense_reference computes in the same
float32 operation order.  The two forms agree except where alpha lies within rounding of the
threshold: the oracle flags those pixels (AMB_ALPHA; AMB_ALPHA_FLIP where the decision differs)
as it does pixels whose early stop lies within rounding (AMB_STOP).

Here, for configs 1-3 at full size (seed 0, the benchmark scenes), dense_reference renders
at least 2,000 sampled tiles of each, plus every tile that holds a flagged pixel, with early
stop and no gradient.  Each tile gets every splat that a conservative distance cull (not the
binning) leaves: a splat whose alpha can reach the threshold somewhere in the tile.  Every
unflagged pixel must match the oracle's image at the image bar (rtol 1e-4, atol 1e-5); a
flagged pixel may differ by what its flipped decisions allow (FLAG_ATOL below).
"""
import numpy as np
import pytest
import torch

from oracle import parity
from oracle import tile_oracle as TO
from oracle.dense_reference import dense_reference
from torch_gsplat_bridge_fast.scenes import make_scene_2d

KEYS = ("means2d", "conics", "colors", "opacities", "depths")
SAMPLED_TILES = 2000
# Pixels flagged AMB_ALPHA / AMB_STOP: one decision may go either way.  A flipped alpha test adds
# or removes a blend of alpha ~ alpha_threshold (1/255): the pixel moves by at most
# alpha_threshold * T * (|colour| + |what is behind|) <= 2 / 255 for colours and background in
# [0, 1]; a flipped early stop moves it by at most T * alpha * |c| with T ~ 1e-4.
FLAG_ATOL = 2.0 / 255.0


def _reach(s_means, s_conics, s_opac, thr):
    """Per splat: the distance from its mean beyond which o*exp(power) < thr (power <= -lmin/2 |d|^2
    for the conic's smaller eigenvalue lmin), with a relative margin of 1e-3 plus 0.01 px that
    dwarfs float32 rounding; +inf for a conic that is not positive definite; -1 for a splat
    whose opacity is below the threshold (never visible)."""
    a, b, c = (s_conics[:, k].astype(np.float64) for k in range(3))
    lmin = 0.5 * (a + c) - np.sqrt((0.5 * (a - c)) ** 2 + b * b)
    o = s_opac.astype(np.float64)
    log_ratio = np.log(np.maximum(o, 1e-38) / thr)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.sqrt(np.maximum(2.0 * log_ratio, 0.0) / lmin) * 1.001 + 0.01
    r = np.where(lmin > 0, r, np.inf)
    return np.where(o >= thr * (1.0 - 1e-6), r, -1.0)


def _tile_candidates(m, reach, tx, ty, H, W):
    """Indices (original order) of the splats whose reach meets the tile's pixel-centre rectangle."""
    rx0, ry0 = 16 * tx + 0.5, 16 * ty + 0.5
    rx1, ry1 = min(16 * tx + 15.5, W - 0.5), min(16 * ty + 15.5, H - 0.5)
    mx, my = m[:, 0].astype(np.float64), m[:, 1].astype(np.float64)
    ddx = np.maximum(np.maximum(rx0 - mx, mx - rx1), 0.0)
    ddy = np.maximum(np.maximum(ry0 - my, my - ry1), 0.0)
    return np.flatnonzero(ddx * ddx + ddy * ddy <= reach * reach)


@pytest.mark.parametrize("cfg", [1, 2, 3])
def test_oracle_matches_dense_torch_form_per_tile(cfg):
    sc = make_scene_2d(cfg, seed=0)
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    meta = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(sc[k].numpy() for k in KEYS), B, G)
    bins = TO.bin_scene(meta, s)
    img, T, last, stop, amb = TO.render_forward(meta, s, bins, with_ambiguity=True)
    flag_alpha = (amb & TO.AMB_ALPHA) != 0
    flagged = (amb & (TO.AMB_ALPHA | TO.AMB_STOP)) != 0
    tiles_x, tiles_y = (W + 15) // 16, (H + 15) // 16
    tpi = tiles_x * tiles_y
    rng = np.random.default_rng(cfg)
    sample = set(rng.choice(B * tpi, size=min(SAMPLED_TILES, B * tpi), replace=False).tolist())
    for b, y, x in np.argwhere(flag_alpha):
        sample.add(int(b) * tpi + (int(y) // 16) * tiles_x + int(x) // 16)
    thr = meta.alpha_threshold
    reach = [_reach(sc["means2d"][b].numpy(), sc["conics"][b].numpy(), sc["opacities"][b].numpy(), thr)
             for b in range(B)]
    print(f"cfg{cfg}: {len(sample)} tiles, {int(flag_alpha.sum())} AMB_ALPHA pixels "
          f"({int(((amb & TO.AMB_ALPHA_FLIP) != 0).sum())} flipped), {int(((amb & TO.AMB_STOP) != 0).sum())} AMB_STOP",
          flush=True)
    # tiles with their candidate splats, rendered GROUP at a time in order of candidate count; a
    # group's lists are padded with splats of opacity 0 and depth +inf (sorted last, never visible:
    # they leave T and the colour unchanged)
    work = []
    for t in sorted(sample):
        b, lt = divmod(t, tpi)
        ty, tx = divmod(lt, tiles_x)
        work.append((t, b, tx, ty, _tile_candidates(sc["means2d"][b].numpy(), reach[b], tx, ty, H, W)))
    work.sort(key=lambda w: w[4].size)
    worst_clear = worst_flag = worst_flag_bar = 0.0
    n_flag = 0
    GROUP = 64
    with torch.no_grad():
        for g0 in range(0, len(work), GROUP):
            grp = work[g0:g0 + GROUP]
            K = max(1, max(w[4].size for w in grp))
            pad = {"means2d": torch.zeros(len(grp), K, 2), "conics": torch.tensor([1.0, 0.0, 1.0]).repeat(len(grp), K, 1),
                   "colors": torch.zeros(len(grp), K, 3), "opacities": torch.zeros(len(grp), K),
                   "depths": torch.full((len(grp), K), float("inf"))}
            for j, (t, b, tx, ty, idx) in enumerate(grp):
                for k in KEYS:
                    pad[k][j, :idx.size] = sc[k][b][torch.from_numpy(idx)]
            ref = dense_reference(*(pad[k] for k in KEYS), 16, 16, background=meta_bg(meta), alpha_threshold=thr,
                                  max_alpha=meta.max_alpha, early_stop=True,
                                  transmittance_threshold=meta.transmittance_threshold,
                                  x0=[16 * w[2] for w in grp], y0=[16 * w[3] for w in grp]).numpy()
            for j, (t, b, tx, ty, idx) in enumerate(grp):
                h, w = min(16, H - 16 * ty), min(16, W - 16 * tx)
                got = img[b, 16 * ty:16 * ty + h, 16 * tx:16 * tx + w].astype(np.float64)
                fl = flagged[b, 16 * ty:16 * ty + h, 16 * tx:16 * tx + w]
                r = ref[j, :h, :w]
                err = np.abs(got - r)
                bar = parity.IMAGE_ATOL + parity.IMAGE_RTOL * np.abs(r)
                clear = err[~fl] / bar[~fl]
                if clear.size:
                    worst_clear = max(worst_clear, float(clear.max()))
                    assert clear.max() <= 1.0, (
                        f"cfg{cfg} tile {t} (b={b}, tx={tx}, ty={ty}): unflagged pixel off the dense reference by "
                        f"{float((err[~fl]).max()):.3g}")
                if fl.any():
                    n_flag += int(fl.sum())
                    worst_flag = max(worst_flag, float(err[fl].max()))
                    worst_flag_bar = max(worst_flag_bar, float((err[fl] / bar[fl]).max()))
                    assert err[fl].max() <= FLAG_ATOL
    print(f"cfg{cfg}: worst unflagged error / bar {worst_clear:.3f}; {n_flag} flagged pixels, "
          f"worst flagged error {worst_flag:.3g} ({worst_flag_bar:.1f} x the bar)")
    if (amb & TO.AMB_ALPHA_FLIP).any():
        # the flags are not vacuous: where the two forms decide differently the images differ
        # beyond the bar
        assert worst_flag_bar > 1.0


def meta_bg(meta):
    return tuple(float(v) for v in meta.bg)
