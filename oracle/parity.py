"""TEST INFRASTRUCTURE ONLY -- the parity bar the GPU results are held to.

Used by tests/, __graft_entry__.smoke() and nothing in the product path.

Image: rtol 1e-4 / atol 1e-5 at every pixel.

Gradients: every entry of every splat satisfies

    |got - ref| <= 1e-5 + 1e-3 |ref|
                   + 2^-24 (K_CHAIN chain + K_SUM (16 + tiles) mag) + slack

with ref, mag, chain and slack from tile_oracle.render_backward (double sums
of float32 contributions; see oracle_render_backward in tile_oracle.c):
  * 1e-5 + 1e-3 |ref| is the stated gradient bar;
  * mag (sum of cancellation-free magnitudes of the entry's contributions)
    times 16 + tiles bounds the float32 summation of the GPU: a per-lane sum
    of four pixels, a 64-lane tree (6 levels) and one atomic add per tile
    the splat is listed in (`tiles`), each rounding by at most 2^-24 of the
    magnitude sum;
  * chain (magnitudes weighted by the first-order relative error of the
    T_prev and gT each contribution used, in units of 2^-24) times K_CHAIN
    covers the different rounding of those recurrences (hardware exp2 and
    reciprocal within 1 ulp, the segment closed form of gT) -- K_CHAIN = 4:
    one ulp of exp2 moves 1 - alpha by up to alpha/(1-alpha) ulps and the
    reciprocal adds about 2 per division, against the 1 + alpha/(1-alpha)
    per blend that chain counts;
  * slack: contributions whose max_alpha gate lies within rounding (either
    decision is valid).
Both extra terms matter only where contributions cancel; elsewhere rtol
1e-3 dominates.  No splat is excluded: pixels whose stop decision lies in
exp's last-ulp window are re-walked by the oracle with the GPU's decision
(gpu_decisions), which the oracle accepts only inside that window.
"""
from __future__ import annotations

import numpy as np

from . import tile_oracle as TO

U = 2.0 ** -24
K_CHAIN = 4.0
K_SUM = 1.0
IMAGE_RTOL, IMAGE_ATOL = 1e-4, 1e-5
GRAD_RTOL, GRAD_ATOL = 1e-3, 1e-5
# At most this fraction of pixels may have a stop decision inside the window.
MAX_AMBIGUOUS_FRACTION = 1e-4

ENTRY_NAMES = ("means2d", "conics", "colors", "opacities")


def tiles_per_splat(bins: TO.OracleBins, B: int, G: int) -> np.ndarray:
    """int64 [B*G] in original order: how many tile lists hold the splat."""
    per_gid = np.bincount(bins.binned_ids, minlength=B * G).astype(np.int64)
    orig = (np.arange(B * G, dtype=np.int64) // G) * G + bins.perm.astype(np.int64)
    out = np.empty(B * G, dtype=np.int64)
    out[orig] = per_gid
    return out


def grad_allowance(ref9: np.ndarray, bounds: dict, tiles: np.ndarray) -> np.ndarray:
    """[BG, 9] allowed |got - ref| per entry (module docstring)."""
    return (GRAD_ATOL + GRAD_RTOL * np.abs(ref9)
            + U * (K_CHAIN * bounds["chain"] + K_SUM * (16.0 + tiles[:, None]) * bounds["mag"])
            + bounds["slack"])


def _as9(grads, n):
    gm, gq, gc, go = (np.asarray(g, dtype=np.float64).reshape(n, -1) for g in grads)
    return np.concatenate([gm, gq, gc, go], axis=1)


def check_grads(got, ref, bounds: dict, tiles: np.ndarray, label: str = "") -> dict:
    """Asserts the gradient bar on every entry of every splat.  got / ref:
    (means2d, conics, colors, opacities) in original order, any shapes with
    B*G leading elements.  Returns a report: the largest |got - ref| relative
    to the stated bar alone and to the whole allowance, per quantity."""
    n = tiles.size
    g9, r9 = _as9(got, n), _as9(ref, n)
    err = np.abs(g9 - r9)
    allow = grad_allowance(r9, bounds, tiles)
    stated = GRAD_ATOL + GRAD_RTOL * np.abs(r9)
    report = {}
    for name, sl in TO.GRAD_SLICES.items():
        e, a, s = err[:, sl], allow[:, sl], stated[:, sl]
        report[name] = {"max_over_allowance": float((e / a).max()), "max_over_stated_bar": float((e / s).max()),
                        "entries_beyond_stated_bar": int((e > s).sum())}
        bad = e > a
        if bad.any():
            i, j = np.argwhere(bad)[0]
            raise AssertionError(
                f"{label} grad {name}: {int(bad.sum())} of {e.size} entries beyond the bar; first splat {i} "
                f"entry {j}: got {g9[i, sl][j]:.9g} ref {r9[i, sl][j]:.9g} allowance {a[i, j]:.3g} "
                f"(mag {bounds['mag'][i, sl][j]:.3g}, chain {bounds['chain'][i, sl][j]:.3g}, tiles {tiles[i]})")
    return report


def gpu_decisions(meta, s, bins, gpu_last, max_ambiguous_fraction=MAX_AMBIGUOUS_FRACTION):
    """The oracle's forward with the GPU's stop decisions at ambiguous pixels.

    Runs the oracle forward, finds pixels whose stop decision lies inside
    exp's last-ulp window and whose GPU stop count differs, and re-walks
    them with the GPU's count.  Asserts that every other pixel's count
    matches the GPU's exactly, that the forced decisions lie inside the
    window, and that at most max_ambiguous_fraction of the pixels are
    ambiguous.  Returns (force_last or None, forward outputs, report); the
    report also counts the pixels where the reference's own form of the
    alpha test lies within rounding of the threshold (alpha_flagged_pixels)
    or decides differently from the base-2 form the GPU and the oracle share
    (alpha_flipped_pixels): there the GPU matches the oracle, and the
    reference may differ by up to T * alpha_threshold * |colour - bg|."""
    img, T, last, stop, amb = TO.render_forward(meta, s, bins, with_ambiguity=True)
    gpu_last = np.asarray(gpu_last, dtype=np.int32).reshape(last.shape)
    ambiguous = (amb & (TO.AMB_STOP | TO.AMB_GATE)) != 0
    assert ambiguous.mean() <= max_ambiguous_fraction, f"ambiguous pixel fraction {ambiguous.mean():.3g}"
    differ = gpu_last != last
    clear = differ & ~((amb & TO.AMB_STOP) != 0)
    assert not clear.any(), (f"{int(clear.sum())} pixels stop differently although their decision is clear; "
                             f"first at {tuple(np.argwhere(clear)[0])}: gpu {gpu_last[clear][0]} oracle {last[clear][0]}")
    report = {"ambiguous_pixels": int(ambiguous.sum()), "forced_pixels": int(differ.sum()),
              "alpha_flagged_pixels": int(((amb & TO.AMB_ALPHA) != 0).sum()),
              "alpha_flipped_pixels": int(((amb & TO.AMB_ALPHA_FLIP) != 0).sum())}
    if not differ.any():
        return None, (img, T, last, stop), report
    force = np.where(differ, gpu_last, -1).astype(np.int32)
    img, T, last, stop, amb2 = TO.render_forward(meta, s, bins, with_ambiguity=True, force_last=force)
    bad = (amb2 & TO.AMB_FORCED_BAD) != 0
    assert not bad.any(), f"{int(bad.sum())} forced stops lie outside the ambiguity window"
    np.testing.assert_array_equal(last, gpu_last)
    return force, (img, T, last, stop), report


def check_image(got, ref, label: str = "") -> None:
    np.testing.assert_allclose(np.asarray(got).reshape(-1, 3), np.asarray(ref).reshape(-1, 3),
                               rtol=IMAGE_RTOL, atol=IMAGE_ATOL, err_msg=f"{label} image")
