"""TEST INFRASTRUCTURE ONLY -- numpy interface to the CPU oracle tile_oracle.c.

Used by tests/ as the parity checker and by bench.py's cpu_baseline leg;
never by the product path.  See tile_oracle.c for the reference lines each
function restates.  Build: ``make -C oracle`` (also done by
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libtile_oracle.so")


class OracleMeta(ctypes.Structure):
    _fields_ = [
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("gpb", ctypes.c_int32),
        ("alpha_threshold", ctypes.c_float),
        ("transmittance_threshold", ctypes.c_float),
        ("bg", ctypes.c_float * 3),
        ("eps", ctypes.c_float),
        ("max_alpha", ctypes.c_float),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing at {LIB_PATH}; run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        vp = ctypes.c_void_p
        pm = ctypes.POINTER(OracleMeta)
        L.oracle_logf.restype = ctypes.c_float
        L.oracle_logf.argtypes = [ctypes.c_float]
        L.oracle_plim.restype = ctypes.c_float
        L.oracle_plim.argtypes = [ctypes.c_float] * 3
        L.oracle_opacity_log2.restype = ctypes.c_float
        L.oracle_opacity_log2.argtypes = [ctypes.c_float]
        L.oracle_depth_order.restype = None
        L.oracle_depth_order.argtypes = [vp, ctypes.c_int32, ctypes.c_int32, vp]
        L.oracle_bin_count.restype = ctypes.c_int64
        L.oracle_bin_count.argtypes = [pm, vp, vp, vp, vp, vp, vp]
        L.oracle_bin_fill.restype = None
        L.oracle_bin_fill.argtypes = [pm, vp, vp, vp, vp, vp, vp]
        L.oracle_render_forward.restype = None
        L.oracle_render_forward.argtypes = [pm] + [vp] * 13
        L.oracle_render_backward.restype = None
        L.oracle_render_backward.argtypes = [pm] + [vp] * 16
        L.oracle_render_backward_serial.restype = None
        L.oracle_render_backward_serial.argtypes = [pm] + [vp] * 12
        L.oracle_threads.restype = ctypes.c_int
        L.oracle_threads.argtypes = []
        L.oracle_set_threads.restype = None
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a, shape=None):
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    return a if shape is None else a.reshape(shape)


def make_meta(height, width, batch, gpb, alpha_threshold=1.0 / 255.0, transmittance_threshold=1e-4,
              background=(0.0, 0.0, 0.0), eps=1e-8, max_alpha=0.99) -> OracleMeta:
    m = OracleMeta()
    m.height, m.width, m.batch, m.gpb = int(height), int(width), int(batch), int(gpb)
    m.alpha_threshold = float(alpha_threshold)
    m.transmittance_threshold = float(transmittance_threshold)
    for i in range(3):
        m.bg[i] = float(background[i])
    m.eps = float(eps)
    m.max_alpha = float(max_alpha)
    return m


def logf(x: float) -> float:
    return float(lib().oracle_logf(ctypes.c_float(x)))


def plim(opacity: float, alpha_threshold: float, max_alpha: float) -> float:
    """Base-2 exponent limit of the alpha test (float32 value as a Python float)."""
    return float(lib().oracle_plim(ctypes.c_float(opacity), ctypes.c_float(alpha_threshold),
                                   ctypes.c_float(max_alpha)))


def opacity_log2(opacity: float) -> float:
    """log2(e)_f32 * oracle_logf(opacity): the packed record's lo (the compositors evaluate
    o * 2^p as 2^(p + lo))."""
    return float(lib().oracle_opacity_log2(ctypes.c_float(opacity)))


def strip_consts(a, b, c, plim) -> np.ndarray:
    """float32 [n, 4] (dxt, beta, gamma, delta): the per-splat strip-culling constants of a packed
    record, restating strip_consts_t of fast-mac-gsplat_amd/csrc/gs_strip.h with correctly rounded
    float32 operations in its order (numpy fuses nothing).  Invisible splats (plim > 0) get
    (0, NaN, inf, 0), never-culled ones (0, 0, inf, 0).  The strips these constants select have no
    reference counterpart (they only skip work; tests/test_strip_mask_cpu.py checks on the C source
    that no strip with a visible pixel is skipped); this restatement pins the device's arithmetic
    to that source bit for bit."""
    f = np.float32
    a, b, c, plim = (np.asarray(x, np.float32).reshape(-1) for x in (a, b, c, plim))
    out = np.zeros((a.size, 4), np.float32)
    out[:, 2] = np.inf
    with np.errstate(all="ignore"):
        tau = f(-1.38629436) * plim
        det = a * c - b * b
        ok = (a > 0) & (c > 0) & (det > f(1e-3) * (a * c)) & (tau < f(3.0e38)) & ~(plim > 0)
        tc = tau * f(1.02) + f(1e-3)
        hy = np.sqrt((a * tc) / det)
        vals = np.stack([(-b * hy) / a, (-b) / c, tc / c, det / (c * c)], axis=1).astype(np.float32)
    out[ok] = vals[ok]
    out[plim > 0, 1] = np.float32(np.nan)
    return out


def plain_flags(a, b, c, mx, my, o, max_alpha) -> np.ndarray:
    """bool [n]: the packed record's plain flag, restating plain_record of gs_strip.h on the
    compositors' base-2 coefficients A = (-a/2) L, B = (-b) L, C = (-c/2) L (float32, L = log2(e)
    rounded), with o_plain = min(max_alpha, 1) (1 - 2^-16).  The flag only selects a shorter but
    equivalent evaluation of the same alpha test (the bound is proved in gs_strip.h and exercised by
    the plain/general GPU tests); this restatement pins the device's flag bit for bit."""
    f = np.float32
    a, b, c, mx, my, o = (np.asarray(x, np.float32).reshape(-1) for x in (a, b, c, mx, my, o))
    L = f(1.44269502)
    with np.errstate(all="ignore"):
        A = (f(-0.5) * a) * L
        B = (-b) * L
        C = (f(-0.5) * c) * L
        aa, cc = -A, -C
        s = aa + cc
        o_plain = np.minimum(f(max_alpha), f(1.0)) * f(1.0 - 2.0 ** -16)
        big, tiny, lim = f(2.0 ** 40), f(2.0 ** -60), f(2.0 ** 32)
        return ((o >= f(2.0 ** -20)) & (o <= o_plain) & (aa >= tiny) & (cc >= tiny) & (aa <= big) & (cc <= big)
                & (B <= big) & (B >= -big) & (f(4.0) * aa * cc - B * B >= f(2.0 ** -16) * s * s)
                & (mx <= lim) & (mx >= -lim) & (my <= lim) & (my >= -lim))


@dataclass
class OracleBins:
    perm: np.ndarray         # int32 [BG]
    tile_counts: np.ndarray  # int32 [T]
    tile_offsets: np.ndarray # int32 [T+1]
    binned_ids: np.ndarray   # int32 [N]

    def sorted_keys(self) -> np.ndarray:
        """64-bit keys (tile << 32) | gid of the sorted pair list."""
        tiles = np.repeat(np.arange(self.tile_counts.size, dtype=np.uint64), self.tile_counts.astype(np.int64))
        return (tiles << np.uint64(32)) | self.binned_ids.astype(np.uint64)


class Scene:
    """Flat float32 inputs in original order: means2d [BG,2], conics [BG,3],
    colors [BG,3], opacities [BG], depths [BG]."""

    def __init__(self, means2d, conics, colors, opacities, depths, B, G):
        self.B, self.G = int(B), int(G)
        n = self.B * self.G
        self.means2d = _f32(means2d, (n, 2))
        self.conics = _f32(conics, (n, 3))
        self.colors = _f32(colors, (n, 3))
        self.opacities = _f32(opacities, (n,))
        self.depths = _f32(depths, (n,))


def depth_order(depths, B, G) -> np.ndarray:
    d = _f32(depths, (B * G,))
    perm = np.empty(B * G, dtype=np.int32)
    lib().oracle_depth_order(_p(d), B, G, _p(perm))
    return perm


def bin_scene(meta: OracleMeta, s: Scene) -> OracleBins:
    L = lib()
    perm = depth_order(s.depths, s.B, s.G)
    tiles = meta.batch * ((meta.width + 15) // 16) * ((meta.height + 15) // 16)
    counts = np.empty(tiles, dtype=np.int32)
    offsets = np.empty(tiles + 1, dtype=np.int32)
    n = L.oracle_bin_count(ctypes.byref(meta), _p(s.means2d), _p(s.conics), _p(s.opacities), _p(perm), _p(counts),
                           _p(offsets))
    ids = np.empty(max(n, 0), dtype=np.int32)
    L.oracle_bin_fill(ctypes.byref(meta), _p(s.means2d), _p(s.conics), _p(s.opacities), _p(perm), _p(offsets),
                      _p(ids))
    return OracleBins(perm, counts, offsets, ids)


AMB_ALPHA, AMB_STOP, AMB_GATE, AMB_FORCED_BAD, AMB_ALPHA_FLIP = 1, 2, 4, 8, 16

# Gradient entries per splat in the bound arrays of render_backward:
# means2d x, y; conics a, b, c; colors r, g, b; opacity.
GRAD_SLICES = {"means2d": slice(0, 2), "conics": slice(2, 5), "colors": slice(5, 8), "opacities": slice(8, 9)}


def threads() -> int:
    """Threads the oracle's parallel loops use (OMP_NUM_THREADS or the core count)."""
    return int(lib().oracle_threads())


def set_threads(n: int) -> None:
    """Thread count of the oracle's parallel loops (results do not depend on it)."""
    lib().oracle_set_threads(int(n))


def _force(meta: OracleMeta, force_last):
    if force_last is None:
        return None
    f = np.ascontiguousarray(force_last, dtype=np.int32)
    assert f.shape == (meta.batch, meta.height, meta.width)
    return f


def render_forward(meta: OracleMeta, s: Scene, bins: OracleBins, with_ambiguity: bool = False, force_last=None):
    """Returns (img, final_T, last, tile_stop[, ambiguity]).  ambiguity[b,y,x] is a
    bit mask: AMB_STOP when an early-stop decision of the pixel lies within
    exp's last-ulp window (another implementation with a 1-ulp exp2 may decide
    it the other way), AMB_GATE likewise for the max_alpha gradient gate.  The
    alpha-threshold decision is exact for the base-2 form the oracle and the
    HIP compositors share (tile_oracle.c: eval_alpha), not for the reference's
    own form min(max_alpha, o exp(power)) >= alpha_threshold
    (gsplat_v8_kernels.metal:121-139): AMB_ALPHA marks pixels where, before
    the pixel stopped, the reference's form was within AMB_ALPHA_ULPS ulps of
    the threshold or decided otherwise, and AMB_ALPHA_FLIP those where it
    decided otherwise.  Such pixels may differ from the reference by up to
    T * alpha_threshold * |colour - background| per flagged evaluation.

    force_last [B,H,W] int32 (-1 = the oracle decides): walk exactly that many
    records of the pixel's tile list (another implementation's stop count);
    AMB_FORCED_BAD marks pixels where that decision lies outside the window."""
    B, H, W = meta.batch, meta.height, meta.width
    img = np.empty((B, H, W, 3), dtype=np.float32)
    T = np.empty((B, H, W), dtype=np.float32)
    last = np.empty((B, H, W), dtype=np.int32)
    stop = np.empty(bins.tile_counts.size, dtype=np.int32)
    amb = np.empty((B, H, W), dtype=np.uint8)
    f = _force(meta, force_last)
    lib().oracle_render_forward(ctypes.byref(meta), _p(s.means2d), _p(s.conics), _p(s.colors), _p(s.opacities),
                                _p(bins.perm), _p(bins.tile_offsets), _p(bins.binned_ids), _p(f), _p(img), _p(T),
                                _p(last), _p(stop), _p(amb))
    if with_ambiguity:
        return img, T, last, stop, amb
    return img, T, last, stop


def render_backward(meta: OracleMeta, s: Scene, bins: OracleBins, grad_img, force_last=None,
                    with_bounds: bool = False):
    """Gradients (original order) (g_means2d [BG,2], g_conics [BG,3], g_colors
    [BG,3], g_opacities [BG]); with_bounds adds a dict of float64 [BG, 9]
    arrays "mag", "chain" and "slack" (tile_oracle.c: oracle_render_backward)
    from which parity.grad_bound forms each entry's rounding allowance."""
    n = s.B * s.G
    g = _f32(grad_img, (meta.batch, meta.height, meta.width, 3))
    gm = np.empty((n, 2), dtype=np.float32)
    gq = np.empty((n, 3), dtype=np.float32)
    gc = np.empty((n, 3), dtype=np.float32)
    go = np.empty((n,), dtype=np.float32)
    bounds = {k: np.empty((n, 9), dtype=np.float64) for k in ("mag", "chain", "slack")} if with_bounds else None
    f = _force(meta, force_last)
    lib().oracle_render_backward(ctypes.byref(meta), _p(s.means2d), _p(s.conics), _p(s.colors), _p(s.opacities),
                                 _p(bins.perm), _p(bins.tile_offsets), _p(bins.binned_ids), _p(f), _p(g), _p(gm),
                                 _p(gq), _p(gc), _p(go), *(_p(bounds[k]) if bounds else None
                                                           for k in ("mag", "chain", "slack")))
    if with_bounds:
        return (gm, gq, gc, go), bounds
    return gm, gq, gc, go


def render_backward_serial(meta: OracleMeta, s: Scene, bins: OracleBins, grad_img):
    """The same gradients accumulated as the reference kernels do (float32
    sums in pixel order, one thread): the restatement render_backward is
    checked against."""
    n = s.B * s.G
    g = _f32(grad_img, (meta.batch, meta.height, meta.width, 3))
    gm = np.zeros((n, 2), dtype=np.float32)
    gq = np.zeros((n, 3), dtype=np.float32)
    gc = np.zeros((n, 3), dtype=np.float32)
    go = np.zeros((n,), dtype=np.float32)
    lib().oracle_render_backward_serial(ctypes.byref(meta), _p(s.means2d), _p(s.conics), _p(s.colors),
                                        _p(s.opacities), _p(bins.perm), _p(bins.tile_offsets), _p(bins.binned_ids),
                                        _p(g), _p(gm), _p(gq), _p(gc), _p(go))
    return gm, gq, gc, go
