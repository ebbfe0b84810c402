"""CPU check that the compositors' strip culling is conservative.

A host build of gs::strip_mask_t (fast-mac-gsplat_amd/csrc/gs_strip.h, the
same source the compositors compile) is compared with brute force over the
64 pixels of each strip: every strip holding a pixel where the splat passes
the alpha test (the compositors' exact exponent chain, e <= 0 and
p >= plim + lo, plim and lo from the oracle) must keep its bit.  The masks are taken with the
reciprocal and square root rounded 2 ulp down, to nearest and 2 ulp up (the
hardware operations are within 1 ulp), in builds with and without FP
contraction, on random splats around a tile: sizes from 0.3 to 40 px, any
orientation, opacities from the threshold to 1, and conics near and past the
culling limit det = 1e-3 a c.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from oracle import tile_oracle as TO

HERE = os.path.dirname(os.path.abspath(__file__))
THR = 1.0 / 255.0


@pytest.fixture(scope="module", params=["-ffp-contract=off", "-ffp-contract=fast"])
def helper(request, tmp_path_factory):
    out = tmp_path_factory.mktemp("strip") / "libstripcheck.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-mfma", request.param,
                    os.path.join(HERE, "strip_mask_check.cpp"), "-o", str(out)], check=True)
    lib = ctypes.CDLL(str(out))
    lib.strip_mask_check.restype = ctypes.c_int
    lib.strip_mask_check.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] + [ctypes.c_void_p] * 2
    return lib


def _splats(rng, n, degenerate=False):
    sx = np.exp(rng.uniform(np.log(0.3), np.log(40.0), n))
    sy = np.exp(rng.uniform(np.log(0.3), np.log(40.0), n))
    th = rng.uniform(0, np.pi, n)
    c, s = np.cos(th), np.sin(th)
    ix, iy = 1 / sx ** 2, 1 / sy ** 2
    a = c * c * ix + s * s * iy
    b = c * s * (ix - iy)
    cc = s * s * ix + c * c * iy
    if degenerate:
        # |b| close to the culling limit: det = a c - b^2 within a factor of 3 of 1e-3 a c
        ratio = np.exp(rng.uniform(np.log(3e-4), np.log(3e-3), n))
        b = np.sign(rng.uniform(-1, 1, n)) * np.sqrt(a * cc * (1 - ratio))
    o = np.exp(rng.uniform(np.log(THR), 0.0, n))
    reach = 3.5 * np.maximum(sx, sy)
    m = rng.uniform(-reach, 16 + reach, (2, n)).T
    out = np.zeros((n, 6), np.float32)
    out[:, 0], out[:, 1], out[:, 2], out[:, 3], out[:, 4] = m[:, 0], m[:, 1], a, b, cc
    return out, o.astype(np.float32)


@pytest.mark.parametrize("degenerate", [False, True])
def test_strip_mask_keeps_every_visible_strip(helper, degenerate):
    rng = np.random.default_rng(17 + degenerate)
    n = 40_000
    sp, o = _splats(rng, n, degenerate)
    tiles = rng.integers(-2, 3, size=(n, 2)).astype(np.int32) * 16   # tile origins around the splats' frame
    # half of the sample far from the origin (up to 2^13 px), where the centre's rounding is coarser
    far = (rng.integers(0, 2, size=(n, 1)) * rng.integers(0, 512, size=(n, 2)) * 16).astype(np.int32)
    tiles += far
    sp[:, 0] = (sp[:, 0] + tiles[:, 0]).astype(np.float32)
    sp[:, 1] = (sp[:, 1] + tiles[:, 1]).astype(np.float32)
    plims = np.array([TO.plim(float(v), THR, 0.99) for v in o], np.float32)
    sp[:, 5] = [TO.opacity_log2(float(v)) for v in o]
    masks = np.zeros((n, 3), np.uint32)
    needed = np.zeros(n, np.uint32)
    helper.strip_mask_check(sp.ctypes.data, plims.ctypes.data, tiles.ctypes.data, n, masks.ctypes.data,
                            needed.ctypes.data)
    for v in range(3):
        missed = needed & ~masks[:, v] & 0xF
        assert not missed.any(), (v, np.nonzero(missed)[0][:5])
    visible = needed != 0
    assert visible.mean() > 0.2                      # the sample exercises visible splats
    kept = np.unpackbits(masks[:, 1].astype(np.uint8)[:, None], axis=1)[:, 4:].sum()
    need = np.unpackbits(needed.astype(np.uint8)[:, None], axis=1)[:, 4:].sum()
    print(f"degenerate={degenerate}: strips needed {need}, kept {kept} ({kept / max(need, 1) - 1:.1%} extra)")
    if not degenerate:
        assert kept <= 1.2 * need                    # the culling is not vacuous
