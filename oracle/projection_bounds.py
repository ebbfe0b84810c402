"""TEST INFRASTRUCTURE ONLY -- the pinhole projection and its vector-Jacobian
product evaluated in float64 with a first-order running error bound.

Each quantity is a pair (value, err): value is computed in float64, err
bounds the deviation of a float32 evaluation of the same sequence of
operations (unit roundoff u = 2^-24 per rounded operation, correctly
rounded division and square root) from value, to first order
(Wilkinson's running error analysis):

    a + b:  err_a + err_b + u |a + b|
    a * b:  |a| err_b + |b| err_a + u |a b|
    a / b:  (err_a + |a / b| err_b) / |b| + u |a / b|

Inputs carry err = 0 (they are float32 values given exactly) unless an
input error is supplied (e.g. the rounding allowance of gradients that come
from the compositor).  The operation sequence follows the reference's
projection (variants/v9_project3d_train/csrc/metal/
gsplat_v9_project3d_train_kernels.metal:66-174 forward, :217-501 backward)
written in the matrix form of the VJP, so err bounds a float32
implementation that evaluates these expressions in this order.  The values
are pinned against float64 autograd through oracle/dense_reference.py's
project_pinhole_reference (tests/test_oracle_bounds_cpu.py).

Used by tests/ only.
"""
from __future__ import annotations

import numpy as np

U = 2.0 ** -24


class RE:
    """A float64 value with a first-order bound on float32 rounding error."""

    __slots__ = ("v", "e")

    def __init__(self, v, e=None):
        self.v = np.asarray(v, dtype=np.float64)
        self.e = np.zeros_like(self.v) if e is None else np.asarray(e, dtype=np.float64)

    @staticmethod
    def _c(x):
        return x if isinstance(x, RE) else RE(x)

    def __add__(self, o):
        o = RE._c(o)
        v = self.v + o.v
        return RE(v, self.e + o.e + U * np.abs(v))

    __radd__ = __add__

    def __sub__(self, o):
        o = RE._c(o)
        v = self.v - o.v
        return RE(v, self.e + o.e + U * np.abs(v))

    def __rsub__(self, o):
        return RE._c(o) - self

    def __neg__(self):
        return RE(-self.v, self.e)

    def __mul__(self, o):
        if not isinstance(o, RE) and np.all(np.isin(np.abs(np.asarray(o, dtype=np.float64)), (0.5, 1.0, 2.0, 4.0))):
            # exact scaling by a power of two
            return RE(self.v * o, self.e * np.abs(o))
        o = RE._c(o)
        v = self.v * o.v
        return RE(v, np.abs(self.v) * o.e + np.abs(o.v) * self.e + U * np.abs(v))

    __rmul__ = __mul__

    def __truediv__(self, o):
        o = RE._c(o)
        v = self.v / o.v
        return RE(v, (self.e + np.abs(v) * o.e) / np.abs(o.v) + U * np.abs(v))

    def __rtruediv__(self, o):
        return RE._c(o) / self


def where(mask, a, b):
    a, b = RE._c(a), RE._c(b)
    return RE(np.where(mask, a.v, b.v), np.where(mask, a.e, b.e))


def maximum(a, floor):
    """max(a, floor) with a constant floor (exact)."""
    return RE(np.maximum(a.v, floor), np.where(a.v > floor, a.e, 0.0))


def _dot3(a, b):
    return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]


def quat_to_rot(r, i, j, k):
    return [[1.0 - 2.0 * (j * j + k * k), 2.0 * (i * j - r * k), 2.0 * (i * k + r * j)],
            [2.0 * (i * j + r * k), 1.0 - 2.0 * (i * i + k * k), 2.0 * (j * k - r * i)],
            [2.0 * (i * k - r * j), 2.0 * (j * k + r * i), 1.0 - 2.0 * (i * i + j * j)]]


def _split(x, n):
    x = np.asarray(x, dtype=np.float64)
    return [RE(x[..., c]) for c in range(n)]


def _state(means3d, scales, quats, c2w, cam, near):
    """Forward quantities per splat.  means3d [N,3], scales [N,3], quats [N,4]
    (r,i,j,k), c2w [N,4,4] and cam [N,4] (each splat's camera)."""
    S = {}
    r, i, j, k = _split(quats, 4)
    R = quat_to_rot(r, i, j, k)
    s = _split(scales, 3)
    M = [[R[a][c] * s[c] for c in range(3)] for a in range(3)]
    Sig = [[_dot3(M[a], M[b]) for b in range(3)] for a in range(3)]
    c2w = np.asarray(c2w, dtype=np.float64)
    W = [[RE(c2w[:, a, c]) for c in range(3)] for a in range(3)]
    t = [RE(c2w[:, a, 3]) for a in range(3)]
    x = _split(means3d, 3)
    d = [x[a] - t[a] for a in range(3)]
    xc = [d[0] * W[0][q] + d[1] * W[1][q] + d[2] * W[2][q] for q in range(3)]
    SW = [[Sig[a][0] * W[0][q] + Sig[a][1] * W[1][q] + Sig[a][2] * W[2][q] for q in range(3)] for a in range(3)]
    Sc = [[W[0][p] * SW[0][q] + W[1][p] * SW[1][q] + W[2][p] * SW[2][q] for q in range(3)] for p in range(3)]
    z = xc[2]
    front = z.v > near
    amb = np.abs(z.v - near) <= 2 * z.e
    zs = where(front, maximum(z, near), 1.0)
    xp = where(front, xc[0], 0.0)
    yp = where(front, xc[1], 0.0)
    fx, fy, cx, cy = _split(cam, 4)
    iz = 1.0 / zs
    J = [[fx * iz, RE(np.zeros_like(iz.v)), -(fx * xp) * iz * iz],
         [RE(np.zeros_like(iz.v)), fy * iz, -(fy * yp) * iz * iz]]
    JS = [[J[r_][0] * Sc[0][c] + J[r_][1] * Sc[1][c] + J[r_][2] * Sc[2][c] for c in range(3)] for r_ in range(2)]
    cov00 = _dot3(JS[0], J[0]) + 0.3
    cov01 = _dot3(JS[0], J[1])
    cov11 = _dot3(JS[1], J[1]) + 0.3
    det_raw = cov00 * cov11 - cov01 * cov01
    det = maximum(det_raw, 1e-6)
    amb |= np.abs(det_raw.v - 1e-6) <= 2 * det_raw.e
    S.update(R=R, s=s, M=M, Sig=Sig, W=W, d=d, xc=xc, Sc=Sc, front=front, zs=zs, xp=xp, yp=yp, J=J,
             cov00=cov00, cov01=cov01, cov11=cov11, det_raw=det_raw, det=det, fx=fx, fy=fy, cx=cx, cy=cy,
             quat=(r, i, j, k), ambiguous=amb)
    return S


def _per_splat_camera(c2w, cam, B, G):
    c2w = np.asarray(c2w, dtype=np.float64).reshape(B, 4, 4)
    cam = np.asarray(cam, dtype=np.float64).reshape(B, 4)
    return np.repeat(c2w, G, axis=0), np.repeat(cam, G, axis=0)


def project_forward(means3d, scales, quats, opacities, c2w, cam, near=1e-4):
    """Batched [B,G,..] inputs -> dict of RE outputs ([B*G,..] flattened):
    means2d (2), conics (3), opacities, depths; plus 'ambiguous' [B*G] (a
    near-plane or det-clamp decision within rounding)."""
    m = np.asarray(means3d, dtype=np.float64)
    B, G = m.shape[:2]
    c2w_n, cam_n = _per_splat_camera(c2w, cam, B, G)
    S = _state(m.reshape(-1, 3), np.asarray(scales).reshape(-1, 3), np.asarray(quats).reshape(-1, 4), c2w_n, cam_n,
               near)
    means2d = [(S["fx"] * S["xp"]) / S["zs"] + S["cx"], (S["fy"] * S["yp"]) / S["zs"] + S["cy"]]
    conics = [S["cov11"] / S["det"], -S["cov01"] / S["det"], S["cov00"] / S["det"]]
    op = np.asarray(opacities, dtype=np.float64).reshape(-1)
    return {"means2d": means2d, "conics": conics, "opacities": RE(np.where(S["front"], op, 0.0)),
            "depths": S["xc"][2], "ambiguous": S["ambiguous"]}


def project_vjp(means3d, scales, quats, opacities, c2w, cam, g_means2d, g_conics, g_opac, g_depths, near=1e-4,
                g_err=None):
    """VJP of the projection for cotangents [B,G,2], [B,G,3], [B,G], [B,G]
    (g_err: optional dict of the same shapes bounding the cotangents'
    errors).  Returns a dict of RE: means3d [N][3], scales [N][3], quats
    [N][4], opacities [N], camera_to_world [B][16] (rows 0-2 of the 4x4,
    row-major, then the zero last row) and camera_params [B][4], plus
    'ambiguous'."""
    m = np.asarray(means3d, dtype=np.float64)
    B, G = m.shape[:2]
    N = B * G
    c2w_n, cam_n = _per_splat_camera(c2w, cam, B, G)
    S = _state(m.reshape(-1, 3), np.asarray(scales).reshape(-1, 3), np.asarray(quats).reshape(-1, 4), c2w_n, cam_n,
               near)
    ge = g_err or {}

    def cot(x, name, n):
        v = np.asarray(x, dtype=np.float64).reshape(N, n)
        e = np.asarray(ge[name], dtype=np.float64).reshape(N, n) if name in ge else np.zeros_like(v)
        return [RE(v[:, c], e[:, c]) for c in range(n)]

    gq0, gq1, gq2 = cot(g_conics, "conics", 3)
    gmx, gmy = cot(g_means2d, "means2d", 2)
    (gop,) = cot(g_opac, "opacities", 1)
    (gdp,) = cot(g_depths, "depths", 1)
    cov00, cov01, cov11, det = S["cov00"], S["cov01"], S["cov11"], S["det"]
    idet = 1.0 / det
    g00 = gq2 * idet
    g11 = gq0 * idet
    g01 = -gq1 * idet
    gdet = -(gq0 * cov11 - gq1 * cov01 + gq2 * cov00) * idet * idet
    live = S["det_raw"].v > 1e-6
    g00 = where(live, g00 + gdet * cov11, g00)
    g11 = where(live, g11 + gdet * cov00, g11)
    g01 = where(live, g01 + gdet * (-2.0 * cov01), g01)
    Gm = [[g00, 0.5 * g01], [0.5 * g01, g11]]
    J, Sc = S["J"], S["Sc"]
    GJ = [[Gm[r][0] * J[0][c] + Gm[r][1] * J[1][c] for c in range(3)] for r in range(2)]
    dSc = [[J[0][p] * GJ[0][q] + J[1][p] * GJ[1][q] for q in range(3)] for p in range(3)]
    dJ = [[2.0 * (GJ[r][0] * Sc[0][c] + GJ[r][1] * Sc[1][c] + GJ[r][2] * Sc[2][c]) for c in range(3)]
          for r in range(2)]
    fx, fy = S["fx"], S["fy"]
    x, y, z = S["xc"]
    front = S["front"]
    zsafe = where(front, z, 1.0)
    iz = 1.0 / zsafe
    iz2 = iz * iz
    iz3 = iz2 * iz
    zero = RE(np.zeros(N))
    g_fx_f = gmx * x * iz + (dJ[0][0] * iz - dJ[0][2] * x * iz2)
    g_fy_f = gmy * y * iz + (dJ[1][1] * iz - dJ[1][2] * y * iz2)
    gxc0_f = gmx * fx * iz - dJ[0][2] * fx * iz2
    gxc1_f = gmy * fy * iz - dJ[1][2] * fy * iz2
    gxc2_f = (gdp - gmx * fx * x * iz2 - gmy * fy * y * iz2
              + (-dJ[0][0] * fx * iz2 + 2.0 * dJ[0][2] * fx * x * iz3 - dJ[1][1] * fy * iz2
                 + 2.0 * dJ[1][2] * fy * y * iz3))
    g_fx = where(front, g_fx_f, dJ[0][0])
    g_fy = where(front, g_fy_f, dJ[1][1])
    gxc = [where(front, gxc0_f, zero), where(front, gxc1_f, zero), where(front, gxc2_f, gdp)]
    W, d, Sig, M, R, s = S["W"], S["d"], S["Sig"], S["M"], S["R"], S["s"]
    gmean = [W[a][0] * gxc[0] + W[a][1] * gxc[1] + W[a][2] * gxc[2] for a in range(3)]
    gW = [[d[a] * gxc[j] for j in range(3)] for a in range(3)]
    WdS = [[W[a][0] * dSc[0][q] + W[a][1] * dSc[1][q] + W[a][2] * dSc[2][q] for q in range(3)] for a in range(3)]
    dSig = [[WdS[a][0] * W[b][0] + WdS[a][1] * W[b][1] + WdS[a][2] * W[b][2] for b in range(3)] for a in range(3)]
    gW = [[gW[a][q] + 2.0 * (Sig[a][0] * WdS[0][q] + Sig[a][1] * WdS[1][q] + Sig[a][2] * WdS[2][q])
           for q in range(3)] for a in range(3)]
    dM = [[2.0 * (dSig[a][0] * M[0][c] + dSig[a][1] * M[1][c] + dSig[a][2] * M[2][c]) for c in range(3)]
          for a in range(3)]
    gs = [dM[0][c] * R[0][c] + dM[1][c] * R[1][c] + dM[2][c] * R[2][c] for c in range(3)]
    dR = [[dM[a][c] * s[c] for c in range(3)] for a in range(3)]
    qr, qi, qj, qk = S["quat"]
    gqr = 2.0 * (-qk * dR[0][1] + qj * dR[0][2] + qk * dR[1][0] - qi * dR[1][2] - qj * dR[2][0] + qi * dR[2][1])
    gqi = (2.0 * (qj * dR[0][1] + qk * dR[0][2] + qj * dR[1][0] - qr * dR[1][2] + qk * dR[2][0] + qr * dR[2][1])
           - 4.0 * qi * (dR[1][1] + dR[2][2]))
    gqj = (2.0 * (qi * dR[0][1] + qr * dR[0][2] + qi * dR[1][0] + qk * dR[1][2] - qr * dR[2][0] + qk * dR[2][1])
           - 4.0 * qj * (dR[0][0] + dR[2][2]))
    gqk = (2.0 * (-qr * dR[0][1] + qi * dR[0][2] + qr * dR[1][0] + qj * dR[1][2] + qi * dR[2][0] + qj * dR[2][1])
           - 4.0 * qk * (dR[0][0] + dR[1][1]))
    g_opac_in = where(front, gop, zero)
    # camera: per-splat values summed per image (float32 tree / sequential
    # sums of at most G terms: log2(G) + 8 roundings of the magnitude sum)
    per = [gW[a][j] for a in range(3) for j in range(3)] + [-gmean[a] for a in range(3)] + \
          [g_fx, g_fy, gmx, gmy]
    levels = float(np.ceil(np.log2(max(G, 2)))) + 8.0
    cam_sums = []
    for v in per:
        vv, ee = v.v.reshape(B, G), v.e.reshape(B, G)
        cam_sums.append(RE(vv.sum(axis=1), ee.sum(axis=1) + levels * U * np.abs(vv).sum(axis=1)))
    c2w_g = [cam_sums[3 * r + c] if c < 3 else cam_sums[9 + r] for r in range(3) for c in range(4)]
    c2w_g += [RE(np.zeros(B))] * 4
    return {"means3d": gmean, "scales": gs, "quats": [gqr, gqi, gqj, gqk], "opacities": g_opac_in,
            "camera_to_world": c2w_g, "camera_params": cam_sums[12:16], "ambiguous": S["ambiguous"]}


def stack(parts):
    """[RE, ...] per component -> (values [N, k], errs [N, k])."""
    if isinstance(parts, RE):
        return parts.v[:, None], parts.e[:, None]
    return np.stack([p.v for p in parts], axis=1), np.stack([p.e for p in parts], axis=1)


def assert_close(got, ref_parts, name, rtol=1e-3, atol=1e-5, k_err=2.0):
    """|got - ref| <= atol + rtol |ref| + k_err err for every entry (the
    gradient bar plus twice the first-order float32 rounding bound)."""
    v, e = stack(ref_parts)
    g = np.asarray(got, dtype=np.float64).reshape(v.shape)
    allow = atol + rtol * np.abs(v) + k_err * e
    bad = np.abs(g - v) > allow
    if bad.any():
        i, j = np.argwhere(bad)[0]
        raise AssertionError(f"{name}: {int(bad.sum())} of {bad.size} entries beyond the bar; first [{i},{j}] "
                             f"got {g[i, j]:.9g} ref {v[i, j]:.9g} allowance {allow[i, j]:.3g} (err {e[i, j]:.3g})")
    return float((np.abs(g - v) / allow).max())
