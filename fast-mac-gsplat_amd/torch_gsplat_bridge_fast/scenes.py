"""Seeded synthetic scenes for the benchmark/parity configurations.

All tensors are generated in float32 on the CPU with torch.Generator seeds
(image b of a batch uses seed + b) and then moved to the requested device, so
every backend sees identical inputs.

Configs (BASELINE.json ``configs``):
  0  512x512, B=1, G=512, sigma_x,sigma_y ~ U(1,8) px, theta ~ U(0,pi)
  1  1920x1080, B=1, G=65536, sigma ~ U(0.5,6)
  2  4096x4096, B=1, G=65536, sigma ~ U(1,12)            (headline)
  3  1024x512 (W x H), B=4, G=65536 per image, 80% of means from 8 isotropic
     clusters (std 20 px, centres uniform), 20% uniform; depth on 10 planes
     (1..10) + N(0, 0.05); sigma ~ U(1,8)
  4  3D: 4096x4096, B=1, G=2^20, means3d ~ U([-5,5]^3), quats normalize(N(0,I4)),
     scales exp(N(-3,0.5)) with 10% of splats scaled x10, pinhole fx=fy=3500,
     cx=cy=2048, camera at (0,0,-15) with identity rotation
Common: opacity sigmoid(N(0,1)), colors U(0,1), depth U(0.1,10) (configs 0-2).

"log-scales sigma ~ U(1,8)" in the config text is read as sigma ~ U(1,8) px
(a literal log-scale would give sigmas up to e^8 px); conic =
(R diag(sigma^2) R^T)^-1.
"""
from __future__ import annotations

import math
from typing import Dict, Tuple

import torch

CONFIGS: Dict[int, dict] = {
    0: dict(name="cfg0_512sq_512", H=512, W=512, B=1, G=512, sigma=(1.0, 8.0), kind="uniform"),
    1: dict(name="cfg1_1080p_64k", H=1080, W=1920, B=1, G=65536, sigma=(0.5, 6.0), kind="uniform"),
    2: dict(name="cfg2_4096sq_64k", H=4096, W=4096, B=1, G=65536, sigma=(1.0, 12.0), kind="uniform"),
    3: dict(name="cfg3_1024x512_b4_clustered", H=512, W=1024, B=4, G=65536, sigma=(1.0, 8.0), kind="clustered"),
    4: dict(name="cfg4_4096sq_1m_3d", H=4096, W=4096, B=1, G=1 << 20, kind="3d"),
}


def _conics_from_sigmas(sx, sy, theta):
    c, s = torch.cos(theta), torch.sin(theta)
    ix, iy = 1.0 / (sx * sx), 1.0 / (sy * sy)
    a = c * c * ix + s * s * iy
    b = c * s * (ix - iy)
    cc = s * s * ix + c * c * iy
    return torch.stack([a, b, cc], dim=-1)


def _one_image_2d(g: torch.Generator, G: int, H: int, W: int, sigma: Tuple[float, float], kind: str):
    f64 = torch.float64
    if kind == "clustered":
        n_cl = int(round(0.8 * G))
        centers = torch.rand(8, 2, generator=g, dtype=f64) * torch.tensor([W, H], dtype=f64)
        which = torch.randint(0, 8, (n_cl,), generator=g)
        cl = centers[which] + torch.randn(n_cl, 2, generator=g, dtype=f64) * 20.0
        uni = torch.rand(G - n_cl, 2, generator=g, dtype=f64) * torch.tensor([W, H], dtype=f64)
        means = torch.cat([cl, uni], dim=0)
        means = means[torch.randperm(G, generator=g)]
        planes = torch.randint(0, 10, (G,), generator=g).to(f64) + 1.0
        depths = planes + torch.randn(G, generator=g, dtype=f64) * 0.05
    else:
        means = torch.rand(G, 2, generator=g, dtype=f64) * torch.tensor([W, H], dtype=f64)
        depths = 0.1 + torch.rand(G, generator=g, dtype=f64) * 9.9
    lo, hi = sigma
    sig = lo + torch.rand(G, 2, generator=g, dtype=f64) * (hi - lo)
    theta = torch.rand(G, generator=g, dtype=f64) * math.pi
    conics = _conics_from_sigmas(sig[:, 0], sig[:, 1], theta)
    opac = torch.sigmoid(torch.randn(G, generator=g, dtype=f64))
    colors = torch.rand(G, 3, generator=g, dtype=f64)
    return [t.to(torch.float32) for t in (means, conics, colors, opac, depths)]


def make_scene_2d(config_id: int, seed: int = 0, device="cpu", *, G: int | None = None, B: int | None = None,
                  H: int | None = None, W: int | None = None):
    """Returns dict(means2d, conics, colors, opacities, depths [B,G,..], H, W, B, G)."""
    cfg = CONFIGS[config_id]
    if cfg["kind"] == "3d":
        raise ValueError("config 4 is a 3D scene; use make_scene_3d")
    H = cfg["H"] if H is None else H
    W = cfg["W"] if W is None else W
    B = cfg["B"] if B is None else B
    G = cfg["G"] if G is None else G
    parts = []
    for b in range(B):
        g = torch.Generator().manual_seed(seed + b)
        parts.append(_one_image_2d(g, G, H, W, cfg["sigma"], cfg["kind"]))
    names = ("means2d", "conics", "colors", "opacities", "depths")
    out = {n: torch.stack([p[i] for p in parts], dim=0).contiguous().to(device) for i, n in enumerate(names)}
    out.update(H=H, W=W, B=B, G=G)
    return out


def make_scene_3d(seed: int = 0, device="cpu", *, G: int | None = None, H: int = 4096, W: int = 4096,
                  adversarial_fraction: float = 0.1, adversarial_scale: float = 10.0):
    """Config 4 (B=1).  Returns dict(means3d, scales, quats, opacities, colors [1,G,..], fx, fy, cx, cy,
    camera_to_world [4,4], H, W, B, G)."""
    G = CONFIGS[4]["G"] if G is None else G
    g = torch.Generator().manual_seed(seed)
    f64 = torch.float64
    means3d = (torch.rand(G, 3, generator=g, dtype=f64) * 10.0 - 5.0)
    q = torch.randn(G, 4, generator=g, dtype=f64)
    quats = q / q.norm(dim=-1, keepdim=True)
    scales = torch.exp(-3.0 + 0.5 * torch.randn(G, 3, generator=g, dtype=f64))
    n_adv = int(round(adversarial_fraction * G))
    adv = torch.randperm(G, generator=g)[:n_adv]
    scales[adv] *= adversarial_scale
    opac = torch.sigmoid(torch.randn(G, generator=g, dtype=f64))
    colors = torch.rand(G, 3, generator=g, dtype=f64)
    c2w = torch.eye(4, dtype=torch.float32)
    c2w[2, 3] = -15.0
    out = {k: v.to(torch.float32).unsqueeze(0).contiguous().to(device) for k, v in
           dict(means3d=means3d, scales=scales, quats=quats, opacities=opac, colors=colors).items()}
    out.update(fx=3500.0, fy=3500.0, cx=W / 2.0, cy=H / 2.0, camera_to_world=c2w.to(device), H=H, W=W, B=1, G=G)
    return out


TRACE_KEYS = ("means2d", "conics", "colors", "opacities", "depths")


def load_trace(path: str, device="cpu", *, batch: int = 0, gaussians: int = 0) -> Dict[str, torch.Tensor]:
    """Loads a recorded scene: a ``torch.save`` dict with means2d, conics, colors, opacities and depths,
    shaped [G,...] or [B,G,...] (the format of the reference's real-trace benchmark case,
    variants/v8/benchmarks/benchmark_mps.py:26-47).  The tensors are converted to float32 on
    ``device``; [G,...] inputs become B=1; ``batch`` / ``gaussians`` > 0 keep only the first that many
    images / splats.  The file is read with ``weights_only=True``: nothing in it is executed."""
    if not path:
        raise ValueError("a trace file is required for the real-trace case")
    data = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(data, dict):
        raise ValueError("trace file must hold a dict of tensors")
    out = {}
    for key in TRACE_KEYS:
        if key not in data:
            raise ValueError(f"trace file is missing {key!r}")
        out[key] = torch.as_tensor(data[key]).to(dtype=torch.float32)
    if out["means2d"].ndim == 2:
        out = {k: v.unsqueeze(0) for k, v in out.items()}
    B0, G0 = out["means2d"].shape[:2]
    B = min(B0, batch) if batch > 0 else B0
    G = min(G0, gaussians) if gaussians > 0 else G0
    return {k: v[:B, :G].contiguous().to(device) for k, v in out.items()}
