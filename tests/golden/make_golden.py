"""Writes the golden fixtures in this directory.

  reference_hand_cases.json     input values of the reference's hand-written
                                16x16 case, variants/v8/tests/reference_check.py:
                                118-144 (means, conics, opacities, depths;
                                the reference draws colors on its GPU, so the
                                tests redraw them on the CPU with seed 0)
  reference_saturated_case.json the reference's saturated 32x32 / 64-splat case
                                (reference_check.py:180-206), drawn from the same
                                distributions with a CPU generator, seed 123
  config0_oracle.npz            config 0 (seed 0) through the CPU oracle: tile
                                counts, sorted pair ids, a 64x64 image crop,
                                final-T crop, and the four gradients for
                                loss = sum(img * w), w ~ U(0,1) seed 123
  projection_cases.json         three hand-picked 3D splats (one behind the
                                near plane) and their float64 projection

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "fast-mac-gsplat_amd"))

from oracle import tile_oracle as TO  # noqa: E402
from oracle.dense_reference import project_pinhole_reference  # noqa: E402
from torch_gsplat_bridge_fast.scenes import make_scene_2d  # noqa: E402


def hand_cases():
    return {
        "means2d": [[[4.2, 5.1], [8.0, 7.5], [11.2, 8.1], [6.4, 12.0]],
                    [[3.7, 4.4], [7.1, 10.2], [12.2, 3.4], [10.4, 12.5]]],
        "conics": [[[0.35, 0.02, 0.42], [0.28, -0.01, 0.33], [0.25, 0.04, 0.31], [0.40, 0.00, 0.27]],
                   [[0.31, 0.03, 0.38], [0.45, 0.01, 0.29], [0.22, -0.02, 0.35], [0.27, 0.05, 0.41]]],
        "opacities": [[0.8, 0.6, 0.5, 0.7], [0.65, 0.55, 0.75, 0.45]],
        "depths": [[0.1, 0.2, 0.3, 0.4], [0.3, 0.1, 0.4, 0.2]],
    }


def saturated_case():
    g = torch.Generator().manual_seed(123)
    B, G, H, W = 1, 64, 32, 32
    means = torch.randn(B, G, 2, generator=g) * torch.tensor([W * 0.2, H * 0.2]) + torch.tensor([W * 0.5, H * 0.5])
    means[..., 0].clamp_(0, W - 1)
    means[..., 1].clamp_(0, H - 1)
    sig = torch.rand(B, G, 2, generator=g) * 8.0 + 3.0
    conics = torch.stack([1.0 / sig[..., 0].square(), torch.zeros(B, G), 1.0 / sig[..., 1].square()], dim=-1)
    colors = torch.rand(B, G, 3, generator=g)
    opac = torch.rand(B, G, generator=g) * 0.45 + 0.45
    depths = (torch.arange(G, dtype=torch.float32) / float(G - 1)).view(1, G)
    return {k: v.tolist() for k, v in dict(means2d=means, conics=conics, colors=colors, opacities=opac,
                                            depths=depths).items()}


def config0():
    sc = make_scene_2d(0, seed=0)
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    keys = ("means2d", "conics", "colors", "opacities", "depths")
    meta = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(sc[k].numpy() for k in keys), B, G)
    bins = TO.bin_scene(meta, s)
    img, T, last, stop = TO.render_forward(meta, s, bins)
    w = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(123)).numpy()
    gm, gq, gc, go = TO.render_backward(meta, s, bins, w[None])
    return dict(perm=bins.perm, tile_counts=bins.tile_counts, binned_ids=bins.binned_ids,
                img_crop=img[0, 200:264, 300:364], T_crop=T[0, 200:264, 300:364], tile_stop=stop,
                g_means2d=gm, g_conics=gq, g_colors=gc, g_opacities=go)


def projection_cases():
    means3d = torch.tensor([[[0.3, -0.2, 2.0], [1.0, 0.5, 6.0], [0.0, 0.0, -1.0]]], dtype=torch.float64)
    scales = torch.tensor([[[0.1, 0.2, 0.05], [0.3, 0.3, 0.3], [0.2, 0.1, 0.1]]], dtype=torch.float64)
    quats = torch.tensor([[[0.9, 0.1, -0.3, 0.2], [1.0, 0.0, 0.0, 0.0], [0.5, 0.5, 0.5, 0.5]]], dtype=torch.float64)
    opac = torch.tensor([[0.7, 0.4, 0.9]], dtype=torch.float64)
    c2w = torch.eye(4, dtype=torch.float64).unsqueeze(0)
    c2w[0, :3, 3] = torch.tensor([0.1, -0.05, -0.5], dtype=torch.float64)
    cam = torch.tensor([[500.0, 480.0, 320.0, 240.0]], dtype=torch.float64)
    m2, cq, op, dp = project_pinhole_reference(means3d, scales, quats, opac, c2w, cam, 1e-4)
    inputs = dict(means3d=means3d, scales=scales, quats=quats, opacities=opac, camera_to_world=c2w,
                  camera_params=cam)
    outputs = dict(means2d=m2, conics=cq, opacities_out=op, depths=dp)
    return {"inputs": {k: v.tolist() for k, v in inputs.items()},
            "outputs": {k: v.tolist() for k, v in outputs.items()}, "near_plane": 1e-4}


def main():
    with open(os.path.join(HERE, "reference_hand_cases.json"), "w") as f:
        json.dump(hand_cases(), f, indent=1)
    with open(os.path.join(HERE, "reference_saturated_case.json"), "w") as f:
        json.dump(saturated_case(), f)
    np.savez_compressed(os.path.join(HERE, "config0_oracle.npz"), **config0())
    with open(os.path.join(HERE, "projection_cases.json"), "w") as f:
        json.dump(projection_cases(), f, indent=1)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
