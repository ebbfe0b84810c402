"""GPU parity of the reference's operator namespace, torch.ops.gsplat_metal_v8.* (v8_ops.py).

The operators are composed here in the order of the reference's autograd Function and eval path
(variants/v8/torch_gsplat_bridge_v8/rasterize.py:465-680 and :684-786, restated in this file, not
imported): stable depth sort and flattening; bin; the fast (or active-tile) state forward; the
overflow forward for the tiles above max_fast_pairs, scattered into a clone of the fast image;
then the fast (or active) backward plus the overflow backward on the gathered gradient tiles,
summed and unsorted.  With B = 2 and max_fast_pairs = 64 a clustered scene has overflow tiles
(some above 128 pairs, the HIP forward's hand-off length) next to ordinary ones.  Checked:
tile counts, offsets and ids bit-exact against the oracle; the fast stop counts (the oracle's,
and 0 above max_fast_pairs); image and every splat's gradients against the oracle at the parity
bar (oracle/parity.py); the eval composition equal to the training one; the state forward's
in-place sort of binned ids that arrive shuffled inside their tiles.
"""
import numpy as np
import pytest
import torch

from oracle import tile_oracle as TO
from test_gpu_raster import gpu_state, oracle_parity
from torch_gsplat_bridge_fast.scenes import make_scene_2d

pytestmark = pytest.mark.gpu

KEYS = ("means2d", "conics", "colors", "opacities", "depths")
OPS = torch.ops.gsplat_metal_v8


def _v8_meta(H, W, B, G, max_fast_pairs, bg):
    """The reference's meta tensors (v8 rasterize.py:129-173 layout): device and host copies."""
    ty, tx = (H + 15) // 16, (W + 15) // 16
    i32 = torch.tensor([H, W, ty, tx, 16, B * G, B * ty * tx, max_fast_pairs, B, G, ty * tx, 0, 64, 0],
                       dtype=torch.int32)
    f32 = torch.tensor([1.0 / 255.0, 1e-4, bg[0], bg[1], bg[2], 1e-8, 0.99], dtype=torch.float32)
    return i32.cuda(), f32.cuda(), i32, f32


def _sorted_flat(sc, B, G):
    """Stable depth order per image and the depth-sorted flat attributes (the reference's gathers)."""
    dev = torch.device("cuda:0")
    d = sc["depths"].to(dev)
    perm = torch.argsort(d, dim=1, stable=True)
    flat = []
    for k, w in (("means2d", 2), ("conics", 3), ("colors", 3), ("opacities", 0)):
        x = sc[k].to(dev)
        g = torch.gather(x, 1, perm[..., None].expand(-1, -1, w)) if w else torch.gather(x, 1, perm)
        flat.append(g.reshape(B * G, w).contiguous() if w else g.reshape(B * G).contiguous())
    return perm, flat


def _overflow_lists(counts, offsets, ids, mfp):
    """Tiles above max_fast_pairs, their offsets into the concatenated lists and each list's ids in
    ascending order (what the reference's Python hands to the overflow operators)."""
    tiles = torch.nonzero(counts > mfp).flatten()
    segs, lens = [], []
    for t in tiles.tolist():
        s, e = int(offsets[t]), int(offsets[t + 1])
        segs.append(torch.sort(ids[s:e]).values)
        lens.append(e - s)
    dev = counts.device
    seg_off = torch.zeros(len(lens) + 1, dtype=torch.int32, device=dev)
    if lens:
        seg_off[1:] = torch.cumsum(torch.tensor(lens, device=dev), 0)
    seg_ids = torch.cat(segs) if segs else torch.empty(0, dtype=torch.int32, device=dev)
    return tiles.to(torch.int32), seg_off, seg_ids.to(torch.int32).contiguous()


def _tile_slices(t, tpi, tiles_x, H, W):
    b, lt = divmod(int(t), tpi)
    y0, x0 = (lt // tiles_x) * 16, (lt % tiles_x) * 16
    return b, y0, min(y0 + 16, H), x0, min(x0 + 16, W)


def _forward(flat, metas, mfp, H, W, *, active, train, shuffle=False):
    counts, offsets, ids = OPS.bin(*flat, *metas)
    act = None
    if active:
        act = torch.nonzero((counts > 0) & (counts <= mfp)).flatten().to(torch.int32)
        act = act[torch.argsort(counts[act.long()], stable=True)]        # sorted by count
    if shuffle:
        # ids inside each tile in a scrambled order, as the reference's atomic cursors leave them
        g = torch.Generator(device="cuda").manual_seed(3)
        key = torch.repeat_interleave(torch.arange(counts.numel(), device=ids.device), counts.long()) * 2.0 \
            + torch.rand(ids.numel(), generator=g, device=ids.device)
        ids = ids[torch.argsort(key)].contiguous()
    stop = None
    if train:
        if active:
            out_fast, stop = OPS.render_active_forward_state(*flat, *metas, ids, act, counts, offsets)
        else:
            out_fast, stop = OPS.render_fast_forward_state(*flat, *metas, ids, counts, offsets)
    else:
        if active:
            out_fast = OPS.render_active_forward_eval(*flat, *metas, act, counts, offsets, ids)
        else:
            out_fast = OPS.render_fast_forward_eval(*flat, *metas, counts, offsets, ids)
    ov = _overflow_lists(counts, offsets, ids, mfp)
    out = out_fast
    if ov[0].numel():
        tiles_img = OPS.render_overflow_forward(*flat, *metas, *ov)
        out = out_fast.clone()
        ty, tx = (H + 15) // 16, (W + 15) // 16
        for i, t in enumerate(ov[0].tolist()):
            b, y0, y1, x0, x1 = _tile_slices(t, ty * tx, tx, H, W)
            out[b, y0:y1, x0:x1] = tiles_img[i, :y1 - y0, :x1 - x0]
    return out, stop, (counts, offsets, ids, act, ov)


def _backward(grad, flat, metas, perm, saved, stop, H, W, B, G, *, active):
    counts, offsets, ids, act, ov = saved
    if active:
        g = OPS.render_active_backward_saved(grad, *flat, *metas, act, counts, offsets, ids, stop)
    else:
        g = OPS.render_fast_backward_saved(grad, *flat, *metas, counts, offsets, ids, stop)
    g = list(g)
    if ov[0].numel():
        ty, tx = (H + 15) // 16, (W + 15) // 16
        gt = torch.zeros((ov[0].numel(), 16, 16, 3), dtype=torch.float32, device=grad.device)
        for i, t in enumerate(ov[0].tolist()):
            b, y0, y1, x0, x1 = _tile_slices(t, ty * tx, tx, H, W)
            gt[i, :y1 - y0, :x1 - x0] = grad[b, y0:y1, x0:x1]
        go = OPS.render_overflow_backward(gt, *flat, *metas, *ov)
        g = [a + b for a, b in zip(g, go)]
    out = []
    for t, w in zip(g, (2, 3, 3, 0)):
        t = t.reshape(B, G, w) if w else t.reshape(B, G)
        u = torch.empty_like(t)
        u.scatter_(1, perm[..., None].expand_as(t) if w else perm, t)
        out.append(u.cpu().numpy())
    return out


@pytest.mark.parametrize("active", [False, True])
def test_reference_ops_compose_like_the_reference(gpu, active):
    B, G, H, W, mfp = 2, 3000, 144, 200, 64
    bg = (0.1, 0.2, 0.3)
    sc = make_scene_2d(3, seed=7, G=G, B=B, H=H, W=W)
    print(f"gsplat_metal_v8 ops, active={active}: {W}x{H} B={B} G={G} max_fast_pairs={mfp}", flush=True)
    metas = _v8_meta(H, W, B, G, mfp, bg)
    perm, flat = _sorted_flat(sc, B, G)
    img, stop, saved = _forward(flat, metas, mfp, H, W, active=active, train=True)
    counts, offsets, ids = saved[:3]
    # binning bit-exact: gids of the flat depth-sorted arrays are the oracle's gids
    ometa = TO.make_meta(H, W, B, G, background=bg)
    s = TO.Scene(*(sc[k].numpy() for k in KEYS), B, G)
    ob = TO.bin_scene(ometa, s)
    np.testing.assert_array_equal(perm.cpu().numpy().reshape(-1), ob.perm)
    np.testing.assert_array_equal(counts.cpu().numpy(), ob.tile_counts)
    np.testing.assert_array_equal(offsets.cpu().numpy(), ob.tile_offsets)
    np.testing.assert_array_equal(ids.cpu().numpy(), ob.binned_ids)
    oc = ob.tile_counts
    assert (oc > mfp).sum() >= 4 and (oc > 128).any() and ((oc > 0) & (oc <= mfp)).sum() >= 50
    # stop counts: the oracle's for rendered tiles, 0 for tiles left to the overflow operators
    gT, glast, gstop, _ = gpu_state(sc, H, W, B, G, bg)
    fast = (oc > 0) & (oc <= mfp)
    want = np.where(fast, gstop, 0)
    np.testing.assert_array_equal(stop.cpu().numpy(), want)
    # image and gradients against the oracle
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(17))
    grads = _backward(w.cuda(), flat, metas, perm, saved, stop, H, W, B, G, active=active)
    torch.cuda.synchronize()
    _, ostop, _ = oracle_parity(sc, H, W, B, G, bg, w.numpy(), img.cpu().numpy(), grads, f"v8 ops active={active}",
                                gpu_last=glast)
    np.testing.assert_array_equal(np.where(fast, ostop, 0), want)
    # the eval composition renders the same image, bit for bit
    ev, _, _ = _forward(flat, metas, mfp, H, W, active=active, train=False)
    assert torch.equal(ev, img)
    # ids scrambled inside their tiles: the state forward sorts the rendered tiles' ids in place
    img2, _, saved2 = _forward(flat, metas, mfp, H, W, active=active, train=True, shuffle=True)
    assert torch.equal(img2, img)
    ids2 = saved2[2].cpu().numpy()
    fast_pair = np.repeat(fast, oc)
    np.testing.assert_array_equal(ids2[fast_pair], ob.binned_ids[fast_pair])


def test_reference_ops_without_overflow_and_errors(gpu):
    """A scene with no tile above max_fast_pairs: bin + fast forward + fast backward alone match
    the whole-image path; malformed calls raise RuntimeError before anything is launched."""
    B, G, H, W, mfp = 2, 400, 64, 96, 2048
    bg = (0.0, 0.0, 0.0)
    sc = make_scene_2d(1, seed=5, G=G, B=B, H=H, W=W)
    metas = _v8_meta(H, W, B, G, mfp, bg)
    perm, flat = _sorted_flat(sc, B, G)
    img, stop, saved = _forward(flat, metas, mfp, H, W, active=False, train=True)
    assert saved[4][0].numel() == 0
    w = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(2))
    grads = _backward(w.cuda(), flat, metas, perm, saved, stop, H, W, B, G, active=False)
    oracle_parity(sc, H, W, B, G, bg, w.numpy(), img.cpu().numpy(), grads, "v8 ops, no overflow")
    counts, offsets, ids = saved[:3]
    bad_ids = ids.clone()
    bad_ids[0] = B * G + 5
    with pytest.raises(RuntimeError, match="binned id out of range"):
        OPS.render_fast_forward_eval(*flat, *metas, counts, offsets, bad_ids)
    with pytest.raises(RuntimeError, match="tile range outside binned ids"):
        OPS.render_fast_forward_eval(*flat, *metas, counts, offsets, ids[:-10])
    with pytest.raises(RuntimeError, match="tile id out of range"):
        OPS.render_overflow_forward(*flat, *metas, torch.tensor([10 ** 6], dtype=torch.int32, device="cuda"),
                                    torch.tensor([0, 0], dtype=torch.int32, device="cuda"), ids[:0])
    with pytest.raises(RuntimeError, match="grad_out must be"):
        OPS.render_fast_backward_saved(torch.zeros(B, H, W, 4, device="cuda"), *flat, *metas, counts, offsets, ids,
                                       stop)
    i32, f32, hi, hf = metas
    bad = hi.clone()
    bad[7] = 4096
    with pytest.raises(RuntimeError, match="exceeds shader compile-time cap 2048"):
        OPS.bin(*flat, i32, f32, bad, hf)
    torch.cuda.synchronize()
