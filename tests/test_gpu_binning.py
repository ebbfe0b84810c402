"""GPU parity: scan, radix sort, depth order and tile binning vs the CPU oracle.

Bar: bit-exact (integer / index work).  Calls go through the C ABI
(libgsplat_hip.so via torch_gsplat_bridge_fast._ops / _lib).
"""
import numpy as np
import pytest
import torch

from oracle import tile_oracle as TO
from torch_gsplat_bridge_fast import _lib, _ops
from torch_gsplat_bridge_fast.scenes import make_scene_2d

pytestmark = pytest.mark.gpu

KEYS = ("means2d", "conics", "colors", "opacities", "depths")


@pytest.mark.parametrize("n", [0, 1, 63, 8191, 8192, 8193, 100_000, (1 << 18), (1 << 18) + 1, 3_000_017])
def test_exclusive_scan(gpu, n):
    print(f"scan n={n}", flush=True)
    rng = np.random.default_rng(n)
    x = rng.integers(0, 50, size=n).astype(np.int32)
    out = _ops.exclusive_scan_i32(torch.from_numpy(x).to(gpu)).cpu().numpy()
    ref = np.concatenate([[0], np.cumsum(x, dtype=np.int64)]).astype(np.int32)
    np.testing.assert_array_equal(out, ref)


def test_exclusive_scan_in_place(gpu):
    x = torch.randint(0, 9, (300_001,), dtype=torch.int32)
    ref = np.concatenate([[0], np.cumsum(x.numpy(), dtype=np.int64)]).astype(np.int32)
    buf = torch.zeros(300_002, dtype=torch.int32, device=gpu)
    buf[:-1] = x.to(gpu)
    L = _lib.lib()
    wsb = L.gsplat_hip_scan_workspace_bytes(300_001)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    _lib.check(L.gsplat_hip_exclusive_scan_i32(buf.data_ptr(), buf.data_ptr(), 300_001, None, ws.data_ptr(), wsb,
                                               _lib.stream_of(buf)), "scan")
    np.testing.assert_array_equal(buf.cpu().numpy(), ref)


@pytest.mark.parametrize("n,segments,begin,end,keyrange", [
    (1, 1, 0, 32, 1 << 32),
    (5000, 1, 0, 16, 1 << 16),
    (4096, 1, 0, 32, 1 << 32),
    (100_003, 1, 0, 13, 37),          # many duplicates, partial digit
    (700_001, 1, 0, 16, 1 << 16),
    (1_048_576, 1, 0, 32, 1 << 32),   # 4096-element blocks (at 2^20 elements)
    (1_048_577, 1, 0, 20, 1 << 20),   # 8192-element blocks (above 2^20), a last block of one element
    (2_500_003, 1, 0, 32, 1 << 32),   # 32-bit keys, 8192-element blocks
    (4_200_001, 1, 0, 16, 1 << 16),   # 8192-element blocks above 2^22 elements
    (3_000_000, 2, 0, 24, 1 << 24),   # segmented, 8192-element blocks
    (65536, 4, 0, 32, 1 << 32),       # segmented
    (10_000, 3, 8, 24, 1 << 32),      # bit window
    (1000, 2, 0, 0, 1 << 32),         # zero passes: copy
])
def test_radix_sort_stable(gpu, n, segments, begin, end, keyrange):
    print(f"radix n={n} seg={segments} bits=[{begin},{end})", flush=True)
    rng = np.random.default_rng(n + segments)
    keys = rng.integers(0, keyrange, size=n * segments, dtype=np.uint64).astype(np.uint32)
    vals = rng.integers(0, 1 << 31, size=n * segments).astype(np.int32)
    ko, vo = _ops.radix_sort_pairs_u32(torch.from_numpy(keys.view(np.int32)).to(gpu), torch.from_numpy(vals).to(gpu),
                                       segments=segments, begin_bit=begin, end_bit=end)
    ko = ko.cpu().numpy().view(np.uint32)
    vo = vo.cpu().numpy()
    mask = np.uint64(((1 << end) - 1) - ((1 << begin) - 1)) if end > begin else np.uint64(0)
    for s in range(segments):
        sl = slice(s * n, (s + 1) * n)
        sub = keys[sl].astype(np.uint64) & mask
        order = np.argsort(sub, kind="stable")
        np.testing.assert_array_equal(ko[sl], keys[sl][order])
        np.testing.assert_array_equal(vo[sl], vals[sl][order])


def _gpu_bins(scene, H, W, B, G, background=(0.0, 0.0, 0.0)):
    dev = torch.device("cuda:0")
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, background)
    flat = [scene[k].reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for k in KEYS]
    return _ops.bin_gaussians(meta, *flat)


def _oracle_bins(scene, H, W, B, G):
    meta = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(scene[k].numpy() for k in KEYS), B, G)
    return meta, s, TO.bin_scene(meta, s)


def _assert_bins_equal(st, ob, scene, B, G):
    np.testing.assert_array_equal(st.perm.cpu().numpy(), ob.perm, err_msg="depth order")
    np.testing.assert_array_equal(st.tile_counts.cpu().numpy(), ob.tile_counts, err_msg="tile counts")
    np.testing.assert_array_equal(st.tile_offsets.cpu().numpy(), ob.tile_offsets, err_msg="tile ranges")
    assert st.n_pairs == ob.binned_ids.size
    np.testing.assert_array_equal(st.binned_ids.cpu().numpy(), ob.binned_ids, err_msg="sorted pair ids")
    # packed records are exact copies of the inputs in gid order
    packed = st.packed.cpu().numpy()
    orig = (np.arange(B * G) // G) * G + ob.perm
    m = scene["means2d"].reshape(-1, 2).numpy()
    q = scene["conics"].reshape(-1, 3).numpy()
    c = scene["colors"].reshape(-1, 3).numpy()
    o = scene["opacities"].reshape(-1).numpy()
    np.testing.assert_array_equal(packed[:, 0:2], m[orig])
    np.testing.assert_array_equal(packed[:, 2:5], q[orig])
    np.testing.assert_array_equal(packed[:, 5], o[orig])
    np.testing.assert_array_equal(packed[:, 6:9], c[orig])
    meta = TO.make_meta(8, 8, 1, 1)
    qm, om, mm = q[orig], o[orig], m[orig]
    word = packed[:, 9].view(np.uint32)
    np.testing.assert_array_equal((word & np.uint32(0x7FFFFFFF)).astype(np.int32), orig.astype(np.int32))
    # bit 31: the plain flag, bit-exact with its restatement (and not vacuous on these scenes)
    plain = TO.plain_flags(qm[:, 0], qm[:, 1], qm[:, 2], mm[:, 0], mm[:, 1], om, meta.max_alpha)
    np.testing.assert_array_equal((word >> np.uint32(31)).astype(bool), plain, err_msg="plain flag")
    # the alpha test's bounds are bit-exact with the oracle's: q = plim + lo and lo
    plim = np.array([TO.plim(float(v), meta.alpha_threshold, meta.max_alpha) for v in om], dtype=np.float32)
    lo = np.array([TO.opacity_log2(float(v)) for v in om], dtype=np.float32)
    np.testing.assert_array_equal(packed[:, 10].view(np.uint32), (plim + lo).view(np.uint32), err_msg="q")
    np.testing.assert_array_equal(packed[:, 11].view(np.uint32), lo.view(np.uint32), err_msg="lo")
    # the strip-culling constants, bit-exact with their restatement
    want = TO.strip_consts(qm[:, 0], qm[:, 1], qm[:, 2], plim)
    np.testing.assert_array_equal(packed[:, 12:16].view(np.uint32), want.view(np.uint32), err_msg="strip constants")
    # sorted 64-bit keys (tile << 32 | gid) strictly increase
    keys = ob.sorted_keys()
    assert np.all(keys[1:] > keys[:-1])


@pytest.mark.parametrize("cfg_id,kw", [
    (0, {}),
    (1, {}),
    (2, {}),
    (3, {}),
    (0, dict(H=37, W=53, G=777)),       # ragged image, G not a multiple of 64
    (3, dict(B=3, G=1000, H=100, W=90)),
])
def test_binning_bit_exact(gpu, cfg_id, kw):
    sc = make_scene_2d(cfg_id, seed=11, **kw)
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    print(f"binning cfg{cfg_id} {W}x{H} B={B} G={G}", flush=True)
    st = _gpu_bins(sc, H, W, B, G)
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    _assert_bins_equal(st, ob, sc, B, G)


@pytest.mark.parametrize("B,G,H,W", [
    (1, 2000, 256, 256),     # 256 tiles: 8 tile bits, one onesweep pass
    (1, 2000, 16, 4112),     # 257 tiles: 9 bits, buckets of 2 tiles, a last bucket of one
    (1, 2000, 100, 1000),    # 441 tiles: 9 bits, ragged rows
    (1, 3000, 4096, 4096),   # 65,536 tiles: 16 bits, 256 buckets of 256 tiles
    (2, 3000, 4096, 4096),   # 131,072 tiles: 17 bits, two onesweep passes and the range launch
])
def test_pair_sort_path_boundaries(gpu, B, G, H, W):
    """The pair sort takes one onesweep pass for images of at most 2^8 tiles, a pass on the high
    bits plus a counting sort per bucket of 2^(bits-8) tiles for 2^9..2^16 tiles, and two passes
    plus the tile-range launch above 2^16: binnings at both sides of each boundary (the first of a
    shape, which reads N before emitting, and the second, with the remembered capacity) are bit-exact
    against the oracle."""
    print(f"pair sort path B={B} G={G} {H}x{W}", flush=True)
    sc = make_scene_2d(1, seed=31, G=G, B=B, H=H, W=W)
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    _ops._capacity.pop(_capacity_key(B, G, H, W), None)
    for _ in range(2):
        _assert_bins_equal(_gpu_bins(sc, H, W, B, G), ob, sc, B, G)


@pytest.mark.parametrize("B,G,H,W,cap", [
    (1, 3000, 512, 512, 9_000_000),     # 1,024 tiles (10 bits), few pairs in a large buffer: many
                                        # low-byte boundaries inside the first sort blocks
    (1, 40_000, 512, 512, None),        # above 2^23 pairs: this path from the binning's own count
    (1, 2000, 16, 4112, 9_000_000),     # 257 tiles: 9 bits, one bit in the second pass
    (2, 3000, 2048, 4096, 9_000_000),   # 65,536 tiles in two images: 16 bits
    (3, 5000, 300, 520, 9_000_000),     # 3 x 19 x 33 = 1,881 tiles: 11 bits, ragged rows
])
def test_two_pass_pair_sort(gpu, B, G, H, W, cap):
    """Images of 2^9..2^16 tiles whose pair buffer holds at least 2^23 pairs (and more than 4096 per
    bucket) sort the pairs in two passes over packed words (low tile byte, then the high bits, with
    gids below 2^24), the second of which writes every tile range from the first pass's digit
    boundaries: bit-exact against the oracle, with the boundaries sparse (a large count) or dense (a
    buffer far larger than the pairs, so that many low-byte ranges start inside one sort block)."""
    print(f"two-pass pair sort B={B} G={G} {H}x{W} cap={cap}", flush=True)
    sc = make_scene_2d(1, seed=37, G=G, B=B, H=H, W=W)
    if cap is None:   # splats 18 times larger: about 1.2e7 pairs
        sc["conics"] = sc["conics"] / 324.0
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    if cap is None:
        assert ob.binned_ids.size > (1 << 23)
    key = _capacity_key(B, G, H, W)
    _ops._capacity.pop(key, None)
    if cap is not None:
        _ops._capacity[key] = cap
    for _ in range(2):
        _assert_bins_equal(_gpu_bins(sc, H, W, B, G), ob, sc, B, G)


def _check_short_buffer(st, ob, n, cap):
    """A binning into a buffer of cap < N pairs: the first `cap` pairs of the full order, each
    tile's kept pairs in order, and every pair of a splat whose range ends by cap kept."""
    assert st.capacity == cap
    offsets = st.tile_offsets.cpu().numpy()
    assert offsets[0] == 0 and offsets[-1] == cap and np.all(np.diff(offsets) >= 0)
    assert not st.confirm() and st.n_pairs == n
    got = st.pairs[:cap].cpu().numpy()
    splat_end = st.splat_offsets.cpu().numpy()[1:]
    for t in range(ob.tile_offsets.size - 1):
        want = ob.binned_ids[ob.tile_offsets[t]:ob.tile_offsets[t + 1]]
        have = got[offsets[t]:offsets[t + 1]]
        assert np.all(np.diff(have) > 0) and np.isin(have, want).all()
        assert np.isin(want[splat_end[want] <= cap], have).all()


def test_large_image_short_buffer(gpu):
    """Images above 131,072 splats bin with the emit in original order over the count's records
    and recorded ballots: with a pair buffer below N the one-call binning keeps exactly the first
    `capacity` pairs, as the depth-order emit does."""
    B, G, H, W = 1, 140_000, 512, 512
    print(f"large image, short buffer B={B} G={G} {H}x{W}", flush=True)
    sc = make_scene_2d(1, seed=43, G=G, B=B, H=H, W=W)
    sc["conics"] = sc["conics"] / 16.0   # splats 4 times larger
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    n = ob.binned_ids.size
    print(f"  pairs {n}", flush=True)
    key = _capacity_key(B, G, H, W)
    dev = torch.device("cuda:0")
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    flat = [sc[k].reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for k in KEYS]
    cap = n // 2
    _ops._capacity[key] = cap
    _check_short_buffer(_ops.bin_gaussians(meta, *flat, defer_check=True), ob, n, cap)
    _ops._capacity[key] = n + 1000   # and a buffer that holds them all: bit-exact
    _assert_bins_equal(_gpu_bins(sc, H, W, B, G), ob, sc, B, G)


def test_two_pass_pair_sort_empty_and_short(gpu):
    """The two-pass sort with no pair at all (every splat culled, a large remembered buffer) leaves
    every range empty, and with a buffer below N keeps exactly the first `capacity` pairs."""
    B, G, H, W = 1, 80_000, 512, 512
    print(f"two-pass pair sort: empty and short buffers B={B} G={G} {H}x{W}", flush=True)
    sc = make_scene_2d(1, seed=41, G=G, B=B, H=H, W=W)
    sc["conics"] = sc["conics"] / 324.0
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    n = ob.binned_ids.size
    assert n // 2 >= (1 << 23)
    key = _capacity_key(B, G, H, W)
    dev = torch.device("cuda:0")
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    # a buffer below N (still at least 2^23 pairs): the first `cap` pairs, consistent ranges
    cap = n // 2
    _ops._capacity[key] = cap
    flat = [sc[k].reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for k in KEYS]
    st = _ops.bin_gaussians(meta, *flat, defer_check=True)
    _check_short_buffer(st, ob, n, cap)
    # every splat culled, the buffer remembered from above
    _ops._capacity[key] = 2 * n
    sc0 = dict(sc)
    sc0["opacities"] = torch.zeros_like(sc["opacities"])
    st = _gpu_bins(sc0, H, W, B, G)
    assert st.n_pairs == 0
    assert not st.tile_offsets.cpu().numpy().any() and int(st.tile_counts.sum()) == 0


def test_bucket_sort_skewed(gpu):
    """The pair sort of images of 2^9..2^16 tiles ends in one counting sort per bucket of
    2^(bits-8) tiles.  Here 1024x1024 (4096 tiles: 256 buckets of 16) with most splats packed into
    a 128x96-pixel patch, so that a few buckets hold tens of thousands of pairs (counted in a sweep,
    then sorted 4096 at a time) while the others hold few: sorted ids, ranges and counts bit-exact,
    on the first binning of the shape and on the one sized from it."""
    rng = np.random.default_rng(21)
    B, H, W = 1, 1024, 1024
    G_hot, G_rest = 24_000, 6_000
    G = G_hot + G_rest
    m = np.concatenate([rng.uniform([300, 500], [428, 596], size=(G_hot, 2)),
                        rng.uniform(-20, 1044, size=(G_rest, 2))]).astype(np.float32)
    sig = rng.uniform(2.0, 14.0, size=(G, 2))
    th = rng.uniform(0, np.pi, size=G)
    c, s_ = np.cos(th), np.sin(th)
    ix, iy = 1 / sig[:, 0] ** 2, 1 / sig[:, 1] ** 2
    q = np.stack([c * c * ix + s_ * s_ * iy, c * s_ * (ix - iy), s_ * s_ * ix + c * c * iy], -1).astype(np.float32)
    perm = rng.permutation(G)
    sc = dict(means2d=m[perm][None], conics=q[perm][None],
              colors=rng.uniform(0, 1, size=(1, G, 3)).astype(np.float32),
              opacities=rng.uniform(0.05, 1, size=(1, G)).astype(np.float32),
              depths=rng.uniform(0.5, 20, size=(1, G)).astype(np.float32))
    sc = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sc.items()}
    print(f"bucket sort skewed {W}x{H} G={G}", flush=True)
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    per_bucket = np.add.reduceat(np.diff(ob.tile_offsets), np.arange(0, 4096, 16))
    assert per_bucket.max() > 4 * 4096 and ob.binned_ids.size <= 256 * 4096
    _ops._capacity.pop(_capacity_key(B, G, H, W), None)
    for _ in range(2):
        st = _gpu_bins(sc, H, W, B, G)
        _assert_bins_equal(st, ob, sc, B, G)


SENTINEL = -123_456_789


def _banded_scene(seed, G, H, W, bands):
    """Config-1 style splats (sigma U(0.5,6) px, support radius at most ~20 px) whose centres lie in
    the given pixel-row bands only, 40 px clear of each band's edges."""
    sc = make_scene_2d(1, seed=seed, G=G, B=1, H=H, W=W)
    rng = np.random.default_rng(seed)
    lo = np.array([b[0] + 40 for b in bands], dtype=np.float64)
    hi = np.array([b[1] - 40 for b in bands], dtype=np.float64)
    pick = rng.choice(len(bands), size=G, p=(hi - lo) / (hi - lo).sum())
    y = rng.uniform(lo[pick], hi[pick]).astype(np.float32)
    sc["means2d"][0, :, 1] = torch.from_numpy(y)
    return sc


def _bin_capi_sentinel(sc, H, W, B, G, cap, staged):
    """Binning through the C ABI with tile_offsets pre-filled with SENTINEL: the one-call
    gsplat_hip_bin, or the four staged calls (count, depth order, pack, emit)."""
    dev = torch.device("cuda:0")
    L = _lib.lib()
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    flat = [sc[k].reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for k in KEYS]
    BG, T = B * G, B * ((H + 15) // 16) * ((W + 15) // 16)
    perm = torch.empty(BG, dtype=torch.int32, device=dev)
    packed = torch.empty((BG, _lib.RECORD_FLOATS), dtype=torch.float32, device=dev)
    offs = torch.empty(BG + 1, dtype=torch.int32, device=dev)
    tiles = torch.full((T + 1,), SENTINEL, dtype=torch.int32, device=dev)
    pairs = torch.full((cap,), SENTINEL, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    if staged:
        wsb = L.gsplat_hip_bin_count_workspace_bytes(meta)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        n_dev = torch.empty(1, dtype=torch.int32, device=dev)
        _lib.check(L.gsplat_hip_bin_count(meta, _lib.ptr(flat[0]), _lib.ptr(flat[1]), _lib.ptr(flat[3]),
                                          n_dev.data_ptr(), ws.data_ptr(), wsb, s), "bin_count")
        _lib.check(L.gsplat_hip_bin_depth_order(meta, _lib.ptr(flat[4]), perm.data_ptr(), ws.data_ptr(), wsb, s),
                   "bin_depth_order")
        _lib.check(L.gsplat_hip_bin_pack(meta, *[_lib.ptr(t) for t in flat[:4]], perm.data_ptr(),
                                         packed.data_ptr(), offs.data_ptr(), ws.data_ptr(), wsb, s), "bin_pack")
        ws2b = L.gsplat_hip_bin_emit_workspace_bytes(meta, cap)
        ws2 = torch.empty(max(ws2b, 1), dtype=torch.uint8, device=dev)
        counts = torch.full((T,), SENTINEL, dtype=torch.int32, device=dev)
        status = torch.full((1,), SENTINEL, dtype=torch.int32, device=dev)
        _lib.check(L.gsplat_hip_bin_emit(meta, packed.data_ptr(), offs.data_ptr(), cap, pairs.data_ptr(),
                                         counts.data_ptr(), tiles.data_ptr(), status.data_ptr(), ws.data_ptr(), wsb,
                                         ws2.data_ptr(), ws2b, s), "bin_emit")
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        return perm, tiles, pairs, counts
    wsb = L.gsplat_hip_bin_workspace_bytes(meta, cap)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    words = torch.zeros((4,), dtype=torch.int32, pin_memory=True)
    ev_st = torch.cuda.Event()
    ev_st.record(torch.cuda.current_stream(dev))
    _lib.check(L.gsplat_hip_bin(meta, *[_lib.ptr(t) for t in flat], cap, perm.data_ptr(), packed.data_ptr(),
                                offs.data_ptr(), pairs.data_ptr(), tiles.data_ptr(), words.data_ptr(),
                                ws.data_ptr(), wsb, s, None, None, None, ev_st.cuda_event), "gsplat_hip_bin")
    ev_st.synchronize()
    assert int(words[1]) == 0 and int(words[3]) == 1
    return perm, tiles, pairs, None


@pytest.mark.parametrize("H,W,G,bands,empty", [
    # 4096 tiles: 256 buckets of 16 tiles (a quarter tile row each)
    (1024, 1024, 6000, [(0, 512)], "last"),                  # splats in the top half only
    (1024, 1024, 6000, [(512, 1024)], "first"),              # bottom half only
    (1024, 1024, 6000, [(100, 400), (600, 900)], "both"),    # empty first, middle and last buckets
    # 65,536 tiles: 256 buckets of one tile row each
    (4096, 4096, 8000, [(300, 1800), (2500, 3900)], "both"),
])
def test_bucket_sort_empty_buckets(gpu, H, W, G, bands, empty):
    """The bucket counting sort writes the tile ranges of buckets that hold no pair (an image band
    with no splats): every such tile's range is empty and starts where the next non-empty one does.
    tile_offsets, tile counts and the sorted ids are pre-filled with a sentinel and compared
    bit-exact with the oracle, for the one-call binning, the four staged calls and binning +
    forward (whose image must be the background exactly on the empty tiles)."""
    B = 1
    print(f"bucket sort empty buckets {W}x{H} G={G} bands={bands}", flush=True)
    sc = _banded_scene(41, G, H, W, bands)
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    n = int(ob.binned_ids.size)
    T = ob.tile_offsets.size - 1
    low = (T - 1).bit_length() - 8
    per_bucket = np.add.reduceat(np.diff(ob.tile_offsets), np.arange(0, T, 1 << low))
    assert per_bucket.size == 256 and n <= 256 * 4096
    if empty in ("first", "both"):
        assert per_bucket[0] == 0
    if empty in ("last", "both"):
        assert per_bucket[-1] == 0
    assert (per_bucket > 0).any() and (per_bucket == 0).sum() >= 16
    for staged in (False, True):
        for cap in (n, n + 777):
            perm, tiles, pairs, counts = _bin_capi_sentinel(sc, H, W, B, G, cap, staged)
            np.testing.assert_array_equal(perm.cpu().numpy(), ob.perm)
            np.testing.assert_array_equal(tiles.cpu().numpy(), ob.tile_offsets, err_msg=f"ranges staged={staged}")
            np.testing.assert_array_equal(pairs[:n].cpu().numpy(), ob.binned_ids, err_msg="sorted pair ids")
            if counts is not None:
                np.testing.assert_array_equal(counts.cpu().numpy(), np.diff(ob.tile_offsets), err_msg="counts")
    # binning + forward in one call: empty tiles show the background
    dev = torch.device("cuda:0")
    L = _lib.lib()
    bg = (0.25, 0.5, 0.75)
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, bg)
    flat = [sc[k].reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for k in KEYS]
    cap = n + 100
    perm = torch.empty(G, dtype=torch.int32, device=dev)
    packed = torch.empty((G, _lib.RECORD_FLOATS), dtype=torch.float32, device=dev)
    offs = torch.empty(G + 1, dtype=torch.int32, device=dev)
    tiles = torch.full((T + 1,), SENTINEL, dtype=torch.int32, device=dev)
    pairs = torch.empty(cap, dtype=torch.int32, device=dev)
    wsb = L.gsplat_hip_bin_workspace_bytes(meta, cap)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    img = torch.full((B, H, W, 3), -1.0, dtype=torch.float32, device=dev)
    rwsb = L.gsplat_hip_render_workspace_bytes(meta, 0)
    rws = torch.empty(max(rwsb, 1), dtype=torch.uint8, device=dev)
    words = torch.zeros((4,), dtype=torch.int32, pin_memory=True)
    ev_st = torch.cuda.Event()
    ev_st.record(torch.cuda.current_stream(dev))
    _lib.check(L.gsplat_hip_bin_render_forward(
        meta, *[_lib.ptr(t) for t in flat], cap, perm.data_ptr(), packed.data_ptr(), offs.data_ptr(),
        pairs.data_ptr(), tiles.data_ptr(), words.data_ptr(), ws.data_ptr(), wsb, img.data_ptr(), None, None, None,
        rws.data_ptr(), rwsb, torch.cuda.current_stream(dev).cuda_stream, None, None, None, ev_st.cuda_event),
        "gsplat_hip_bin_render_forward")
    ev_st.synchronize()
    assert [int(v) for v in words] == [n, 0, int(np.max(np.diff(ob.tile_offsets)) > _lib.HANDOFF_PAIRS), 1]
    np.testing.assert_array_equal(tiles.cpu().numpy(), ob.tile_offsets)
    tiles_x = (W + 15) // 16
    im = img[0].cpu().numpy()
    for t in np.flatnonzero(np.diff(ob.tile_offsets) == 0)[::7]:
        ty, tx = divmod(int(t), tiles_x)
        blk = im[16 * ty:16 * ty + 16, 16 * tx:16 * tx + 16]
        np.testing.assert_array_equal(blk, np.broadcast_to(np.array(bg, np.float32), blk.shape))


def test_binning_edge_cases(gpu):
    """Off-screen, zero/threshold opacity, degenerate and huge conics, depth ties, -0/+0, NaN depth."""
    rng = np.random.default_rng(5)
    B, G, H, W = 2, 300, 70, 45
    m = rng.uniform(-60, 110, size=(B, G, 2)).astype(np.float32)
    sig = rng.uniform(0.2, 40, size=(B, G, 2))
    th = rng.uniform(0, np.pi, size=(B, G))
    c, s = np.cos(th), np.sin(th)
    ix, iy = 1 / sig[..., 0] ** 2, 1 / sig[..., 1] ** 2
    q = np.stack([c * c * ix + s * s * iy, c * s * (ix - iy), s * s * ix + c * c * iy], -1).astype(np.float32)
    q[:, :10] = [1e-9, 0.0, 1e-9]           # near-zero conic: huge support
    q[:, 10:20] = [50.0, 0.0, 50.0]         # tiny support
    o = rng.uniform(0, 1, size=(B, G)).astype(np.float32)
    o[:, 20:30] = 0.0
    o[:, 30:40] = 1.0 / 255.0
    o[:, 40:50] = 1.0
    d = rng.integers(0, 5, size=(B, G)).astype(np.float32)   # many ties
    d[:, 50] = -0.0
    d[:, 51] = 0.0
    d[:, 52] = np.nan
    d[:, 53] = -np.inf
    col = rng.uniform(0, 1, size=(B, G, 3)).astype(np.float32)
    sc = {k: torch.from_numpy(v) for k, v in
          dict(means2d=m, conics=q, colors=col, opacities=o, depths=d).items()}
    st = _gpu_bins(sc, H, W, B, G)
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    _assert_bins_equal(st, ob, sc, B, G)
    # stable argsort semantics: ties by index, -0 == +0, NaN last
    for b in range(B):
        np.testing.assert_array_equal(ob.perm[b * G:(b + 1) * G], np.argsort(d[b], kind="stable"))


@pytest.mark.parametrize("seed,H,W,G,elong", [
    (51, 640, 1000, 2000, False),   # large round splats, centres also off-screen
    (52, 512, 8192, 1500, True),    # elongated and rotated, far from the origin (x up to 8k)
    (53, 300, 300, 800, True),
])
def test_binning_large_splats(gpu, seed, H, W, G, elong):
    """Splats of 10-150 px, round or thin (axis ratio down to 0.02) at any angle, opacities from
    just above the threshold (small support) to 1: most of their candidate tiles lie in the
    rectangle of certain hits that the walk skips (counted and written without the test), the rest
    are tested.  The binning is bit-exact against the oracle, which tests every tile."""
    rng = np.random.default_rng(seed)
    print(f"large splats seed={seed} {W}x{H} G={G} elongated={elong}", flush=True)
    m = np.stack([rng.uniform(-200, W + 200, G), rng.uniform(-200, H + 200, G)], -1)
    s1 = np.exp(rng.uniform(np.log(10.0), np.log(150.0), G))
    s2 = s1 * (rng.uniform(0.02, 1.0, G) if elong else rng.uniform(0.5, 1.0, G))
    th = rng.uniform(0, np.pi, G)
    c, s = np.cos(th), np.sin(th)
    ix, iy = 1 / s1 ** 2, 1 / s2 ** 2
    q = np.stack([c * c * ix + s * s * iy, c * s * (ix - iy), s * s * ix + c * c * iy], -1)
    o = np.exp(rng.uniform(np.log(1.0 / 255.0 * 1.001), 0.0, G))
    o[: G // 10] = 1.0 / 255.0 * (1 + rng.uniform(1e-4, 1e-2, G // 10))   # tiny support
    sc = {k: torch.from_numpy(np.asarray(v, np.float32)[None]) for k, v in dict(
        means2d=m, conics=q, colors=rng.uniform(0, 1, (G, 3)), opacities=o,
        depths=rng.uniform(0.1, 10, G)).items()}
    _, _, ob = _oracle_bins(sc, H, W, 1, G)
    print(f"  pairs {ob.binned_ids.size}", flush=True)
    key = _capacity_key(1, G, H, W)
    _ops._capacity.pop(key, None)
    for _ in range(2):   # the four-call binning, then the one-call path with the remembered buffer
        _assert_bins_equal(_gpu_bins(sc, H, W, 1, G), ob, sc, 1, G)


def test_large_image_emit_with_recorded_ballots(gpu):
    """Images above 131,072 splats: the one-call binning's count records each wavefront's first 128
    walk-step hit ballots, and the emit walks the count's wavefronts in original order, taking a
    recorded step's hits from its ballot (a step without hits is skipped) and testing the steps past
    the record itself.  The first 32 splats (one count wavefront) are long thin splats at about 45
    degrees, each with thousands of candidate tiles and few hits, so that wavefront walks thousands
    of steps past its record; the rest are ordinary small splats.  Bit-exact against the oracle on
    the four-call binning and on the one-call path."""
    rng = np.random.default_rng(61)
    H, W, B, G = 2048, 2048, 1, 140_000
    print(f"large image, recorded ballots {W}x{H} G={G}", flush=True)
    sc = make_scene_2d(1, seed=61, G=G, B=B, H=H, W=W)
    n = 32
    s1 = rng.uniform(500.0, 700.0, n)     # along the axis (px)
    s2 = rng.uniform(1.5, 3.0, n)         # across it
    th = np.pi / 4 + rng.uniform(-0.05, 0.05, n)
    c, s = np.cos(th), np.sin(th)
    ix, iy = 1 / s1 ** 2, 1 / s2 ** 2
    q = np.stack([c * c * ix + s * s * iy, c * s * (ix - iy), s * s * ix + c * c * iy], -1)
    o = rng.uniform(0.5, 1.0, n)
    sc["means2d"][0, :n] = torch.from_numpy(rng.uniform(700.0, 1300.0, (n, 2)).astype(np.float32))
    sc["conics"][0, :n] = torch.from_numpy(q.astype(np.float32))
    sc["opacities"][0, :n] = torch.from_numpy(o.astype(np.float32))
    # the wavefront's candidates (its splats' clipped boxes, a lower bound) far exceed its record's
    # 128 steps of 64
    a_, b_, c_ = q[:, 0], q[:, 1], q[:, 2]
    det = a_ * c_ - b_ * b_
    tau = 2.0 * np.log(o * 255.0)
    hx, hy = np.sqrt(tau * c_ / det), np.sqrt(tau * a_ / det)
    mx, my = sc["means2d"][0, :n, 0].numpy(), sc["means2d"][0, :n, 1].numpy()
    bw = np.floor(np.minimum(mx + hx, W - 1) / 16) - np.floor(np.maximum(mx - hx, 0) / 16) + 1
    bh = np.floor(np.minimum(my + hy, H - 1) / 16) - np.floor(np.maximum(my - hy, 0) / 16) + 1
    assert (bw * bh).sum() > 4 * 128 * 64
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    print(f"  pairs {ob.binned_ids.size}, wavefront 0 candidates >= {int((bw * bh).sum())}", flush=True)
    key = _capacity_key(B, G, H, W)
    _ops._capacity.pop(key, None)
    for _ in range(2):   # the four-call binning, then the one-call path with the remembered buffer
        _assert_bins_equal(_gpu_bins(sc, H, W, B, G), ob, sc, B, G)


def test_binning_all_culled(gpu):
    B, G, H, W = 1, 100, 32, 32
    sc = make_scene_2d(0, seed=1, G=G, H=H, W=W)
    sc["opacities"] = torch.zeros_like(sc["opacities"])
    st = _gpu_bins(sc, H, W, B, G)
    assert st.n_pairs == 0
    assert int(st.tile_counts.sum()) == 0


def _capacity_key(B, G, H, W):
    return (0, B, G, H, W)


@pytest.mark.parametrize("B,G,H,W", [(2, 3000, 200, 264), (1, 70_000, 512, 384), (3, 9_000, 160, 200),
                                     (4, 131_072, 64, 96), (5, 104_858, 64, 96)])
def test_binning_from_remembered_capacity(gpu, B, G, H, W):
    """The second binning of a shape sizes its pair buffers from the first one's count and reads N
    only afterwards (one C-ABI call: for these sizes the count and the depth runs share a launch and N
    comes from the pack scan); the result is bit-identical and the capacity covers N.  Sizes: one
    depth run per image, 18 runs with a partial last one, three images of three runs, and both sides
    of the bound on the emit workgroups of that path (4096 x 128 splats in the batch: at it the
    path above, one splat more and the one-call binning takes the look-back path)."""
    print(f"capacity B={B} G={G} {H}x{W}", flush=True)
    sc = make_scene_2d(1, seed=5, G=G, B=B, H=H, W=W)
    _ops._capacity.pop(_capacity_key(B, G, H, W), None)
    first = _gpu_bins(sc, H, W, B, G)
    assert first.capacity == first.n_pairs > 0
    st = _gpu_bins(sc, H, W, B, G)
    assert st.capacity > st.n_pairs == first.n_pairs
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    _assert_bins_equal(st, ob, sc, B, G)


def _wait_word(words, timeout_s=5.0):
    """Polls pinned host word 3 (set by the device after words 0-2), bounded in time."""
    import time
    t_end = time.perf_counter() + timeout_s
    while words[3] == 0:
        if time.perf_counter() > t_end:
            torch.cuda.synchronize()
            break
    return [int(v) for v in words]


def test_report_ring_wraps(gpu):
    """The Python layer's binnings report N through a ring of pinned host rows, one row per call,
    reused every RING calls.  RING + 8 binnings alternating between two scenes of different pair
    counts each read their own N (the oracle's) across the wrap, and the last binning of each scene
    equals the oracle's."""
    H, W, B, G = 64, 96, 1, 500
    dev = torch.device("cuda:0")
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    scenes, flats, obs = [], [], []
    for seed in (21, 22):
        sc = make_scene_2d(1, seed=seed, G=G, B=B, H=H, W=W)
        scenes.append(sc)
        flats.append([sc[k].reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for k in KEYS])
        obs.append(_oracle_bins(sc, H, W, B, G)[2])
    n_ref = [int(ob.binned_ids.size) for ob in obs]
    assert n_ref[0] != n_ref[1]
    calls = _ops._DeviceBinState.RING + 8
    print(f"report ring: {calls} binnings, N = {n_ref}", flush=True)
    last = [None, None]
    for i in range(calls):
        st = _ops.bin_gaussians(meta, *flats[i % 2])
        assert st.n_pairs == n_ref[i % 2], f"call {i}"
        last[i % 2] = st
    for k in range(2):
        _assert_bins_equal(last[k], obs[k], scenes[k], B, G)


@pytest.mark.parametrize("cfg,G,H,W,B", [(1, 3000, 200, 264, 1), (3, 150_000, 256, 256, 1)])
def test_host_report_words(gpu, cfg, G, H, W, B):
    """gsplat_hip_bin and gsplat_hip_bin_render_forward report {N, status, long-range flag} to four
    pinned host words with word 3 set last.  The words read after polling word 3 (no event, no
    synchronisation) and after waiting for status_event hold the oracle's N, status 0 and whether some
    tile range exceeds HANDOFF_PAIRS; word 3 is cleared by the call before it launches.  Sizes: the
    one-stream small-image path and the two-stream path above 131,072 splats."""
    print(f"host report cfg={cfg} G={G} {H}x{W}", flush=True)
    dev = torch.device("cuda:0")
    sc = make_scene_2d(cfg, seed=11, G=G, B=B, H=H, W=W)
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    n = int(ob.binned_ids.size)
    long_ref = int(np.max(np.diff(ob.tile_offsets)) > _lib.HANDOFF_PAIRS)
    L = _lib.lib()
    meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    flat = [sc[k].reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for k in KEYS]
    BG, T = B * G, B * ((H + 15) // 16) * ((W + 15) // 16)
    cap = n + 1000
    perm = torch.empty(BG, dtype=torch.int32, device=dev)
    packed = torch.empty((BG, _lib.RECORD_FLOATS), dtype=torch.float32, device=dev)
    offs = torch.empty(BG + 1, dtype=torch.int32, device=dev)
    tiles = torch.empty(T + 1, dtype=torch.int32, device=dev)
    pairs = torch.empty(cap, dtype=torch.int32, device=dev)
    wsb = L.gsplat_hip_bin_workspace_bytes(meta, cap)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    words = torch.full((4,), 7, dtype=torch.int32, pin_memory=True)
    host = words.numpy()
    main = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(device=dev)
    ev_in, ev_n, ev_st = torch.cuda.Event(), torch.cuda.Event(), torch.cuda.Event()
    for e in (ev_in, ev_n, ev_st):
        e.record(main)
    torch.cuda.synchronize()
    args = [_lib.ptr(t) for t in flat] + [cap, perm.data_ptr(), packed.data_ptr(), offs.data_ptr(),
                                         pairs.data_ptr(), tiles.data_ptr(), words.data_ptr(),
                                         ws.data_ptr(), wsb]
    streams = [main.cuda_stream, side.cuda_stream, ev_in.cuda_event, ev_n.cuda_event]
    expect = [n, 0, long_ref, 1]
    # standalone binning, polled
    _lib.check(L.gsplat_hip_bin(meta, *args, *streams, None), "gsplat_hip_bin")
    assert _wait_word(host) == expect
    np.testing.assert_array_equal(tiles.cpu().numpy(), ob.tile_offsets)
    # standalone binning, waited for through status_event
    host[:] = 7
    _lib.check(L.gsplat_hip_bin(meta, *args, *streams, ev_st.cuda_event), "gsplat_hip_bin")
    ev_st.synchronize()
    assert [int(v) for v in host] == expect
    # binning + forward: the forward's first workgroup reports
    img = torch.empty((B, H, W, 3), dtype=torch.float32, device=dev)
    rwsb = L.gsplat_hip_render_workspace_bytes(meta, 0)
    rws = torch.empty(max(rwsb, 1), dtype=torch.uint8, device=dev)
    for ev in (None, ev_st.cuda_event):
        host[:] = 7
        _lib.check(L.gsplat_hip_bin_render_forward(meta, *args, img.data_ptr(), None, None, None, rws.data_ptr(),
                                                   rwsb, *streams, ev), "gsplat_hip_bin_render_forward")
        if ev is None:
            assert _wait_word(host) == expect
        else:
            ev_st.synchronize()
            assert [int(v) for v in host] == expect
    torch.cuda.synchronize()


def test_binning_capacity_too_small(gpu):
    """With buffers below N the binning holds exactly the first `capacity` pairs (every pair of the
    gids whose range ends below it, part of the one range that straddles it), confirm() reports it,
    and binning again fits and is exact."""
    B, G, H, W = 1, 4000, 256, 256
    print(f"capacity overflow B={B} G={G} {H}x{W}", flush=True)
    sc = make_scene_2d(2, seed=9, G=G, B=B, H=H, W=W)
    _, _, ob = _oracle_bins(sc, H, W, B, G)
    n = ob.binned_ids.size
    key = _capacity_key(B, G, H, W)
    for cap in (n // 3, n - 1):
        _ops._capacity[key] = cap
        dev = torch.device("cuda:0")
        meta = _lib.make_raster_meta(H, W, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
        flat = [sc[k].reshape(B * G, -1).squeeze(-1).contiguous().to(dev) for k in KEYS]
        st = _ops.bin_gaussians(meta, *flat, defer_check=True)
        assert st.capacity == cap
        offsets = st.tile_offsets.cpu().numpy()
        assert offsets[0] == 0 and offsets[-1] == cap and np.all(np.diff(offsets) >= 0)
        assert not st.confirm() and st.n_pairs == n
        assert _ops._capacity[key] >= n
        # the truncated pairs: tile t holds a depth-ordered subset of the oracle's tile t
        got = st.pairs[:cap].cpu().numpy()
        splat_end = st.splat_offsets.cpu().numpy()[1:]
        for t in range(ob.tile_offsets.size - 1):
            want = ob.binned_ids[ob.tile_offsets[t]:ob.tile_offsets[t + 1]]
            have = got[offsets[t]:offsets[t + 1]]
            assert np.all(np.diff(have) > 0) and np.isin(have, want).all()
            full = want[splat_end[want] <= cap]
            assert np.isin(full, have).all()
        st2 = _ops.bin_gaussians(meta, *flat)
        _assert_bins_equal(st2, ob, sc, B, G)


@pytest.mark.parametrize("B,G", [(3, 70_001), (1, 4_200_001)])
def test_depth_order_segments_and_large(gpu, B, G):
    """Stable depth order of bin_depth_order (torch.argsort(stable=True) semantics: ties by index,
    -0.0 == +0.0) for several images of 1024-element workgroups and for 4.2M splats in one image
    (4096-element workgroups, more of them than the device holds at once)."""
    print(f"depth order B={B} G={G}", flush=True)
    rng = np.random.default_rng(G)
    d = rng.uniform(0.1, 10.0, size=(B, G)).astype(np.float32)
    d[:, ::7] = d[:, 3:4]          # ties keep index order
    d[:, 5] = -0.0
    d[:, 6] = 0.0
    meta = _lib.make_raster_meta(64, 64, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    L = _lib.lib()
    wsb = L.gsplat_hip_bin_count_workspace_bytes(meta)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    dd = torch.from_numpy(d).to(gpu)
    perm = torch.empty(B * G, dtype=torch.int32, device=gpu)
    _lib.check(L.gsplat_hip_bin_depth_order(meta, _lib.ptr(dd), _lib.ptr(perm), _lib.ptr(ws), wsb,
                                            _lib.stream_of(dd)), "gsplat_hip_bin_depth_order")
    got = perm.cpu().numpy().reshape(B, G)
    for b in range(B):
        np.testing.assert_array_equal(got[b], np.argsort(d[b], kind="stable"))


@pytest.mark.parametrize("B,G,kind", [
    (1, 1, "uniform"), (1, 37, "few"), (2, 4095, "uniform"), (1, 4096, "equal"),
    (3, 4097, "few"), (1, 65536, "uniform"), (2, 65536, "special"), (1, 131072, "few"),
    (2, 131072, "uniform"),     # largest image of the two-launch sort (32 runs)
    (1, 131073, "special"),     # smallest image of the onesweep path
])
def test_depth_order_small_images(gpu, B, G, kind):
    """Images of up to 131072 splats take the two-launch sort (4096-splat runs sorted in LDS, merge
    ranks from sampled binary searches): permutation equal to a stable argsort for uniform depths,
    all-equal depths, few distinct depths and NaN / +-inf / +-0 mixes, at and around the run and
    path boundaries."""
    print(f"depth order small B={B} G={G} {kind}", flush=True)
    rng = np.random.default_rng(G + B)
    if kind == "uniform":
        d = rng.uniform(0.1, 10.0, size=(B, G))
    elif kind == "equal":
        d = np.full((B, G), 2.5)
    elif kind == "few":
        d = rng.integers(0, 4, size=(B, G)) * 0.75 + 1.0
    else:
        d = rng.uniform(-5.0, 5.0, size=(B, G))
        specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-30, -1e-30])
        pick = rng.random((B, G)) < 0.2
        d[pick] = rng.choice(specials, size=int(pick.sum()))
    d = d.astype(np.float32)
    meta = _lib.make_raster_meta(64, 64, B, G, 1.0 / 255.0, 1e-4, (0.0, 0.0, 0.0))
    L = _lib.lib()
    wsb = L.gsplat_hip_bin_count_workspace_bytes(meta)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    dd = torch.from_numpy(d).to(gpu)
    perm = torch.full((B * G,), -1, dtype=torch.int32, device=gpu)
    _lib.check(L.gsplat_hip_bin_depth_order(meta, _lib.ptr(dd), _lib.ptr(perm), _lib.ptr(ws), wsb,
                                            _lib.stream_of(dd)), "gsplat_hip_bin_depth_order")
    got = perm.cpu().numpy().reshape(B, G)
    for b in range(B):
        # numpy: -0.0 == +0.0, NaN last, stable
        np.testing.assert_array_equal(got[b], np.argsort(d[b], kind="stable"))


def test_lookback_giveup_reaches_the_caller(gpu):
    """A look-back wait whose predecessor never publishes its status (forced
    from the host: the diagnostic scan never runs its first blocks) gives up
    after its poll budget, every kernel finishes, and the status word says
    so; the same scan without a stall reports 0 and is exact."""
    L = _lib.lib()
    n = 10 * 4096 + 123
    x = torch.ones(n, dtype=torch.int32, device=gpu)
    wsb = L.gsplat_hip_scan_workspace_bytes(n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    for stalled, spin_limit in ((0, 1 << 20), (3, 64)):
        print(f"stalled scan: {stalled} stalled blocks, spin limit {spin_limit}", flush=True)
        out = torch.full((n + 1,), -7, dtype=torch.int32, device=gpu)
        status = torch.full((1,), -1, dtype=torch.int32, device=gpu)
        _lib.check(L.gsplat_hip_debug_stalled_scan(x.data_ptr(), out.data_ptr(), n, stalled, spin_limit,
                                                   status.data_ptr(), ws.data_ptr(), wsb, _lib.stream_of(x)),
                   "gsplat_hip_debug_stalled_scan")
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        if stalled == 0:
            assert int(status.item()) == 0
            np.testing.assert_array_equal(o, np.arange(n + 1, dtype=np.int32))
        else:
            assert int(status.item()) == _lib.STATUS_LOOKBACK_TIMEOUT
            # the stalled blocks were never scanned; the first block after them gave up with an
            # empty prefix (later ones may give up too: each block is only consistent in itself)
            assert np.all(o[: stalled * 4096] == -7)
            assert o[stalled * 4096] == 0
            for b in range(stalled, (n + 4095) // 4096):
                blk = o[b * 4096: min((b + 1) * 4096, n)]
                np.testing.assert_array_equal(np.diff(blk), np.ones(blk.size - 1, dtype=np.int32))
    # invalid diagnostics are refused before launching
    rc = L.gsplat_hip_debug_stalled_scan(x.data_ptr(), x.data_ptr(), n, 11, 1, x.data_ptr(), ws.data_ptr(), wsb,
                                         _lib.stream_of(x))
    assert rc == 1


def test_binning_reports_status_zero(gpu):
    """The status word of a normal binning (fast path and four-call path) is 0."""
    sc = make_scene_2d(1, seed=3, G=20000, H=300, W=500)
    from torch_gsplat_bridge_fast import _ops as ops

    key = (0, 1, 20000, 300, 500)
    ops._capacity.pop(key, None)
    for _ in range(2):                      # first call: four-call path; second: one call
        st = _gpu_bins(sc, 300, 500, 1, 20000)
        assert st._status_ready is None      # checked by bin_gaussians
        assert int(st._status_host[st._status_index]) == 0
