"""Tensor-level wrappers over the C ABI.

Each function allocates its outputs with torch's caching allocator on the
inputs' device, enqueues the HIP work on the current stream and returns the
tensors.  The raster path holds one host synchronisation: the pair count N,
which sizes the pair buffers (the reference reads it before emitting,
variants/v8/csrc/metal/gsplat_metal.mm:188).  Here the buffers are sized from
the count of an earlier call of the same shape and N is checked only after
the compositor has been enqueued (bin_and_render), so the host does not stall
the GPU between binning stages; the first call of a shape reads N first.

Every binning also reports a status word (GSPLAT_STATUS_*, set when a
look-back wait gave up, which empties every tile range of that binning).
It reaches pinned memory in the same transfer as N, and BinState.confirm()
raises RuntimeError when it is set, so the call that bins fails.
"""
from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from ._lib import check, ptr, stream_of


# Optional per-op timing: when enabled, the C-ABI calls below (all, or those
# named in `ops`) are bracketed by timing events recorded on the stream the
# work is enqueued on; the compositor calls instead hand the events to their
# kernel launch (gsplat_hip_time_next_launch), which times the compositing
# kernels themselves and adds no stream command.  The events come from a pool
# created up front, so a timed call creates no event.  With every = k
# only every k-th of those calls is bracketed (each event record costs the
# stream a few microseconds, so a sample keeps that out of most steps).
_timing: Optional[list] = None
_timing_ops: Optional[set] = None
_pool: list = []
_every = 1
_seen = 0


def set_timing(enabled: bool, ops=None, pool: int = 0, every: int = 1) -> None:
    """Starts (or stops) recording; `pool` events are created now and used first."""
    global _timing, _timing_ops, _pool, _every, _seen
    _timing = [] if enabled else None
    _timing_ops = set(ops) if ops is not None else None
    _every, _seen = max(1, int(every)), 0
    _pool = []
    if enabled and pool:
        _pool = [torch.cuda.Event(enable_timing=True) for _ in range(pool)]
        for e in _pool:          # creates the underlying HIP events
            e.record()
        torch.cuda.synchronize()
        _pool.reverse()


def _event():
    return _pool.pop() if _pool else torch.cuda.Event(enable_timing=True)


def pop_timing() -> list:
    """Returns [(op_name, start_event, end_event)] recorded since set_timing(True)."""
    global _timing
    out = _timing or []
    _timing = None
    return out


class LaunchTrace:
    """Kernel-level timing of everything the library launches inside a `with` block
    (gsplat_hip_trace_launches): each of the first `capacity` launches, from any thread (the
    autograd engine runs backward launches on its own), records a pair of this object's HIP
    events at its kernel's start and end.  After the block, `launches` holds
    [(kernel name, ms)] in launch order.  Traced launches cost the stream ~10 us each, so a
    trace never brackets a timed region."""

    def __init__(self, capacity: int = 128):
        if not 0 < capacity <= _lib.TRACE_MAX:
            raise ValueError(f"capacity must lie in [1, {_lib.TRACE_MAX}]")
        self.capacity = capacity
        self._events = [torch.cuda.Event(enable_timing=True) for _ in range(2 * capacity)]
        for e in self._events:   # creates the underlying HIP events
            e.record()
        torch.cuda.synchronize()
        self._handles = (ctypes.c_void_p * (2 * capacity))(*[e.cuda_event for e in self._events])
        self.launches: list = []

    def __enter__(self):
        torch.cuda.synchronize()
        check(_lib.lib().gsplat_hip_trace_launches(self._handles, self.capacity), "gsplat_hip_trace_launches")
        return self

    def __exit__(self, *exc):
        L = _lib.lib()
        torch.cuda.synchronize()
        n = int(L.gsplat_hip_trace_count())
        names = [L.gsplat_hip_trace_name(k).decode() for k in range(n)]
        check(L.gsplat_hip_trace_launches(None, 0), "gsplat_hip_trace_launches")
        self.launches = [(names[k], self._events[2 * k].elapsed_time(self._events[2 * k + 1])) for k in range(n)]
        return False


_LAUNCH_TIMED = {"render_forward": _lib.TIME_FORWARD, "render_backward": _lib.TIME_BACKWARD}


class _timed:
    def __init__(self, name):
        global _seen
        self.name = name
        self.on = _timing is not None and (_timing_ops is None or name in _timing_ops)
        if self.on:
            self.on = _seen % _every == _every - 1
            _seen += 1

    def __enter__(self):
        if self.on:
            self.e0 = _event()
            self.which = _LAUNCH_TIMED.get(self.name)
            if self.which is None:
                self.e0.record()
            else:
                self.e1 = _event()
                for e in (self.e0, self.e1):
                    if not e.cuda_event:
                        e.record()   # creates the HIP event
                check(_lib.lib().gsplat_hip_time_next_launch(self.which, self.e0.cuda_event, self.e1.cuda_event),
                      "gsplat_hip_time_next_launch")
        return self

    def __exit__(self, *exc):
        if self.on:
            if self.which is None:
                e1 = _event()
                e1.record()
            else:
                e1 = self.e1
                _lib.lib().gsplat_hip_time_next_launch(self.which, None, None)   # disarm if unused
            if exc[0] is None:
                _timing.append((self.name, self.e0, e1))
        return False


# Pair-buffer capacity per (device, B, G, H, W), from the pair counts of
# earlier calls: binning then needs no host read of N before the compositors
# are enqueued.
_capacity: dict = {}

# Largest pair count the pair sort takes (radix_size_ok in radix_sort.hip).
MAX_PAIRS = 1 << 29


def _headroom(n: int) -> int:
    """Capacity remembered for a shape whose last count was n: 25% + 4096 of
    headroom, but never above the sort's limit when n itself fits it (a
    larger capacity would make every later call of the shape fail)."""
    cap = n + n // 4 + 4096
    return min(cap, MAX_PAIRS) if n <= MAX_PAIRS else cap


@dataclass
class BinState:
    perm: Optional[Tensor]          # int32 [BG]  depth rank -> original index within image
    packed: Tensor                  # float32 [BG, 12]  packed records in gid order
    splat_offsets: Optional[Tensor] # int32 [BG+1]
    tile_offsets: Tensor            # int32 [T+1]
    pairs: Tensor                   # int32 [capacity]; the first N entries are the binned gids
    capacity: int                   # pair capacity the buffers and workspaces were sized for
    _n_host: Optional[Tensor] = None                 # pinned int32: N at _n_index once _n_ready completes
    _n_ready: Optional[object] = None                 # torch.cuda.Event or _ReportReady (synchronize())
    _n: Optional[int] = None
    _key: Optional[tuple] = None
    _n_index: tuple = (0,)
    _status_host: Optional[Tensor] = None            # pinned int32: the status at _status_index
    _status_index: tuple = (0,)
    _status_ready: Optional[object] = None
    _ring: Optional["_DeviceBinState"] = None        # owner of the pinned words (fast path)
    _generation: int = 0
    _long_index: Optional[tuple] = None              # where _n_host holds the long-range flag

    def _words_current(self) -> bool:
        """False if the pinned ring slot has been reused by later binnings."""
        return self._ring is None or self._ring.calls - self._generation < self._ring.RING

    @property
    def n_pairs(self) -> int:
        """The pair count N (waits for the transfer that carries it)."""
        if self._n is None:
            self._n_ready.synchronize()
            if not self._words_current():
                raise RuntimeError("binning state read after its pinned slot was reused")
            self._n = int(self._n_host[self._n_index])
        return self._n

    def confirm(self) -> bool:
        """True if all N pairs fit in the buffers.  Otherwise the binning holds only the first
        `capacity` pairs and must be redone; the capacity for this shape has then been raised, so
        binning the same inputs again fits.  Raises if N overflowed int32."""
        n = self.n_pairs
        self.check_status()
        if n < 0:
            raise RuntimeError("pair count overflowed int32")
        if self._key is not None:
            cap = _capacity.get(self._key, 0)
            if n > cap or 2 * _headroom(n) < cap:
                _capacity[self._key] = _headroom(n)
        return n <= self.capacity

    @property
    def long_tiles(self) -> bool:
        """Whether some tile range is longer than HANDOFF_PAIRS pairs (the forward then hands tiles
        to its continuation); True when the binning did not report it.  Waits like n_pairs."""
        if self._long_index is None:
            return True
        self.n_pairs  # the transfer that carries N carries the flag too
        if not self._words_current():
            return True
        return bool(self._n_host[self._long_index])

    def check_status(self) -> None:
        """Raises RuntimeError if a look-back wait of this binning gave up (its tile ranges are then
        all empty).  Waits for the transfer that carries the status; a no-op once read."""
        if self._status_ready is None:
            return
        self._status_ready.synchronize()
        if not self._words_current():
            return  # the slot was reused; its status can no longer be read
        status = int(self._status_host[self._status_index])
        self._status_ready = None
        if status & _lib.STATUS_LOOKBACK_TIMEOUT:
            raise RuntimeError("binning failed: a decoupled look-back wait gave up (a predecessor workgroup "
                               "did not make progress for ~1 s); the results of this call are invalid")
        if status:
            raise RuntimeError(f"binning failed with device status {status:#x}")

    @property
    def binned_ids(self) -> Tensor:
        """int32 [N] gids grouped by tile, depth order inside each tile."""
        return self.pairs[: self.n_pairs]

    @property
    def num_tiles(self) -> int:
        return self.tile_offsets.numel() - 1

    @property
    def tile_counts(self) -> Tensor:
        """int32 [T] pairs per tile (computed on demand; the compositors use the offsets)."""
        return self.tile_offsets[1:] - self.tile_offsets[:-1]


def _empty(n, dtype, device):
    return torch.empty((n,), dtype=dtype, device=device)


_side_streams: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for the per-splat count,
    which runs concurrently with the depth sort."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    st = _side_streams.get(key)
    if st is None:
        st = torch.cuda.Stream(device=device)
        _side_streams[key] = st
    return st


def bin_gaussians(meta: _lib.RasterMeta, means2d: Tensor, conics: Tensor, colors: Tensor,
                  opacities: Tensor, depths: Tensor, *, defer_check: bool = False) -> BinState:
    """Tile binning + stable depth order + record packing + pair sort + tile ranges.

    Inputs are flat contiguous fp32 [BG,2], [BG,3], [BG,3], [BG], [BG] in the
    original splat order.  The per-splat tile-hit count runs on a side stream
    while the depth sort runs on the caller's stream; packing waits for both.
    The pair count N is copied to pinned memory right after the count.  The
    pair buffers are sized from earlier calls of the same shape; the first call
    reads N before emitting (like the reference's tile_offsets[-1] read,
    variants/v8/csrc/metal/gsplat_metal.mm:188).  Unless defer_check, N is then
    checked against the capacity (binning again if it did not fit); with
    defer_check the caller must call confirm() (and check_status()) before using the result;
    otherwise both run here."""
    st = _bin(meta, means2d, conics, colors, opacities, depths)
    if not defer_check:
        if not st.confirm():
            st = _bin(meta, means2d, conics, colors, opacities, depths)
            if not st.confirm():
                raise RuntimeError("binning: pair count changed between two binnings of the same inputs")
        st.check_status()
    return st


def bin_and_render(meta: _lib.RasterMeta, flat, *, save_state: bool):
    """Binning then render_forward with the capacity check after the forward is enqueued, so
    that the host never waits on the GPU in between.  Returns (BinState, render_forward outputs);
    the caller runs st.check_status() before the results are relied on.  With the shape's pair
    capacity known, both go through one C-ABI call (gsplat_hip_bin_render_forward) and the
    continuation of long tiles is launched only if the binning reports a tile range longer than
    HANDOFF_PAIRS."""
    dev = flat[0].device
    key = (dev.index, meta.batch, meta.gaussians_per_batch, meta.height, meta.width)
    cap = _capacity.get(key)
    if cap is not None and not _staged():
        st, out, rws = _bin_render_fast(meta, flat, cap, key, save_state)
        if st.confirm():
            if st.long_tiles:
                render_forward_long(meta, st, out, rws)
            return st, out
        st = bin_gaussians(meta, *flat)
        return st, render_forward(meta, st, save_state=save_state)
    st = bin_gaussians(meta, *flat, defer_check=True)
    out = render_forward(meta, st, save_state=save_state)
    if not st.confirm():
        st = bin_gaussians(meta, *flat)
        out = render_forward(meta, st, save_state=save_state)
    return st, out


def _staged() -> bool:
    """True while per-stage timing of the binning or the forward is on: those calls then run one
    by one, each bracketed by its events."""
    return _timing is not None and (_timing_ops is None or
                                    bool(_timing_ops & {"bin_count", "bin_pack", "bin_emit", "render_forward"}))


class _DeviceBinState:
    """Per-device objects reused by every binning call: the two events that order gsplat_hip_bin's
    count stream (re-recording them is safe: a stream wait takes the event's state when it is
    enqueued) and a ring of pinned host words, one row per call, that the device fills with the
    binning's report (N, status, long-range flag, then the ready word)."""
    RING = 1024

    def __init__(self, device: torch.device):
        main = torch.cuda.current_stream(device)
        self.device = device
        self.inputs = torch.cuda.Event()
        self.count = torch.cuda.Event()
        for e in (self.inputs, self.count):
            e.record(main)      # creates the HIP event
        # {N, status, long-range flag, ready} per call, read through a numpy view
        self.ring_t = torch.zeros((self.RING, 4), dtype=torch.int32, pin_memory=True)
        self.ring = self.ring_t.numpy()
        self.ring_base = self.ring_t.data_ptr()
        self.calls = 0

    def slot(self) -> int:
        i = self.calls % self.RING
        self.calls += 1
        return i


class _ReportReady:
    """Host wait for the binning's report in one ring row: the device writes words 0-2 and then
    word 3 = 1, with system-scope stores in that order, so the host reads the row once word 3 is
    set.  The wait polls the pinned word (no HIP event, no stream synchronisation).  A wait that
    lasts over a second synchronises the device instead (which raises if the device failed) and
    then requires the word to be set."""
    __slots__ = ("row", "device")
    POLL_S = 1.0

    def __init__(self, row, device: torch.device):
        self.row = row
        self.device = device

    def synchronize(self) -> None:
        row = self.row
        spins = 0
        limit = None
        while not row[3]:
            spins += 1
            if spins & 4095 == 0:
                now = time.perf_counter()
                if limit is None:
                    limit = now + self.POLL_S
                elif now > limit:
                    torch.cuda.synchronize(self.device)
                    if not row[3]:
                        raise RuntimeError("binning: the device did not write its report to the host words")
                    return


_device_bin: dict = {}


def _bin_fast(meta: _lib.RasterMeta, means2d: Tensor, conics: Tensor, colors: Tensor,
              opacities: Tensor, depths: Tensor, cap: int, key: tuple) -> BinState:
    """All of binning in one C-ABI call (gsplat_hip_bin) with buffers of the known capacity."""
    L = _lib.lib()
    dev = means2d.device
    B, G = meta.batch, meta.gaussians_per_batch
    BG = B * G
    tiles = B * ((meta.height + 15) // 16) * ((meta.width + 15) // 16)
    d = _device_bin.get(dev.index)
    if d is None:
        d = _device_bin[dev.index] = _DeviceBinState(dev)
    perm = _empty(BG, torch.int32, dev)
    packed = torch.empty((BG, _lib.RECORD_FLOATS), dtype=torch.float32, device=dev)
    splat_offsets = _empty(BG + 1, torch.int32, dev)
    tile_offsets = _empty(tiles + 1, torch.int32, dev)
    pairs = _empty(cap, torch.int32, dev)
    ws_bytes = L.gsplat_hip_bin_workspace_bytes(meta, cap)
    ws = _empty(max(ws_bytes, 1), torch.uint8, dev)
    slot = d.slot()
    # The side stream's work (the count) is waited for by the launch stream inside the call, so
    # every later use of these buffers on the launch stream is ordered after it.
    check(L.gsplat_hip_bin(meta, ptr(means2d), ptr(conics), ptr(colors), ptr(opacities), ptr(depths), cap,
                           ptr(perm), ptr(packed), ptr(splat_offsets), ptr(pairs), ptr(tile_offsets),
                           d.ring_base + 16 * slot, ptr(ws), ws_bytes,
                           torch.cuda.current_stream(dev).cuda_stream, _side_stream(dev).cuda_stream,
                           d.inputs.cuda_event, d.count.cuda_event, None),
          "gsplat_hip_bin")
    ready = _ReportReady(d.ring[slot], dev)
    return BinState(perm, packed, splat_offsets, tile_offsets, pairs, cap, d.ring, ready, None, key, (slot, 0),
                    d.ring, (slot, 1), ready, d, d.calls - 1, (slot, 2))


_fast_ws_bytes: dict = {}


def _fast_workspace_bytes(L, meta: _lib.RasterMeta, cap: int, key: tuple, save_state: bool) -> tuple:
    """(binning, render) workspace bytes of the one-call path for a shape key and capacity."""
    k = (key, cap, save_state)
    v = _fast_ws_bytes.get(k)
    if v is None:
        v = (L.gsplat_hip_bin_workspace_bytes(meta, cap),
             L.gsplat_hip_render_workspace_bytes(meta, cap if save_state else 0))
        if len(_fast_ws_bytes) > 256:
            _fast_ws_bytes.clear()
        _fast_ws_bytes[k] = v
    return v


def _bin_render_fast(meta: _lib.RasterMeta, flat, cap: int, key: tuple, save_state: bool):
    """Binning with buffers of the known capacity and the forward in one C-ABI call
    (gsplat_hip_bin_render_forward).  Returns (BinState, render_forward outputs, render workspace);
    the continuation of long tiles is left to the caller."""
    L = _lib.lib()
    means2d, conics, colors, opacities, depths = flat
    dev = means2d.device
    B, G, H, W = meta.batch, meta.gaussians_per_batch, meta.height, meta.width
    BG = B * G
    tiles = B * ((H + 15) // 16) * ((W + 15) // 16)
    d = _device_bin.get(dev.index)
    if d is None:
        d = _device_bin[dev.index] = _DeviceBinState(dev)
    perm = _empty(BG, torch.int32, dev)
    packed = torch.empty((BG, _lib.RECORD_FLOATS), dtype=torch.float32, device=dev)
    splat_offsets = _empty(BG + 1, torch.int32, dev)
    tile_offsets = _empty(tiles + 1, torch.int32, dev)
    pairs = _empty(cap, torch.int32, dev)
    ws_bytes, rws_bytes = _fast_workspace_bytes(L, meta, cap, key, save_state)
    ws = _empty(max(ws_bytes, 1), torch.uint8, dev)
    img = torch.empty((B, H, W, 3), dtype=torch.float32, device=dev)
    final_T = last = tile_stop = None
    if save_state:
        final_T = torch.empty((B, H, W), dtype=torch.float32, device=dev)
        last = torch.empty((B, H, W), dtype=torch.int32, device=dev)
        tile_stop = _empty(tiles, torch.int32, dev)
    rws = _empty(max(rws_bytes, 1), torch.uint8, dev)
    slot = d.slot()
    check(L.gsplat_hip_bin_render_forward(
        meta, ptr(means2d), ptr(conics), ptr(colors), ptr(opacities), ptr(depths), cap, ptr(perm), ptr(packed),
        ptr(splat_offsets), ptr(pairs), ptr(tile_offsets), d.ring_base + 16 * slot, ptr(ws), ws_bytes, ptr(img),
        ptr(final_T), ptr(last), ptr(tile_stop), ptr(rws), rws_bytes,
        torch.cuda.current_stream(dev).cuda_stream, _side_stream(dev).cuda_stream,
        d.inputs.cuda_event, d.count.cuda_event, None), "gsplat_hip_bin_render_forward")
    ready = _ReportReady(d.ring[slot], dev)
    st = BinState(perm, packed, splat_offsets, tile_offsets, pairs, cap, d.ring, ready, None, key, (slot, 0),
                  d.ring, (slot, 1), ready, d, d.calls - 1, (slot, 2))
    return st, (img, final_T, last, tile_stop, (rws if save_state else None)), rws


def _bin(meta: _lib.RasterMeta, means2d: Tensor, conics: Tensor, colors: Tensor,
         opacities: Tensor, depths: Tensor) -> BinState:
    dev = means2d.device
    key = (dev.index, meta.batch, meta.gaussians_per_batch, meta.height, meta.width)
    cap = _capacity.get(key)
    staged = _timing is not None and (_timing_ops is None or
                                      bool(_timing_ops & {"bin_count", "bin_pack", "bin_emit"}))
    if cap is not None and not staged:
        return _bin_fast(meta, means2d, conics, colors, opacities, depths, cap, key)
    L = _lib.lib()
    dev = means2d.device
    B, G = meta.batch, meta.gaussians_per_batch
    BG = B * G
    tiles = B * ((meta.height + 15) // 16) * ((meta.width + 15) // 16)
    perm = _empty(BG, torch.int32, dev)
    packed = torch.empty((BG, _lib.RECORD_FLOATS), dtype=torch.float32, device=dev)
    splat_offsets = _empty(BG + 1, torch.int32, dev)
    tile_offsets = _empty(tiles + 1, torch.int32, dev)
    pair_count = _empty(1, torch.int32, dev)
    ws_bytes = L.gsplat_hip_bin_count_workspace_bytes(meta)
    ws = _empty(max(ws_bytes, 1), torch.uint8, dev)
    n_host = torch.empty((1,), dtype=torch.int32, pin_memory=True)
    main = torch.cuda.current_stream(dev)
    side = _side_stream(dev)
    inputs_ready = torch.cuda.Event()
    inputs_ready.record(main)
    side.wait_event(inputs_ready)
    n_ready = torch.cuda.Event()
    with torch.cuda.stream(side):
        with _timed("bin_count"):
            check(L.gsplat_hip_bin_count(meta, ptr(means2d), ptr(conics), ptr(opacities), ptr(pair_count),
                                         ptr(ws), ws_bytes, side.cuda_stream), "gsplat_hip_bin_count")
        n_host.copy_(pair_count, non_blocking=True)
        n_ready.record(side)
    s = main.cuda_stream
    with _timed("bin_pack"):
        check(L.gsplat_hip_bin_depth_order(meta, ptr(depths), ptr(perm), ptr(ws), ws_bytes, s),
              "gsplat_hip_bin_depth_order")
        main.wait_event(n_ready)
        check(L.gsplat_hip_bin_pack(meta, ptr(means2d), ptr(conics), ptr(colors), ptr(opacities), ptr(perm),
                                    ptr(packed), ptr(splat_offsets), ptr(ws), ws_bytes, s),
              "gsplat_hip_bin_pack")
    n_known = None
    if cap is None:
        # first binning of this shape: size the buffers from N itself
        n_ready.synchronize()
        n_known = int(n_host[0])
        if n_known < 0:
            raise RuntimeError("pair count overflowed int32")
        cap = n_known
    pairs = _empty(cap, torch.int32, dev)
    ws2_bytes = L.gsplat_hip_bin_emit_workspace_bytes(meta, cap)
    ws2 = _empty(max(ws2_bytes, 1), torch.uint8, dev)
    status = _empty(1, torch.int32, dev)
    with _timed("bin_emit"):
        check(L.gsplat_hip_bin_emit(meta, ptr(packed), ptr(splat_offsets), cap, ptr(pairs), None,
                                    ptr(tile_offsets), ptr(status), ptr(ws), ws_bytes, ptr(ws2), ws2_bytes, s),
              "gsplat_hip_bin_emit")
    status_host = torch.empty((1,), dtype=torch.int32, pin_memory=True)
    status_host.copy_(status, non_blocking=True)
    status_ready = torch.cuda.Event()
    status_ready.record(main)
    return BinState(perm, packed, splat_offsets, tile_offsets, pairs, cap, n_host, n_ready, n_known, key, (0,),
                    status_host, (0,), status_ready)


def render_forward(meta: _lib.RasterMeta, st: BinState, *, save_state: bool):
    """Returns (img, final_T, last, tile_stop, workspace); the state tensors are None unless
    save_state.  The workspace lets long tiles be continued by four wavefronts and, with the state,
    holds the segment records the backward reads."""
    L = _lib.lib()
    dev = st.packed.device
    B, H, W = meta.batch, meta.height, meta.width
    tiles = st.num_tiles
    img = torch.empty((B, H, W, 3), dtype=torch.float32, device=dev)
    final_T = last = tile_stop = None
    if save_state:
        final_T = torch.empty((B, H, W), dtype=torch.float32, device=dev)
        last = torch.empty((B, H, W), dtype=torch.int32, device=dev)
        tile_stop = _empty(tiles, torch.int32, dev)
    # the eval forward records no segments: its workspace has no record area
    wsb = L.gsplat_hip_render_workspace_bytes(meta, st.capacity if save_state else 0)
    ws = _empty(max(wsb, 1), torch.uint8, dev)
    with _timed("render_forward"):
        check(L.gsplat_hip_render_forward(meta, ptr(st.packed), ptr(st.tile_offsets), ptr(st.pairs), ptr(img),
                                          ptr(final_T), ptr(last), ptr(tile_stop), st.capacity, ptr(ws), wsb,
                                          stream_of(img)),
              "gsplat_hip_render_forward")
    return img, final_T, last, tile_stop, (ws if save_state else None)


def render_forward_long(meta: _lib.RasterMeta, st: BinState, out, workspace: Tensor) -> None:
    """Continues the tiles that the forward of gsplat_hip_bin_render_forward handed off (out: its
    (img, final_T, last, tile_stop, ...) outputs, workspace: its render workspace)."""
    L = _lib.lib()
    img, final_T, last, tile_stop = out[:4]
    check(L.gsplat_hip_render_forward_long(meta, ptr(st.packed), ptr(st.tile_offsets), ptr(st.pairs), ptr(img),
                                           ptr(final_T), ptr(last), ptr(tile_stop), st.capacity, ptr(workspace),
                                           workspace.numel(), stream_of(img)),
          "gsplat_hip_render_forward_long")


def gradient_buffers(B: int, G: int, device) -> tuple:
    """The four gradient outputs of render_backward, [B,G,2], [B,G,3], [B,G,3], [B,G] (allocated
    ahead, e.g. by the forward before it waits on the binning, to keep them off the path from the
    forward's return to the backward's launch)."""
    return (torch.empty((B, G, 2), dtype=torch.float32, device=device),
            torch.empty((B, G, 3), dtype=torch.float32, device=device),
            torch.empty((B, G, 3), dtype=torch.float32, device=device),
            torch.empty((B, G), dtype=torch.float32, device=device))


def render_backward(meta: _lib.RasterMeta, st: BinState, final_T: Tensor, last: Tensor, tile_stop: Tensor,
                    grad_img: Tensor, workspace: Optional[Tensor] = None, out: Optional[tuple] = None):
    """Returns (g_means2d [B,G,2], g_conics [B,G,3], g_colors [B,G,3], g_opacities [B,G]) in ORIGINAL
    order.  They are allocated in the leaves' batched shapes (not as views of flat buffers) so that
    autograd can hand them to .grad without a copy; out: such buffers from gradient_buffers (written
    in full), or None.  workspace: the one render_forward returned for the same binning (heavy tiles
    are then split into segments), or None."""
    L = _lib.lib()
    dev = st.packed.device
    B, G = meta.batch, meta.gaussians_per_batch
    g_m, g_q, g_c, g_o = out if out is not None else gradient_buffers(B, G, dev)
    grad_img = grad_img.contiguous()
    with _timed("render_backward"):
        check(L.gsplat_hip_render_backward(meta, ptr(st.packed), ptr(st.tile_offsets), ptr(st.pairs),
                                           ptr(final_T), ptr(last), ptr(tile_stop), ptr(grad_img), ptr(g_m), ptr(g_q),
                                           ptr(g_c), ptr(g_o), st.capacity, ptr(workspace),
                                           0 if workspace is None else workspace.numel(), stream_of(grad_img)),
              "gsplat_hip_render_backward")
    return g_m, g_q, g_c, g_o


def project_forward(meta: _lib.ProjectMeta, means3d, scales, quats, opacities, c2w, cam):
    L = _lib.lib()
    dev = means3d.device
    BG = meta.batch * meta.gaussians_per_batch
    m2 = torch.empty((BG, 2), dtype=torch.float32, device=dev)
    cq = torch.empty((BG, 3), dtype=torch.float32, device=dev)
    op = torch.empty((BG,), dtype=torch.float32, device=dev)
    dp = torch.empty((BG,), dtype=torch.float32, device=dev)
    with _timed("project_forward"):
        check(L.gsplat_hip_project_forward(meta, ptr(means3d), ptr(scales), ptr(quats), ptr(opacities), ptr(c2w),
                                           ptr(cam), ptr(m2), ptr(cq), ptr(op), ptr(dp), stream_of(means3d)),
              "gsplat_hip_project_forward")
    return m2, cq, op, dp


def project_backward(meta: _lib.ProjectMeta, g_m2, g_cq, g_op, g_dp, means3d, scales, quats, opacities, c2w, cam):
    L = _lib.lib()
    dev = means3d.device
    B = meta.batch
    BG = B * meta.gaussians_per_batch
    gm3 = torch.empty((BG, 3), dtype=torch.float32, device=dev)
    gs = torch.empty((BG, 3), dtype=torch.float32, device=dev)
    gq = torch.empty((BG, 4), dtype=torch.float32, device=dev)
    go = torch.empty((BG,), dtype=torch.float32, device=dev)
    gc2w = torch.empty((B, 4, 4), dtype=torch.float32, device=dev)
    gcam = torch.empty((B, 4), dtype=torch.float32, device=dev)
    wsb = L.gsplat_hip_project_backward_workspace_bytes(meta)
    ws = _empty(max(wsb, 1), torch.uint8, dev)
    with _timed("project_backward"):
        check(L.gsplat_hip_project_backward(meta, ptr(g_m2), ptr(g_cq), ptr(g_op), ptr(g_dp), ptr(means3d),
                                            ptr(scales), ptr(quats), ptr(opacities), ptr(c2w), ptr(cam), ptr(gm3),
                                            ptr(gs), ptr(gq), ptr(go), ptr(gc2w), ptr(gcam), ptr(ws), wsb,
                                            stream_of(means3d)),
              "gsplat_hip_project_backward")
    return gm3, gs, gq, go, gc2w, gcam


def _raise_on_status(status: Tensor, what: str) -> None:
    """Synchronises on the device status word of a primitive call."""
    v = int(status.item())
    if v:
        raise RuntimeError(f"{what}: device status {v:#x} (a decoupled look-back wait gave up)")


def exclusive_scan_i32(x: Tensor) -> Tensor:
    """out[0..n]: exclusive prefix sum of int32 x with the total at out[n]."""
    L = _lib.lib()
    n = x.numel()
    out = _empty(n + 1, torch.int32, x.device)
    status = _empty(1, torch.int32, x.device)
    wsb = L.gsplat_hip_scan_workspace_bytes(n)
    ws = _empty(max(wsb, 1), torch.uint8, x.device)
    check(L.gsplat_hip_exclusive_scan_i32(ptr(x), ptr(out), n, ptr(status), ptr(ws), wsb, stream_of(x)),
          "gsplat_hip_exclusive_scan_i32")
    _raise_on_status(status, "gsplat_hip_exclusive_scan_i32")
    return out


def radix_sort_pairs_u32(keys: Tensor, vals: Optional[Tensor], *, segments: int = 1, begin_bit: int = 0,
                         end_bit: int = 32):
    """Stable per-segment LSD sort of int32-typed (bit pattern uint32) keys."""
    L = _lib.lib()
    n = keys.numel()
    assert n % segments == 0
    n_seg = n // segments
    ko = torch.empty_like(keys)
    vo = torch.empty((n,), dtype=torch.int32, device=keys.device)
    wsb = L.gsplat_hip_radix_sort_workspace_bytes(n_seg, segments)
    ws = _empty(max(wsb, 1), torch.uint8, keys.device)
    status = _empty(1, torch.int32, keys.device)
    check(L.gsplat_hip_radix_sort_pairs_u32(ptr(keys), ptr(vals), ptr(ko), ptr(vo), n_seg, segments, begin_bit,
                                            end_bit, ptr(status), ptr(ws), wsb, stream_of(keys)),
          "gsplat_hip_radix_sort_pairs_u32")
    _raise_on_status(status, "gsplat_hip_radix_sort_pairs_u32")
    return ko, vo
