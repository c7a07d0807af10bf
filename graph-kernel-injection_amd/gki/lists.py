"""GPU-resident kept-block lists and kernel schedules.

The reference visits every ``(i, j)`` tile and skips it after a per-iteration
int32 gate load (``sparse_triton_kernel.py:283-285, 448-450, 563-565``). Here the
mask is turned once, on the GPU, into int32 lists:

* ``build_block_lists(mask)`` -- CSR (row -> ascending kept columns) and CSC
  (column -> ascending kept rows) of a 0/1 block mask. The CSR order is exactly
  ``mask.nonzero()``.
* ``fwd_schedule`` / ``bwd_schedule`` / ``decode_schedule`` -- the same lists
  over the kernels' fixed tiles (forward 128x64 for 16-bit inputs, 64x64 for
  fp32; backward 64x64; decode 16x64). A mask of any block size is first
  classified per tile by ``gki_tile_mask`` (token-rule aware when causal, so
  tiles with nothing visible are not visited). The backward schedule adds the
  dK/dV work list (``gki_dkdv_items``: long kv-tile walks cut into near-equal
  items whose fp32 partials are summed in order); the decode schedule adds the
  token-exact stream of visible positions.

Schedules are cached per mask content (one build per model, not per layer):
each mask tensor is matched to a content class once, then found by identity.
Building a schedule synchronises the stream once (to size the lists).
"""

from __future__ import annotations

import ctypes

import threading
import weakref
from collections import OrderedDict
from dataclasses import dataclass
from typing import Tuple

import torch

from . import _lib


@dataclass(frozen=True)
class BlockLists:
    """CSR + CSC kept-block lists of an int32 ``[n_rows, n_cols]`` matrix.

    ``row_idx`` / ``col_idx`` are the nnz-long views; ``row_buf`` / ``col_buf``
    their allocations (at least one element), whose addresses the kernels take:
    an empty view reports a null data pointer, which the C ABI rejects, while
    an empty list (nothing kept or visible) is legal and gives zero outputs."""

    row_ptr: torch.Tensor  # [n_rows + 1] int32
    row_idx: torch.Tensor  # [nnz] int32, column | partial << 30
    col_ptr: torch.Tensor  # [n_cols + 1] int32
    col_idx: torch.Tensor  # [nnz] int32, row | partial << 30
    n_rows: int
    n_cols: int
    nnz: int
    row_buf: torch.Tensor  # [max(nnz, 1)]
    col_buf: torch.Tensor  # [max(nnz, 1)]


@dataclass(frozen=True)
class FwdSchedule:
    lists: BlockLists         # CSR used; over fwd tiles (n_qt x n_kt)
    n_qt: int
    key: tuple = ()           # its schedule-cache key (the order tables extend it)


@dataclass(frozen=True)
class BwdSchedule:
    lists: BlockLists         # over 64x64 tiles (n_qt x n_kt)
    items: torch.Tensor       # [n_items, 4] int32 (kv tile, first it, end it, slot | -1)
    n_items: int
    split: torch.Tensor       # [max(n_split, 1), 3] int32 (kv tile, first slot, slots)
    n_split: int
    n_pslots: int             # fp32 partial slots per (b, kv head)
    n_qt: int
    n_kt: int
    dq_order: torch.Tensor    # [n_qt * B * H] int32, the dQ grid's workgroup order


@dataclass(frozen=True)
class DecodeSchedule:
    tiles: torch.Tensor       # [n_tiles] int32 kept kv tiles of q tile 0
    n_tiles: int
    tokens: torch.Tensor      # [n_tokens] int32 visible token positions (| partial << 30)
    n_tokens: int
    # > 0 when the stream is exactly the causal StreamingLLM one of (n_kv, sink,
    # window) -- the sinks, then the last positions any of the n_q rows can see --
    # so the decode can compute it instead of reading the list: the full cache
    # then decodes as a sink + ring cache with ring length n_kv - sink (slot =
    # position). 0 otherwise (custom masks, partial tiles, short caches).
    ring: int = 0


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _lists_of(matrix: torch.Tensor, need_cols: bool = True) -> BlockLists:
    """CSR/CSC of a {0,1,2}-valued int32 device matrix (2 marks partial)."""
    lib = _lib.load()
    n_rows, n_cols = (int(s) for s in matrix.shape)
    dev = matrix.device
    stream = _stream(dev)
    row_cnt = torch.empty(n_rows, dtype=torch.int32, device=dev)
    col_cnt = torch.empty(n_cols, dtype=torch.int32, device=dev)
    row_ptr = torch.empty(n_rows + 1, dtype=torch.int32, device=dev)
    col_ptr = torch.empty(n_cols + 1, dtype=torch.int32, device=dev)
    _lib.check(lib.gki_block_list_counts(matrix.data_ptr(), n_rows, n_cols, row_cnt.data_ptr(),
                                         col_cnt.data_ptr(), row_ptr.data_ptr(), col_ptr.data_ptr(),
                                         stream), "gki_block_list_counts")
    nnz = int(row_ptr[-1].item())  # one sync per (cached) schedule
    row_idx = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)
    col_idx = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)
    _lib.check(lib.gki_block_list_fill(matrix.data_ptr(), n_rows, n_cols, row_ptr.data_ptr(),
                                       col_ptr.data_ptr(), row_idx.data_ptr(),
                                       col_idx.data_ptr() if need_cols else None, stream),
               "gki_block_list_fill")
    return BlockLists(row_ptr, row_idx[:nnz], col_ptr, col_idx[:nnz], n_rows, n_cols, nnz, row_idx,
                      col_idx)


def build_block_lists(block_mask: torch.Tensor) -> BlockLists:
    """Kept-block lists of a block mask, computed by the gfx950 library.

    ``block_mask`` must be a 2-D tensor on a GPU (any integer dtype; non-zero
    means kept). ``row_idx`` equals ``block_mask.nonzero()[:, 1]`` and
    ``col_idx`` equals ``block_mask.t().nonzero()[:, 1]``, bit for bit.
    """
    if block_mask.dim() != 2:
        raise ValueError("block_mask must be 2-D")
    if not block_mask.is_cuda:
        raise ValueError("block_mask must live on a CUDA device")
    m = (block_mask != 0).to(torch.int32).contiguous()
    with torch.cuda.device(m.device):
        return _lists_of(m)


def tile_matrix(mask: torch.Tensor, n_q: int, n_kv: int, block_m: int, block_n: int, tile_m: int,
                tile_n: int, is_causal: bool, sink: int, window: int) -> torch.Tensor:
    """{0, 1, 2} classification of the tile_m x tile_n tiles (see gki_tile_mask)."""
    lib = _lib.load()
    n_qb, n_kb = (int(s) for s in mask.shape)
    n_qt, n_kt = -(-n_q // tile_m), -(-n_kv // tile_n)
    out = torch.empty((n_qt, n_kt), dtype=torch.int32, device=mask.device)
    _lib.check(lib.gki_tile_mask(mask.data_ptr(), n_qb, n_kb, block_m, block_n, n_q, n_kv, tile_m,
                                 tile_n, int(bool(is_causal)), sink, window, out.data_ptr(),
                                 _stream(mask.device)), "gki_tile_mask")
    return out


class _ScheduleCache:
    """Schedules keyed by mask content, resolved once per mask tensor.

    A mask tensor is mapped to a content class once per (tensor, version): on
    later calls the alias table answers by identity (it sits outside the LRU
    and holds the tensors weakly, so every layer's mask buffer stays resolved
    however many layers a model has). An unresolved tensor is compared exactly
    (``torch.equal``) with the representative of each known class of the same
    shape, dtype and device; a match joins that class, otherwise the tensor
    founds a new one. Schedules live in an LRU keyed by (class, schedule key).
    So the per-layer device copies of one injected mask (the FX pass gives
    every ``_triton_attn_i`` its own buffer, which ``.to(device)`` copies
    separately, fx_compiler_pass.py:346-368, 566, 592) share one schedule per
    key, and a steady-state step makes no comparison and no build.

    A representative modified in place (version bump) retires its class and
    the class's schedules. The class table holds each representative strongly,
    so a retired mask's storage cannot be recycled under a live class.
    """

    def __init__(self, capacity: int = 64, max_classes: int = 16) -> None:
        self._sched: "OrderedDict[tuple, object]" = OrderedDict()
        self._classes: "OrderedDict[int, Tuple[torch.Tensor, int, tuple]]" = OrderedDict()
        self._alias: dict = {}       # id(tensor) -> (weakref, version, class id)
        self._next = 0
        self._cap = capacity
        self._max_classes = max_classes
        self._lock = threading.RLock()

    def _drop_class(self, cid: int) -> None:
        self._classes.pop(cid, None)
        for k in [k for k in self._sched if k[0] == cid]:
            del self._sched[k]

    def _forget(self, key: int, ref) -> None:
        with self._lock:
            ent = self._alias.get(key)
            if ent is not None and ent[0] is ref:
                del self._alias[key]

    def _class_of(self, mask: torch.Tensor) -> int:
        ent = self._alias.get(id(mask))
        if ent is not None and ent[0]() is mask and ent[1] == mask._version:
            cls = self._classes.get(ent[2])
            if cls is not None and cls[0]._version == cls[1]:
                self._classes.move_to_end(ent[2])
                return ent[2]
        meta = (tuple(mask.shape), mask.dtype, mask.device)
        found = None
        for cid, (rep, ver, m) in list(self._classes.items()):
            if rep._version != ver:                      # representative changed in place
                self._drop_class(cid)
            elif found is None and m == meta and (rep is mask or torch.equal(rep, mask)):
                found = cid
        if found is None:
            found = self._next
            self._next += 1
            self._classes[found] = (mask, mask._version, meta)
            while len(self._classes) > self._max_classes:
                self._drop_class(next(iter(self._classes)))
        self._classes.move_to_end(found)
        key = id(mask)
        ref = weakref.ref(mask, lambda r, k=key: self._forget(k, r))
        self._alias[key] = (ref, mask._version, found)
        return found

    def get(self, mask: torch.Tensor, key: tuple, build):
        with self._lock:
            full = (self._class_of(mask),) + key
            hit = self._sched.get(full)
            if hit is not None:
                self._sched.move_to_end(full)
                return hit
        value = build()
        # The build's kernels ran on this thread's current stream; a schedule
        # becomes visible to every stream and thread once cached, so it is
        # complete on the device before it is published (builds are rare and
        # already wait once for their list sizes).
        if mask.is_cuda:
            torch.cuda.current_stream(mask.device).synchronize()
        with self._lock:
            self._sched[full] = value
            self._sched.move_to_end(full)
            while len(self._sched) > self._cap:
                self._sched.popitem(last=False)
        return value

    def clear(self) -> None:
        with self._lock:
            self._sched.clear()
            self._classes.clear()
            self._alias.clear()


_CACHE = _ScheduleCache()


def clear_schedule_cache() -> None:
    _CACHE.clear()


def fwd_schedule(mask: torch.Tensor, n_q: int, n_kv: int, block_m: int, block_n: int,
                 is_causal: bool, sink: int, window: int, fp32: bool) -> FwdSchedule:
    """CSR schedule of the prefill forward kernel."""
    ts = _lib.tile_sizes()
    tm = ts["fwd_tile_m_32"] if fp32 else ts["fwd_tile_m_16"]
    tn = ts["tile_n"]

    key = ("fwd", n_q, n_kv, block_m, block_n, tm, tn, bool(is_causal), sink, window)

    def build() -> FwdSchedule:
        tiles = tile_matrix(mask, n_q, n_kv, block_m, block_n, tm, tn, is_causal, sink, window)
        lists = _lists_of(tiles, need_cols=False)
        return FwdSchedule(lists, lists.n_rows, key)

    return _CACHE.get(mask, key, build)


def _grid_order(row_ptr: torch.Tensor, n_qt: int, bh: int, device) -> torch.Tensor:
    """``gki_fwd_order`` over a CSR's q tiles and ``bh`` = B * H heads: each
    XCD's share of (b, h, q tile) units, longest kept-tile list first, as a
    device int32 tensor [n_qt * bh]."""
    lib = _lib.load()
    host = row_ptr.to("cpu").contiguous()
    order = torch.empty(n_qt * bh, dtype=torch.int32)
    _lib.check(lib.gki_fwd_order(host.data_ptr(), n_qt, bh, order.data_ptr()), "gki_fwd_order")
    return order.to(device)


def fwd_order(mask: torch.Tensor, sched: FwdSchedule, bh: int) -> torch.Tensor:
    """Workgroup order of the forward launch over ``bh`` = B * H heads,
    cached with the schedule."""
    return _CACHE.get(mask, sched.key + ("order", bh),
                      lambda: _grid_order(sched.lists.row_ptr, sched.n_qt, bh, mask.device))


def dkdv_items(col_ptr_host: torch.Tensor, group: int, bh_kv: int, max_chunk: int = 0):
    """The dK/dV work list of CSC column pointers (a host int32 tensor):
    (items [n_items, 4], split [max(n_split, 1), 3], n_items, n_split, n_pslots),
    host int32 tensors, from ``gki_dkdv_items`` (items of at most ``max_chunk``
    iterations when positive)."""
    lib = _lib.load()
    ptr = col_ptr_host.to(torch.int32).contiguous()
    n_kt = ptr.numel() - 1
    counts = [ctypes.c_int32() for _ in range(3)]
    refs = [ctypes.addressof(c) for c in counts]
    _lib.check(lib.gki_dkdv_items(ptr.data_ptr(), n_kt, group, bh_kv, max_chunk, None, refs[0], None,
                                  refs[1], refs[2]), "gki_dkdv_items")
    n_items, n_split, _ = (c.value for c in counts)
    items = torch.empty((n_items, 4), dtype=torch.int32)
    split = torch.zeros((max(n_split, 1), 3), dtype=torch.int32)
    _lib.check(lib.gki_dkdv_items(ptr.data_ptr(), n_kt, group, bh_kv, max_chunk, items.data_ptr(),
                                  refs[0], split.data_ptr(), refs[1], refs[2]), "gki_dkdv_items")
    return items, split, counts[0].value, counts[1].value, counts[2].value


def spread_chunk(col_ptr_host: torch.Tensor, group: int, bh_kv: int, target: int) -> int:
    """Iterations per dK/dV work item that spread the column walks over about
    ``target`` items (at least two iterations each) when the ``bh_kv`` x
    columns are fewer than ``target``; 0 (the library's own chunk) otherwise."""
    n_cols = (col_ptr_host.numel() - 1) * bh_kv
    if target <= 0 or n_cols >= target:
        return 0
    total = int(col_ptr_host[-1]) * group * bh_kv
    return max(2, -(-total // target))


def bwd_schedule(mask: torch.Tensor, n_q: int, n_kv: int, block_m: int, block_n: int,
                 is_causal: bool, sink: int, window: int, group: int = 1,
                 bh_kv: int = 1, max_chunk: int = 0, spread_to: int = 0) -> BwdSchedule:
    """CSR + CSC schedules of the dQ and dK/dV kernels (64x64 tiles) and the
    dK/dV work list for ``group`` q heads per kv head over ``bh_kv`` = B * H_kv
    (b, kv head) pairs (items of at most ``max_chunk`` iterations when positive;
    with ``spread_to``, short grids are cut into about that many items, see
    ``spread_chunk``)."""
    ts = _lib.tile_sizes()
    tm, tn = ts["bwd_tile_m"], ts["tile_n"]

    def build() -> BwdSchedule:
        tiles = tile_matrix(mask, n_q, n_kv, block_m, block_n, tm, tn, is_causal, sink, window)
        lists = _lists_of(tiles)
        col_ptr = lists.col_ptr.cpu()
        chunk = max_chunk or spread_chunk(col_ptr, group, bh_kv, spread_to)
        items, split, n_items, n_split, n_pslots = dkdv_items(col_ptr, group, bh_kv, chunk)
        dev = mask.device
        dq_order = _grid_order(lists.row_ptr, lists.n_rows, group * bh_kv, dev)
        return BwdSchedule(lists, items.to(dev), n_items, split.to(dev), n_split, n_pslots,
                           lists.n_rows, lists.n_cols, dq_order)

    key = ("bwd", n_q, n_kv, block_m, block_n, tm, tn, bool(is_causal), sink, window, group, bh_kv,
           max_chunk, spread_to)
    return _CACHE.get(mask, key, build)


def decode_schedule(mask: torch.Tensor, n_q: int, n_kv: int, block_m: int, block_n: int,
                    is_causal: bool, sink: int, window: int) -> DecodeSchedule:
    """Kept kv tiles (64 keys each) of the single decode q tile (n_q rows) and
    the token-exact stream of positions the decode kernel reads."""
    ts = _lib.tile_sizes()
    tm, tn = ts["decode_tile_m"], ts["tile_n"]

    def build() -> DecodeSchedule:
        lib = _lib.load()
        tiles = tile_matrix(mask, n_q, n_kv, block_m, block_n, tm, tn, is_causal, sink, window)
        lists = _lists_of(tiles, need_cols=False)
        tokens = torch.empty(max(lists.nnz * tn, 1), dtype=torch.int32, device=mask.device)
        count = torch.zeros(1, dtype=torch.int32, device=mask.device)
        n_qb, n_kb = (int(s) for s in mask.shape)
        _lib.check(lib.gki_decode_tokens(lists.row_buf.data_ptr(), lists.nnz, n_q, n_kv,
                                         mask.data_ptr(), n_qb, n_kb, block_m, block_n,
                                         int(bool(is_causal)), sink, window, tokens.data_ptr(),
                                         count.data_ptr(), _stream(mask.device)), "gki_decode_tokens")
        n_tokens = int(count.item())
        toks = tokens[:n_tokens]
        ring = 0
        r = n_kv - sink
        if is_causal and n_kv >= n_q and r >= 1 and r >= window + n_q - 1 and n_kv < (1 << 30):
            a, b, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
            _lib.check(lib.gki_rolling_stream(n_kv, n_q, sink, window, r, ctypes.byref(a),
                                              ctypes.byref(b), ctypes.byref(c)), "gki_rolling_stream")
            if c.value == n_tokens:
                arith = torch.cat([torch.arange(a.value, dtype=torch.int32, device=mask.device),
                                   torch.arange(b.value, n_kv, dtype=torch.int32, device=mask.device)])
                if torch.equal(toks, arith):
                    ring = r
        return DecodeSchedule(lists.row_idx, lists.nnz, toks, n_tokens, ring)

    key = ("decode", n_q, n_kv, block_m, block_n, tm, tn, bool(is_causal), sink, window)
    return _CACHE.get(mask, key, build)
