"""EXL3 routed experts on MI355X: every expert of every MoE layer has a host record in pinned, device-mapped memory
(read zero-copy over PCIe by the kernels), and a subset also lives in HBM slots (the expert cache). The kernels reach an
expert only through the layer's pointer table, so moving an expert between HBM and host is one 8-byte table entry.

Public API (the reference's plugin/exl3xpu/moe_offload.py:14-30, same names and meaning; device work goes to the
current stream unless a stream is given, and nothing synchronises the host unless noted):

  store = ExpertStore(H, I, K, n_experts, n_slots)       n_slots HBM slots shared by every layer
  store.add_layer(key, blobs)                             host records of a layer ([E, blob] uint8, or filled later)
  store.host_view(key)[e]                                 uint8 view of expert e's host record
  store.ptrs(key)                                         int64 [E] device pointer table of the layer
  store.make_resident(key, experts, stream=None)          copy experts into free slots and repoint them
  store.evict(key, experts)                               repoint to host; the slot is reused in stream order
  store.forward(key, x, topk_ids, topk_w)                 routed-MoE output (routing weights applied)
  store.forward_cached(key, x, topk_ids, topk_w)          decode through the device-managed LRU cache
  store.prefetch / start_copy_prefetch / plan_prefetch / stop_copy_prefetch    predicted experts into slots early
  store.stage_layer(key, buf, stream)                     prefill: stage the layer's non-HBM experts into HBM
  store.forward_prefill_staged(key, x, topk_ids, topk_w)  prefill with the next layer staged on a copy stream
  store.slot_of[key]                                      host mirror of the layer's slot map (int32 [E], -1 = host)
  store.check_device_status()                             raise if a decode kernel's bounded wait timed out (also
                                                          done by forward / forward_cached / prefetch)

Expert blob (blob_bytes(H, I, K) bytes; 1,195,008 for H 2048, I 512, K 3), the reference's format:
  gate|up trellis u32 [H/16][2I/16][8K] | down trellis u32 [I/16][H/16][8K] | fp16 suh_g[H] suh_u[H] svh_g[I] svh_u[I]
  suh_d[I] svh_d[H]; trellis words of odd K in PLANAR4 order (see planar4).
"""
from __future__ import annotations

import ctypes
import heapq
import logging
import os
import re
import threading
from dataclasses import dataclass

import numpy as np
import torch

__all__ = ["ops", "s64", "planar4", "pack_expert", "plan_copies", "BlobLayout", "ExpertStore", "STAGE_VERIFIED_BYTES",
           "staging_fits"]

_HERE = os.path.dirname(os.path.abspath(__file__))
_ops_lock = threading.Lock()
_ops_ns = None
# ops whose meta output is shaped like x (registered for torch.compile / fake tensors)
_X_SHAPED_OPS = ("moe_forward", "moe_forward_cached")

# Staged prefill (copy-stream streaming into HBM staging buffers) has been verified on the GPU with staging buffers of
# up to this many bytes per layer. A full-size run (8,192 tokens x 48 layers, 512 experts of 1.2 MB) ended in a GPU
# memory fault whose cause has not been found (a CPU replay of that sequence found every copy, table entry and stream
# order in bounds), so larger staging is never enqueued: the staged entry points serve such layers through the
# zero-copy route instead (the prefill kernels read non-HBM experts straight from their pinned host records; the
# same blob bytes, so the same output bits), and _Stager itself refuses larger buffers.
STAGE_VERIFIED_BYTES = 2 << 20

log = logging.getLogger("exl3xpu")
_route_logged = set()


def staging_fits(n_experts: int, rec: int) -> bool:
    """True when a layer's staging buffer (n_experts records of rec bytes) is within the GPU-verified size."""
    return int(n_experts) * int(rec) <= STAGE_VERIFIED_BYTES


def _log_zero_copy_route(what: str, nbytes: int) -> None:
    if what not in _route_logged:
        _route_logged.add(what)
        log.warning("exl3xpu: %s: staging buffer of %d B is above the verified %d B; the layer runs zero-copy from "
                    "the pinned host records instead (same output)", what, nbytes, STAGE_VERIFIED_BYTES)


def ops():
    """torch.ops.exl3xpu_moe with _moe.so (or $EXL3_MOE_LIB) loaded on first use (reference ops(),
    moe_offload.py:44-61). Raises RuntimeError when the HIP library is missing: nothing falls back to the CPU."""
    global _ops_ns
    with _ops_lock:
        if _ops_ns is None:
            path = os.environ.get("EXL3_MOE_LIB") or os.path.join(_HERE, "_moe.so")
            if not os.path.isfile(path):
                raise RuntimeError(f"exl3xpu: HIP op library not built ({path}); run "
                                   "qwen38-flash-next-b70-offload_amd/build.py")
            torch.ops.load_library(path)
            for name in _X_SHAPED_OPS:
                torch.library.register_fake(f"exl3xpu_moe::{name}")(lambda x, *rest: torch.empty_like(x))
            _ops_ns = torch.ops.exl3xpu_moe
    return _ops_ns


def s64(p: int) -> int:
    """A 64-bit address as the signed int64 that an int64 tensor element or op argument holds."""
    return ctypes.c_int64(p).value


# ---- blob format ------------------------------------------------------------------------------------------------------

@dataclass(frozen=True)
class BlobLayout:
    """Byte layout of one expert blob (kernels/moe-a8/exl3_moe.a8.sycl:3-13, 42-54)."""
    H: int
    I: int  # noqa: E741
    K: int

    @property
    def words_per_tile(self) -> int:
        return 8 * self.K

    @property
    def fields(self):
        """(name, offset, nbytes) in blob order."""
        H, I, W = self.H, self.I, self.words_per_tile
        sizes = [("gate_up", (H // 16) * (2 * I // 16) * W * 4), ("down", (I // 16) * (H // 16) * W * 4),
                 ("suh_g", 2 * H), ("suh_u", 2 * H), ("svh_g", 2 * I), ("svh_u", 2 * I), ("suh_d", 2 * I),
                 ("svh_d", 2 * H)]
        out, off = [], 0
        for name, n in sizes:
            out.append((name, off, n))
            off += n
        return out

    @property
    def nbytes(self) -> int:
        _, off, n = self.fields[-1]
        return off + n


_planar_index_cache: dict = {}


def _planar4_index(tiles: int, K: int) -> np.ndarray:
    """Source word of every PLANAR4 position within one tile-row of `tiles` tiles (odd K): a group of 4 tiles stores
    its 4 x 8K words plane-major, position (group q, plane i, tile t, period g) <- word g K + i of tile 4 q + t."""
    key = (tiles, K)
    idx = _planar_index_cache.get(key)
    if idx is None:
        q, i, t, g = np.meshgrid(np.arange(tiles // 4), np.arange(K), np.arange(4), np.arange(8), indexing="ij")
        idx = ((4 * q + t) * 8 * K + g * K + i).reshape(-1).astype(np.int64)
        _planar_index_cache[key] = idx
    return idx


def planar4(tr: torch.Tensor, K: int) -> torch.Tensor:
    """Checkpoint trellis int16 [rows, tiles, 16K] -> int32 words in PLANAR4 order (reference moe_offload.py:68-73):
    each tile-row's tiles in groups of 4 whose 4 x 8K words are stored [plane i][tile][period g] rather than
    [tile][period g][plane i]. For even K a period is one word, and PLANAR4 is the natural order."""
    rows, tiles, _ = tr.shape
    words = tr.contiguous().view(torch.int32).reshape(rows, tiles * 8 * K)
    if K % 2 == 0:
        return words.reshape(rows, tiles, 8 * K).contiguous()
    if K not in (1, 3, 5, 7) or tiles % 4:
        raise ValueError(f"planar4: odd K in (1, 3, 5, 7) and a multiple of 4 tiles per row (K={K}, tiles={tiles})")
    idx = torch.from_numpy(_planar4_index(tiles, K))
    return words.index_select(1, idx).reshape(rows, tiles // 4, K, 4, 8).contiguous()


def pack_expert(gate: dict, up: dict, down: dict, K: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """One expert's checkpoint tensors {trellis, suh, svh} -> its blob (uint8 CPU tensor, or written into `out`)
    (reference moe_offload.py:76-89). gate and up trellises are joined along the output (tile-column) axis."""
    H = gate["trellis"].shape[0] * 16
    I = gate["trellis"].shape[1] * 16  # noqa: E741
    lay = BlobLayout(H, I, K)
    if out is None:
        out = torch.empty(lay.nbytes, dtype=torch.uint8)
    elif out.numel() != lay.nbytes:
        raise ValueError(f"pack_expert: out has {out.numel()} bytes, the blob {lay.nbytes}")
    src = {
        "gate_up": planar4(torch.cat([gate["trellis"], up["trellis"]], dim=1), K),
        "down": planar4(down["trellis"], K),
        "suh_g": gate["suh"], "suh_u": up["suh"], "svh_g": gate["svh"], "svh_u": up["svh"],
        "suh_d": down["suh"], "svh_d": down["svh"],
    }
    for name, off, n in lay.fields:
        t = src[name]
        if name not in ("gate_up", "down"):
            t = t.to(torch.float16)
        raw = t.contiguous().view(torch.uint8).reshape(-1)
        if raw.numel() != n:
            raise ValueError(f"pack_expert: {name} has {raw.numel()} bytes, the layout {n}")
        out[off:off + n].copy_(raw)
    return out


# ---- process-wide strides -----------------------------------------------------------------------------------------------

class _Strides:
    """The library's slot and host strides are process-wide (moe_set_slot_stride / moe_set_host_stride, the
    reference's globals a8:765). Each store states its own before every call that uses them, so stores of different
    geometry can alternate; a HIP graph keeps the values it was captured with."""
    lock = threading.Lock()
    slot = None
    host = None

    @classmethod
    def use(cls, X, slot: int, host: int) -> None:
        with cls.lock:
            if cls.slot != slot:
                X.moe_set_slot_stride(slot)
                cls.slot = slot
            if cls.host != host:
                X.moe_set_host_stride(host)
                cls.host = host


def _capi():
    from . import capi
    return capi


def _stream_handle(stream) -> int:
    return int(stream.cuda_stream)


# ---- device health ---------------------------------------------------------------------------------------------------------

class _StatusWatch:
    """Watches the host mirror of the decode kernels' timeout count (exl3_set_status_mirror): a word of pinned host
    memory that the device raises whenever a bounded wait gives up, so that an output was computed from incomplete
    data. check() reads that word (host memory: no copy, no synchronisation, nothing enqueued) and raises
    RuntimeError when it moved since the previous check."""

    def __init__(self, word):
        self.word = word                                # int32 CPU view of the mirror, [>= 1]
        self.seen = int(word[0])

    def check(self, what: str = "exl3xpu") -> None:
        v = int(self.word[0])
        if v != self.seen:
            n, self.seen = v - self.seen, v
            raise RuntimeError(f"{what}: {n} bounded waits of the decode kernels timed out on the device since the "
                               "last check (an output was computed from incomplete data); the device state is not "
                               "trustworthy")


_mirror_lock = threading.Lock()
_mirrors: dict = {}


def _status_mirror(dev) -> torch.Tensor:
    """The pinned timeout-count mirror of `dev`, set up (and registered with the library) on first use."""
    idx = torch.device(dev).index
    idx = torch.cuda.current_device() if idx is None else idx
    with _mirror_lock:
        t = _mirrors.get(idx)
        if t is None:
            t = ops().host_alloc(16).view(torch.int32)
            t.zero_()
            capi = _capi()
            with torch.cuda.device(idx):
                capi.check(capi.lib().exl3_set_status_mirror(t.data_ptr()), "status mirror")
            _mirrors[idx] = t
    return t


# ---- HBM slots -----------------------------------------------------------------------------------------------------------

class _SlotPool:
    """Free HBM slots, lowest index first. A slot released by evict() carries the event recorded after the work that
    could still read it; whoever takes the slot orders its copy after that event."""

    def __init__(self, n: int):
        self.owner = np.full(n, -1, dtype=np.int64)        # key (layer row * E + e) or -1
        self._heap = list(range(n))
        self._release = {}

    def __len__(self) -> int:
        return len(self._heap)

    def free_list(self) -> list:
        return sorted(self._heap)

    def take(self, n: int):
        if n > len(self._heap):
            raise RuntimeError("ExpertStore: no free slot (evict first or raise n_slots)")
        slots = [heapq.heappop(self._heap) for _ in range(n)]
        events = {id(ev): ev for ev in (self._release.pop(s, None) for s in slots) if ev is not None}
        return slots, list(events.values())

    def give(self, slots, event) -> None:
        for s in slots:
            self.owner[s] = -1
            self._release[s] = event
            heapq.heappush(self._heap, s)

    def reset(self) -> None:
        self.owner[:] = -1
        self._heap = list(range(len(self.owner)))
        self._release.clear()

    def rebuild(self, slot_key: np.ndarray) -> None:
        self.owner[:] = slot_key
        self._heap = np.nonzero(slot_key < 0)[0].tolist()
        heapq.heapify(self._heap)
        self._release.clear()


@dataclass
class _HostRecords:
    """Where a layer's experts live in host memory: record e at base + e * stride, inside [lo, hi)."""
    base: int
    stride: int
    lo: int
    hi: int
    view: torch.Tensor | None          # uint8 [E, >= blob] CPU view of the records (None: not addressable here)

    def addr(self, e) -> np.ndarray:
        return self.base + np.asarray(e, dtype=np.int64) * self.stride


# ---- staging (prefill streaming) --------------------------------------------------------------------------------------------

def plan_copies(dst_base: int, rec: int, src_addr, missing):
    """Copies that stage experts `missing` (ascending) into a buffer of records of `rec` bytes at dst_base, from host
    records at src_addr[e]: one (dst, src, nbytes) per run of consecutive experts whose host records are also
    consecutive at `rec` bytes; returns three int64 arrays."""
    m = np.asarray(missing, dtype=np.int64)
    if m.size == 0:
        z = np.zeros(0, dtype=np.int64)
        return z, z, z
    src = np.asarray(src_addr, dtype=np.int64)[m]
    new_run = np.ones(m.size, dtype=bool)
    new_run[1:] = (np.diff(m) != 1) | (np.diff(src) != rec)
    starts = np.nonzero(new_run)[0]
    lengths = np.diff(np.append(starts, m.size))
    return dst_base + m[starts] * rec, src[starts], lengths * rec


class _Stager:
    """Two HBM staging buffers of E records of `rec` bytes, filled from host records on a dedicated copy stream.
    A buffer's fill waits for the event after the last kernel that read it (release()); the consumer waits for the
    fill's event. Copies of consecutive experts whose host records are contiguous are merged, and every copy is
    bounds-checked by the library before anything is enqueued."""

    def __init__(self, dev, E: int, rec: int):
        if not staging_fits(E, rec):
            raise RuntimeError(
                f"exl3xpu: staged prefill with {E} x {rec} B staging buffers is disabled: a full-size staged run "
                f"faulted the GPU and its cause has not been found; staging has been verified up to "
                f"{STAGE_VERIFIED_BYTES} B per buffer. Use ensure_for_prefill + forward (zero-copy) instead")
        self.dev, self.E, self.rec = dev, E, rec
        self.stream = torch.cuda.Stream(dev)
        self._buf = [None, None]
        self._released = [None, None]
        self.bytes = 0
        self.copies = 0

    def base(self, b: int) -> int:
        if self._buf[b] is None:
            self._buf[b] = torch.empty(self.E * self.rec, dtype=torch.uint8, device=self.dev)
        return self._buf[b].data_ptr()

    def bounds(self, b: int):
        lo = self.base(b)
        return lo, lo + self.E * self.rec

    def plan(self, b: int, src_addr: np.ndarray, missing: np.ndarray):
        """(dst, src, nbytes) arrays of the copies that stage experts `missing` (ascending) into buffer b."""
        return plan_copies(self.base(b), self.rec, src_addr, missing)

    def fill(self, b: int, src_addr: np.ndarray, missing: np.ndarray, src_lo: int, src_hi: int):
        """Enqueue the copies on the copy stream; returns the event that marks them done."""
        dst, src, nb = self.plan(b, src_addr, missing)
        lo, hi = self.bounds(b)
        capi = _capi()
        with torch.cuda.stream(self.stream):
            if self._released[b] is not None:
                self.stream.wait_event(self._released[b])
                self._released[b] = None
            if dst.size:
                arr = lambda a: (ctypes.c_void_p * a.size)(*[int(v) for v in a])     # noqa: E731
                capi.check(capi.lib().exl3_copy_batch(arr(dst), arr(src), (ctypes.c_int64 * nb.size)(*nb.tolist()),
                                                      dst.size, lo, hi, src_lo, src_hi, _stream_handle(self.stream)),
                           "staging copies")
            ready = torch.cuda.Event()
            ready.record(self.stream)
        self.bytes += int(nb.sum())
        self.copies += int(nb.size)
        return ready

    def table(self, b: int, slot_of: np.ndarray, slot_base: int, slot_stride: int) -> torch.Tensor:
        """Pointer table: the HBM slot of a resident expert, else its record in staging buffer b."""
        so = np.asarray(slot_of, dtype=np.int64)
        staged = self.base(b) + np.arange(self.E, dtype=np.int64) * self.rec
        t = np.where(so >= 0, slot_base + np.maximum(so, 0) * slot_stride, staged)
        return torch.from_numpy(t).to(self.dev)

    def release(self, b: int, stream) -> None:
        ev = torch.cuda.Event()
        ev.record(stream)
        self._released[b] = ev


_LAYER_NO = re.compile(r"layers\.(\d+)\.")


class _PrefillPipeline:
    """forward_prefill_staged's schedule: layers in model order (the number in "layers.N." keys, else registration
    order; "mtp." layers are staged on demand only). A layer's experts are staged into one buffer while the previous
    layer computes from the other; after each layer the next one in order is staged, wrapping to the first so that
    chunked prefill runs forwards back to back."""

    def __init__(self, store: "ExpertStore"):
        self.st = store
        self.stager = _Stager(store.dev, store.E, store._records_stride())
        self.ready = {}                 # key -> (buffer, table, event)
        self.tick = None
        self._order_n = -1
        self.order = []

    def _layers(self):
        idx = self.st.layer_index
        if self._order_n != len(idx):
            num = {k: (int(m.group(1)) if (m := _LAYER_NO.search(str(k))) else idx[k]) for k in idx}
            self.order = sorted((k for k in idx if not str(k).startswith("mtp.")), key=lambda k: (num[k], idx[k]))
            self._order_n = len(idx)
        return self.order

    def reset(self) -> None:
        self.ready.clear()

    def _stage(self, key, b: int) -> None:
        for k in [k for k, v in self.ready.items() if v[0] == b]:
            del self.ready[k]           # an unconsumed staging in this buffer is overwritten
        st = self.st
        st._refresh_mirror()
        so = st.slot_of[key].numpy()
        rec = st._host[key]
        missing = np.nonzero(so < 0)[0]
        ev = self.stager.fill(b, rec.addr(np.arange(st.E)), missing, rec.lo, rec.hi)
        self.ready[key] = (b, self.stager.table(b, so, st.slot_base, st.slot_stride), ev)

    def run(self, key, x, topk_ids, topk_w):
        st, order = self.st, self._layers()
        cs = torch.cuda.current_stream(st.dev)
        if order and key == order[0]:
            # start of a forward: decode replays may have moved the cache since the last staging (no Python runs
            # inside a graph replay), so the staged tables are dropped if the tick moved
            torch.cuda.synchronize(st.dev)
            t = int(st.tick.item())
            if t != self.tick or st._mirror_stale:
                st.sync_mirror()
                self.ready.clear()
                self.tick = t
        if key not in self.ready:
            busy = {v[0] for v in self.ready.values()}
            self._stage(key, 1 if 0 in busy else 0)
        b, table, ev = self.ready.pop(key)
        cs.wait_event(ev)
        y = st.forward(key, x, topk_ids, topk_w, ptrs=table)
        self.stager.release(b, cs)
        if key in order:
            nxt = order[(order.index(key) + 1) % len(order)]
            if nxt != key and nxt not in self.ready:
                self._stage(nxt, 1 - b)
        return y


# ---- the store ---------------------------------------------------------------------------------------------------------------

class ExpertStore:
    """HBM slot arena + host expert records + the device cache state (reference ExpertStore, moe_offload.py:92-485)."""

    _own_host_arrays = True            # one host allocation per layer, listed in `host` (a TierStore has one arena)

    def __init__(self, H: int, I: int, K: int, n_experts: int, n_slots: int, device=None,  # noqa: E741
                 max_layers: int = 64):
        self.H, self.I, self.K, self.E = H, I, K, n_experts
        self.dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.X = ops()
        self.blob = int(self.X.blob_bytes(H, I, K))
        self.n_slots, self.max_layers = int(n_slots), int(max_layers)
        self.slot_stride = self.blob                    # bytes between slots (mixed_bitrates raises it)
        self._slot_stride_arg = 0                       # the library's slot stride (0: the blob of the call)
        self.slots = (torch.empty((self.n_slots, self.blob), dtype=torch.uint8, device=self.dev)
                      if self.n_slots else None)
        self.slot_base = s64(self.slots.data_ptr()) if self.n_slots else 0
        self._pool = _SlotPool(self.n_slots)
        self.layer_index: dict = {}                     # key -> row of the device tables
        self.host: dict = {}                            # key -> uint8 [E, blob] host records (CPU view)
        self.slot_of: dict = {}                         # key -> int32 [E] host mirror of the slot map
        self.K_of: dict = {}                            # key -> bitrate of the layer when it differs from K
        self._host: dict = {}                           # key -> _HostRecords
        self._mirror_stale = False                      # the device cache moved since the mirror was built
        self._pipeline = None
        n = self.max_layers * self.E
        d = self.dev
        # device cache state (authoritative for forward_cached; moe_offload.py:110-123)
        self.ptrs_all = torch.zeros(n, dtype=torch.int64, device=d)
        self.slot_of_dev = torch.full((n,), -1, dtype=torch.int32, device=d)
        self.slot_key = torch.full((self.n_slots,), -1, dtype=torch.int32, device=d)
        self.slot_last = torch.full((self.n_slots,), -1, dtype=torch.int32, device=d)
        self.tick = torch.zeros(1, dtype=torch.int32, device=d)
        self.host_base = torch.zeros(self.max_layers, dtype=torch.int64, device=d)
        self.fill_all = torch.zeros(n, dtype=torch.int64, device=d)
        self.fill_list = torch.zeros(1 + self.E, dtype=torch.int32, device=d)
        self.pf_list = torch.zeros(1 + self.E, dtype=torch.int32, device=d)
        self.pf_slot = torch.zeros(self.E, dtype=torch.int32, device=d)
        self.pend = torch.zeros(self.max_layers * 35, dtype=torch.int32, device=d)
        self.done_seq = torch.zeros(0, dtype=torch.int32, device=d)
        self._watch = _StatusWatch(_status_mirror(d))

    # ---- geometry and strides
    def _host_stride(self) -> int:
        """The library's host stride (0: host records at the slot stride)."""
        return 0

    def _records_stride(self) -> int:
        return self._host_stride() or self.slot_stride

    def _bind_strides(self) -> None:
        _Strides.use(self.X, self._slot_stride_arg, self._host_stride())

    def mixed_bitrates(self) -> None:
        """Layers of this store use bitrates K <= the store's K: every slot (and host record) keeps the size of the
        largest blob and the device cache addresses slots at that stride; smaller layers read and write their own
        blob bytes, victims are written back as whole slots."""
        self._slot_stride_arg = self.blob

    def k_of(self, key) -> int:
        return self.K_of.get(key, self.K)

    @property
    def free_slots(self) -> list:
        return self._pool.free_list()

    # ---- layers
    def _new_records(self, li: int, blobs) -> _HostRecords:
        view = self.X.host_alloc(self.E * self.blob).view(self.E, self.blob)
        if blobs is not None:
            view.copy_(blobs)
        base = view.data_ptr()
        return _HostRecords(base, self.blob, base, base + self.E * self.blob, view)

    def add_layer(self, key, blobs: torch.Tensor | None = None):
        li = len(self.layer_index)
        if li >= self.max_layers:
            raise RuntimeError(f"ExpertStore: more than max_layers={self.max_layers} MoE layers")
        rec = self._new_records(li, blobs)
        self.layer_index[key] = li
        self._host[key] = rec
        if self._own_host_arrays:
            self.host[key] = rec.view
        self.ptrs_all[li * self.E:(li + 1) * self.E].copy_(torch.from_numpy(rec.addr(np.arange(self.E))))
        self.host_base[li] = s64(rec.base)
        self.slot_of[key] = torch.full((self.E,), -1, dtype=torch.int32)
        return self.host.get(key)

    def host_view(self, key) -> torch.Tensor:
        return self._host[key].view

    def ptrs(self, key) -> torch.Tensor:
        li = self.layer_index[key]
        return self.ptrs_all[li * self.E:(li + 1) * self.E]

    def slot_ptr(self, s: int) -> int:
        return self.slot_base + s * self.slot_stride

    # ---- static residency (load time and host-driven policies; moe_offload.py:154-216)
    def make_resident(self, key, experts, stream=None) -> int:
        """Copy experts of `key` into free slots, then repoint them; copies and table update are ordered on `stream`
        (default: the current stream). Returns the number copied."""
        s_ = stream or torch.cuda.current_stream(self.dev)
        self._refresh_mirror()
        so = self.slot_of[key]
        todo = [e for e in dict.fromkeys(int(e) for e in experts) if int(so[e]) < 0]
        if not todo:
            return 0
        slots, waits = self._pool.take(len(todo))
        li, rec = self.layer_index[key], self._host[key]
        es = np.asarray(todo, dtype=np.int64)
        sl = np.asarray(slots, dtype=np.int64)
        dst = self.slot_base + sl * self.slot_stride
        capi = _capi()
        h = _stream_handle(s_)
        with torch.cuda.stream(s_):
            for ev in waits:
                s_.wait_event(ev)
            arr = lambda a: (ctypes.c_void_p * a.size)(*[int(v) for v in a])     # noqa: E731
            capi.check(capi.lib().exl3_copy_batch(
                arr(dst), arr(rec.addr(es)), (ctypes.c_int64 * es.size)(*([self.blob] * es.size)), es.size,
                self.slot_base, self.slot_base + self.n_slots * self.slot_stride, rec.lo, rec.hi, h), "make_resident")
            self._table_update(li * self.E + es, sl, dst, h)
        for e, s in zip(todo, slots):
            so[e] = s
            self._pool.owner[s] = li * self.E + e
        return len(todo)

    def evict(self, key, experts) -> None:
        """Repoint experts of `key` to their host records; their slots are reused only after the work already queued
        on the current stream."""
        self._refresh_mirror()
        so = self.slot_of[key]
        es = [e for e in dict.fromkeys(int(e) for e in experts) if int(so[e]) >= 0]
        if not es:
            return
        li, rec = self.layer_index[key], self._host[key]
        e_np = np.asarray(es, dtype=np.int64)
        slots = so[e_np].numpy().astype(np.int64)
        cs = torch.cuda.current_stream(self.dev)
        self._table_update(li * self.E + e_np, -1 - slots, rec.addr(e_np), _stream_handle(cs))
        so[e_np] = -1
        ev = torch.cuda.Event()
        ev.record(cs)
        self._pool.give(slots.tolist(), ev)

    def _table_update(self, keys: np.ndarray, slots: np.ndarray, ptrs: np.ndarray, stream: int) -> None:
        """One launch on `stream` (the current stream) for the records (key, slot or -1 - old slot, pointer). The
        records' device copy is allocated and filled on that stream, so its memory is reused only after the launch."""
        rec = np.ascontiguousarray(np.stack([keys, slots, np.asarray(ptrs, dtype=np.int64)], axis=1))
        rec_d = torch.from_numpy(rec).to(self.dev)
        capi = _capi()
        capi.check(capi.lib().exl3_table_update(self.ptrs_all.data_ptr(), self.slot_of_dev.data_ptr(),
                                                self.slot_key.data_ptr(), self.slot_last.data_ptr(), rec_d.data_ptr(),
                                                len(rec), stream), "table update")

    def resident_count(self, key=None) -> int:
        maps = self.slot_of.values() if key is None else [self.slot_of[key]]
        return int(sum(int((m >= 0).sum()) for m in maps))

    def device_resident_count(self, key) -> int:
        """From the device slot map (synchronises; for metrics and tests)."""
        li = self.layer_index[key]
        return int((self.slot_of_dev[li * self.E:(li + 1) * self.E] >= 0).sum().item())

    # ---- compute (moe_offload.py:228-249)
    @staticmethod
    def _ids32(ids: torch.Tensor) -> torch.Tensor:
        flat = ids.reshape(-1)
        return flat if flat.dtype == torch.int32 and flat.is_contiguous() else flat.contiguous().to(torch.int32)

    @staticmethod
    def _routing(topk_ids: torch.Tensor, topk_w: torch.Tensor):
        """int32 / fp32 contiguous routing as the ops take it; tensors already in that form are passed through, so
        the tier mask's rewrite of masked picks lands in the caller's tensors."""
        ids = topk_ids if topk_ids.dtype == torch.int32 and topk_ids.is_contiguous() else \
            topk_ids.contiguous().to(torch.int32)
        w = topk_w if topk_w.dtype == torch.float32 and topk_w.is_contiguous() else topk_w.contiguous().to(torch.float32)
        return ids, w

    def check_device_status(self) -> None:
        """Raise RuntimeError if a bounded wait of a decode kernel timed out on this store's device since the last
        check. Reads host memory only. forward, forward_cached and prefetch run it before enqueueing anything."""
        self._watch.check("exl3xpu")

    def forward(self, key, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, ptrs=None) -> torch.Tensor:
        self._watch.check("exl3xpu.forward")
        ids, w = self._routing(topk_ids, topk_w)
        return self.X.moe_forward(x, ids, w, self.ptrs(key) if ptrs is None else ptrs, self.I, self.k_of(key), self.E)

    def forward_cached(self, key, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor,
                       max_fill: int | None = None) -> torch.Tensor:
        """Decode through the device-managed LRU cache: hits read their slot, misses read the host record zero-copy
        and are written through into their new slot, committed at the end of the call (no host sync; graph-safe).
        With the RAM tier on, masked picks are rewritten in topk_ids / topk_w when those are int32 / fp32
        contiguous (else in the converted copies)."""
        self._watch.check("exl3xpu.forward_cached")
        ids, w = self._routing(topk_ids, topk_w)
        self._mirror_stale = True
        self._bind_strides()
        return self.X.moe_forward_cached(x, ids, w, self.ptrs_all, self.layer_index[key], self.slot_of_dev,
                                         self.slot_key, self.slot_last, self.tick, self.host_base, self.slot_base,
                                         self.fill_all, self.fill_list, self.E if max_fill is None else int(max_fill),
                                         self.I, self.k_of(key), self.E, self.pend, self.done_seq)

    def prefetch(self, key, ids: torch.Tensor, max_fill: int = 16) -> None:
        """Claim exact-LRU slots for up to max_fill predicted experts `ids` of `key` that are not resident (the tick is
        not advanced, so the last call's slots stay protected), copy them from their host records and repoint the
        table (moe_offload.py:251-262). All on the current stream: run it on a side stream that waited for the
        previous MoE call, and make the compute stream wait for it before the next."""
        if not self.n_slots:
            return
        self._watch.check("exl3xpu.prefetch")
        flat = self._ids32(ids)
        self._mirror_stale = True
        self._bind_strides()
        self.X.moe_prefetch(flat, self.ptrs_all, self.layer_index[key], self.slot_of_dev, self.slot_key,
                            self.slot_last, self.tick, self.host_base, self.slot_base, self.pf_list, self.pf_slot,
                            int(max_fill), self.E, int(self.X.blob_bytes(self.H, self.I, self.k_of(key))))

    # ---- copy-engine prefetch (moe_offload.py:264-302): device plan -> host worker -> copies -> device commit
    def start_copy_prefetch(self) -> None:
        """Start the host worker that copies the experts of published plans into their slots on its own stream; the
        next ensure of a layer (forward_cached or plan_prefetch) commits the plans whose copies finished."""
        n_layers = len(self.layer_index)
        self._plans = self.X.host_alloc(n_layers * (4 + 2 * self.E) * 4)
        self._plans.zero_()
        self._plan_seq = torch.zeros(n_layers, dtype=torch.int32, device=self.dev)
        self.done_seq = torch.zeros(n_layers, dtype=torch.int32, device=self.dev)
        self.pend.zero_()
        self._commit_host = self.X.host_alloc(n_layers * 2 * 4)
        bases = torch.zeros(n_layers, dtype=torch.int64)
        for key, li in self.layer_index.items():
            bases[li] = s64(self._host[key].base)
        torch.cuda.synchronize(self.dev)
        self._bind_strides()
        self._pf_stream = torch.cuda.Stream(self.dev)
        with torch.cuda.stream(self._pf_stream):                # the worker enqueues its copies on this stream
            self.X.moe_prefetch_worker_start(self._plans, bases, self.slot_base, self.blob, self.ptrs_all,
                                             self.slot_last, self._commit_host, self.done_seq, n_layers, self.E)

    def plan_prefetch(self, key, ids: torch.Tensor, max_fill: int = 16) -> None:
        """On the compute stream (for instance right after the previous layer's MoE call): claim and pin slots for up
        to 16 predicted experts of `key` and publish the plan to the worker; the compute stream never waits for the
        copies, and the experts are read from their slots once a later ensure has committed the plan."""
        flat = self._ids32(ids)
        self._mirror_stale = True
        self._bind_strides()
        self.X.moe_prefetch_plan(flat, self.ptrs_all, self.layer_index[key], self.slot_of_dev, self.slot_key,
                                 self.slot_last, self.tick, self.host_base, self.slot_base, self.pf_list, self.pf_slot,
                                 self._plans, self._plan_seq, self.pend, self.done_seq, int(max_fill), self.E,
                                 self.blob)

    def stop_copy_prefetch(self):
        """Stop the worker (its stream drained), commit what finished with one ensure pass that fills nothing, and
        return [plans handled, experts copied]; forward_cached then runs without plan commits."""
        counts = self.X.moe_prefetch_worker_stop()
        if self.done_seq.numel():
            self._commit_pass()
            self.done_seq = torch.zeros(0, dtype=torch.int32, device=self.dev)
        return counts

    def _commit_pass(self) -> None:
        first = next(iter(self.layer_index))
        d = self.dev
        self.forward_cached(first, torch.zeros((1, self.H), dtype=torch.bfloat16, device=d),
                            torch.zeros((1, 1), dtype=torch.int32, device=d),
                            torch.ones((1, 1), dtype=torch.float32, device=d), max_fill=0)
        torch.cuda.synchronize(d)

    # ---- prefill staging (moe_offload.py:305-462)
    def stage_layer(self, key, buf: int, stream) -> torch.Tensor:
        """Copy every non-resident expert of `key` into staging buffer `buf` (0 or 1) on `stream`; returns the
        pointer table (slots for residents, staging otherwise) to pass to forward(ptrs=...) once `stream` has been
        waited on. Uses the host mirror of the slot map (refreshed from the device after cached calls). A staging
        buffer above STAGE_VERIFIED_BYTES is not used: the returned table is then the layer's own (HBM slot, else the
        pinned host record, read zero-copy), with nothing enqueued on `stream`."""
        if not staging_fits(self.E, self._records_stride()):
            _log_zero_copy_route("stage_layer", self.E * self._records_stride())
            return self.ptrs(key).clone()
        if self._pipeline is None:
            self._pipeline = _PrefillPipeline(self)
        stg = self._pipeline.stager
        self._refresh_mirror()
        so = self.slot_of[key].numpy()
        rec = self._host[key]
        src = rec.addr(np.arange(self.E))
        dst, srcs, nb = stg.plan(buf, src, np.nonzero(so < 0)[0])
        lo, hi = stg.bounds(buf)
        capi = _capi()
        arr = lambda a: (ctypes.c_void_p * a.size)(*[int(v) for v in a])     # noqa: E731
        capi.check(capi.lib().exl3_copy_batch(arr(dst), arr(srcs), (ctypes.c_int64 * nb.size)(*nb.tolist()),
                                              dst.size, lo, hi, rec.lo, rec.hi, _stream_handle(stream)),
                   "stage_layer copies")
        return stg.table(buf, so, self.slot_base, self.slot_stride)

    def forward_prefill_staged(self, key, x: torch.Tensor, topk_ids: torch.Tensor,
                               topk_w: torch.Tensor) -> torch.Tensor:
        """Prefill-size MoE for `key` from a staging buffer: its non-resident experts were copied on the copy stream
        (normally while the previous layer computed); the next layer is staged into the other buffer now. With a
        staging buffer above STAGE_VERIFIED_BYTES the layer runs on its own table instead (HBM slot, else the pinned
        host record, read zero-copy by the prefill kernels): the same blob bytes, so the same output."""
        if not staging_fits(self.E, self._records_stride()):
            _log_zero_copy_route("forward_prefill_staged", self.E * self._records_stride())
            return self.forward(key, x, topk_ids, topk_w)
        if self._pipeline is None:
            self._pipeline = _PrefillPipeline(self)
        return self._pipeline.run(key, x, topk_ids, topk_w)

    def prefill_reset(self) -> None:
        """Drop staged layers: their tables hold slot pointers that are valid only until the cache moves."""
        if self._pipeline is not None:
            self._pipeline.reset()

    # ---- host mirror of the slot map
    def reset_cache(self) -> None:
        """Empty every slot and repoint all tables to the host records (waits for the current stream's work)."""
        torch.cuda.current_stream(self.dev).synchronize()
        for key, li in self.layer_index.items():
            self.ptrs_all[li * self.E:(li + 1) * self.E].copy_(
                torch.from_numpy(self._host[key].addr(np.arange(self.E))))
            self.slot_of[key].fill_(-1)
        for t, v in ((self.slot_of_dev, -1), (self.slot_key, -1), (self.slot_last, -1), (self.fill_all, 0),
                     (self.pend, 0), (self.tick, 0)):
            t.fill_(v)
        self._pool.reset()
        self._mirror_stale = False

    def sync_mirror(self) -> None:
        """Rebuild the host mirror (slot_of, slot owners, free slots) from the device cache state (synchronises)."""
        slot_key = self.slot_key.cpu().numpy().astype(np.int64)
        sod = self.slot_of_dev.cpu()
        for key, li in self.layer_index.items():
            self.slot_of[key] = sod[li * self.E:(li + 1) * self.E].clone()
        self._pool.rebuild(slot_key)
        self._mirror_stale = False

    def _refresh_mirror(self) -> None:
        if self._mirror_stale:
            self.sync_mirror()
