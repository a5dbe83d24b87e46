"""RAM expert tier below the device-managed HBM expert cache (the reference's plugin/exl3xpu/nvtier.py API).

Three tiers: HBM slots (device LRU, write-through on a miss) -> RAM records (one pinned, device-mapped host arena with
a fixed address per expert, read zero-copy by the kernels) -> the expert store (every expert; a fill source: the
packed on-disk expert file, or a seeded synthetic source with a deterministic completion latency in host steps).

Device side (csrc/moe_cache.hip, csrc/exl3_ensure.cuh): a pick whose expert is in neither HBM nor RAM is masked to
(the layer's safe expert, weight 0) and logged in a miss ring; an HBM victim whose RAM copy is not valid is written
back to its record and flagged. Host side, after every decode step (NvTierAsync.step): consume the previous step's
device snapshot, complete fills, admit the most-missed keys into free budget, evict RAM copies of HBM-resident
experts first and then keys older than AGE steps, and upload the changed flags. The arena is never unmapped, so an
evicted record's bytes stay readable until a fill overwrites them; eviction is bookkeeping only.
"""
from __future__ import annotations

import ctypes
import json
import logging
import os
import threading
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from .moe_offload import ExpertStore, _HostRecords, _Stager, _log_zero_copy_route, s64, staging_fits

log = logging.getLogger("exl3xpu")
_REC_ALIGN = 4096


def record_bytes(blob: int) -> int:
    """Size of one expert record on disk and in the RAM arena: the blob rounded up to 4 KiB (direct I/O alignment)."""
    return -(-int(blob) // _REC_ALIGN) * _REC_ALIGN


def _env_int(name: str, default: int) -> int:
    return int(os.environ.get(name, str(default)))


class RecordPool:
    """Pinned, device-mapped host records of one stride, allocated `chunk` records at a time when none is free and
    reused through a free list, so that the RAM tier pins the records it holds (its budget plus a bounded headroom)
    rather than one record per expert (the reference keeps a sparse memfd of every expert and punches the pages of
    evicted ones, nvtier.py:19-53, 109-126). Records are 4 KiB aligned when the stride is (direct I/O)."""

    def __init__(self, X, stride: int, chunk: int = 32):
        self.X, self.stride, self.chunk = X, int(stride), max(1, int(chunk))
        self.arenas = []
        self.free = []                                  # addresses; the last one is taken first
        self.in_use = 0
        self.high = 0

    def _grow(self) -> None:
        a = self.X.host_alloc(self.chunk * self.stride)
        self.arenas.append(a)
        base = a.data_ptr()
        self.free.extend(base + (self.chunk - 1 - i) * self.stride for i in range(self.chunk))

    def take(self, n: int) -> np.ndarray:
        n = int(n)
        while len(self.free) < n:
            self._grow()
        out = np.array(self.free[len(self.free) - n:][::-1], dtype=np.int64)
        del self.free[len(self.free) - n:]
        self.in_use += n
        self.high = max(self.high, self.in_use)
        return out

    def give(self, addrs) -> None:
        a = [int(v) for v in np.asarray(addrs, dtype=np.int64).reshape(-1) if v]
        self.free.extend(a)
        self.in_use -= len(a)

    @property
    def records(self) -> int:
        return len(self.arenas) * self.chunk

    @property
    def pinned_bytes(self) -> int:
        return self.records * self.stride

    def view(self, addr: int, nbytes: int) -> torch.Tensor:
        """CPU uint8 view of nbytes at a record address (tests and tools)."""
        for a in self.arenas:
            lo = a.data_ptr()
            if lo <= addr < lo + a.numel():
                off = addr - lo
                return a[off:off + nbytes]
        raise KeyError(f"RecordPool: {addr:#x} is not a record")


class TierStore(ExpertStore):
    """ExpertStore whose host records sit at fixed-stride addresses of one pinned arena: key li * E + e at
    base + key * stride (the reference maps a sparse 2 MiB-stride memfd, nvtier.py:22-53). The stride defaults to the
    blob rounded up to 4 KiB, the record size of the expert file. Ks: the bitrate of each layer in add_layer order
    when layers differ; slots and records then take the largest blob.

    pool=True: no arena; the RAM tier (NvTierAsync) takes a record from a RecordPool for each key it holds and the
    device tables follow it (host_addr_dev: record of every key, set by the tier; victims are written back into free
    records the tier queues per step). Until a key has a record its table entry points at one zeroed null record.
    The fixed-record paths (make_resident, evict, stage_layer, forward_prefill_staged, the prefetch ops) raise."""

    _own_host_arrays = False

    def __init__(self, H, I, K, E, n_slots, n_layers, stride=None, device=None, Ks=None,  # noqa: E741
                 pool: bool = False, pool_chunk: int = 32):
        self.Ks = [int(k) for k in Ks] if Ks is not None else None
        if self.Ks is not None and len(self.Ks) != n_layers:
            raise ValueError(f"TierStore: {len(self.Ks)} bitrates for {n_layers} layers")
        super().__init__(H, I, max(self.Ks) if self.Ks else K, E, n_slots, device=device, max_layers=n_layers)
        if self.Ks and len(set(self.Ks)) > 1:
            self.mixed_bitrates()
        self.stride = int(stride) if stride else record_bytes(self.blob)
        if self.stride < self.blob or self.stride % 16:
            raise ValueError(f"TierStore: stride {self.stride} must hold a blob ({self.blob} B), 16-byte multiple")
        self.L = n_layers
        if pool:
            self.pool = RecordPool(self.X, self.stride, pool_chunk)
            self.null_record = self.X.host_alloc(self.stride)
            self.null_record.zero_()
            self.base = self.null_record.data_ptr()
            self.size = 0
            n = n_layers * E
            self.rec_of = np.zeros(n, dtype=np.int64)          # host record of every key (0: none)
            self.host_addr_dev = torch.full((n,), s64(self.base), dtype=torch.int64, device=self.dev)
        else:
            self.pool = None
            self.size = n_layers * E * self.stride
            self.arena = self.X.host_alloc(self.size)
            self.base = self.arena.data_ptr()

    def _host_stride(self) -> int:
        return self.stride

    def _new_records(self, li: int, blobs) -> _HostRecords:
        if self.pool is not None:
            if blobs is not None:
                raise ValueError("TierStore(pool=True): records are filled by the tier from its source")
            return _HostRecords(self.base, 0, self.base, self.base + self.stride, None)
        span = self.E * self.stride
        view = self.arena[li * span:(li + 1) * span].view(self.E, self.stride)[:, :self.blob]
        if blobs is not None:
            view.copy_(blobs)
        return _HostRecords(self.base + li * span, self.stride, self.base, self.base + self.size, view)

    def _fixed_records(self, what: str) -> None:
        if self.pool is not None:
            raise RuntimeError(f"TierStore.{what}: needs fixed host records (this store uses the record pool)")

    def make_resident(self, key, experts, stream=None) -> int:
        self._fixed_records("make_resident")
        return super().make_resident(key, experts, stream)

    def evict(self, key, experts) -> None:
        self._fixed_records("evict")
        return super().evict(key, experts)

    def stage_layer(self, key, buf: int, stream):
        self._fixed_records("stage_layer")
        return super().stage_layer(key, buf, stream)

    def forward_prefill_staged(self, key, x, topk_ids, topk_w):
        self._fixed_records("forward_prefill_staged")
        return super().forward_prefill_staged(key, x, topk_ids, topk_w)

    def prefetch(self, key, ids, max_fill: int = 16) -> None:
        self._fixed_records("prefetch")
        return super().prefetch(key, ids, max_fill)

    def start_copy_prefetch(self) -> None:
        self._fixed_records("start_copy_prefetch")
        return super().start_copy_prefetch()

    def reset_cache(self) -> None:
        super().reset_cache()
        if self.pool is not None:                       # tables back to each key's record (or the null record)
            n = self.L * self.E
            self.ptrs_all[:n].copy_(self.host_addr_dev)

    def publish_records(self, keys) -> None:
        """Device side of new records (synchronous callers): host_addr_dev[key] = rec_of[key], and the table entry of
        each key not in an HBM slot, on the current stream."""
        keys = np.asarray(keys, dtype=np.int64).reshape(-1)
        if keys.size == 0:
            return
        k = torch.from_numpy(keys).to(self.dev)
        a = torch.from_numpy(self.rec_of[keys].copy()).to(self.dev)
        self.host_addr_dev[k] = a
        self.ptrs_all[k] = torch.where(self.slot_of_dev[k] < 0, a, self.ptrs_all[k])

    def add_layer(self, key, blobs=None):
        if len(self.layer_index) >= self.L:
            raise RuntimeError(f"TierStore: more than n_layers={self.L} MoE layers")
        li = len(self.layer_index)
        super().add_layer(key, blobs)
        if self.Ks:
            self.K_of[key] = self.Ks[li]
        return None

    def addr(self, key: int) -> int:
        """Host record address of key = layer row * E + e (with the record pool: the record it holds)."""
        if self.pool is not None:
            a = int(self.rec_of[int(key)])
            if not a:
                raise KeyError(f"TierStore: key {key} holds no record")
            return a
        return self.base + int(key) * self.stride


# ---- fill sources ---------------------------------------------------------------------------------------------------------

class SyntheticExpertSource:
    """Seeded stand-in for the expert file: record r holds the blob of synthetic expert r % n_distinct of workload
    `seed`; read(r, dst, room) copies it to a host address (room: bytes writable at dst, at least the blob)."""

    def __init__(self, H, I, K, seed: int, n_distinct: int = 64):  # noqa: E741
        from .synth import expert_blob
        self.n = int(n_distinct)
        self.buf = np.stack([expert_blob(seed, i, H, I, K).numpy() for i in range(self.n)])
        self.blob = int(self.buf.shape[1])
        self.rec = self.blob

    def read(self, rec_index: int, dst: int, room: int | None = None) -> None:
        src = self.buf[rec_index % self.n]
        ctypes.memmove(dst, src.ctypes.data, self.blob)

    def blob_of(self, rec_index: int) -> np.ndarray:
        return self.buf[rec_index % self.n]


class LayeredExpertSource:
    """Fill source for a store whose layers differ in bitrate: record r = layer * E + e comes from sources[layer]."""

    def __init__(self, sources, E: int):
        self.sources, self.E = list(sources), int(E)
        self.blob = max(s.blob for s in self.sources)

    def read(self, rec_index: int, dst: int, room: int | None = None) -> None:
        self.sources[rec_index // self.E].read(rec_index, dst, room)

    def blob_of(self, rec_index: int) -> np.ndarray:
        return self.sources[rec_index // self.E].blob_of(rec_index)


class ExpertFile:
    """The packed expert store on disk (reference serve/pack_store.py:1-90, read by nvtier.py:96-112, 460-486):
    record r = checkpoint layer * E + e, each `rec` = blob rounded up to 4 KiB bytes at offset r * rec, so every
    record can be read with direct I/O into a 4 KiB-aligned buffer. meta (JSON beside the file, or a dict):
    {"blob", "rec", "layers", "experts", "H", "I", "K"}.

    read(r, dst, room) reads record r into host memory at dst, where `room` bytes are writable (default: the blob).
    With O_DIRECT (default where the file system supports it) the whole record goes straight into dst when dst is
    4 KiB aligned, room holds the record and the kernel can pin the memory; otherwise it goes through an aligned
    bounce buffer of this thread and only the blob's bytes are written at dst. Buffered reads without O_DIRECT."""

    def __init__(self, path: str, meta=None, direct: bool | None = None):
        if meta is None:
            meta = os.path.splitext(path)[0] + ".json"
        if isinstance(meta, (str, os.PathLike)):
            with open(meta) as f:
                meta = json.load(f)
        self.meta = dict(meta)
        self.blob, self.rec = int(meta["blob"]), int(meta["rec"])
        if self.rec % _REC_ALIGN or self.rec < self.blob:
            raise ValueError(f"ExpertFile: record size {self.rec} must be a 4 KiB multiple holding the blob")
        self.path = path
        want_direct = direct if direct is not None else _env_int("EXL3_NVTIER_DIRECT", 1) == 1
        self.fd, self.direct = None, False
        if want_direct and hasattr(os, "O_DIRECT"):
            try:
                self.fd = os.open(path, os.O_RDONLY | os.O_DIRECT)
                self.direct = True
            except OSError:
                self.fd = None
        if self.fd is None:
            self.fd = os.open(path, os.O_RDONLY)
        self._tls = threading.local()
        self.reads = 0

    def _bounce(self):
        b = getattr(self._tls, "buf", None)
        if b is None:
            import mmap
            b = mmap.mmap(-1, self.rec)                 # page-aligned anonymous memory
            self._tls.buf = b
            self._tls.addr = ctypes.addressof(ctypes.c_char.from_buffer(b))
        return b, self._tls.addr

    def read(self, rec_index: int, dst: int, room: int | None = None) -> None:
        off = int(rec_index) * self.rec
        if self.direct and dst % _REC_ALIGN == 0 and room is not None and room >= self.rec:
            try:
                n = os.preadv(self.fd, [(ctypes.c_char * self.rec).from_address(dst)], off)
                if n == self.rec:
                    self.reads += 1
                    return
            except OSError:
                pass                                    # memory the kernel cannot pin for direct I/O: bounce
        buf, addr = self._bounce()
        n = os.preadv(self.fd, [buf], off)
        if n != self.rec:
            raise OSError(f"ExpertFile: short read of record {rec_index} ({n} of {self.rec} bytes)")
        ctypes.memmove(dst, addr, self.blob)
        self.reads += 1

    def close(self) -> None:
        if self.fd is not None:
            os.close(self.fd)
            self.fd = None


def write_expert_file(path: str, source, n_layers: int, n_experts: int, H: int, I: int, K: int) -> dict:  # noqa: E741
    """Write the expert file of `source` (records 0 .. n_layers * n_experts - 1) and its JSON meta; returns meta."""
    rec = record_bytes(source.blob)
    zero = bytes(rec - source.blob)
    with open(path, "wb") as f:
        for r in range(n_layers * n_experts):
            f.write(np.ascontiguousarray(source.blob_of(r)).tobytes())
            f.write(zero)
    meta = {"blob": int(source.blob), "rec": rec, "layers": n_layers, "experts": n_experts, "H": H, "I": I, "K": K}
    with open(os.path.splitext(path)[0] + ".json", "w") as f:
        json.dump(meta, f)
    return meta


# ---- the tier ----------------------------------------------------------------------------------------------------------------

class _TierDevice:
    """The tier's device tensors (the reference's moe_set_tier / moe_set_victims globals, nvtier.py:69-87):
    RAM flags, the miss ring, the safe expert per layer and the victim list; attached to the library while the tier
    is open."""

    def __init__(self, dev, n_keys: int, ring_cap: int, n_layers: int, n_experts: int, safe: int):
        self.res = torch.zeros(n_keys, dtype=torch.uint8, device=dev)
        self.ring = torch.zeros(1 + ring_cap, dtype=torch.int32, device=dev)
        self.safe = torch.full((n_layers,), safe, dtype=torch.int32, device=dev)
        self.vict = torch.zeros(1 + 2 * n_experts, dtype=torch.int32, device=dev)
        self.dev = dev

    def attach(self, X, victims: bool) -> None:
        X.moe_set_tier(self.res, self.ring, self.safe)
        X.moe_set_victims(self.vict if victims else torch.zeros(0, dtype=torch.int32, device=self.dev))

    def detach(self, X) -> None:
        none = torch.zeros(0, dtype=torch.int32, device=self.dev)
        X.moe_set_tier(torch.zeros(0, dtype=torch.uint8, device=self.dev), none, none)
        X.moe_set_victims(none)


def _evict_order(over: int, classes, age: np.ndarray) -> np.ndarray:
    """The `over` keys to evict: candidates of class 0 first, then class 1, ...; within a class by ascending age, ties
    by ascending key. `classes` is a list of boolean masks over the keys."""
    if over <= 0:
        return np.zeros(0, dtype=np.int64)
    keys, rank = [], []
    for c, m in enumerate(classes):
        k = np.nonzero(m)[0]
        keys.append(k)
        rank.append(np.full(k.size, c, dtype=np.int64))
    keys, rank = np.concatenate(keys), np.concatenate(rank)
    order = np.lexsort((keys, age[keys], rank))
    return keys[order[:over]].astype(np.int64)


class NvTier:
    """RAM tier base (the reference's NvTier, nvtier.py:56-112): flags, miss ring, safe expert per layer (pinned in
    RAM from the start), fills from the source into the arena, prefill-time fills (ensure_for_prefill), warm-up from
    a routing prior (warm) and tier-mode prefill streaming (stage_forward).

    source: a fill source with read(rec_index, dst) (ExpertFile, SyntheticExpertSource), or the path of an expert
    file (meta: its JSON, default beside it). The RAM budget is ram_budget_bytes // stride records (the reference's
    rule), or budget_records when given. ckpt_layer[li] is the checkpoint layer of store row li (record = that
    layer * E + e)."""

    _pool_ok = False                               # the record pool's queue protocol lives in NvTierAsync.step

    def __init__(self, store: TierStore, source, meta=None, ram_budget_bytes=2 << 30, ring_cap=1 << 16, safe=0,
                 dev=None, ckpt_layer=None, budget_records: int | None = None, latency: int = 8):
        self.st, self.E = store, store.E
        self.pool = store.pool
        if self.pool is not None:
            if not self._pool_ok:
                raise ValueError(f"{type(self).__name__}: a TierStore with the record pool needs NvTierAsync")
            if _env_int("EXL3_NVTIER_NO_VICTIM", 0) == 1:
                raise ValueError("NvTier: the record pool needs victim write-back (EXL3_NVTIER_NO_VICTIM=1 is set)")
        self._own_src = isinstance(source, (str, os.PathLike))   # a file opened here is closed by close()
        self.src = ExpertFile(source, meta) if self._own_src else source
        self.ckpt = np.asarray(ckpt_layer if ckpt_layer is not None else range(store.L), dtype=np.int64)
        self.L = int(self.ckpt.size)
        self.dev = torch.device(dev) if dev is not None else store.dev
        self.blob = store.blob
        self.budget = int(budget_records) if budget_records else max(1, int(ram_budget_bytes // store.stride))
        self.latency = max(1, int(latency))
        n = self.L * self.E
        self._d = _TierDevice(self.dev, n, int(ring_cap), self.L, self.E, int(safe))
        self.res_dev, self.ring, self.safe, self.vict = self._d.res, self._d.ring, self._d.safe, self._d.vict
        self.res = np.zeros(n, dtype=np.uint8)
        self.pinned = {li * self.E + int(safe) for li in range(self.L)}
        self.ring_seen = 0
        self.stats = dict(nvme_reads=0, nvme_ms=0.0, evicts=0, masked=0, steps=0, fill_ms=0.0, ring_overflow=0)
        self._readers = None
        self._streamer = None
        self.fill_many(sorted(self.pinned))
        self.res_dev.copy_(torch.from_numpy(self.res))
        self._d.attach(store.X, victims=_env_int("EXL3_NVTIER_NO_VICTIM", 0) != 1)

    def close(self) -> None:
        """Detach the tier from the library (no masking, no write-back afterwards), stop the reader threads and close
        an expert file the tier opened from a path. The store's strides are the store's and stay as they are."""
        self._d.detach(self.st.X)
        if self._readers is not None:
            self._readers.shutdown(wait=True)
            self._readers = None
        if self._own_src:
            self.src.close()

    # ---- records
    def rec_index(self, key: int) -> int:
        return int(self.ckpt[key // self.E]) * self.E + key % self.E

    def _pool(self) -> ThreadPoolExecutor:
        if self._readers is None:
            self._readers = ThreadPoolExecutor(_env_int("EXL3_NVTIER_FILL_THREADS", 16))
        return self._readers

    def _read(self, key: int) -> None:
        self.src.read(self.rec_index(key), self.st.addr(key), self.st.stride)

    def _fill(self, key: int) -> None:
        self.fill_many([key])

    def fill_many(self, keys) -> None:
        """Read the records of `keys` into the arena (reader threads) and mark them RAM-resident (host books). With
        the record pool, keys without a record take one first and the device tables follow (current stream)."""
        keys = [int(k) for k in keys]
        if not keys:
            return
        if self.pool is not None:
            need = [k for k in keys if not self.st.rec_of[k]]
            if need:
                self.st.rec_of[need] = self.pool.take(len(need))
        t = time.perf_counter()
        if len(keys) < 4:
            for k in keys:
                self._read(k)
        else:
            list(self._pool().map(self._read, keys))
        self.res[keys] = 1
        self.stats["nvme_reads"] += len(keys)
        self.stats["nvme_ms"] += (time.perf_counter() - t) * 1e3
        if self.pool is not None:
            self.st.publish_records(keys)

    def ram_bytes(self) -> int:
        return int(self.res.sum()) * self.st.stride

    def pinned_bytes(self) -> int:
        """Pinned host memory holding expert records: the record pool's chunks, or the whole fixed arena."""
        return self.pool.pinned_bytes if self.pool is not None else self.st.size

    def _flags_changed(self, keys, val: int) -> None:
        """Host-side hook after a synchronous path set device flags of `keys` to val (the device is idle)."""

    def warm(self, keys_ckpt, max_bytes):
        """Fill the RAM tier with the hottest experts of a routing prior (checkpoint keys layer * E + e, hottest
        first) until max_bytes of records are resident (reference nvtier.py:492-509); returns (filled, seconds)."""
        t0 = time.perf_counter()
        kc = np.asarray(list(keys_ckpt), dtype=np.int64)
        row_of = np.full(int(self.ckpt.max()) + 1 if self.ckpt.size else 1, -1, dtype=np.int64)
        row_of[self.ckpt] = np.arange(self.L)
        lay = kc // self.E
        known = (lay >= 0) & (lay < row_of.size)
        rows = np.where(known, row_of[np.clip(lay, 0, row_of.size - 1)], -1)
        keys = (rows * self.E + kc % self.E)[rows >= 0]
        keys = keys[self.res[keys] == 0]
        _, first = np.unique(keys, return_index=True)
        keys = keys[np.sort(first)]                     # distinct, in prior order
        room = max(0, int(max_bytes // self.st.stride) - int(self.res.sum()))
        todo = keys[:room]
        if self.pool is not None and todo.size:
            torch.cuda.synchronize(self.dev)
        self.fill_many(todo)
        if hasattr(self, "age"):
            self.age[todo] = 0
        if todo.size:
            self.res_dev.index_fill_(0, torch.from_numpy(todo.astype(np.int64)).to(self.dev), 1)
            self._flags_changed(todo, 1)
        return int(todo.size), time.perf_counter() - t0

    # ---- prefill
    def ensure_for_prefill(self, li: int, ids) -> int:
        """Make every expert of layer row li that `ids` routes to RAM-resident and flag it on the device, so that the
        prefill kernels read it zero-copy (reference nvtier.py:389-457). The budget holds: over budget, evict first
        the transient (prefill-only) fills, then RAM copies of HBM-resident experts, then the rest, each by ascending
        age with ties by ascending key; never this layer's keys, pinned keys or fills in flight. Synchronous;
        returns the number of records filled."""
        n = self.L * self.E
        if not hasattr(self, "transient"):
            self.transient = np.zeros(n, dtype=bool)
        ids_np = ids.reshape(-1).to("cpu", torch.int64).numpy() if torch.is_tensor(ids) else np.asarray(ids).reshape(-1)
        keys = np.unique(ids_np) + li * self.E
        miss = keys[self.res[keys] == 0]
        pool = self.pool is not None
        ready = set()
        if pool and miss.size:
            # the record pool: the device is idle from here on (records released below are read by nothing), and
            # fills in flight for these keys are finished here instead of at their step
            torch.cuda.synchronize(self.dev)
            ready = self._take_inflight(miss)
        inflight = getattr(self, "inflight", np.zeros(n, dtype=bool))
        over = int(self.res.sum()) + int(inflight.sum()) + miss.size - self.budget
        if miss.size and over > 0:
            torch.cuda.synchronize(self.dev)
            age = getattr(self, "age", np.zeros(n, dtype=np.int64))
            if not pool:
                # victims written back since the last step (with the record pool the step adopts them, when it
                # learns their records)
                back = (self.res_dev.cpu().numpy() == 1) & (self.res == 0)
                self.res[back] = 1
                if hasattr(self, "age"):
                    age[back] = self.tick
            ok = (self.res == 1) & ~inflight
            ok[list(self.pinned)] = False
            ok[keys] = False
            vram = self.st.slot_of_dev[:n].cpu().numpy() >= 0
            ev = _evict_order(over, [ok & self.transient, ok & ~self.transient & vram,
                                     ok & ~self.transient & ~vram], age)
            if ev.size:
                self.res[ev] = 0
                self.transient[ev] = False
                self.res_dev.index_fill_(0, torch.from_numpy(ev).to(self.dev), 0)
                if pool:
                    r = self.st.rec_of[ev]
                    self.pool.give(r[r != 0])
                    self.st.rec_of[ev] = 0
                    self._flags_changed(ev, 0)
            self.stats["prefill_evicts"] = self.stats.get("prefill_evicts", 0) + int(ev.size)
        self.fill_many([k for k in miss.tolist() if k not in ready])
        if ready:
            self.res[sorted(ready)] = 1
            self.st.publish_records(sorted(ready))
        if miss.size:
            if hasattr(self, "inflight"):
                self.inflight[miss] = False
            if hasattr(self, "age"):
                self.age[miss] = self.tick
            self.transient[miss] = True
            self.res_dev.index_fill_(0, torch.from_numpy(miss.astype(np.int64)).to(self.dev), 1)
            self._flags_changed(miss, 1)
        self.stats["prefill_fills"] = self.stats.get("prefill_fills", 0) + int(miss.size)
        return int(miss.size)

    def stage_forward(self, store, key, li: int, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """Prefill-size MoE for layer row li with its non-HBM experts streamed: reader threads read their records into
        a pinned host ring (read-ahead of the following layers), the copy stream moves them into an HBM staging
        buffer, and the layer runs on the table (HBM slot, else staging). The first layer of a forward synchronises
        once and snapshots the slot map (reference nvtier.py:534-640). A staging buffer above STAGE_VERIFIED_BYTES
        is not used: the layer's experts are made RAM-resident (ensure_for_prefill) and the prefill kernels read the
        non-HBM ones zero-copy from their records, which gives the same output."""
        if not staging_fits(self.E, store.stride):
            _log_zero_copy_route("NvTier.stage_forward", self.E * store.stride)
            self.ensure_for_prefill(li, ids)
            return store.forward(key, x, ids, w)
        if self._streamer is None:
            self._streamer = _TierStreamer(self)
        return self._streamer.run(store, key, li, x, ids, w)

    # ---- reporting
    def log_stats(self, logger=None, every=200):
        """Every `every` host steps: per-step rates of masked picks, fills and evictions over the last period, the
        host time per step and the RAM in use (reference nvtier.py:512-526)."""
        steps = self.stats["steps"]
        if not steps or steps % every:
            return
        prev = getattr(self, "_stats_mark", {})
        d = {k: v - prev.get(k, 0) for k, v in self.stats.items() if isinstance(v, (int, float))}
        per = max(1, int(d.get("steps", 0)))
        (logger or log).info(
            "exl3xpu tier: %d steps | per step: masked %.2f, fills %.2f, evictions %.2f, host %.3f ms (waiting %.3f) | "
            "admissions dropped %d | RAM %.2f GiB of %.2f", per, d.get("masked", 0) / per, d.get("nvme_reads", 0) / per,
            d.get("evicts", 0) / per, d.get("fill_ms", 0.0) / per, d.get("wait_ms", 0.0) / per,
            int(d.get("admit_dropped", 0)), self.ram_bytes() / 2 ** 30, self.budget * self.st.stride / 2 ** 30)
        self._stats_mark = dict(self.stats)


class _TierStreamer:
    """Tier-mode prefill streaming: per layer, the records of its non-HBM experts are read by the reader threads into
    one of NB pinned host buffers (NB = EXL3_NVTIER_STAGE_HOSTBUF, default 4: NB - 1 layers of read-ahead), then the
    copy stream moves them into one of the two HBM staging buffers. Layers run in checkpoint order; the first layer of
    a forward (or a layer whose reads were not started) synchronises, snapshots the HBM slot map and restarts the
    read-ahead."""

    def __init__(self, tier: NvTier):
        st = tier.st
        self.tier, self.E, self.rec = tier, tier.E, st.stride
        self.stager = _Stager(tier.dev, tier.E, self.rec)
        self.nb = max(2, _env_int("EXL3_NVTIER_STAGE_HOSTBUF", 4))
        self.host = [st.X.host_alloc(self.E * self.rec) for _ in range(self.nb)]
        self.host_free = [None] * self.nb          # event of the copy that last read host buffer i
        self.order = [int(li) for li in np.argsort(tier.ckpt, kind="stable")]
        self.pos = {li: i for i, li in enumerate(self.order)}
        self.pending = {}                          # layer row -> (host buffer, missing experts, futures)
        self.next_host = 0
        self.next_dev = 0
        self.snap = None                           # host copy of the slot map at the start of the forward

    def _kick(self, li: int) -> None:
        hb = self.next_host
        self.next_host = (hb + 1) % self.nb
        if self.host_free[hb] is not None:
            self.host_free[hb].synchronize()       # the copy that read this buffer NB - 1 layers ago is done
            self.host_free[hb] = None
        missing = np.nonzero(self.snap[li * self.E:(li + 1) * self.E] < 0)[0]
        base, tier = self.host[hb].data_ptr(), self.tier
        chunks = np.array_split(missing, min(8, max(1, missing.size)))

        def read(part):
            for e in part.tolist():
                tier.src.read(tier.rec_index(li * self.E + e), base + e * self.rec, self.rec)
        self.pending[li] = (hb, missing, [tier._pool().submit(read, c) for c in chunks if c.size])

    def _restart(self, pos: int) -> None:
        torch.cuda.synchronize(self.tier.dev)
        self.snap = self.tier.st.slot_of_dev[:self.tier.L * self.E].cpu().numpy()
        for _, _, futs in self.pending.values():
            for f in futs:
                f.result()
        self.pending.clear()
        for q in range(pos, min(pos + self.nb, len(self.order))):
            self._kick(self.order[q])

    def run(self, store, key, li, x, ids, w):
        pos = self.pos[li]
        if pos == 0 or li not in self.pending:
            self._restart(pos)
        hb, missing, futs = self.pending.pop(li)
        for f in futs:
            f.result()
        b = self.next_dev
        self.next_dev ^= 1
        base = self.host[hb].data_ptr()
        src = base + np.arange(self.E, dtype=np.int64) * self.rec
        ready = self.stager.fill(b, src, missing, base, base + self.E * self.rec)
        self.host_free[hb] = ready
        cs = torch.cuda.current_stream(self.tier.dev)
        cs.wait_event(ready)
        table = self.stager.table(b, self.snap[li * self.E:(li + 1) * self.E], store.slot_base, store.slot_stride)
        y = store.forward(key, x, ids, w, ptrs=table)
        self.stager.release(b, cs)
        self.tier.stats["stage_bytes"] = self.tier.stats.get("stage_bytes", 0) + int(missing.size) * self.rec
        nq = pos + self.nb
        if nq < len(self.order) and self.order[nq] not in self.pending:
            self._kick(self.order[nq])
        return y


class NvTierFast(NvTier):
    """Vectorised bookkeeping with background fills (the reference's NvTierFast, nvtier.py:175-278): per-key age,
    in-flight and pinned masks; the fills admitted at host step n are read by worker tasks and become resident at
    host step n + latency (a deterministic completion time in place of wall-clock NVMe reads), or, with
    completion="wallclock" (EXL3_NVTIER_COMPLETION=wallclock), at the first host step after their own read finished:
    each key is read on FIFO queue key % N of N single-reader queues (N = EXL3_NVTIER_DECODE_FILL_QUEUES, default 8;
    the reference's decode-fill queues, nvtier.py:643-693), so the admissions then depend on the disk's timing. With
    the record pool the admitted keys take their records, and their reads start, at the next host step, once the
    records of the keys evicted with them are free again."""

    FILL_CHUNKS = 4

    def __init__(self, *a, completion: str | None = None, **k):
        super().__init__(*a, **k)
        n = self.L * self.E
        self.age = np.zeros(n, dtype=np.int64)
        self.tick = 1
        self.pin_mask = np.zeros(n, dtype=bool)
        self.pin_mask[sorted(self.pinned)] = True
        self.inflight = np.zeros(n, dtype=bool)
        self.completion = completion or os.environ.get("EXL3_NVTIER_COMPLETION", "steps")
        if self.completion not in ("steps", "wallclock"):
            raise ValueError(f"NvTierFast: completion {self.completion!r} is 'steps' or 'wallclock'")
        self._due = {}                              # host step -> [(keys, future)]
        self._fut_of = {}                           # key -> (keys, future) of its started fill
        self._fifos = None                          # wall-clock mode: the decode-fill queues
        self._to_start = []                         # record pool: [(keys, due step)] admitted, not started
        self._hstep = 0

    def _read_keys(self, keys) -> None:
        for key in keys:
            self._read(key)

    def _queue_fills(self, keys, hs: int) -> None:
        """Fills admitted at host step hs: read by workers, resident from host step hs + latency."""
        keys = [int(k) for k in keys]
        if not keys:
            return
        self.stats["nvme_reads"] += len(keys)
        if self.pool is not None:
            self._to_start.append((keys, hs + self.latency))
            return
        self._submit(keys, hs + self.latency)

    def _submit(self, keys, due: int) -> None:
        lst = self._due.setdefault(due, [])
        if self.completion == "wallclock":
            if self._fifos is None:
                self._fifos = [ThreadPoolExecutor(1) for _ in range(max(1, _env_int("EXL3_NVTIER_DECODE_FILL_QUEUES",
                                                                                   8)))]
            for key in keys:
                kl = [int(key)]
                fut = self._fifos[int(key) % len(self._fifos)].submit(self._read, int(key))
                lst.append((kl, fut))
                self._fut_of[int(key)] = (kl, fut)
            return
        for part in np.array_split(np.asarray(keys, dtype=np.int64), min(self.FILL_CHUNKS, len(keys))):
            kl = part.tolist()
            fut = self._pool().submit(self._read_keys, list(kl))
            lst.append((kl, fut))
            for key in kl:
                self._fut_of[key] = (kl, fut)

    def close(self) -> None:
        if self._fifos is not None:
            for q in self._fifos:
                q.shutdown(wait=True)
            self._fifos = None
        super().close()

    def _start_fills(self) -> None:
        """Record pool: the admissions of the previous host step take their records and start their reads."""
        for keys, due in self._to_start:
            keys = [k for k in keys if self.inflight[k]]        # a prefill may have filled some meanwhile
            if keys:
                self.st.rec_of[keys] = self.pool.take(len(keys))
                self._submit(keys, due)
        self._to_start = []

    def _take_inflight(self, keys) -> set:
        """Finish the fills in flight of `keys` now (synchronous paths): admissions not started are dropped from the
        start list, started reads are waited for and leave their step; returns the keys whose record is filled."""
        ks = {int(k) for k in keys if self.inflight[int(k)]}
        if not ks:
            return set()
        rest = []
        for kl, due in self._to_start:
            kl = [k for k in kl if k not in ks]
            if kl:
                rest.append((kl, due))
        self._to_start = rest
        ready = set()
        for key in ks:
            ent = self._fut_of.pop(key, None)
            if ent is not None:
                ent[1].result()
                ent[0].remove(key)
                ready.add(key)
        self.inflight[sorted(ks)] = False
        return ready

    def _completed(self, hs: int) -> list:
        done = []
        if self.completion == "wallclock":
            for d in sorted(self._due):
                keep = []
                for keys, fut in self._due[d]:
                    if fut.done():
                        fut.result()
                        done.extend(keys)
                    else:
                        keep.append((keys, fut))
                if keep:
                    self._due[d] = keep
                else:
                    del self._due[d]
        else:
            for keys, fut in self._due.pop(hs, []):
                fut.result()
                done.extend(keys)
        for key in done:
            self._fut_of.pop(key, None)
        return done


class _AdmitState(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int64) for f in ("n", "budget", "admit_age", "admit_qmax", "ring_cap", "tick",
                                               "ring_seen", "masked", "evicts", "admit_dropped", "ring_overflow")]


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


class AdmissionPolicy:
    """Host books of the admission-controlled tier step (_async_step_admit, nvtier.py:708-806); the decision runs
    natively (exl3_admit_decide in libexl3moe.so) over the numpy books held here.

    decide() consumes the device state of the PREVIOUS step (flags with the previous upload overlaid, miss ring, HBM
    slot map) plus the keys whose fills completed now, and returns (admitted keys, evicted keys, flag diff keys, flag
    diff values). Ordering contract: misses by descending count, ties by ascending key; evictions by ascending age,
    ties by ascending key (the reference's numpy argsort default is not stable)."""

    def __init__(self, n, pinned, budget, age=4, qmax=256, ring_cap=1 << 16):
        from . import capi
        self._lib = capi.lib()
        self.n = int(n)
        self.res = np.zeros(n, dtype=np.uint8)
        self.age = np.zeros(n, dtype=np.int64)
        self.inflight = np.zeros(n, dtype=bool)
        self.pin_mask = np.zeros(n, dtype=bool)
        self.pin_mask[list(pinned)] = True
        self.res[list(pinned)] = 1
        self._st = _AdmitState(n=self.n, budget=int(budget), admit_age=int(age), admit_qmax=int(qmax),
                               ring_cap=int(ring_cap), tick=1)
        self._out = np.empty((3, self.n), dtype=np.int64)
        self._vals = np.empty(self.n, dtype=np.uint8)
        self._cnt = np.zeros(3, dtype=np.int64)

    def _field(name):
        return property(lambda self: int(getattr(self._st, name)),
                        lambda self, v: setattr(self._st, name, int(v)))

    budget = _field("budget")
    admit_age = _field("admit_age")
    admit_qmax = _field("admit_qmax")
    cap = _field("ring_cap")
    tick = _field("tick")
    ring_seen = _field("ring_seen")
    del _field

    @property
    def stats(self):
        st = self._st
        return dict(masked=st.masked, evicts=st.evicts, admit_dropped=st.admit_dropped, ring_overflow=st.ring_overflow)

    def decide(self, view, ring, slot_of, done_keys):
        """view u8 [n], ring i32 [1 + cap], slot_of i32 [n] (>= 0: resident in HBM), done_keys: completed fills."""
        view = np.ascontiguousarray(view, dtype=np.uint8)
        ring = np.ascontiguousarray(ring, dtype=np.int32)
        slot_of = np.ascontiguousarray(slot_of, dtype=np.int32)
        done = np.ascontiguousarray(np.asarray(done_keys, dtype=np.int64).reshape(-1))
        assert view.size == self.n and slot_of.size == self.n and ring.size == self.cap + 1
        c = self._cnt
        cp = _ptr(c)
        rc = self._lib.exl3_admit_decide(ctypes.byref(self._st), _ptr(self.res), _ptr(self.age), _ptr(self.inflight),
                                         _ptr(self.pin_mask), _ptr(view), _ptr(ring), _ptr(slot_of), _ptr(done),
                                         done.size, _ptr(self._out[0]), cp, _ptr(self._out[1]), cp + 8,
                                         _ptr(self._out[2]), _ptr(self._vals), cp + 16)
        if rc != 0:
            raise RuntimeError(f"exl3_admit_decide: error {rc} (corrupt snapshot or bad done key)")
        na, ne, nd = int(c[0]), int(c[1]), int(c[2])
        return (self._out[0, :na].copy(), self._out[1, :ne].copy(), self._out[2, :nd].copy(),
                self._vals[:nd].copy())


class NvTierAsync(NvTierFast):
    """One-step-lagged, event-ordered bookkeeping without a per-step device sync (nvtier.py:282-386) with the
    admission policy (AdmissionPolicy): AGE = EXL3_NVTIER_ADMIT_AGE (default 4), QMAX = EXL3_NVTIER_ADMIT_QMAX
    (default 256). Host step n snapshots the device state after decode step n and acts on the snapshot of step n-1.

    Per step on the stream: one exchange kernel (exl3_tier_exchange) that applies the step's (key, value) flag diff,
    read in place from a pinned double buffer, mirrors the miss-ring entries appended since the last snapshot into a
    pinned ring mirror, and copies the RAM flags, the slot table and the device status words into pinned double
    buffers; no host allocation, no extra synchronisation. A non-zero status (a bounded wait of a decode kernel timed
    out, so an output was computed from incomplete data) raises RuntimeError at the next step.

    With a TierStore(pool=True) the tier pins a RecordPool instead of a record per expert (exl3_tier_exchange_pool):
    every key it holds owns one record; a victim written back takes the next record of the step's write-back queue
    (wb_queue records, EXL3_NVTIER_WB_QUEUE, default 48; the exchange installs the next queue and mirrors what the
    last one gave to which key); the records of evicted keys return to the pool after the exchange that clears their
    flags has run; admitted fills take records at the next step. The pool then holds at most budget + 3 * wb_queue
    records (two queues outstanding and one step of adopted write-backs), rounded up to its chunk. A write-back that
    finds the queue used up is dropped (stats["wb_dropped"]): the victim leaves HBM without a copy and stays masked
    until a fill brings it back.

    victim_ring=K (or EXL3_NVTIER_VICTIM_RING=1 with EXL3_NVTIER_VRING_K, default 128; the reference's
    NvTierAsyncRing, experimental/n111-victim-ring/nvtier.py:655-884): victims go to a ring of K slots in HBM
    (exl3_set_victim_ring) instead of to host memory, and the host drains them. From each snapshot the step takes the
    ring's new claims (a slot whose claim number it has not handled), marks their keys in flight (so that the policy
    neither admits them nor forgets them in the budget, and a miss on them waits for the data that is about to land),
    gives each a record (its fixed record, or one from the pool) and copies the slot there on a side stream once the
    decode step that wrote it has finished. A drain lands at the next host step (completion "steps"; at the first
    step after its copy finished with "wallclock"): the key becomes RAM-resident like a completed fill and its slot
    is freed (key = -1 written on the compute stream before the next decode step). The device never flags a ring
    victim resident and only claims free slots; a full ring drops the write-back (stats["vr_drops"])."""

    _pool_ok = True

    def __init__(self, *a, wb_queue: int | None = None, victim_ring: int | None = None, **k):
        super().__init__(*a, **k)
        from . import capi
        self._capi = capi
        n = self.L * self.E
        self._n = n
        X = self.st.X
        self._h_res = [X.host_alloc(n) for _ in range(2)]
        self._h_ring = X.host_alloc(4 * self.ring.numel()).view(torch.int32)
        self._h_ring.zero_()
        self._ring_from = 0                # ring count (mod 2^32) of the last snapshot read
        self._h_slot = [X.host_alloc(4 * n).view(torch.int32) for _ in range(2)]
        self._h_status = [X.host_alloc(16).view(torch.int32) for _ in range(2)]
        for t in self._h_status:
            t.zero_()
        self._np_res = [t.numpy() for t in self._h_res]
        self._np_ring = self._h_ring.numpy()
        self._np_slot = [t.numpy() for t in self._h_slot]
        self._h_diff = [X.host_alloc(4 * n).view(torch.int32) for _ in range(2)]
        self._np_diff = [t.numpy() for t in self._h_diff]
        self._snap_ev = [torch.cuda.Event(), torch.cuda.Event()]
        dev_status = ctypes.c_void_p()
        capi.check(capi.lib().exl3_device_status_address(ctypes.byref(dev_status)), "device status address")
        self._xargs = []                   # (src, dst, nbytes) ctypes arrays of the snapshot copies per buffer
        for b in range(2):
            copies = ((self.res_dev.data_ptr(), self._h_res[b].data_ptr(), n),
                      (self.st.slot_of_dev.data_ptr(), self._h_slot[b].data_ptr(), 4 * n),
                      (dev_status.value, self._h_status[b].data_ptr(), 16))
            self._xargs.append(((ctypes.c_void_p * 3)(*[c[0] for c in copies]),
                                (ctypes.c_void_p * 3)(*[c[1] for c in copies]),
                                (ctypes.c_int64 * 3)(*[c[2] for c in copies])))
        self._have = [False, False]
        self._k = 0
        self._last_diff = None
        self._view = np.empty(n, dtype=np.uint8)
        self.policy = AdmissionPolicy(n, self.pinned, self.budget, _env_int("EXL3_NVTIER_ADMIT_AGE", 4),
                                      _env_int("EXL3_NVTIER_ADMIT_QMAX", 256), self.ring.numel() - 1)
        self.policy.res[:] = self.res
        self.res = self.policy.res
        self.log_decisions = False
        self.decisions = []                # (admitted keys, evicted keys) per step when log_decisions
        if self.pool is not None:
            self._pool_init(int(wb_queue) if wb_queue else _env_int("EXL3_NVTIER_WB_QUEUE", 48))
        self.vr_K = 0
        if victim_ring is None and _env_int("EXL3_NVTIER_VICTIM_RING", 0) == 1:
            victim_ring = _env_int("EXL3_NVTIER_VRING_K", 128)
        if victim_ring:
            self._ring_init(int(victim_ring))

    # ---- victim ring
    def _ring_init(self, K: int) -> None:
        if not 1 <= K <= 256:
            raise ValueError(f"NvTierAsync: victim ring of {K} slots (1..256)")
        if _env_int("EXL3_NVTIER_NO_VICTIM", 0) == 1:
            raise ValueError("NvTierAsync: the victim ring needs victim write-back (EXL3_NVTIER_NO_VICTIM=1 is set)")
        X, d, st = self.st.X, self.dev, self.st
        self.vr_K = K
        meta = torch.full((4 + 2 * K,), -1, dtype=torch.int32)
        meta[:4] = torch.tensor([0, 0, 0, K], dtype=torch.int32)
        meta[4 + K:] = 0
        self.vr_meta = meta.to(d)
        self.vr_sel = torch.full((self.E,), -1, dtype=torch.int32, device=d)
        self.vr_stride = int(st.slot_stride)
        self.vr_buf = torch.empty(K * self.vr_stride, dtype=torch.uint8, device=d)
        self._h_vr = [X.host_alloc(4 * (4 + 2 * K)).view(torch.int32) for _ in range(2)]
        for t in self._h_vr:
            t.fill_(-1)
        self._np_vr = [t.numpy() for t in self._h_vr]
        self._h_vfree = [X.host_alloc(8 * K).view(torch.int64) for _ in range(2)]
        self._np_vfree = [t.numpy() for t in self._h_vfree]
        self._d_vfree = torch.zeros(K, dtype=torch.int64, device=d)
        self._vr_events = []                             # free events for the drains
        self._vr_seen = np.zeros(K, dtype=np.int64)      # claim number handled per slot (claims count from 1)
        self._vr_fly = []                                # [(event, due host step, [(slot, key), ...])]
        self._vr_cs = torch.cuda.Stream(d)
        self._vr_claims = self._vr_drops = 0
        for key in ("vr_claims", "vr_drops", "vr_issued", "vr_landed", "vr_ms", "vr_sync_ms"):
            self.stats[key] = 0
        if not hasattr(self, "_vict_addr"):
            self._vict_addr = torch.zeros(self.E, dtype=torch.int64, device=d)
        L = self._capi.lib()
        for b in range(2):                               # the ring's meta joins the snapshot copies
            srcs, dsts, nbs = self._xargs[b]
            self._xargs[b] = ((ctypes.c_void_p * 4)(*list(srcs), self.vr_meta.data_ptr()),
                              (ctypes.c_void_p * 4)(*list(dsts), self._h_vr[b].data_ptr()),
                              (ctypes.c_int64 * 4)(*list(nbs), 4 * (4 + 2 * K)))
        torch.cuda.synchronize(d)
        self._capi.check(L.exl3_set_victim_addrs(self._vict_addr.data_ptr()), "set_victim_addrs")
        self._capi.check(L.exl3_set_victim_ring(self.vr_meta.data_ptr(), self.vr_sel.data_ptr(),
                                                self.vr_buf.data_ptr(), self.vr_buf.numel(), K), "set_victim_ring")

    def _ring_landed(self, hs: int, wait_all: bool = False) -> tuple:
        """Drains that have landed: (keys, ring slots); with wait_all every drain in flight."""
        keys, slots, keep = [], [], []
        for ev, due, items in self._vr_fly:
            if wait_all or (due <= hs if self.completion == "steps" else ev.query()):
                t = time.perf_counter()
                ev.synchronize()
                self.stats["vr_sync_ms"] += (time.perf_counter() - t) * 1e3
                self._vr_events.append(ev)
                for r, key in items:
                    slots.append(r)
                    keys.append(key)
            else:
                keep.append((ev, due, items))
        self._vr_fly = keep
        self.stats["vr_landed"] += len(keys)
        return keys, slots

    def _ring_claims(self, m: np.ndarray, k: int, hs: int, after) -> list:
        """New claims in the ring meta m (a snapshot, or the live meta with the device idle): their keys go in flight
        with a record each, and copies slot -> record start on the side stream after the event `after` (the end of
        the decode step that wrote the slots). A claim whose key a synchronous path has made RAM-resident meanwhile
        needs no copy: its slot is returned, to be freed."""
        K = self.vr_K
        if int(m[3]) != K:                               # the snapshot holds the meta only after the first exchange
            return []
        self.stats["vr_claims"] += int(m[1]) - self._vr_claims
        self.stats["vr_drops"] += int(m[2]) - self._vr_drops
        self._vr_claims, self._vr_drops = int(m[1]), int(m[2])
        vk, vs = m[4:4 + K], m[4 + K:4 + 2 * K].astype(np.int64)
        new = np.nonzero((vk >= 0) & (vs != self._vr_seen))[0]
        if not new.size:
            return []
        self._vr_seen[new] = vs[new]
        st, pol = self.st, self.policy
        keys = vk[new].astype(np.int64)
        have = pol.res[keys] == 1
        if pol.inflight[keys[~have]].any():
            raise RuntimeError("exl3xpu tier: a victim ring claim for a key whose fill is in flight")
        skip = new[have].tolist()
        new, keys = new[~have], keys[~have]
        if not new.size:
            return skip
        if self.pool is not None:
            old = st.rec_of[keys]
            if (old != 0).any():
                self._pending[k].extend(old[old != 0].tolist())
            st.rec_of[keys] = self.pool.take(keys.size)
        pol.inflight[keys] = True
        cs = self._vr_cs
        if after is not None:
            cs.wait_event(after)
        L, h = self._capi.lib(), ctypes.c_void_p(cs.cuda_stream)
        base = self.vr_buf.data_ptr()
        for r, key in zip(new.tolist(), keys.tolist()):
            self._capi.check(L.exl3_memcpy_async(st.addr(key), base + r * self.vr_stride, self.vr_stride, h),
                             "victim ring drain")
        ev = self._vr_events.pop() if self._vr_events else torch.cuda.Event()
        ev.record(cs)
        self._vr_fly.append((ev, hs + 1, list(zip(new.tolist(), keys.tolist()))))
        self.stats["vr_issued"] += int(new.size)
        return skip

    def _ring_free(self, slots, k: int) -> None:
        """Free ring slots on the compute stream (their copies have completed), before the next decode step."""
        if not slots:
            return
        n = len(slots)
        self._np_vfree[k][:n] = np.asarray(slots, dtype=np.int64) + 4
        idx = self._d_vfree[:n]
        idx.copy_(self._h_vfree[k][:n], non_blocking=True)
        self.vr_meta.index_fill_(0, idx, -1)

    def ring_settle(self) -> None:
        """Drain the whole ring now (synchronous paths; the device goes idle): the claims of the device's current
        meta are copied too, every drain lands, the keys become RAM-resident on the host and the device, their
        records are published and their slots freed."""
        if not self.vr_K:
            return
        torch.cuda.synchronize(self.dev)
        skip = self._ring_claims(self.vr_meta.cpu().numpy(), self._k, self._hstep, None)
        keys, slots = self._ring_landed(self._hstep, wait_all=True)
        slots = slots + skip
        if keys:
            pol = self.policy
            ka = np.asarray(keys, dtype=np.int64)
            pol.res[ka] = 1
            pol.age[ka] = pol.tick
            pol.inflight[ka] = False
            if self.pool is not None:
                self.st.publish_records(keys)
            self.res_dev.index_fill_(0, torch.from_numpy(ka).to(self.dev), 1)
            self._flags_changed(ka, 1)
        self._ring_free(slots, self._k)
        torch.cuda.synchronize(self.dev)

    def ensure_for_prefill(self, li: int, ids) -> int:
        self.ring_settle()
        return super().ensure_for_prefill(li, ids)

    # ---- record pool
    def _pool_init(self, cap: int) -> None:
        if cap <= 0:
            raise ValueError(f"NvTierAsync: write-back queue of {cap} records")
        X, d, n = self.st.X, self.dev, self._n
        self.wb_cap = cap
        self._vict_addr = torch.zeros(self.E, dtype=torch.int64, device=d)
        self._wbq = torch.zeros(cap, dtype=torch.int64, device=d)
        self._wbq_state = torch.zeros(2 + cap, dtype=torch.int32, device=d)
        self._h_next = [X.host_alloc(8 * cap).view(torch.int64) for _ in range(2)]
        self._h_wbm = [X.host_alloc(4 * (2 + cap)).view(torch.int32) for _ in range(2)]
        for t in self._h_wbm:
            t.zero_()
        self._np_next = [t.numpy() for t in self._h_next]
        self._np_wbm = [t.numpy() for t in self._h_wbm]
        self._h_upd = [X.host_alloc(16 * n).view(torch.int64) for _ in range(2)]
        self._np_upd = [t.numpy() for t in self._h_upd]
        self._pending = [[], []]           # records of keys evicted by the step that used buffer b
        self._q_recs = [np.zeros(0, np.int64), np.zeros(0, np.int64)]    # the queue installed by exchange b
        q0 = self.pool.take(cap)           # the queue of the first decode step, as if installed by exchange 1
        self._wbq.copy_(torch.from_numpy(q0))
        self._q_recs[1] = q0
        for key in ("wb_taken", "wb_dropped", "pool_rebind"):
            self.stats[key] = 0
        L = self._capi.lib()
        torch.cuda.synchronize(d)
        self._capi.check(L.exl3_set_victim_addrs(self._vict_addr.data_ptr()), "set_victim_addrs")
        self._capi.check(L.exl3_set_record_pool(self.st.host_addr_dev.data_ptr(), self._wbq.data_ptr(),
                                                self._wbq_state.data_ptr(), cap), "set_record_pool")

    def _pool_collect(self, j: int, k: int) -> None:
        """After the exchange of buffer j has run: free the records of the keys its step evicted, and settle the
        queue that exchange found in use (installed by exchange k): taken records belong to the keys written back
        into them, the rest return to the pool."""
        st, pool, cap = self.st, self.pool, self.wb_cap
        pool.give(self._pending[j])
        self._pending[j] = []
        m = self._np_wbm[j]
        taken = int(m[0])
        q = self._q_recs[k]
        if taken > q.size:
            raise RuntimeError(f"exl3xpu tier: the device took {taken} write-back records of a queue of {q.size}")
        if taken:
            keys = m[1:1 + taken].astype(np.int64)
            old = st.rec_of[keys]
            if (old != 0).any():           # a key written back while the books still gave it a record
                self._pending[k].extend(old[old != 0].tolist())
                self.stats["pool_rebind"] += int((old != 0).sum())
            st.rec_of[keys] = q[:taken]
        pool.give(q[taken:])
        self._q_recs[k] = np.zeros(0, np.int64)
        self.stats["wb_taken"] += taken
        self.stats["wb_dropped"] += int(m[1 + cap])

    def _flags_changed(self, keys, val: int) -> None:
        """A synchronous path changed device flags while the device is idle: make the snapshot the next step will
        read show them (the previous upload overlaid first), so that the step does not mistake them for write-backs
        or reverse them."""
        keys = np.asarray(keys, dtype=np.int64).reshape(-1)
        for b in range(2):
            if self._have[b]:
                if self._last_diff is not None:
                    dk, dv = self._last_diff
                    self._np_res[b][dk] = dv
                self._np_res[b][keys] = val
        self._last_diff = None

    def close(self) -> None:
        if self.vr_K:
            torch.cuda.synchronize(self.dev)
            self._capi.check(self._capi.lib().exl3_set_victim_ring(None, None, None, 0, 0), "set_victim_ring")
            if self.pool is None:
                self._capi.check(self._capi.lib().exl3_set_victim_addrs(None), "set_victim_addrs")
            self.vr_K = 0
        if self.pool is not None:
            torch.cuda.synchronize(self.dev)
            L = self._capi.lib()
            self._capi.check(L.exl3_set_record_pool(None, None, None, 0), "set_record_pool")
            self._capi.check(L.exl3_set_victim_addrs(None), "set_victim_addrs")
        super().close()

    @property
    def inflight_keys(self):
        return np.nonzero(self.policy.inflight)[0]

    def step(self) -> int:
        """The host step after a decode step; returns the number of masked picks it consumed."""
        t0 = time.perf_counter()
        pol = self.policy
        pol.tick += 1
        self.tick = pol.tick
        hs = self._hstep
        self._hstep += 1
        cur = torch.cuda.current_stream(self.dev)
        k, j = self._k, self._k ^ 1
        self._k = j
        n_diff = 0
        n_upd = 0
        pool = self.pool is not None
        seen0 = pol.ring_seen
        if self._have[j]:
            tw = time.perf_counter()
            self._snap_ev[j].synchronize()
            self.stats["wait_ms"] = self.stats.get("wait_ms", 0.0) + (time.perf_counter() - tw) * 1e3
            bad = int(self._h_status[j][0])
            if bad:
                raise RuntimeError(f"exl3xpu: {bad} bounded waits of the decode kernels timed out on the device "
                                   "(outputs computed from incomplete data); the device state is not trustworthy")
            if pool:
                self._pool_collect(j, k)
                self._start_fills()
            tv = time.perf_counter()
            vr_keys, vr_slots = self._ring_landed(hs) if self.vr_K else ([], [])
            if self.vr_K:
                vr_slots += self._ring_claims(self._np_vr[j], k, hs, self._snap_ev[j])
                self.stats["vr_ms"] += (time.perf_counter() - tv) * 1e3
            view = self._view
            np.copyto(view, self._np_res[j])
            if self._last_diff is not None:         # the flags uploaded with that snapshot
                dk, dv = self._last_diff
                view[dk] = dv
            done = self._completed(hs) + vr_keys
            adm, ev_keys, diff, vals = pol.decide(view, self._np_ring, self._np_slot[j], done)
            if self.vr_K:
                tv = time.perf_counter()
                self._ring_free(vr_slots, k)
                self.stats["vr_ms"] += (time.perf_counter() - tv) * 1e3
            self._ring_from = int(self._np_ring[0]) & 0xFFFFFFFF
            self._queue_fills(adm, hs)
            if pool:
                st = self.st
                r = st.rec_of[ev_keys]
                self._pending[k].extend(r[r != 0].tolist())
                st.rec_of[ev_keys] = 0
                dn = np.asarray(done, dtype=np.int64)
                dn = dn[pol.res[dn] == 1]
                if dn.size:                         # completed fills: their records go up with their flags
                    u = self._np_upd[k]
                    u[0:2 * dn.size:2] = dn
                    u[1:2 * dn.size:2] = st.rec_of[dn]
                    n_upd = int(dn.size)
            if len(diff):
                # buffer k was last read by the exchange of step n-2, which ran before the snapshot just waited for
                self._np_diff[k][:len(diff)] = (diff << 1) | vals
                n_diff = len(diff)
                self._last_diff = (diff, vals)
            else:
                self._last_diff = None
            self.res = pol.res
            self.age, self.inflight, self.ring_seen = pol.age, pol.inflight, pol.ring_seen
            if self.log_decisions:
                self.decisions.append((adm.copy(), ev_keys.copy()))
            for key, v in pol.stats.items():
                self.stats[key] = v
        elif self.log_decisions:
            self.decisions.append((np.zeros(0, np.int64), np.zeros(0, np.int64)))
        # this step's diff and the snapshot of the device state after decode step n, in one launch
        srcs, dsts, nbs = self._xargs[k]
        L = self._capi.lib()
        if pool:
            q = self.pool.take(self.wb_cap)         # the write-back queue of decode step n + 1
            self._np_next[k][:] = q
            self._q_recs[k] = q
            st = self.st
            self._capi.check(L.exl3_tier_exchange_pool(
                self.res_dev.data_ptr(), self._n, self._h_diff[k].data_ptr(), n_diff, self.ring.data_ptr(),
                self.ring.numel() - 1, self._ring_from, self._h_ring.data_ptr(), srcs, dsts, nbs, len(nbs),
                self._h_upd[k].data_ptr(), n_upd, st.host_addr_dev.data_ptr(), st.ptrs_all.data_ptr(),
                st.slot_of_dev.data_ptr(), self._h_next[k].data_ptr(), self._wbq.data_ptr(),
                self._wbq_state.data_ptr(), self._h_wbm[k].data_ptr(), self.wb_cap, cur.cuda_stream),
                "nvtier exchange")
        else:
            self._capi.check(L.exl3_tier_exchange(self.res_dev.data_ptr(), self._n, self._h_diff[k].data_ptr(),
                                                  n_diff, self.ring.data_ptr(), self.ring.numel() - 1,
                                                  self._ring_from, self._h_ring.data_ptr(), srcs, dsts, nbs,
                                                  len(nbs), cur.cuda_stream), "nvtier exchange")
        self._snap_ev[k].record(cur)
        self._have[k] = True
        self.stats["steps"] += 1
        self.stats["fill_ms"] += (time.perf_counter() - t0) * 1e3
        return int((pol.ring_seen - seen0) & 0xFFFFFFFF)
