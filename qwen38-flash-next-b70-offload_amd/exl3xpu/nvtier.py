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


class TierStore(ExpertStore):
    """ExpertStore whose host records sit at fixed-stride addresses of one pinned arena: key li * E + e at
    base + key * stride (the reference maps a sparse 2 MiB-stride memfd, nvtier.py:22-53). The stride defaults to the
    blob rounded up to 4 KiB, the record size of the expert file. Ks: the bitrate of each layer in add_layer order
    when layers differ; slots and records then take the largest blob."""

    _own_host_arrays = False

    def __init__(self, H, I, K, E, n_slots, n_layers, stride=None, device=None, Ks=None):  # noqa: E741
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
        self.size = n_layers * E * self.stride
        self.arena = self.X.host_alloc(self.size)
        self.base = self.arena.data_ptr()

    def _host_stride(self) -> int:
        return self.stride

    def _new_records(self, li: int, blobs) -> _HostRecords:
        span = self.E * self.stride
        view = self.arena[li * span:(li + 1) * span].view(self.E, self.stride)[:, :self.blob]
        if blobs is not None:
            view.copy_(blobs)
        return _HostRecords(self.base + li * span, self.stride, self.base, self.base + self.size, view)

    def add_layer(self, key, blobs=None):
        if len(self.layer_index) >= self.L:
            raise RuntimeError(f"TierStore: more than n_layers={self.L} MoE layers")
        li = len(self.layer_index)
        super().add_layer(key, blobs)
        if self.Ks:
            self.K_of[key] = self.Ks[li]
        return None

    def addr(self, key: int) -> int:
        """Host record address of key = layer row * E + e."""
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

    def __init__(self, store: TierStore, source, meta=None, ram_budget_bytes=2 << 30, ring_cap=1 << 16, safe=0,
                 dev=None, ckpt_layer=None, budget_records: int | None = None, latency: int = 8):
        self.st, self.E = store, store.E
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
        """Read the records of `keys` into the arena (reader threads) and mark them RAM-resident (host books)."""
        keys = [int(k) for k in keys]
        if not keys:
            return
        t = time.perf_counter()
        if len(keys) < 4:
            for k in keys:
                self._read(k)
        else:
            list(self._pool().map(self._read, keys))
        self.res[keys] = 1
        self.stats["nvme_reads"] += len(keys)
        self.stats["nvme_ms"] += (time.perf_counter() - t) * 1e3

    def ram_bytes(self) -> int:
        return int(self.res.sum()) * self.st.stride

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
        self.fill_many(todo)
        if hasattr(self, "age"):
            self.age[todo] = 0
        self.res_dev.copy_(torch.from_numpy(self.res))
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
        inflight = getattr(self, "inflight", np.zeros(n, dtype=bool))
        over = int(self.res.sum()) + int(inflight.sum()) + miss.size - self.budget
        if miss.size and over > 0:
            torch.cuda.synchronize(self.dev)
            back = (self.res_dev.cpu().numpy() == 1) & (self.res == 0)       # victims written back since the last step
            self.res[back] = 1
            age = getattr(self, "age", np.zeros(n, dtype=np.int64))
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
            self.stats["prefill_evicts"] = self.stats.get("prefill_evicts", 0) + int(ev.size)
        self.fill_many(miss)
        if miss.size:
            if hasattr(self, "inflight"):
                self.inflight[miss] = False
            if hasattr(self, "age"):
                self.age[miss] = self.tick
            self.transient[miss] = True
            self.res_dev.index_fill_(0, torch.from_numpy(miss.astype(np.int64)).to(self.dev), 1)
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
    host step n + latency (a deterministic completion time in place of wall-clock NVMe reads)."""

    FILL_CHUNKS = 4

    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        n = self.L * self.E
        self.age = np.zeros(n, dtype=np.int64)
        self.tick = 1
        self.pin_mask = np.zeros(n, dtype=bool)
        self.pin_mask[sorted(self.pinned)] = True
        self.inflight = np.zeros(n, dtype=bool)
        self._due = {}                              # host step -> [(keys, future)]
        self._hstep = 0

    def _read_keys(self, keys) -> None:
        for key in keys:
            self._read(key)

    def _queue_fills(self, keys, hs: int) -> None:
        """Fills admitted at host step hs: read by workers, resident from host step hs + latency."""
        keys = [int(k) for k in keys]
        if not keys:
            return
        due = self._due.setdefault(hs + self.latency, [])
        for part in np.array_split(np.asarray(keys), min(self.FILL_CHUNKS, len(keys))):
            due.append((part.tolist(), self._pool().submit(self._read_keys, part.tolist())))
        self.stats["nvme_reads"] += len(keys)

    def _completed(self, hs: int) -> list:
        done = []
        for keys, fut in self._due.pop(hs, []):
            fut.result()
            done.extend(keys)
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
    out, so an output was computed from incomplete data) raises RuntimeError at the next step."""

    def __init__(self, *a, **k):
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
        seen0 = pol.ring_seen
        if self._have[j]:
            tw = time.perf_counter()
            self._snap_ev[j].synchronize()
            self.stats["wait_ms"] = self.stats.get("wait_ms", 0.0) + (time.perf_counter() - tw) * 1e3
            bad = int(self._h_status[j][0])
            if bad:
                raise RuntimeError(f"exl3xpu: {bad} bounded waits of the decode kernels timed out on the device "
                                   "(outputs computed from incomplete data); the device state is not trustworthy")
            view = self._view
            np.copyto(view, self._np_res[j])
            if self._last_diff is not None:         # the flags uploaded with that snapshot
                dk, dv = self._last_diff
                view[dk] = dv
            adm, ev_keys, diff, vals = pol.decide(view, self._np_ring, self._np_slot[j], self._completed(hs))
            self._ring_from = int(self._np_ring[0]) & 0xFFFFFFFF
            self._queue_fills(adm, hs)
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
        self._capi.check(L.exl3_tier_exchange(self.res_dev.data_ptr(), self._n, self._h_diff[k].data_ptr(), n_diff,
                                              self.ring.data_ptr(), self.ring.numel() - 1, self._ring_from,
                                              self._h_ring.data_ptr(), srcs, dsts, nbs, 3, cur.cuda_stream),
                         "nvtier exchange")
        self._snap_ev[k].record(cur)
        self._have[k] = True
        self.stats["steps"] += 1
        self.stats["fill_ms"] += (time.perf_counter() - t0) * 1e3
        return int((pol.ring_seen - seen0) & 0xFFFFFFFF)
