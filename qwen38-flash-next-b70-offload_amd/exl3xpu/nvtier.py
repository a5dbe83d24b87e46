"""RAM expert tier for the MI355X device-managed expert cache (reference plugin/exl3xpu/nvtier.py).

Tiers: HBM slots (device LRU, write-through on miss) -> RAM tier (one pinned, device-mapped host arena with a fixed
address per expert, read zero-copy by the kernels) -> expert store (all experts; a pluggable fill source with a
deterministic completion latency in host steps, standing in for the reference's O_DIRECT NVMe reads).

Device side (csrc/moe_cache.hip): picks whose expert is in neither HBM nor RAM are masked to (safe expert, weight 0) and
logged to a miss ring; HBM victims whose RAM copy is not valid are written back to their RAM address and flagged.
Host side (call step() after every decode step): consume the previous step's device snapshot, complete fills, admit the
most-missed keys into free budget, evict RAM copies of HBM-resident experts first and then keys older than AGE steps,
and upload the changed flags. The RAM arena is never unmapped, so an evicted key's bytes stay readable: the reference's
punch/write-back race (its docs/results.md:164-172) cannot corrupt data here; "punch" is bookkeeping only.
"""
from __future__ import annotations

import ctypes
import logging
import os
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from .moe_offload import ExpertStore, s64

MiB2 = 2 << 20
log = logging.getLogger("exl3xpu")


class TierStore(ExpertStore):
    """ExpertStore whose host copies live at fixed-stride addresses of one pinned arena (the reference uses a sparse
    2 MiB-stride memfd, nvtier.py:22-53). stride defaults to the blob size rounded up to 4 KiB."""

    def __init__(self, H, I, K, E, n_slots, n_layers, stride=None, device=None, Ks=None):
        """Ks: bitrate per layer (in add_layer order) when layers differ; slots and records take the largest blob."""
        self.Ks = [int(k) for k in Ks] if Ks is not None else None
        if self.Ks is not None and len(self.Ks) != n_layers:
            raise ValueError(f"TierStore: {len(self.Ks)} bitrates for {n_layers} layers")
        super().__init__(H, I, max(self.Ks) if self.Ks else K, E, n_slots, device=device, max_layers=n_layers)
        if self.Ks and len(set(self.Ks)) > 1:
            self.mixed_bitrates()
        self.stride = int(stride) if stride else (self.blob + 4095) // 4096 * 4096
        assert self.blob <= self.stride and self.stride % 16 == 0
        self.L = n_layers
        self.size = n_layers * E * self.stride
        self.arena = self.X.host_alloc(self.size)
        self.base = s64(self.arena.data_ptr())
        self.X.moe_set_host_stride(self.stride)

    def add_layer(self, key, blobs=None):
        li = len(self.layer_index)
        if li >= self.L:
            raise RuntimeError(f"TierStore: more than n_layers={self.L} MoE layers")
        self.layer_index[key] = li
        if self.Ks:
            self.K_of[key] = self.Ks[li]
        base = self.base + li * self.E * self.stride
        self._host_ptr[key] = base + torch.arange(self.E, dtype=torch.int64) * self.stride
        self.ptrs_all[li * self.E:(li + 1) * self.E].copy_(self._host_ptr[key])
        self.host_base[li] = base
        self.slot_of[key] = torch.full((self.E,), -1, dtype=torch.int32)
        if blobs is not None:
            for e in range(self.E):
                self.arena[(li * self.E + e) * self.stride:(li * self.E + e) * self.stride + self.blob].copy_(blobs[e])
        return None

    def addr(self, key: int) -> int:                       # key = li * E + e
        return self.base + key * self.stride

    def host_view(self, key):
        li = self.layer_index[key]
        return self.arena[li * self.E * self.stride:(li + 1) * self.E * self.stride].view(self.E, self.stride)[:, :self.blob]


class SyntheticExpertSource:
    """Deterministic stand-in for the packed NVMe store (serve/pack_store.py): record r holds the blob of synthetic
    expert r % n_distinct of workload `seed`; `read(r, dst)` copies it to a host address."""

    def __init__(self, H, I, K, seed: int, n_distinct: int = 64):
        from .synth import expert_blob
        self.blob = int(expert_blob(seed, 0, H, I, K).numel())
        self.n = n_distinct
        self.buf = np.stack([expert_blob(seed, i, H, I, K).numpy() for i in range(n_distinct)])
        self.rec = self.blob

    def read(self, rec_index: int, dst: int) -> None:
        src = self.buf[rec_index % self.n]
        ctypes.memmove(dst, src.ctypes.data, self.blob)

    def blob_of(self, rec_index: int) -> np.ndarray:
        return self.buf[rec_index % self.n]


class LayeredExpertSource:
    """Fill source for a store whose layers differ in bitrate: record r = layer * E + e is read from sources[layer]
    (a source of that layer's geometry)."""

    def __init__(self, sources, E: int):
        self.sources, self.E = list(sources), int(E)
        self.blob = max(s.blob for s in self.sources)

    def read(self, rec_index: int, dst: int) -> None:
        self.sources[rec_index // self.E].read(rec_index, dst)

    def blob_of(self, rec_index: int) -> np.ndarray:
        return self.sources[rec_index // self.E].blob_of(rec_index)


class NvTier:
    """Tier base: flags, miss ring, pinned safe expert per layer (nvtier.py:56-87).
    source: object with read(rec_index, dst_addr) (an NVMe store reader or SyntheticExpertSource).
    ram_budget: bytes (records = bytes // stride, like the reference) or, with budget_records, a record count."""

    def __init__(self, store: TierStore, source, meta=None, ram_budget_bytes=2 << 30, ring_cap=1 << 16, safe=0,
                 dev=None, ckpt_layer=None, budget_records: int | None = None, latency: int = 8):
        self.st, self.E = store, store.E
        self.src = source
        self.L = len(ckpt_layer) if ckpt_layer is not None else store.L
        self.ckpt = np.asarray(ckpt_layer if ckpt_layer is not None else range(self.L), dtype=np.int64)
        self.dev = dev or store.dev
        self.blob = store.blob
        self.budget = int(budget_records) if budget_records else max(1, int(ram_budget_bytes // store.stride))
        self.latency = max(1, int(latency))
        n = self.L * self.E
        self.res_dev = torch.zeros(n, dtype=torch.uint8, device=self.dev)
        self.ring = torch.zeros(1 + ring_cap, dtype=torch.int32, device=self.dev)
        self.safe = torch.full((self.L,), safe, dtype=torch.int32, device=self.dev)
        self.vict = torch.zeros(1 + 2 * self.E, dtype=torch.int32, device=self.dev)
        self.res = np.zeros(n, dtype=np.uint8)
        self.pinned = set(li * self.E + safe for li in range(self.L))
        self.ring_seen = 0
        self.stats = dict(nvme_reads=0, nvme_ms=0.0, evicts=0, masked=0, steps=0, fill_ms=0.0, ring_overflow=0)
        for k in sorted(self.pinned):
            self._fill(k)
        self.res_dev.copy_(torch.from_numpy(self.res))
        X = store.X
        X.moe_set_tier(self.res_dev, self.ring, self.safe)
        if os.environ.get("EXL3_NVTIER_NO_VICTIM", "0") != "1":
            X.moe_set_victims(self.vict)
        else:
            X.moe_set_victims(torch.zeros(0, dtype=torch.int32, device=self.dev))

    def close(self):
        X = self.st.X
        X.moe_set_tier(torch.zeros(0, dtype=torch.uint8, device=self.dev), torch.zeros(0, dtype=torch.int32, device=self.dev),
                       torch.zeros(0, dtype=torch.int32, device=self.dev))
        X.moe_set_victims(torch.zeros(0, dtype=torch.int32, device=self.dev))
        X.moe_set_host_stride(0)
        X.moe_set_slot_stride(0)

    def rec_index(self, key: int) -> int:
        return int(self.ckpt[key // self.E]) * self.E + key % self.E

    def _fill(self, key: int) -> None:
        t = time.perf_counter()
        self.src.read(self.rec_index(key), self.st.addr(key))
        self.res[key] = 1
        self.stats["nvme_reads"] += 1
        self.stats["nvme_ms"] += (time.perf_counter() - t) * 1e3

    def fill_many(self, keys) -> None:
        keys = [int(k) for k in keys]
        if not keys:
            return
        if not hasattr(self, "_pool"):
            self._pool = ThreadPoolExecutor(int(os.environ.get("EXL3_NVTIER_FILL_THREADS", "16")))
        t = time.perf_counter()
        list(self._pool.map(lambda k: self.src.read(self.rec_index(k), self.st.addr(k)), keys))
        for k in keys:
            self.res[k] = 1
        self.stats["nvme_reads"] += len(keys)
        self.stats["nvme_ms"] += (time.perf_counter() - t) * 1e3

    def ram_bytes(self) -> int:
        return int(self.res.sum()) * self.st.stride

    def warm(self, keys_ckpt, max_bytes):
        """Fill the RAM tier with the hottest experts (checkpoint keys, hottest first) up to max_bytes
        (nvtier.py:492-509)."""
        inv = {int(c): li for li, c in enumerate(self.ckpt)}
        t = time.perf_counter()
        cap = int(max_bytes // self.st.stride)
        have = int(self.res.sum())
        todo, seen = [], set()
        for kc in keys_ckpt:
            if have + len(todo) >= cap:
                break
            li = inv.get(int(kc) // self.E)
            if li is None:
                continue
            k = li * self.E + int(kc) % self.E
            if not self.res[k] and k not in seen:
                todo.append(k)
                seen.add(k)
        self.fill_many(todo)
        if hasattr(self, "age"):
            self.age[todo] = 0
        self.res_dev.copy_(torch.from_numpy(self.res))
        return len(todo), time.perf_counter() - t

    # ---- tier-mode prefill streaming (nvtier.py:534-640) ------------------------------------------------------------
    def stage_forward(self, store, key, li: int, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """Prefill-size MoE for layer `li` with its non-HBM experts streamed: reader threads copy the layer's records
        from the fill source into a pinned host ring buffer (read-ahead of NB-1 layers, EXL3_NVTIER_STAGE_HOSTBUF,
        default 4), a side stream copies them into one of two HBM staging buffers (runs of consecutive experts in one
        copy), and the layer runs from the device table where(slot_of >= 0, slot, staging). The first layer of a
        forward synchronises once and snapshots the HBM slot map; layers follow the checkpoint order."""
        sg = getattr(self, "_sg", None) or self._stage_setup()
        E, rec = self.E, sg["rec"]
        pos = sg["pos"][li]
        if pos == 0 or li not in sg["pending"]:
            torch.cuda.synchronize(self.dev)
            sod = self.st.slot_of_dev[:self.L * E]
            sg["snap_dev"] = sod.to(torch.int64)
            sg["snap"] = sod.cpu().numpy()
            for _, _, fs in sg["pending"].values():
                for f in fs:
                    f.result()
            sg["pending"].clear()
            for q in range(pos, min(pos + sg["NB"], len(sg["order"]))):
                self._stage_kick(sg["order"][q])
        hb, miss, futs = sg["pending"].pop(li)
        for f in futs:
            f.result()
        buf = sg["dbuf"]
        sg["dbuf"] = 1 - buf
        cur = torch.cuda.current_stream(self.dev)
        dbase, hbase = s64(sg["dev"][buf].data_ptr()), s64(sg["host"][hb].data_ptr())
        with torch.cuda.stream(sg["cs"]):
            if sg["comp_ev"][buf] is not None:
                sg["cs"].wait_event(sg["comp_ev"][buf])      # the layer that last read this staging buffer is done
            m, i = miss.tolist(), 0
            while i < len(m):
                j = i
                while j + 1 < len(m) and m[j + 1] == m[j] + 1:
                    j += 1
                self.st.X.memcpy_async(dbase + m[i] * rec, hbase + m[i] * rec, (j - i + 1) * rec)
                i = j + 1
            ev = torch.cuda.Event()
            ev.record(sg["cs"])
        sg["hfree"][hb] = ev
        cur.wait_event(ev)
        so = sg["snap_dev"][li * E:(li + 1) * E]
        table = torch.where(so >= 0, self.st.slot_base + so.clamp_min(0) * self.st.blob, dbase + sg["ar"])
        y = store.forward(key, x, ids, w, ptrs=table)
        ce = torch.cuda.Event()
        ce.record(cur)
        sg["comp_ev"][buf] = ce
        nq = pos + sg["NB"]
        if nq < len(sg["order"]) and sg["order"][nq] not in sg["pending"]:
            self._stage_kick(sg["order"][nq])
        sg["bytes"] += len(miss) * rec
        return y

    def _stage_setup(self):
        E = self.E
        rec = self.st.stride
        NB = max(2, int(os.environ.get("EXL3_NVTIER_STAGE_HOSTBUF", "4")))
        X = self.st.X
        order = [int(li) for li in np.argsort(self.ckpt, kind="stable")]
        sg = dict(rec=rec, NB=NB, dev=[torch.empty(E * rec, dtype=torch.uint8, device=self.dev) for _ in range(2)],
                  host=[X.host_alloc(E * rec) for _ in range(NB)], cs=torch.cuda.Stream(self.dev),
                  comp_ev=[None, None], hfree={}, pending={}, nexth=0, dbuf=0, order=order,
                  pos={li: i for i, li in enumerate(order)}, snap=None, snap_dev=None, bytes=0,
                  ar=torch.arange(E, dtype=torch.int64, device=self.dev) * rec,
                  pool=ThreadPoolExecutor(int(os.environ.get("EXL3_NVTIER_FILL_THREADS", "16"))))
        self._sg = sg
        return sg

    def _stage_kick(self, li: int) -> None:
        """Start the reads of layer li's non-HBM experts into the next host ring buffer."""
        sg, E, rec = self._sg, self.E, self._sg["rec"]
        hb = sg["nexth"]
        sg["nexth"] = (hb + 1) % sg["NB"]
        ev = sg["hfree"].pop(hb, None)
        if ev is not None:
            ev.synchronize()                        # the copy that last read this host buffer is done
        miss = np.nonzero(sg["snap"][li * E:(li + 1) * E] < 0)[0]
        hp = s64(sg["host"][hb].data_ptr())
        keys = [int(e) for e in miss]
        per = max(1, -(-len(keys) // 8))

        def rd(part):
            for e in part:
                self.src.read(self.rec_index(li * E + e), hp + e * rec)
        sg["pending"][li] = (hb, miss, [sg["pool"].submit(rd, keys[i:i + per]) for i in range(0, len(keys), per)])

    def log_stats(self, logger=None, every=200):
        logger = logger or log
        if self.stats["steps"] % every or not self.stats["steps"]:
            return
        b = getattr(self, "_last", None) or {k: 0 for k in self.stats}
        d = {k: self.stats.get(k, 0) - b.get(k, 0) for k in self.stats}
        n = max(1, d.get("steps", 0))
        logger.info("exl3xpu: nvtier last %d steps: masked/step %.2f fills/step %.2f evicts/step %.1f host ms/step %.2f "
                    "admit_dropped %d ram %.2f GB", n, d.get("masked", 0) / n, d.get("nvme_reads", 0) / n,
                    d.get("evicts", 0) / n, d.get("fill_ms", 0) / n, d.get("admit_dropped", 0), self.ram_bytes() / 2 ** 30)
        self._last = dict(self.stats)


class NvTierFast(NvTier):
    """Vectorised bookkeeping + background fills (nvtier.py:175-278): age, in-flight set, pinned mask; fills complete
    `latency` host steps after admission (deterministic). The fills admitted by one host step are copied by a few
    worker tasks (one future per chunk of keys), since each completes as a group."""

    FILL_CHUNKS = 4

    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        n = self.L * self.E
        self.age = np.zeros(n, dtype=np.int64)
        self.tick = 1
        self.pin_mask = np.zeros(n, dtype=bool)
        self.pin_mask[list(self.pinned)] = True
        self.inflight = np.zeros(n, dtype=bool)
        self._pending = {}                 # host step -> [(keys, future)]
        self._hstep = 0
        self._pool = ThreadPoolExecutor(int(os.environ.get("EXL3_NVTIER_FILL_THREADS", "16")))

    def _read_keys(self, keys) -> None:
        for key in keys:
            self.src.read(self.rec_index(key), self.st.addr(key))

    def _queue_fills(self, keys, hs: int) -> None:
        """fills admitted at host step hs: copied by workers, flagged resident at host step hs + latency"""
        keys = [int(k) for k in keys]
        if not keys:
            return
        per = -(-len(keys) // self.FILL_CHUNKS)
        lst = self._pending.setdefault(hs + self.latency, [])
        for i in range(0, len(keys), per):
            part = keys[i:i + per]
            lst.append((part, self._pool.submit(self._read_keys, part)))
        self.stats["nvme_reads"] += len(keys)

    def _queue_fill(self, key: int, hs: int) -> None:
        self._queue_fills([key], hs)

    def _completed(self, hs: int):
        done = []
        for keys, fut in self._pending.pop(hs, []):
            fut.result()
            done.extend(keys)
        return done

    def close(self):
        self._pool.shutdown(wait=True)
        super().close()


class _AdmitState(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int64) for f in ("n", "budget", "admit_age", "admit_qmax", "ring_cap", "tick",
                                               "ring_seen", "masked", "evicts", "admit_dropped", "ring_overflow")]


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


class AdmissionPolicy:
    """Host bookkeeping of the admission-controlled tier step (_async_step_admit, nvtier.py:708-806); the decision
    runs natively (exl3_admit_decide in libexl3moe.so) over the numpy books held here.

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
    pinned ring mirror, and writes the snapshot of the RAM flags and the slot table into pinned double buffers; no
    host allocation, no extra synchronisation. The host reads the mirror only between the wait for one exchange and
    the launch of the next, so one mirror suffices."""

    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        from . import capi
        self._capi = capi
        n = self.L * self.E
        self._n = n
        X = self.st.X
        # device-mapped pinned buffers: the exchange kernel writes the snapshots and reads the diffs in place
        self._h_res = [X.host_alloc(n) for _ in range(2)]
        self._h_ring = X.host_alloc(4 * self.ring.numel()).view(torch.int32)
        self._h_ring.zero_()
        self._ring_from = 0                # ring count of the last snapshot read (the next exchange mirrors from it)
        self._h_slot = [X.host_alloc(4 * n).view(torch.int32) for _ in range(2)]
        self._np_res = [t.numpy() for t in self._h_res]
        self._np_ring = self._h_ring.numpy()
        self._np_slot = [t.numpy() for t in self._h_slot]
        self._h_diff = [X.host_alloc(4 * n).view(torch.int32) for _ in range(2)]   # device-mapped pinned
        self._np_diff = [t.numpy() for t in self._h_diff]
        self._snap_ev = [torch.cuda.Event(), torch.cuda.Event()]
        import ctypes
        self._xargs = []                   # (src, dst, nbytes) ctypes arrays of the two snapshot copies per buffer
        for b in range(2):
            pairs = ((self.res_dev, self._h_res[b], n), (self.st.slot_of_dev, self._h_slot[b], 4 * n))
            self._xargs.append(((ctypes.c_void_p * 2)(*[p[0].data_ptr() for p in pairs]),
                                (ctypes.c_void_p * 2)(*[p[1].data_ptr() for p in pairs]),
                                (ctypes.c_int64 * 2)(*[p[2] for p in pairs])))
        self._have = [False, False]
        self._k = 0
        self._last_diff = None
        self._view = np.empty(n, dtype=np.uint8)
        self.policy = AdmissionPolicy(n, self.pinned, self.budget, int(os.environ.get("EXL3_NVTIER_ADMIT_AGE", "4")),
                                      int(os.environ.get("EXL3_NVTIER_ADMIT_QMAX", "256")), self.ring.numel() - 1)
        self.policy.res[:] = self.res
        self.res = self.policy.res
        self.log_decisions = False
        self.decisions = []                # (admitted keys, evicted keys) per step when log_decisions

    @property
    def inflight_keys(self):
        return np.nonzero(self.policy.inflight)[0]

    def step(self) -> int:
        t0 = time.perf_counter()
        pol = self.policy
        pol.tick += 1
        self.tick = pol.tick
        hs = self._hstep
        self._hstep += 1
        n = self._n
        cur = torch.cuda.current_stream(self.dev)
        L, sh = self._capi.lib(), cur.cuda_stream
        k = self._k
        self._k ^= 1
        j = k ^ 1
        n_diff = 0
        seen0 = pol.ring_seen
        if self._have[j]:
            tw = time.perf_counter()
            self._snap_ev[j].synchronize()
            self.stats["wait_ms"] = self.stats.get("wait_ms", 0.0) + (time.perf_counter() - tw) * 1e3
            view = self._view
            np.copyto(view, self._np_res[j])
            if self._last_diff is not None:         # the flags uploaded with that snapshot
                dk, dv = self._last_diff
                view[dk] = dv
            adm, ev_keys, diff, vals = pol.decide(view, self._np_ring, self._np_slot[j], self._completed(hs))
            self._ring_from = int(self._np_ring[0])
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
        self._capi.check(L.exl3_tier_exchange(self.res_dev.data_ptr(), n, self._h_diff[k].data_ptr(), n_diff,
                                              self.ring.data_ptr(), self.ring.numel() - 1, self._ring_from,
                                              self._h_ring.data_ptr(), srcs, dsts, nbs, 2, sh), "nvtier exchange")
        self._snap_ev[k].record(cur)
        self._have[k] = True
        self.stats["steps"] += 1
        self.stats["fill_ms"] += (time.perf_counter() - t0) * 1e3
        return int(max(0, pol.ring_seen - seen0))


def _ensure_for_prefill(self, li, ids):
    """Prefill: synchronously make every expert this layer's batch uses RAM-resident and flag it on the device, so
    the prefill kernel can read it zero-copy (nvtier.py:389-457). Evicts, in order: prefill-only fills of other
    layers, RAM copies of HBM-resident experts, the oldest; never this layer's keys, pinned keys or in-flight fills.
    Ties by ascending key (stable sort)."""
    n = self.L * self.E
    if not hasattr(self, "transient"):
        self.transient = np.zeros(n, dtype=bool)
    keys = np.unique(ids.reshape(-1).to("cpu", torch.int64).numpy()) + li * self.E
    miss = keys[self.res[keys] == 0]
    if len(miss):
        inflight = getattr(self, "inflight", np.zeros(n, dtype=bool))
        over = int(self.res.sum()) + int(inflight.sum()) + len(miss) - self.budget
        if over > 0:
            torch.cuda.synchronize(self.dev)
            res_d = self.res_dev.cpu().numpy()
            newly = (res_d == 1) & (self.res == 0)
            self.res[newly] = 1
            if hasattr(self, "age"):
                self.age[newly] = self.tick
            age = getattr(self, "age", np.zeros(n, dtype=np.int64))
            ok = (self.res == 1) & ~inflight
            ok[list(self.pinned)] = False
            ok[keys] = False
            vram = self.st.slot_of_dev[:n].cpu().numpy() >= 0
            ev = []
            for m in (ok & self.transient, ok & ~self.transient & vram, ok & ~self.transient & ~vram):
                if over <= 0:
                    break
                c = np.nonzero(m)[0]
                c = c[np.argsort(age[c], kind="stable")[:over]]
                ev.append(c)
                over -= len(c)
            ev = np.concatenate(ev) if ev else np.zeros(0, dtype=np.int64)
            if len(ev):
                self.res[ev] = 0
                self.transient[ev] = False
                self.res_dev.index_fill_(0, torch.from_numpy(ev.astype(np.int64)).to(self.dev), 0)
            self.stats["prefill_evicts"] = self.stats.get("prefill_evicts", 0) + len(ev)
    miss = [int(k) for k in miss]
    self.fill_many(miss)
    for k in miss:
        if hasattr(self, "inflight"):
            self.inflight[k] = False
        if hasattr(self, "age"):
            self.age[k] = self.tick
        self.transient[k] = True
    if miss:
        idx = torch.tensor(miss, dtype=torch.int64).to(self.dev, non_blocking=True)
        self.res_dev.index_fill_(0, idx, 1)
    self.stats["prefill_fills"] = self.stats.get("prefill_fills", 0) + len(miss)
    return len(miss)


NvTier.ensure_for_prefill = _ensure_for_prefill
