"""ctypes wrapper of cache_oracle.c: canonical device `ensure` + host admission step.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
Restates kernels/moe-a8/exl3_moe.a8.sycl:864-1039, 1168-1189 and plugin/exl3xpu/nvtier.py:57-87, 179-188, 282-386,
708-806 (file-level citations in cache_oracle.c).

Parity pinning (tests/test_oracle_cache.py): a from-scratch pure-Python brute force (LRU by explicit sort of
(u, slot) pairs; host step by direct set arithmetic) on tiny L/E/S; invariants on the full config-1 trace
(slot_of/slot_key bijection, victims never touched this tick, at most S assigned, RAM budget respected after
eviction, at most QMAX in flight). Age-tie order of the reference (numpy default argsort) is NOT pinned: the contract
is the stable order (ascending key): equal ages are admitted/evicted in ascending key order.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "libcache_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    src = os.path.join(_HERE, "cache_oracle.c")
    if force or not os.path.exists(_LIB) or os.path.getmtime(_LIB) < os.path.getmtime(src):
        subprocess.check_call(["gcc", "-O2", "-shared", "-fPIC", "-o", _LIB, src])
    return _LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = ctypes.CDLL(_LIB)
        P, I32, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        L.co_new.restype = P
        L.co_new.argtypes = [I32] * 10
        L.co_free.argtypes = [P]
        for name in ("co_slot_of", "co_slot_key", "co_slot_last", "co_tick", "co_ram_res", "co_ring", "co_safe",
                     "co_res", "co_inflight", "co_age"):
            getattr(L, name).restype = P
            getattr(L, name).argtypes = [P]
        L.co_htick.restype = I64
        L.co_htick.argtypes = [P]
        L.co_stats.argtypes = [P, P]
        L.co_rec_len.restype = I32
        L.co_rec_len.argtypes = [I32]
        L.co_ensure.restype = I32
        L.co_ensure.argtypes = [P, I32, P, P, I32, I32, P]
        L.co_prefetch.restype = I32
        L.co_prefetch.argtypes = [P, I32, P, I32, I32, P]
        L.co_plan.restype = I32
        L.co_plan.argtypes = [P, I32, P, I32, I32, P]
        L.co_host_step.restype = I64
        L.co_host_step.argtypes = [P, P, P, P, P]
        L.co_run.restype = I64
        L.co_run.argtypes = [P, P, P, I32, I32, I32, P, P, I64]
        L.co_set_ring.argtypes = [P, I32]
        for name in ("co_vr_key", "co_vr_seq"):
            getattr(L, name).restype = P
            getattr(L, name).argtypes = [P]
        L.co_vr_stats.argtypes = [P, P]
        _lib = L
    return _lib


def rec_len(P: int) -> int:
    return 3 + 4 * P


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class CacheOracle:
    """Device cache + host tier state machine. L layers x E experts, S slots, ring capacity R.
    tier=False: plain device LRU (no mask, no RAM tier, no write-back flags)."""

    def __init__(self, L, E, S, ring_cap=1 << 16, tier=True, budget=1075, age=4, qmax=256, latency=8, safe=0,
                 victim_ring: int = 0):
        self.L, self.E, self.S, self.R, self.tier = L, E, S, ring_cap, tier
        self.qmax = qmax
        self._c = lib().co_new(L, E, S, ring_cap, int(tier), budget, age, qmax, max(1, latency), safe)
        n = L * E
        self.vr_K = int(victim_ring)
        if self.vr_K:
            lib().co_set_ring(self._c, self.vr_K)

        def arr(name, cnt, dt):
            p = getattr(lib(), name)(self._c)
            return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(np.ctypeslib.as_ctypes_type(dt))), (cnt,))
        self.slot_of = arr("co_slot_of", n, np.int32)
        self.slot_key = arr("co_slot_key", max(S, 1), np.int32)[:S]
        self.slot_last = arr("co_slot_last", max(S, 1), np.int32)[:S]
        self.tick = arr("co_tick", 1, np.int32)
        self.ram_res = arr("co_ram_res", n, np.uint8)
        self.ring = arr("co_ring", 1 + ring_cap, np.int32)
        self.safe = arr("co_safe", L, np.int32)
        self.res = arr("co_res", n, np.uint8)
        self.inflight = arr("co_inflight", n, np.uint8)
        self.age = arr("co_age", n, np.int64)
        if self.vr_K:
            self.vr_key = arr("co_vr_key", self.vr_K, np.int32)
            self.vr_seq = arr("co_vr_seq", self.vr_K, np.int32)

    def ring_stats(self) -> dict:
        """Victim ring: next search position, claims made, write-backs dropped, protocol error flag."""
        o = np.zeros(4, dtype=np.int64)
        lib().co_vr_stats(self._c, _ptr(o))
        return dict(pos=int(o[0]), claims=int(o[1]), drops=int(o[2]), error=int(o[3]))

    def __del__(self):
        if getattr(self, "_c", None):
            lib().co_free(self._c)
            self._c = None

    @property
    def host_tick(self) -> int:
        return int(lib().co_htick(self._c))

    def stats(self) -> dict:
        o = np.zeros(4, dtype=np.int64)
        lib().co_stats(self._c, _ptr(o))
        return dict(masked=int(o[0]), evicts=int(o[1]), admit_dropped=int(o[2]), ring_overflow=int(o[3]))

    def ensure(self, layer: int, ids: np.ndarray, w: np.ndarray, max_fill: int | None = None):
        """One decode-mode ensure call. ids int32 [P] and w fp32 [P] are masked IN PLACE (like the reference's
        topk_ids / topk_w). Returns the decision record (int32 [3 + 4P])."""
        assert ids.dtype == np.int32 and w.dtype == np.float32 and ids.flags.c_contiguous and w.flags.c_contiguous
        P = ids.size
        rec = np.zeros(rec_len(P), dtype=np.int32)
        lib().co_ensure(self._c, layer, _ptr(ids), _ptr(w), P, self.E if max_fill is None else max_fill, _ptr(rec))
        return rec

    def prefetch(self, layer: int, ids: np.ndarray, max_fill: int | None = None):
        """One prefetch-mode ensure (moe_prefetch): tick not advanced, no mask, no write-back. Returns the decision
        record (int32 [3 + 4P]); its assigned experts and slots are the prefetch's fill_list and pf_slot."""
        assert ids.dtype == np.int32 and ids.flags.c_contiguous
        P = ids.size
        rec = np.zeros(rec_len(P), dtype=np.int32)
        lib().co_prefetch(self._c, layer, _ptr(ids), P, self.E if max_fill is None else max_fill, _ptr(rec))
        return rec

    def plan(self, layer: int, ids: np.ndarray, max_fill: int | None = None):
        """One copy-engine plan (moe_prefetch_plan): a prefetch of at most 16 experts whose slots stay pinned until
        the next call commits them (the caller waits for the copy worker in between). Returns the decision record."""
        assert ids.dtype == np.int32 and ids.flags.c_contiguous
        P = ids.size
        rec = np.zeros(rec_len(P), dtype=np.int32)
        lib().co_plan(self._c, layer, _ptr(ids), P, self.E if max_fill is None else max_fill, _ptr(rec))
        return rec

    def host_step(self):
        """-> (admitted keys, evicted keys) of this host step."""
        adm = np.zeros(max(self.qmax, 1), dtype=np.int32)
        ev = np.zeros(self.L * self.E, dtype=np.int32)
        na, ne = np.zeros(1, np.int32), np.zeros(1, np.int32)
        lib().co_host_step(self._c, _ptr(adm), _ptr(na), _ptr(ev), _ptr(ne))
        return adm[:na[0]].copy(), ev[:ne[0]].copy()

    def run(self, ids: np.ndarray, w: np.ndarray, max_fill: int | None = None, host_log_cap: int = 1 << 24):
        """ids int32 [steps, L, P], w fp32 [steps, L, P] -> (records [steps, L, rec_len], host log list of
        (admitted, evicted) per step)."""
        steps, L, P = ids.shape
        assert L == self.L
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        recs = np.zeros((steps, L, rec_len(P)), dtype=np.int32)
        hl = np.zeros(host_log_cap, dtype=np.int32)
        n = lib().co_run(self._c, _ptr(ids), _ptr(w), steps, P, self.E if max_fill is None else max_fill,
                         _ptr(recs), _ptr(hl), host_log_cap)
        assert n >= 0, "host log capacity exceeded"
        log, pos = [], 0
        while pos < n:
            na, ne = int(hl[pos]), int(hl[pos + 1])
            pos += 2
            log.append((hl[pos:pos + na].copy(), hl[pos + na:pos + na + ne].copy()))
            pos += na + ne
        return recs, log
