"""
Two-tier EXL3 routed-expert store for MI355X: every expert of every MoE layer lives in pinned, device-mapped host
memory (tier 1, read zero-copy over PCIe by the kernels), a subset lives in HBM slots (tier 0, the expert cache). The
grouped MoE kernels (`torch.ops.exl3xpu_moe.moe_forward`, csrc/moe_decode.hip) address experts only through a per-layer
POINTER TABLE, so moving an expert between tiers is one 8-byte table write; both pointers stay valid.

Mirrors the reference's plugin/exl3xpu/moe_offload.py (API docstring :14-30) on PyTorch-ROCm streams and events.

Expert blob (`blob_bytes(H, I, K)` bytes; 1,195,008 B for H=2048, I=512, K=3):
  gate|up trellis (u32, [H/16][2I/16][8K], PLANAR4 word order) | down trellis ([I/16][H/16][8K], PLANAR4) |
  suh_g[H] suh_u[H] svh_g[I] svh_u[I] suh_d[I] svh_d[H]   (fp16)

API (device work is enqueued on the current stream unless noted; nothing syncs the host):
  store = ExpertStore(H, I, K, n_experts, n_slots)          # n_slots HBM slots shared by all layers
  store.add_layer(key, blobs_cpu [E, BLOB] uint8 | None)     # allocates the layer's pinned host arena (fills it)
  store.host_view(key)[e]                                    # uint8 view of expert e's host blob
  store.ptrs(key)                                            # int64 [E] device pointer table (fixed address)
  store.make_resident(key, experts, stream=None)             # copy blobs into free slots, then repoint
  store.evict(key, experts)                                  # repoint to host (slot reuse is stream-ordered)
  store.forward(key, x, topk_ids, topk_w) -> out             # routed-MoE output (weights applied)
  store.forward_cached(key, x, topk_ids, topk_w)            # decode through the DEVICE-managed LRU cache
  store.stage_layer(key, buf, stream) -> ptrs                # prefill: stage non-resident experts into buffer buf
  store.forward_prefill_staged(key, x, topk_ids, topk_w)     # prefill with next-layer staging on a copy stream
  store.slot_of[key]  (cpu int32 [E], -1 = host only)        # the slot map mirror
"""
from __future__ import annotations

import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_lib_loaded = False
_lock = threading.Lock()


def ops():
    """torch.ops.exl3xpu_moe, loading exl3xpu/_moe.so (or $EXL3_MOE_LIB) once (moe_offload.py:44-61). Raises if the
    HIP library is missing: there is no fallback path."""
    global _lib_loaded
    with _lock:
        if not _lib_loaded:
            path = os.environ.get("EXL3_MOE_LIB") or os.path.join(_HERE, "_moe.so")
            if not os.path.exists(path):
                raise RuntimeError(f"exl3xpu: HIP op library not built ({path}); run qwen38-flash-next-b70-offload_amd/build.py")
            torch.ops.load_library(path)

            @torch.library.register_fake("exl3xpu_moe::moe_forward")
            def _fake(x, topk_ids, topk_w, ptrs, I, K, n_experts):   # noqa: N803
                return torch.empty_like(x)

            @torch.library.register_fake("exl3xpu_moe::moe_forward_cached")
            def _fake_c(x, *args):
                return torch.empty_like(x)

            _lib_loaded = True
    return torch.ops.exl3xpu_moe


def s64(p: int) -> int:
    return p - (1 << 64) if p >= (1 << 63) else p


def planar4(tr: torch.Tensor, K: int) -> torch.Tensor:
    """int16 trellis [rows, tiles, 16K] -> int32 words in PLANAR4 order (moe_offload.py:68-73): per row, groups of 4
    tiles along n stored [plane i][tile][period g]. Even K (one word per period) keeps the natural order."""
    r, n, _ = tr.shape
    w = tr.contiguous().view(torch.int32)
    if K % 2 == 0:
        return w.contiguous()
    assert K in (1, 3, 5, 7), "PLANAR4 packing for odd K (K words per 32-value period)"
    w = w.view(r, n // 4, 4, 8, K)                                        # [row, group, tile, period g, plane i]
    return w.permute(0, 1, 4, 2, 3).contiguous()                         # [row, group, plane i, tile, g]


def pack_expert(gate: dict, up: dict, down: dict, K: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """Checkpoint tensors {trellis, suh, svh} of one expert -> blob (uint8 CPU tensor, or written into `out`)
    (moe_offload.py:76-89)."""
    b = lambda z: z.contiguous().view(torch.uint8).flatten()     # noqa: E731
    gu = torch.cat([gate["trellis"], up["trellis"]], dim=1)
    parts = [b(planar4(gu, K)), b(planar4(down["trellis"], K)), b(gate["suh"].half()), b(up["suh"].half()),
             b(gate["svh"].half()), b(up["svh"].half()), b(down["suh"].half()), b(down["svh"].half())]
    if out is None:
        return torch.cat(parts)
    o = 0
    for p in parts:
        out[o:o + p.numel()].copy_(p)
        o += p.numel()
    assert o == out.numel(), (o, out.numel())
    return out


def _default_device():
    return torch.device("cuda", torch.cuda.current_device())


class ExpertStore:
    """Slot arena + device cache state (moe_offload.py:92-124)."""

    def __init__(self, H: int, I: int, K: int, n_experts: int, n_slots: int, device=None, max_layers: int = 64):
        self.H, self.I, self.K, self.E = H, I, K, n_experts
        self.dev = torch.device(device) if device is not None else _default_device()
        self.X = ops()
        self.blob = int(self.X.blob_bytes(H, I, K))
        self.n_slots = n_slots
        self.max_layers = max_layers
        self.slots = torch.empty((n_slots, self.blob), dtype=torch.uint8, device=self.dev) if n_slots else None
        self.slot_owner: list = [None] * n_slots            # slot -> (key, e)   (static placement mirror)
        self.free_slots = list(range(n_slots - 1, -1, -1))
        self.host: dict = {}                                # key -> uint8 CPU tensor [E, BLOB] (pinned)
        self.layer_index: dict = {}                         # key -> row in the device tables
        self.slot_of: dict = {}                             # key -> cpu int32 [E] (mirror of static placement)
        self._host_ptr: dict = {}
        self._stage = [None, None]
        self._slot_ready_ev: dict = {}
        LE = max_layers * n_experts
        self.ptrs_all = torch.zeros(LE, dtype=torch.int64, device=self.dev)
        self.slot_of_dev = torch.full((LE,), -1, dtype=torch.int32, device=self.dev)
        self.slot_key = torch.full((n_slots,), -1, dtype=torch.int32, device=self.dev)
        self.slot_last = torch.full((n_slots,), -1, dtype=torch.int32, device=self.dev)
        self.tick = torch.zeros(1, dtype=torch.int32, device=self.dev)
        self.host_base = torch.zeros(max_layers, dtype=torch.int64, device=self.dev)
        self.fill_all = torch.zeros(LE, dtype=torch.int64, device=self.dev)
        self.fill_list = torch.zeros(1 + n_experts, dtype=torch.int32, device=self.dev)
        self.pf_list = torch.zeros(1 + n_experts, dtype=torch.int32, device=self.dev)   # prefetch: [n, e...]
        self.pf_slot = torch.zeros(n_experts, dtype=torch.int32, device=self.dev)       # prefetch: slot of each
        self.pend = torch.zeros(max_layers * 35, dtype=torch.int32, device=self.dev)
        self.done_seq = torch.zeros(0, dtype=torch.int32, device=self.dev)
        self.slot_base = s64(self.slots.data_ptr()) if n_slots else 0
        self._cache_used = False
        self.K_of: dict = {}                                # key -> bitrate of the layer (default K)
        self.X.moe_set_slot_stride(0)                       # slots at the blob size (mixed_bitrates() widens)

    # ---- layers
    def add_layer(self, key, blobs: torch.Tensor | None = None) -> torch.Tensor:
        li = len(self.layer_index)
        if li >= self.max_layers:
            raise RuntimeError(f"ExpertStore: more than max_layers={self.max_layers} MoE layers")
        self.layer_index[key] = li
        h = self.X.host_alloc(self.E * self.blob).view(self.E, self.blob)
        if blobs is not None:
            h.copy_(blobs)
        self.host[key] = h
        base = s64(h.data_ptr())
        self._host_ptr[key] = base + torch.arange(self.E, dtype=torch.int64) * self.blob
        self.ptrs_all[li * self.E:(li + 1) * self.E].copy_(self._host_ptr[key])
        self.host_base[li] = base
        self.slot_of[key] = torch.full((self.E,), -1, dtype=torch.int32)
        return h

    def host_view(self, key) -> torch.Tensor:
        return self.host[key]

    def mixed_bitrates(self) -> None:
        """Layers of this store use different bitrates K <= the store's K: slots (and host records) keep the size of
        the largest blob, and the device cache addresses slots at that stride (moe_set_slot_stride). Layers with a
        smaller K read and write only their own blob bytes; victims are written back as whole slots."""
        self.X.moe_set_slot_stride(self.blob)

    def k_of(self, key) -> int:
        return self.K_of.get(key, self.K)

    def ptrs(self, key) -> torch.Tensor:
        li = self.layer_index[key]
        return self.ptrs_all[li * self.E:(li + 1) * self.E]

    def slot_ptr(self, s: int) -> int:
        return self.slot_base + s * self.blob

    # ---- static residency (load time / host-driven policies), moe_offload.py:154-216
    def make_resident(self, key, experts, stream=None) -> int:
        s_ = stream or torch.cuda.current_stream(self.dev)
        self._resync()
        so = self.slot_of[key]
        li = self.layer_index[key]
        todo = [int(e) for e in experts if so[int(e)] < 0]
        if not todo:
            return 0
        es, sls = [], []
        with torch.cuda.stream(s_):
            for e in todo:
                if not self.free_slots:
                    raise RuntimeError("ExpertStore: no free slot (evict first or raise n_slots)")
                sl = self.free_slots.pop()
                ev = self._slot_ready_ev.pop(sl, None)
                if ev is not None:
                    s_.wait_event(ev)
                self.X.memcpy_async(self.slot_ptr(sl), self._host_addr(key, e), self.blob)
                self.slot_owner[sl] = (key, e)
                so[e] = sl
                es.append(e)
                sls.append(sl)
            keys = torch.tensor([li * self.E + e for e in es], dtype=torch.int64)
            slt = torch.tensor(sls, dtype=torch.int64)
            d = self.dev
            self.ptrs_all.index_copy_(0, keys.to(d), (self.slot_base + slt * self.blob).to(d))
            self.slot_of_dev.index_copy_(0, keys.to(d), slt.to(torch.int32).to(d))
            self.slot_key.index_copy_(0, slt.to(d), keys.to(torch.int32).to(d))
            self.slot_last.index_fill_(0, slt.to(d), 0)
        return len(todo)

    def _host_addr(self, key, e: int) -> int:
        return int(self._host_ptr[key][e])

    def evict(self, key, experts) -> None:
        self._resync()
        so = self.slot_of[key]
        li = self.layer_index[key]
        es, sls = [], []
        for e in experts:
            e = int(e)
            sl = int(so[e])
            if sl < 0:
                continue
            es.append(e)
            sls.append(sl)
            so[e] = -1
            self.slot_owner[sl] = None
        if not es:
            return
        d = self.dev
        et = torch.tensor(es, dtype=torch.int64)
        keys = (li * self.E + et).to(d)
        slt = torch.tensor(sls, dtype=torch.int64).to(d)
        self.ptrs_all.index_copy_(0, keys, self._host_ptr[key][et].to(d))
        self.slot_of_dev.index_fill_(0, keys, -1)
        self.slot_key.index_fill_(0, slt, -1)
        self.slot_last.index_fill_(0, slt, -1)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.dev))
        for sl in sls:
            self._slot_ready_ev[sl] = ev
            self.free_slots.append(sl)

    def resident_count(self, key=None) -> int:
        if key is None:
            return sum(int((v >= 0).sum()) for v in self.slot_of.values())
        return int((self.slot_of[key] >= 0).sum())

    def device_resident_count(self, key) -> int:
        li = self.layer_index[key]
        return int((self.slot_of_dev[li * self.E:(li + 1) * self.E] >= 0).sum().item())

    # ---- compute (moe_offload.py:218-249)
    @staticmethod
    def _rt(topk_ids, topk_w):
        ids = topk_ids if topk_ids.dtype == torch.int32 and topk_ids.is_contiguous() else topk_ids.to(torch.int32).contiguous()
        w = topk_w if topk_w.dtype == torch.float32 and topk_w.is_contiguous() else topk_w.to(torch.float32).contiguous()
        return ids, w

    def forward(self, key, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, ptrs=None) -> torch.Tensor:
        ids, w = self._rt(topk_ids, topk_w)
        return self.X.moe_forward(x, ids, w, self.ptrs(key) if ptrs is None else ptrs, self.I, self.k_of(key), self.E)

    def forward_cached(self, key, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor,
                       max_fill: int | None = None) -> torch.Tensor:
        """Decode with the device-managed LRU expert cache: hits read their slot, misses read host memory zero-copy
        and are written through into the LRU slot (committed at the end of the call). No host sync, graph-safe.
        With the RAM tier on, the masked picks are rewritten in `topk_ids` / `topk_w` when those are int32 / fp32
        contiguous (otherwise in the converted copies)."""
        ids, w = self._rt(topk_ids, topk_w)
        self._cache_used = True
        return self.X.moe_forward_cached(x, ids, w, self.ptrs_all, self.layer_index[key], self.slot_of_dev,
                                         self.slot_key, self.slot_last, self.tick, self.host_base, self.slot_base,
                                         self.fill_all, self.fill_list, self.E if max_fill is None else max_fill,
                                         self.I, self.k_of(key), self.E, self.pend, self.done_seq)

    def prefetch(self, key, ids: torch.Tensor, max_fill: int = 16) -> None:
        """Bring the predicted experts `ids` of layer `key` into HBM slots ahead of their MoE call (moe_offload.py:
        251-262): the device cache claims exact-LRU slots for up to `max_fill` of them that are not resident, without
        advancing the tick (slots used by the last MoE call are never taken), copies them from their host records and
        repoints the layer's table. Everything is enqueued on the current stream; run it on a side stream that has
        waited for the previous MoE call, and make the compute stream wait for that stream before the next one."""
        if not self.n_slots:
            return
        ids = ids if ids.dtype == torch.int32 and ids.is_contiguous() else ids.to(torch.int32).contiguous()
        self._cache_used = True
        self.X.moe_prefetch(ids.flatten(), self.ptrs_all, self.layer_index[key], self.slot_of_dev, self.slot_key,
                            self.slot_last, self.tick, self.host_base, self.slot_base, self.pf_list, self.pf_slot,
                            max_fill, self.E, int(self.X.blob_bytes(self.H, self.I, self.k_of(key))))

    # ---- copy-engine prefetch (moe_offload.py:264-302): device plan -> host worker -> copies -> device commit
    def start_copy_prefetch(self) -> None:
        """Start the host worker that copies the experts of published prefetch plans into their slots on a
        dedicated stream; later ensures (forward_cached, plan_prefetch) commit the plans whose copies finished."""
        L, E = len(self.layer_index), self.E
        self._plans = self.X.host_alloc(L * (4 + 2 * E) * 4)
        self._plans.zero_()
        self._plan_seq = torch.zeros(L, dtype=torch.int32, device=self.dev)
        self.done_seq = torch.zeros(L, dtype=torch.int32, device=self.dev)
        self.pend.zero_()
        self._commit_host = self.X.host_alloc(L * 2 * 4)
        hb = torch.zeros(L, dtype=torch.int64)
        for key, li in self.layer_index.items():
            hb[li] = int(self._host_ptr[key][0])
        torch.cuda.synchronize(self.dev)
        self._pf_stream = torch.cuda.Stream(self.dev)
        with torch.cuda.stream(self._pf_stream):                 # the worker's copies go to this stream
            self.X.moe_prefetch_worker_start(self._plans, hb, self.slot_base, self.blob, self.ptrs_all,
                                             self.slot_last, self._commit_host, self.done_seq, L, E)

    def plan_prefetch(self, key, ids: torch.Tensor, max_fill: int = 16) -> None:
        """On the compute stream (for instance right after the MoE call of the previous layer): claim and pin slots for
        up to 16 predicted experts of `key` and publish the plan to the worker. The compute stream never waits for the
        copies; the experts are used from their slots once a later ensure has committed the plan."""
        ids = ids if ids.dtype == torch.int32 and ids.is_contiguous() else ids.to(torch.int32).contiguous()
        self._cache_used = True
        self.X.moe_prefetch_plan(ids.flatten(), self.ptrs_all, self.layer_index[key], self.slot_of_dev, self.slot_key,
                                 self.slot_last, self.tick, self.host_base, self.slot_base, self.pf_list, self.pf_slot,
                                 self._plans, self._plan_seq, self.pend, self.done_seq, max_fill, self.E, self.blob)

    def stop_copy_prefetch(self):
        """Stop the worker (its stream drained), commit what finished with one empty ensure pass, and return
        [plans handled, experts copied]; forward_cached then runs without plan commits."""
        r = self.X.moe_prefetch_worker_stop()
        if self.done_seq.numel():
            k0 = next(iter(self.layer_index))
            x = torch.zeros((1, self.H), dtype=torch.bfloat16, device=self.dev)
            ids = torch.zeros((1, 1), dtype=torch.int32, device=self.dev)
            self.forward_cached(k0, x, ids, torch.ones((1, 1), device=self.dev), max_fill=0)
            torch.cuda.synchronize(self.dev)
            self.done_seq = torch.zeros(0, dtype=torch.int32, device=self.dev)
        return r

    # ---- prefill staging (moe_offload.py:305-462)
    def stage_layer(self, key, buf: int, stream) -> torch.Tensor:
        """Copy every non-resident expert of `key` into staging buffer `buf` on `stream`; returns the pointer table
        to pass to forward(ptrs=...) once `stream` has been waited on. Contiguous expert runs are copied together."""
        if self._stage[buf] is None:
            self._stage[buf] = torch.empty((self.E, self.blob), dtype=torch.uint8, device=self.dev)
        st = self._stage[buf]
        self._resync()
        so = self.slot_of[key]
        miss = (so < 0).nonzero().flatten().tolist()
        # runs of consecutive experts are one copy when host copies are packed at the blob size (a TierStore arena
        # has a 4 KiB-rounded stride: one copy per expert there)
        packed = self._host_addr(key, 1) - self._host_addr(key, 0) == self.blob if self.E > 1 else True
        with torch.cuda.stream(stream):
            i = 0
            while i < len(miss):
                j = i
                while packed and j + 1 < len(miss) and miss[j + 1] == miss[j] + 1:
                    j += 1
                n = j - i + 1
                self.X.memcpy_async(s64(st[miss[i]].data_ptr()), self._host_addr(key, miss[i]), n * self.blob)
                i = j + 1
        sp = s64(st.data_ptr()) + torch.arange(self.E, dtype=torch.int64) * self.blob
        if self.n_slots:
            dp = self.slot_base + so.clamp_min(0).to(torch.int64) * self.blob
            sp = torch.where(so >= 0, dp, sp)
        return sp.to(self.dev)

    def reset_cache(self) -> None:
        """Empty every slot and repoint all tables to host memory (current stream; waits for queued work)."""
        torch.cuda.current_stream(self.dev).synchronize()
        for key, li in self.layer_index.items():
            self.ptrs_all[li * self.E:(li + 1) * self.E].copy_(self._host_ptr[key])
            self.slot_of[key].fill_(-1)
        self.slot_of_dev.fill_(-1)
        self.slot_key.fill_(-1)
        self.slot_last.fill_(-1)
        self.fill_all.zero_()
        self.pend.zero_()
        self.tick.zero_()
        self.slot_owner = [None] * self.n_slots
        self.free_slots = list(range(self.n_slots - 1, -1, -1))
        self._slot_ready_ev.clear()
        self._cache_used = False

    def forward_prefill_staged(self, key, x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor) -> torch.Tensor:
        """Prefill-size MoE for layer `key` from a device staging buffer: the layer's non-resident experts are copied
        H2D on a side stream (normally already done while the previous layer computed), then this call starts staging
        the NEXT layer into the other buffer. Resident experts are read from their cache slots."""
        if not hasattr(self, "_pf"):
            self._pf = {"stream": torch.cuda.Stream(self.dev), "buf_of": {}, "ready": {}, "free": [None, None],
                        "order": None}
        pf = self._pf
        if pf["order"] is None or len(pf["order"]) != len(self.layer_index):
            pf["order"] = list(self.layer_index)
            import re as _re

            def _lid(k):
                m = _re.search(r"layers\.(\d+)\.", str(k))
                return int(m.group(1)) if m else self.layer_index[k]
            pf["layers"] = sorted((k for k in pf["order"] if not str(k).startswith("mtp.")), key=_lid)
        cs = torch.cuda.current_stream(self.dev)
        if pf["layers"] and key == pf["layers"][0]:
            torch.cuda.synchronize(self.dev)
            t = int(self.tick.item())
            if pf.get("tick") != t or self._cache_used:
                self.sync_mirror()
                self._cache_used = False
                pf["buf_of"].clear()
                pf["ready"].clear()
                pf["tick"] = t
        if key not in pf["buf_of"]:
            used = {b for b, _ in pf["buf_of"].values()}
            self._stage_into(key, 0 if 0 not in used else 1)
        buf, table = pf["buf_of"].pop(key)
        rdy = pf["ready"].pop(key)
        cs.wait_event(rdy)
        ids, w = self._rt(topk_ids, topk_w)
        y = self.X.moe_forward(x, ids, w, table, self.I, self.k_of(key), self.E)
        ev = torch.cuda.Event()
        ev.record(cs)
        pf["free"][buf] = ev
        layers = pf["layers"]
        pos = layers.index(key) if key in layers else -1
        if pos >= 0 and layers:
            nxt = layers[(pos + 1) % len(layers)]
            if nxt not in pf["buf_of"] and nxt != key:
                self._stage_into(nxt, 1 - buf)
        return y

    def _stage_into(self, key, buf: int) -> None:
        pf = self._pf
        st = pf["stream"]
        for k_ in [k_ for k_, (b_, _) in pf["buf_of"].items() if b_ == buf]:
            pf["buf_of"].pop(k_)
            pf["ready"].pop(k_, None)
        if pf["free"][buf] is not None:
            st.wait_event(pf["free"][buf])
            pf["free"][buf] = None
        table = self.stage_layer(key, buf, st)
        ev = torch.cuda.Event()
        ev.record(st)
        pf["buf_of"][key] = (buf, table)
        pf["ready"][key] = ev

    def prefill_reset(self) -> None:
        if hasattr(self, "_pf") and self._pf["buf_of"]:
            self._pf["buf_of"].clear()
            self._pf["ready"].clear()

    def sync_mirror(self) -> None:
        """Rebuild the CPU mirror (slot_of, slot_owner, free list) from the device cache state (syncs)."""
        sk = self.slot_key.cpu()
        sod = self.slot_of_dev.cpu()
        keys = {li: key for key, li in self.layer_index.items()}
        for key, li in self.layer_index.items():
            self.slot_of[key] = sod[li * self.E:(li + 1) * self.E].clone()
        self.slot_owner = [None] * self.n_slots
        free = []
        for sl in range(self.n_slots):
            k = int(sk[sl])
            if k < 0:
                free.append(sl)
            else:
                self.slot_owner[sl] = (keys[k // self.E], k % self.E)
        self.free_slots = free[::-1]

    def _resync(self) -> None:
        if self._cache_used:
            self.sync_mirror()
            self._cache_used = False
