"""CPU replay of the prefill staging pipeline (ExpertStore.forward_prefill_staged) at the full config-3 shape: 48
layers x 512 experts of 1,195,008 B, 8,000 HBM-resident keys, two forwards back to back. Streams, events, the copies
and the MoE calls are recorded instead of run; the test checks from that record that every layer reads a table built
for its own staging, that its copies are ordered before its kernel, and that no later copy into the same staging
buffer can overtake that kernel."""
import numpy as np
import pytest
import torch

from exl3xpu import moe_offload as mo


class _Timeline:
    """Operations in host order on named streams; an event is a position on a stream; wait(e) orders the stream's
    next operations after everything up to e."""

    def __init__(self):
        self.ops = []                    # (stream, kind, payload, vector clock)
        self.vc = {}

    def _clock(self, s):
        return self.vc.setdefault(s, {})

    def op(self, s, kind, payload=None):
        c = self._clock(s)
        c[s] = c.get(s, 0) + 1
        self.ops.append((s, kind, payload, dict(c)))
        return len(self.ops) - 1

    def event(self, s):
        return dict(self._clock(s))

    def wait(self, s, ev):
        c = self._clock(s)
        for k, v in ev.items():
            c[k] = max(c.get(k, 0), v)

    def before(self, i, j):
        """operation i happens before operation j"""
        si, _, _, ci = self.ops[i]
        return self.ops[j][3].get(si, 0) >= ci[si]


class _Event:
    def __init__(self, tl):
        self.tl, self.at = tl, None

    def record(self, stream):
        self.at = self.tl.event(stream.name)

    def synchronize(self):
        pass


class _Stream:
    def __init__(self, tl, name):
        self.tl, self.name = tl, name

    def wait_event(self, ev):
        self.tl.wait(self.name, ev.at)


class _FakeStager:
    """_Stager's interface over the timeline: fill = wait for the buffer's release, one copy op, an event."""

    def __init__(self, tl, E, rec):
        self.tl, self.E, self.rec = tl, E, rec
        self.stream = _Stream(tl, "copy")
        self.released = [None, None]
        self.serial = 0

    def fill(self, b, src_addr, missing, lo, hi):
        if self.released[b] is not None:
            self.stream.wait_event(self.released[b])
            self.released[b] = None
        self.serial += 1
        self.tl.op("copy", "copy", (b, self.serial))
        ev = _Event(self.tl)
        ev.record(self.stream)
        return ev

    def table(self, b, slot_of, slot_base, slot_stride):
        return ("table", b, self.serial)

    def release(self, b, stream):
        ev = _Event(self.tl)
        ev.record(stream)
        self.released[b] = ev


class _FakeStore:
    def __init__(self, tl, L, E, resident):
        self.tl, self.E = tl, E
        self.dev = torch.device("cpu")
        self.layer_index = {f"model.layers.{li}.mlp": li for li in range(L)}
        self.slot_of = {}
        for k, li in self.layer_index.items():
            so = np.full(E, -1, dtype=np.int32)
            r = resident[resident // E == li] % E
            so[r] = np.arange(r.size)
            self.slot_of[k] = torch.from_numpy(so)
        rec = mo._HostRecords(1 << 40, 1196032, 1 << 40, (1 << 40) + L * E * 1196032, None)
        self._host = {k: rec for k in self.layer_index}
        self.slot_base, self.slot_stride = 1 << 44, 1195008
        self.tick = torch.zeros(1, dtype=torch.int32)
        self._mirror_stale = False
        self.compute = _Stream(tl, "compute")
        self.reads = []

    def _refresh_mirror(self):
        pass

    def sync_mirror(self):
        pass

    def forward(self, key, x, ids, w, ptrs=None):
        i = self.tl.op("compute", "read", ptrs)
        self.reads.append((key, i))
        return x


@pytest.mark.parametrize("forwards", [2])
def test_staged_pipeline_order_full_size(monkeypatch, forwards):
    L, E = 48, 512
    tl = _Timeline()
    resident = np.random.default_rng(3).choice(L * E, 8000, replace=False)
    st = _FakeStore(tl, L, E, resident)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a, **k: st.compute)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    pipe = mo._PrefillPipeline.__new__(mo._PrefillPipeline)
    pipe.st, pipe.stager, pipe.ready, pipe.tick, pipe._order_n, pipe.order = st, _FakeStager(tl, E, 1196032), {}, \
        None, -1, []
    keys = list(st.layer_index)
    for _ in range(forwards):
        for k in keys:
            pipe.run(k, None, None, None)
    copies = [(i, op[2]) for i, op in enumerate(tl.ops) if op[1] == "copy"]
    reads = [(i, op[2]) for i, op in enumerate(tl.ops) if op[1] == "read"]
    assert len(reads) == forwards * L and len(copies) >= forwards * L
    for ri, (_, b, serial) in reads:
        own = [ci for ci, (cb, cs) in copies if cs == serial]
        assert len(own) == 1 and copies[[c[0] for c in copies].index(own[0])][1][0] == b
        assert tl.before(own[0], ri), "a layer's kernel is not ordered after its staging copies"
        for ci, (cb, cs) in copies:
            if cb == b and cs > serial:
                assert tl.before(ri, ci), "a later staging into the buffer can overtake the kernel reading it"
    # the first forward reads layers in model order, each from the staging made for it
    assert [k for k, _ in st.reads[:L]] == keys
