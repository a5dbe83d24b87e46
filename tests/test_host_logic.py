"""Product host logic against the oracle, on the CPU: the admission policy, the PLANAR4 packer and the synthetic
expert generator."""
import numpy as np
import pytest
import torch

from exl3xpu import moe_offload, nvtier
from exl3xpu import synth as psynth
from oracle import cache, exl3, synth


def test_pack_expert_matches_oracle():
    for K in (2, 3, 4):
        g, u, d = synth.expert_checkpoint(np.random.default_rng(K), 256, 128, K)
        ref = exl3.pack_expert(g, u, d, K)
        tg = {k: torch.from_numpy(v) for k, v in g.items()}
        tu = {k: torch.from_numpy(v) for k, v in u.items()}
        td = {k: torch.from_numpy(v) for k, v in d.items()}
        got = moe_offload.pack_expert(tg, tu, td, K).numpy()
        assert np.array_equal(got, ref)
        out = torch.empty(ref.size, dtype=torch.uint8)
        moe_offload.pack_expert(tg, tu, td, K, out=out)
        assert np.array_equal(out.numpy(), ref)


def test_product_synth_matches_oracle_synth():
    for K in (2, 3, 4):
        assert np.array_equal(psynth.expert_blob(5, 3, 256, 128, K).numpy(), synth.expert_blob(5, 3, 256, 128, K))
    a = psynth.zipf_trace(9, 3, 4, 64, 6, M=2)
    b = synth.zipf_trace(9, 3, 4, 64, 6, M=2)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


@pytest.mark.parametrize("seed,R", [(0, 256), (1, 256), (2, 16)])
def test_admission_policy_matches_oracle(seed, R):
    """Drive two copies of the oracle's device simulation with the same trace: one uses the oracle's host step, the
    other the product's AdmissionPolicy fed with one-step-lagged snapshots exactly as NvTierAsync.step() takes them."""
    L, E, S, P = 6, 32, 40, 5
    budget, age, qmax, lat = 45, 4, 12, 3
    steps = 300
    ids, w = synth.zipf_trace(100 + seed, steps, L, E, P)
    ids, w = ids[:, :, 0], w[:, :, 0]
    A = cache.CacheOracle(L, E, S, ring_cap=R, budget=budget, age=age, qmax=qmax, latency=lat)
    B = cache.CacheOracle(L, E, S, ring_cap=R, budget=budget, age=age, qmax=qmax, latency=lat)
    pol = nvtier.AdmissionPolicy(L * E, [li * E for li in range(L)], budget, age, qmax, R)
    snaps, last_diff, pending = [], None, {}
    for n in range(steps):
        for li in range(L):
            ra = A.ensure(li, ids[n, li].copy(), w[n, li].copy())
            rb = B.ensure(li, ids[n, li].copy(), w[n, li].copy())
            assert np.array_equal(ra, rb)
        adm_a, ev_a = A.host_step()
        pol.tick += 1
        snaps.append((B.ram_res.copy(), B.ring.copy(), B.slot_of.astype(np.int32)))
        if len(snaps) < 2:
            assert len(adm_a) == 0 and len(ev_a) == 0
            continue
        view, ring, slot_of = snaps[-2][0].copy(), snaps[-2][1], snaps[-2][2]
        if last_diff is not None:
            view[last_diff[0]] = last_diff[1]
        adm, ev, dk, dv = pol.decide(view, ring, slot_of, pending.pop(n, []))
        pending.setdefault(n + lat, []).extend(adm.tolist())
        B.ram_res[dk] = dv
        last_diff = (dk, dv) if len(dk) else None
        assert adm.tolist() == adm_a.tolist(), n
        assert ev.tolist() == ev_a.tolist(), n
        assert np.array_equal(B.ram_res, A.ram_res)
        assert np.array_equal(pol.res, A.res) and np.array_equal(pol.inflight, A.inflight.astype(bool))
    if R == 16:
        assert pol.stats["ring_overflow"] > 0          # the small ring overflowed and was handled like the oracle's


def test_admission_rejects_corrupt_snapshots():
    """A miss-ring key or completed key outside [0, n) is an error, and leaves the books usable."""
    n, R = 64, 32
    pol = nvtier.AdmissionPolicy(n, [0], budget=8, age=4, qmax=4, ring_cap=R)
    view = pol.res.copy()
    slot = np.full(n, -1, dtype=np.int32)
    ring = np.zeros(1 + R, dtype=np.int32)
    ring[0], ring[1], ring[2] = 2, 5, n + 3
    with pytest.raises(RuntimeError):
        pol.decide(view, ring, slot, [])
    with pytest.raises(RuntimeError):
        pol.decide(view, np.zeros(1 + R, dtype=np.int32), slot, [n])
    ring[2] = 5
    adm, ev, dk, dv = pol.decide(view, ring, slot, [])
    assert adm.tolist() == [5] and ev.size == 0 and dk.size == 0
    assert pol.inflight[5] and pol.stats["masked"] == 2



@pytest.mark.parametrize("offset", [(1 << 31) - 40, (1 << 32) - 40])
def test_admission_ring_count_wraps(offset):
    """The device miss-ring count is kept modulo 2^32 (entry c at position (c mod 2^32) % cap). Feeding the policy
    the oracle's snapshots with every count shifted by `offset` (crossing INT32_MAX, or 2^32 back to 0, within the
    first steps) gives the decisions of the unshifted run."""
    L, E, S, P, R = 6, 32, 40, 5, 256                  # R divides 2^32: a shift moves every entry by offset % R
    budget, age, qmax, lat, steps = 45, 4, 12, 3, 120
    ids, w = synth.zipf_trace(300, steps, L, E, P)
    ids, w = ids[:, :, 0], w[:, :, 0]
    A = cache.CacheOracle(L, E, S, ring_cap=R, budget=budget, age=age, qmax=qmax, latency=lat)
    pols = [nvtier.AdmissionPolicy(L * E, [li * E for li in range(L)], budget, age, qmax, R) for _ in range(2)]
    pols[1].ring_seen = offset
    snaps, diffs, pending, crossed = [], [None, None], [{}, {}], False
    for n in range(steps):
        for li in range(L):
            A.ensure(li, ids[n, li].copy(), w[n, li].copy())
        for p in pols:
            p.tick += 1
        snaps.append((A.ram_res.copy(), A.ring.copy(), A.slot_of.astype(np.int32)))
        A.host_step()
        if len(snaps) < 2:
            continue
        view0, ring, slot_of = snaps[-2]
        shifted = np.empty_like(ring)
        cnt = (int(ring[0]) + offset) & 0xFFFFFFFF
        shifted[0] = np.array(cnt, dtype=np.uint32).view(np.int32)
        shifted[1:] = np.roll(ring[1:], offset % R)
        crossed |= cnt < offset or cnt >= (1 << 31) > offset      # wrapped to 0, or negative as an int32
        out = []
        for i, (p, rg) in enumerate(zip(pols, (ring, shifted))):
            view = view0.copy()
            if diffs[i] is not None:
                view[diffs[i][0]] = diffs[i][1]
            adm, ev, dk, dv = p.decide(view, rg, slot_of, pending[i].pop(n, []))
            pending[i].setdefault(n + lat, []).extend(adm.tolist())
            diffs[i] = (dk, dv) if len(dk) else None
            out.append((adm.tolist(), ev.tolist(), dk.tolist(), dv.tolist()))
        assert out[0] == out[1], n
        assert (pols[1].ring_seen - pols[0].ring_seen) & 0xFFFFFFFF == offset % (1 << 32)
    assert crossed and pols[0].stats == pols[1].stats and pols[0].stats["masked"] > 40


def test_plan_copies_merges_contiguous_runs():
    """Staging copies: every missing record is covered exactly once, no copy spans a record that is not missing or a
    gap between host records, and runs are maximal."""
    rng = np.random.default_rng(7)
    rec = 4096 * 3
    for E, stride_gap in [(512, 0), (64, 4096), (33, 0)]:
        src = (1 << 40) + np.arange(E, dtype=np.int64) * (rec + stride_gap)
        src[E // 2:] += 8192 * 7                         # a break in host contiguity halfway
        for _ in range(20):
            missing = np.sort(rng.choice(E, rng.integers(0, E + 1), replace=False))
            dst, srcs, nb = moe_offload.plan_copies(1 << 44, rec, src, missing)
            covered = []
            for d, s, n in zip(dst, srcs, nb):
                assert n % rec == 0 and n > 0
                e0 = (d - (1 << 44)) // rec
                run = list(range(e0, e0 + n // rec))
                covered += run
                assert all(src[e] == s + (e - e0) * rec for e in run)        # host records contiguous along the run
            assert covered == missing.tolist()
            # maximal: two consecutive copies are not mergeable
            for i in range(len(dst) - 1):
                e_end = (dst[i] - (1 << 44)) // rec + nb[i] // rec
                assert not (e_end == (dst[i + 1] - (1 << 44)) // rec and srcs[i] + nb[i] == srcs[i + 1])


def test_evict_order_matches_sequential_classes():
    """_evict_order (one lexsort over class, age, key) equals the eviction loop it replaces: classes in order, each
    by a stable argsort of age over ascending keys, until `over` keys are taken (nvtier.py:414-419)."""
    rng = np.random.default_rng(11)
    for _ in range(200):
        n = int(rng.integers(1, 300))
        age = rng.integers(0, 6, n)
        masks = [rng.random(n) < 0.3 for _ in range(3)]
        masks[1] &= ~masks[0]
        masks[2] &= ~(masks[0] | masks[1])
        over = int(rng.integers(0, n + 2))
        want, left = [], over
        for m in masks:
            if left <= 0:
                break
            c = np.nonzero(m)[0]
            c = c[np.argsort(age[c], kind="stable")[:left]]
            want += c.tolist()
            left -= len(c)
        assert nvtier._evict_order(over, masks, age).tolist() == want


def test_staged_prefill_routes_zero_copy_above_limit():
    """Above STAGE_VERIFIED_BYTES per staging buffer (every real expert count: 512 records of 1,196,032 B need 612
    MB), the staged entry points never build a stager: ExpertStore.forward_prefill_staged runs forward() on the
    layer's own table, stage_layer returns that table, and NvTier.stage_forward makes the batch RAM-resident
    (ensure_for_prefill) and then runs forward(); nothing is staged. At or below the limit they stage."""
    import torch
    from exl3xpu import moe_offload, nvtier
    assert moe_offload.staging_fits(16, 131072) and not moe_offload.staging_fits(16, 131073)
    assert not moe_offload.staging_fits(512, 1196032)
    calls = []
    st = moe_offload.ExpertStore.__new__(moe_offload.ExpertStore)
    st.E, st.slot_stride, st._pipeline = 512, 1196032, None
    st.forward = lambda key, x, ids, w, ptrs=None: calls.append(("forward", key, ptrs)) or "y"
    st.ptrs = lambda key: torch.arange(4)
    assert st.forward_prefill_staged("k0", None, None, None) == "y"
    assert calls == [("forward", "k0", None)] and st._pipeline is None
    assert torch.equal(st.stage_layer("k0", 0, None), torch.arange(4)) and st._pipeline is None
    calls.clear()
    tier = nvtier.NvTier.__new__(nvtier.NvTier)
    tier.E, tier._streamer = 512, None
    tier.ensure_for_prefill = lambda li, ids: calls.append(("ensure", li, ids))

    class _Store:
        stride = 1196032

        def forward(self, key, x, ids, w):
            calls.append(("forward", key))
            return "y"
    assert tier.stage_forward(_Store(), "k3", 3, "x", "ids", "w") == "y"
    assert calls == [("ensure", 3, "ids"), ("forward", "k3")] and tier._streamer is None


def test_status_watch_raises_when_the_mirror_moves():
    """The ExpertStore wrappers read the host mirror of the device timeout count (pinned host memory that a timed-out
    bounded wait raises) before enqueueing anything, and raise RuntimeError once per change of it; forward,
    forward_cached and prefetch all check, and the failed call enqueues nothing."""
    from exl3xpu.moe_offload import ExpertStore, _StatusWatch
    word = np.zeros(4, dtype=np.int32)
    w = _StatusWatch(word)
    w.check()
    word[0] = 3
    with pytest.raises(RuntimeError, match="3 bounded waits"):
        w.check()
    w.check()                                            # reported once
    st = ExpertStore.__new__(ExpertStore)
    st._watch, st.n_slots = _StatusWatch(word), 4
    st._routing = lambda *a: pytest.fail("enqueued after a timeout")
    st._ids32 = st._routing
    for n, call in enumerate((lambda: st.forward_cached("k", None, None, None), lambda: st.forward("k", None, None, None),
                              lambda: st.prefetch("k", None), st.check_device_status)):
        word[0] = 4 + n
        with pytest.raises(RuntimeError, match="1 bounded waits"):
            call()
    st.check_device_status()


def test_record_pool_reuses_records_and_grows_by_chunks():
    """RecordPool bookkeeping on plain CPU memory (host_alloc stubbed): records come lowest address first from each
    chunk, given-back records are reused before the pool grows, the high-water mark and the pinned bytes follow,
    and view() finds a record's bytes."""
    class Stub:
        def __init__(self):
            self.allocs = []

        def host_alloc(self, n):
            t = torch.zeros(n, dtype=torch.uint8)
            self.allocs.append(t)
            return t

    X = Stub()
    pool = nvtier.RecordPool(X, 4096, chunk=4)
    a = pool.take(3)
    base = X.allocs[0].data_ptr()
    assert a.tolist() == [base, base + 4096, base + 8192]
    assert pool.records == 4 and pool.in_use == 3 and pool.high == 3
    b = pool.take(2)                                   # one left in the first chunk, then a second chunk
    assert len(X.allocs) == 2 and pool.records == 8 and pool.pinned_bytes == 8 * 4096
    assert len(set(a.tolist()) | set(b.tolist())) == 5
    pool.give(a[:2])
    pool.give(np.zeros(2, dtype=np.int64))             # zeros (no record) are ignored
    assert pool.in_use == 3 and pool.high == 5
    c = pool.take(2)
    assert sorted(c.tolist()) == sorted(a[:2].tolist()) and pool.records == 8
    pool.view(int(c[0]), 16)[:] = 7
    assert int(X.allocs[0][int(c[0]) - base]) == 7
    with pytest.raises(KeyError):
        pool.view(12345, 16)
