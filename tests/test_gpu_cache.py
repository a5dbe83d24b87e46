"""GPU parity of the device expert cache and the RAM tier: every ensure decision (mask set, miss list, victims with
write-back flags, slot ids, ring count) and every host admission/eviction decision must equal the oracle's, bit for
bit; outputs through the cache must equal outputs of the plain forward on the post-mask picks, bit for bit."""
import os

import numpy as np
import pytest
import torch

from oracle import cache, synth

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _setup(L, E, S, H, I, K, budget, qmax, age, latency, ring_cap, seed, pool=False, wb_queue=None,
           victim_ring=None):
    from exl3xpu import nvtier
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L, pool=pool)
    for li in range(L):
        store.add_layer(f"model.layers.{li}.mlp")
    src = nvtier.SyntheticExpertSource(H, I, K, seed, n_distinct=16)
    tier = nvtier.NvTierAsync(store, src, ring_cap=ring_cap, budget_records=budget, latency=latency,
                              wb_queue=wb_queue, victim_ring=victim_ring)
    tier.policy.admit_age, tier.policy.admit_qmax = age, qmax
    tier.log_decisions = True
    # reference table: every expert's true blob in HBM (independent of the cache)
    blobs = torch.from_numpy(src.buf).cuda()
    ref_ptr = torch.tensor([blobs[r % src.n].data_ptr() for r in range(L * E)], dtype=torch.int64, device="cuda")
    return store, tier, blobs, ref_ptr


def _run(store, tier, ids, w, H, check_out_every=0, ref_ptr=None, M=1):
    """ids/w [steps, L, P]: decode steps of M rows (P = M x top-k picks, row-major) through forward_cached + the host
    step; returns the device decision log (records) and optionally checks outputs against the plain forward."""
    X = store.X
    steps, L, P = ids.shape
    rl = cache.rec_len(P)
    logbuf = torch.zeros(1 + steps * L * rl, dtype=torch.int32, device="cuda")
    X.moe_set_decision_log(logbuf)
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).cuda()
    ids_d = torch.from_numpy(ids).cuda()
    w_d = torch.from_numpy(w).cuda()
    keys = list(store.layer_index)
    bad = 0
    try:
        for n in range(steps):
            for li in range(L):
                it = ids_d[n, li].view(M, P // M).clone()
                wt = w_d[n, li].view(M, P // M).clone()
                out = store.forward_cached(keys[li], x, it, wt)
                if check_out_every and n % check_out_every == 0:
                    E = store.E
                    ref = X.moe_forward(x, it, wt, ref_ptr[li * E:(li + 1) * E], store.I, store.K, E)
                    bad += int(not torch.equal(out, ref))
            tier.step()
        torch.cuda.synchronize()
    finally:
        X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
    lg = logbuf.cpu().numpy()
    assert lg[0] == steps * L
    return lg[1:].reshape(steps, L, rl), bad


@pytest.mark.parametrize("fused,pool", [(1, False), (0, False), (1, True), (0, True)])
def test_cache_golden_small(fused, pool):
    """fused 1: the ensure runs inside the layer kernel; 0: as its own launch before it. pool: the RAM tier keeps
    its records in a RecordPool (write-back queue of 8 records) instead of one fixed record per expert."""
    from pool_checks import check_pool, write_backs
    g = np.load(os.path.join(GOLD, "cache_small.npz"))
    L, E, S, P = int(g["L"]), int(g["E"]), int(g["S"]), int(g["P"])
    print(f"case cache golden L={L} E={E} S={S} fused={fused} pool={pool}", flush=True)
    H = I = 128
    store, tier, blobs, ref_ptr = _setup(L, E, S, H, I, 3, int(g["budget"]), int(g["qmax"]), int(g["age"]),
                                         int(g["latency"]), int(g["ring_cap"]), 3, pool=pool, wb_queue=8)
    store.X.moe_set_fused_ensure(fused)
    try:
        recs, bad = _run(store, tier, g["ids"], g["w"], H, check_out_every=1, ref_ptr=ref_ptr)
    finally:
        store.X.moe_set_fused_ensure(1)
    assert np.array_equal(recs, g["recs"])
    flat, pos = g["host_log"], 0
    for n, (adm, ev) in enumerate(tier.decisions):
        na, ne = int(flat[pos]), int(flat[pos + 1])
        pos += 2
        assert adm.tolist() == flat[pos:pos + na].tolist(), n
        assert ev.tolist() == flat[pos + na:pos + na + ne].tolist(), n
        pos += na + ne
    assert bad == 0
    if pool:
        wb = write_backs(g["recs"], P)
        check_pool(store, tier, tier.src, int(g["budget"]), int(wb[:-1].sum()))
    tier.close()


@pytest.mark.parametrize("pool", [False, True])
def test_cache_config1_trace_bitexact(pool):
    """48 layers x 512 experts, 8,000 slots, RAM budget 1,075 records, 4,000-step Zipf(1.1) trace of 10 picks per
    layer, 8-step fill latency, AGE 4, QMAX 256: every device and host decision equals the oracle's. Experts are tiny
    (H = I = 128): the decisions do not depend on the expert shape. pool: the RAM tier in a RecordPool (write-back
    queue of 48 records; the trace writes back up to 14 victims per step once HBM is full)."""
    from pool_checks import check_pool, write_backs
    L, E, S, P, steps = 48, 512, 8000, 10, int(os.environ.get("EXL3_TEST_C1_STEPS", "4000"))
    print(f"case cache config1 steps={steps} pool={pool}", flush=True)
    ids, w = synth.zipf_trace(20261202, steps, L, E, P)
    ids, w = ids[:, :, 0], w[:, :, 0]
    co = cache.CacheOracle(L, E, S, budget=1075, age=4, qmax=256, latency=8)
    orecs, olog = co.run(ids, w)
    store, tier, blobs, ref_ptr = _setup(L, E, S, 128, 128, 3, 1075, 256, 4, 8, 1 << 16, 7, pool=pool)
    recs, bad = _run(store, tier, ids, w, 128, check_out_every=97, ref_ptr=ref_ptr)
    mism = np.nonzero((recs != orecs).any(axis=-1))
    assert mism[0].size == 0, f"first mismatch at step/layer {mism[0][0]}/{mism[1][0]}"
    for n, ((a1, e1), (a2, e2)) in enumerate(zip(tier.decisions, olog)):
        assert a1.tolist() == a2.tolist() and e1.tolist() == e2.tolist(), n
    assert bad == 0
    if pool:
        check_pool(store, tier, tier.src, 1075, int(write_backs(orecs, P)[:-1].sum()))
    tier.close()


@pytest.mark.parametrize("fused,pool", [(1, False), (0, False), (1, True), (0, True)])
def test_cache_multirow_tier(fused, pool):
    """4 rows x top-10 per call (40 picks, duplicates across rows: the ensure inside the layer kernel when fused),
    6 layers x 128 experts, 150 slots, RAM tier of 160 records (AGE 4, QMAX 64, 3-step fill latency), Zipf(1.1)
    routing: every device record and host decision equals the oracle's and every output equals the plain forward.
    pool: the RAM tier in a RecordPool with a write-back queue of 48 records (the trace writes back up to 40 victims
    per step)."""
    from pool_checks import check_pool, write_backs
    L, E, S, M, TK, steps = 6, 128, 150, 4, 10, 80
    print(f"case cache multirow tier M={M} top-{TK} fused={fused} pool={pool}", flush=True)
    ids, w = synth.zipf_trace(20261203, steps, L, E, TK, M=M)
    ids = np.ascontiguousarray(ids.reshape(steps, L, M * TK))
    w = np.ascontiguousarray(w.reshape(steps, L, M * TK))
    co = cache.CacheOracle(L, E, S, ring_cap=1 << 12, budget=160, age=4, qmax=64, latency=3)
    orecs, olog = co.run(ids, w)
    store, tier, blobs, ref_ptr = _setup(L, E, S, 128, 128, 3, 160, 64, 4, 3, 1 << 12, 11, pool=pool, wb_queue=48)
    store.X.moe_set_fused_ensure(fused)
    try:
        recs, bad = _run(store, tier, ids, w, 128, check_out_every=1, ref_ptr=ref_ptr, M=M)
    finally:
        store.X.moe_set_fused_ensure(1)
    mism = np.nonzero((recs != orecs).any(axis=-1))
    assert mism[0].size == 0, f"first mismatch at step/layer {mism[0][0]}/{mism[1][0]}"
    for n, ((a1, e1), (a2, e2)) in enumerate(zip(tier.decisions, olog)):
        assert a1.tolist() == a2.tolist() and e1.tolist() == e2.tolist(), n
    assert bad == 0
    assert recs[:, :, 1].sum() > 0 and recs[:, :, 2 + M * TK].sum() > 0   # masked picks and fills happened
    if pool:
        wb = write_backs(orecs, M * TK)
        assert wb.sum() > 0
        check_pool(store, tier, tier.src, 160, int(wb[:-1].sum()))
    tier.close()


@pytest.mark.parametrize("H,I,steps", [(128, 128, 200), (4096, 1536, 12)])
def test_cache_mixed_bitrates(H, I, steps):
    """Layers of one store at K = 2, 3, 4 (128 experts, top-8, uniform routing), HBM slots for 30 % of the expert
    bytes (slot stride = the largest blob), every expert in the pinned RAM arena, no tier: each ensure decision equals
    the oracle's (plain device LRU) and every cached output equals the uncached output on the true blobs."""
    import ctypes
    from exl3xpu import nvtier
    L, E, P, Ks, nd = 3, 128, 8, [2, 3, 4], 4
    print(f"case mixed bitrates H={H} I={I} steps={steps}", flush=True)
    blob = [int(_blob(H, I, k)) for k in Ks]
    S = int(0.3 * E * sum(blob) / max(blob))
    store = nvtier.TierStore(H, I, 4, E, S, n_layers=L, Ks=Ks)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    srcs = [nvtier.SyntheticExpertSource(H, I, K, 90 + li, n_distinct=nd) for li, K in enumerate(Ks)]
    for key in range(L * E):
        ctypes.memmove(store.addr(key), srcs[key // E].buf[key % nd].ctypes.data, srcs[key // E].blob)
    dev = [torch.from_numpy(s.buf).cuda() for s in srcs]
    tables = [torch.tensor([dev[li][e % nd].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
              for li in range(L)]
    ids, w = synth.uniform_trace(91, steps, L, E, P)
    ids, w = ids[:, :, 0], w[:, :, 0]
    co = cache.CacheOracle(L, E, S, tier=False)
    orecs = np.stack([np.stack([co.ensure(li, ids[n, li].copy(), w[n, li].copy()) for li in range(L)])
                      for n in range(steps)])
    X = store.X
    rl = cache.rec_len(P)
    logbuf = torch.zeros(1 + steps * L * rl, dtype=torch.int32, device="cuda")
    X.moe_set_decision_log(logbuf)
    x = torch.randn(L, 1, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).cuda()
    bad = 0
    try:
        for n in range(steps):
            for li in range(L):
                it = torch.from_numpy(ids[n, li]).view(1, P).cuda()
                wt = torch.from_numpy(w[n, li]).view(1, P).cuda()
                out = store.forward_cached(keys[li], x[li], it, wt)
                ref = X.moe_forward(x[li], it, wt, tables[li], I, Ks[li], E)
                bad += int(not torch.equal(out, ref))
        torch.cuda.synchronize()
    finally:
        X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
    lg = logbuf.cpu().numpy()
    assert lg[0] == steps * L
    recs = lg[1:].reshape(steps, L, rl)
    mism = np.nonzero((recs != orecs).any(axis=-1))
    assert mism[0].size == 0, f"first mismatch at step/layer {mism[0][0]}/{mism[1][0]}"
    assert recs[:, :, 2 + P].sum() > 0                     # misses (and write-throughs) happened
    assert bad == 0


def _blob(H, I, K):
    from exl3xpu.moe_offload import ops
    return ops().blob_bytes(H, I, K)


@pytest.mark.parametrize("M,topk,fused", [(1, 8, 1), (1, 8, 0), (10, 8, 1)])
def test_cache_pinned_slots(M, topk, fused):
    """Slots pinned mid-trace (slot_last = INT_MAX, the reference's never-evict stamp) keep their stamp through hits
    and are never chosen as victims. 1 x top-8 runs the no-miss fast path and the full path; 10 x top-8 (80 picks)
    runs the full path only (as its own launch: more than 64 picks). fused 0 launches the ensure before the layer
    kernel. Every decision and the final slot_last table equal the oracle's."""
    import ctypes
    from exl3xpu import nvtier
    L, E, H, I, K, nd, steps, n0 = 2, 128, 128, 128, 3, 4, 60, 20
    P = M * topk
    print(f"case cache pinned slots M={M} top-{topk} fused={fused}", flush=True)
    S = 100
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    src = nvtier.SyntheticExpertSource(H, I, K, 77, n_distinct=nd)
    for key in range(L * E):
        ctypes.memmove(store.addr(key), src.buf[key % nd].ctypes.data, src.blob)
    rng = np.random.default_rng(78)
    # skewed routing so that hits (fast-path calls) and misses both occur
    pr = 1.0 / np.arange(1, E + 1) ** 1.5
    pr /= pr.sum()
    ids = np.stack([[np.stack([rng.choice(E, topk, replace=False, p=pr) for _ in range(M)]).reshape(-1)
                     for _ in range(L)] for _ in range(steps)]).astype(np.int32)
    w = rng.random(ids.shape, dtype=np.float32)
    co = cache.CacheOracle(L, E, S, tier=False)
    X = store.X
    rl = cache.rec_len(P)
    logbuf = torch.zeros(1 + steps * L * rl, dtype=torch.int32, device="cuda")
    X.moe_set_decision_log(logbuf)
    X.moe_set_fused_ensure(fused)
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    orecs = []
    try:
        for n in range(steps):
            if n == n0:
                torch.cuda.synchronize()
                held = np.nonzero(store.slot_key.cpu().numpy() >= 0)[0]
                assert held.size > 3 and np.array_equal(store.slot_last.cpu().numpy(), co.slot_last)
                pin = held[::3]
                store.slot_last[torch.from_numpy(pin).cuda()] = 0x7FFFFFFF
                co.slot_last[pin] = 0x7FFFFFFF
            for li in range(L):
                orecs.append(co.ensure(li, ids[n, li].copy(), w[n, li].copy()))
                it = torch.from_numpy(ids[n, li]).view(M, topk).cuda()
                wt = torch.from_numpy(w[n, li]).view(M, topk).cuda()
                store.forward_cached(keys[li], x, it, wt)
        torch.cuda.synchronize()
    finally:
        X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
        X.moe_set_fused_ensure(1)
    lg = logbuf.cpu().numpy()
    assert lg[0] == steps * L
    recs = lg[1:].reshape(steps * L, rl)
    orecs = np.stack(orecs)
    mism = np.nonzero((recs != orecs).any(axis=-1))[0]
    assert mism.size == 0, f"first mismatch at call {mism[0]}"
    sl = store.slot_last.cpu().numpy()
    assert np.array_equal(sl, co.slot_last)
    assert (sl[pin] == 0x7FFFFFFF).all()
    pinned_keys = store.slot_key.cpu().numpy()[pin]
    assert (pinned_keys >= 0).all()
    nm = recs[:, 2 + P]
    assert nm[n0 * L:].sum() > 0
    if P <= 64:
        assert (nm[n0 * L:] == 0).any()                    # no-miss (fast-path) calls after pinning too


def test_tier_exchange():
    """exl3_tier_exchange: the flag diff (keys outside [0, n) and negative entries skipped), the ring mirror (only the
    entries since `from`, wrapping, at most the last cap of them) and up to four copies into device-mapped pinned
    buffers, sizes that are not multiples of 16 included; misaligned copies are refused."""
    import ctypes
    from exl3xpu import capi
    from exl3xpu.moe_offload import ops
    X = ops()
    L = capi.lib()
    print("case tier exchange", flush=True)
    n = 24576
    g = torch.Generator().manual_seed(5)
    flags = torch.randint(0, 2, (n,), generator=g, dtype=torch.uint8).cuda()
    before = flags.cpu().numpy()
    diff = X.host_alloc(4 * 1000).view(torch.int32)
    keys = torch.randperm(n, generator=g)[:990].to(torch.int32)     # unique, as the tier's diffs are
    vals = torch.randint(0, 2, (990,), generator=g, dtype=torch.int32)
    dn = diff.numpy()
    dn[:990] = (keys.numpy() << 1) | vals.numpy()
    dn[990:995] = ((n + np.arange(5)) << 1) | 1          # beyond n_flags: skipped
    dn[995:1000] = -2                                     # negative: skipped
    sizes = [n, 4 * 24577 + 12]
    srcs = [flags, torch.randint(0, 255, (sizes[1],), generator=g, dtype=torch.uint8).cuda()]
    dsts = [X.host_alloc(sz) for sz in sizes]
    for d in dsts:
        d.fill_(0xAB)
    c_src = (ctypes.c_void_p * 2)(*[t.data_ptr() for t in srcs])
    c_dst = (ctypes.c_void_p * 2)(*[t.data_ptr() for t in dsts])
    c_n = (ctypes.c_int64 * 2)(*sizes)
    cap = 1024                                            # a power of two (required)
    ring = torch.randint(0, n, (1 + cap,), generator=g, dtype=torch.int32)
    mirror = X.host_alloc(4 * (1 + cap)).view(torch.int32)
    mirror.fill_(-7)
    st = torch.cuda.current_stream().cuda_stream

    def run(n_diff, cnt, frm, nc=2, src=c_src):
        ring[0] = cnt
        rd = ring.cuda()
        rc = L.exl3_tier_exchange(flags.data_ptr(), n, diff.data_ptr(), n_diff, rd.data_ptr(), cap, frm,
                                  mirror.data_ptr(), src, c_dst, c_n, nc, st)
        torch.cuda.synchronize()
        return rc, rd
    # copies and the ring first: the snapshot of the flags is their state before any diff
    rc, _ = run(0, 700, 650)
    assert rc == 0
    assert np.array_equal(dsts[0].numpy(), before)
    assert np.array_equal(dsts[1].numpy(), srcs[1].cpu().numpy())
    m, r = mirror.numpy(), ring.numpy()
    assert m[0] == 700 and np.array_equal(m[1 + 650:1 + 700], r[1 + 650:1 + 700])
    assert (m[1:1 + 650] == -7).all() and (m[1 + 700:] == -7).all()
    rc, _ = run(0, 1300, 900)                             # wraps: positions 900..1023, then 0..275
    assert rc == 0 and m[0] == 1300
    assert np.array_equal(m[1 + 900:], r[1 + 900:]) and np.array_equal(m[1:1 + 276], r[1:1 + 276])
    assert (m[1 + 276:1 + 650] == -7).all()
    mirror.fill_(-7)
    rc, _ = run(0, 5000, 100)                             # more than cap since `from`: the last cap entries
    assert rc == 0 and m[0] == 5000 and np.array_equal(m[1:], r[1:])
    rc, _ = run(1000, 5000, 5000, nc=0)
    assert rc == 0
    want = before.copy()
    want[keys.numpy()] = vals.numpy()
    assert np.array_equal(flags.cpu().numpy(), want)
    bad = (ctypes.c_void_p * 1)(srcs[1].data_ptr() + 4)
    assert run(0, 5000, 5000, nc=1, src=bad)[0] != 0
    # a capacity that is not a power of two is refused before anything is enqueued
    rd = ring.cuda()
    assert L.exl3_tier_exchange(flags.data_ptr(), n, diff.data_ptr(), 0, rd.data_ptr(), cap - 24, 0, mirror.data_ptr(),
                                c_src, c_dst, c_n, 0, st) != 0


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [1, 0])
def test_cache_prefetch(fused):
    """moe_prefetch between MoE calls, on a side stream ordered after the previous call and before the next one (the
    reference caller's protocol, moe_offload.py:251-262): every prefetch and ensure decision equals the oracle's
    (prefetch mode: tick not advanced, slots of the last call protected, exact LRU, max_fill cap), every slot holds
    its expert's blob, the final slot tables equal the oracle's, and every cached output equals the uncached one."""
    import ctypes
    from exl3xpu import nvtier
    L, E, H, I, K, nd, steps, P, S, mf = 2, 128, 128, 128, 3, 16, 40, 8, 60, 5
    print(f"case cache prefetch fused={fused}", flush=True)
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    src = nvtier.SyntheticExpertSource(H, I, K, 81, n_distinct=nd)
    for key in range(L * E):
        ctypes.memmove(store.addr(key), src.buf[key % nd].ctypes.data, src.blob)
    dev = torch.from_numpy(src.buf).cuda()
    table = torch.tensor([dev[e % nd].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
    rng = np.random.default_rng(82)
    pr = 1.0 / np.arange(1, E + 1) ** 1.2
    pr /= pr.sum()
    ids = np.stack([[rng.choice(E, P, replace=False, p=pr) for _ in range(L)] for _ in range(steps + 1)]).astype(np.int32)
    w = rng.random(ids.shape, dtype=np.float32)
    # predicted experts of the next call: half of the true next picks, the rest drawn uniformly
    pred = np.zeros((steps, L, P), np.int32)
    for n in range(steps):
        for li in range(L):
            keep = list(ids[n + 1, li][:P // 2])
            rest = [e for e in rng.permutation(E) if e not in keep][:P - len(keep)]
            pred[n, li] = np.array(keep + rest, np.int32)
    co = cache.CacheOracle(L, E, S, tier=False)
    X = store.X
    rl = cache.rec_len(P)
    logbuf = torch.zeros(1 + 2 * steps * L * rl, dtype=torch.int32, device="cuda")
    X.moe_set_decision_log(logbuf)
    X.moe_set_fused_ensure(fused)
    side = torch.cuda.Stream()
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    orecs, bad = [], 0
    try:
        for n in range(steps):
            for li in range(L):
                orecs.append(co.ensure(li, ids[n, li].copy(), w[n, li].copy()))
                it = torch.from_numpy(ids[n, li]).view(1, P).cuda()
                wt = torch.from_numpy(w[n, li]).view(1, P).cuda()
                out = store.forward_cached(keys[li], x, it, wt)
                ref = X.moe_forward(x, it, wt, table, I, K, E)
                bad += int(not torch.equal(out, ref))
                orecs.append(co.prefetch(li, pred[n, li].copy(), max_fill=mf))
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    store.prefetch(keys[li], torch.from_numpy(pred[n, li]).cuda(), max_fill=mf)
                torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
    finally:
        X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
        X.moe_set_fused_ensure(1)
    lg = logbuf.cpu().numpy()
    assert lg[0] == 2 * steps * L
    recs = lg[1:].reshape(2 * steps * L, rl)
    orecs = np.stack(orecs)
    mism = np.nonzero((recs != orecs).any(axis=-1))[0]
    assert mism.size == 0, f"first mismatch at call {mism[0]} ({'prefetch' if mism[0] % 2 else 'ensure'})"
    pf_nm = recs[1::2, 2 + P]
    assert pf_nm.sum() > 0 and pf_nm.max() <= mf and (pf_nm == mf).any()   # prefetches claimed slots, capped
    assert (recs[0::2, 2 + P] < P).any()                                   # some picks were already prefetched
    sk = store.slot_key.cpu().numpy()
    assert np.array_equal(sk, co.slot_key) and np.array_equal(store.slot_last.cpu().numpy(), co.slot_last)
    slots = store.slots.cpu().numpy()
    for s in np.nonzero(sk >= 0)[0]:
        assert np.array_equal(slots[s, :src.blob], src.buf[sk[s] % nd]), f"slot {s}"
    assert bad == 0


@pytest.mark.gpu
def test_cache_copy_prefetch():
    """Copy-engine prefetch (moe_offload.py:264-302): after each MoE call the next layer's predicted experts are
    planned on the compute stream (slots claimed and pinned), the host worker copies them on its own stream, and the
    next ensure commits the finished plan. Waiting for the worker between calls makes the sequence deterministic: every
    plan and ensure decision equals the oracle's plan mode, the worker reports the plans and copies the records hold,
    every slot holds its expert's blob, the final tables equal the oracle's, and every output equals the uncached one."""
    import ctypes
    import time
    from exl3xpu import nvtier
    L, E, H, I, K, nd, steps, P, S, mf = 2, 128, 128, 128, 3, 16, 30, 8, 60, 6
    print("case cache copy-engine prefetch", flush=True)
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    src = nvtier.SyntheticExpertSource(H, I, K, 83, n_distinct=nd)
    for key in range(L * E):
        ctypes.memmove(store.addr(key), src.buf[key % nd].ctypes.data, src.blob)
    dev = torch.from_numpy(src.buf).cuda()
    table = torch.tensor([dev[e % nd].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
    rng = np.random.default_rng(84)
    pr = 1.0 / np.arange(1, E + 1) ** 1.2
    pr /= pr.sum()
    ids = np.stack([[rng.choice(E, P, replace=False, p=pr) for _ in range(L)] for _ in range(steps + 1)]).astype(np.int32)
    w = rng.random(ids.shape, dtype=np.float32)
    co = cache.CacheOracle(L, E, S, tier=False)
    X = store.X
    rl = cache.rec_len(P)
    logbuf = torch.zeros(1 + 2 * steps * L * rl, dtype=torch.int32, device="cuda")
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()

    def wait_worker():
        torch.cuda.synchronize()
        t0 = time.monotonic()
        while not torch.equal(store.done_seq.cpu(), store._plan_seq.cpu()):
            assert time.monotonic() - t0 < 10.0, "prefetch worker did not finish its copies"
            time.sleep(0.0005)

    store.start_copy_prefetch()
    X.moe_set_decision_log(logbuf)
    orecs, bad, planned, copied = [], 0, 0, 0
    try:
        for n in range(steps):
            for li in range(L):
                orecs.append(co.ensure(li, ids[n, li].copy(), w[n, li].copy()))
                it = torch.from_numpy(ids[n, li]).view(1, P).cuda()
                wt = torch.from_numpy(w[n, li]).view(1, P).cuda()
                out = store.forward_cached(keys[li], x, it, wt)
                ref = X.moe_forward(x, it, wt, table, I, K, E)
                bad += int(not torch.equal(out, ref))
                # the next call's layer and picks (true picks reversed: the cap of mf takes a different subset)
                nn_, nli = (n, li + 1) if li + 1 < L else (n + 1, 0)
                pred = ids[nn_, nli][::-1].copy()
                r = co.plan(nli, pred.copy(), max_fill=mf)
                orecs.append(r)
                planned += int(r[2 + P] > 0)
                copied += int(r[2 + P])
                store.plan_prefetch(keys[nli], torch.from_numpy(pred).cuda(), max_fill=mf)
                wait_worker()
        torch.cuda.synchronize()
    finally:
        X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
        counts = store.stop_copy_prefetch()
    co.ensure(0, np.zeros(1, np.int32), np.ones(1, np.float32), max_fill=0)      # the stop's commit pass
    lg = logbuf.cpu().numpy()
    assert lg[0] == 2 * steps * L
    recs = lg[1:].reshape(2 * steps * L, rl)
    orecs = np.stack(orecs)
    mism = np.nonzero((recs != orecs).any(axis=-1))[0]
    assert mism.size == 0, f"first mismatch at call {mism[0]} ({'plan' if mism[0] % 2 else 'ensure'})"
    assert list(counts) == [planned, copied] and copied > 0
    assert (recs[1::2, 2 + P] <= mf).all() and (recs[0::2, 2 + P] < P).any()
    sk = store.slot_key.cpu().numpy()
    assert np.array_equal(sk, co.slot_key) and np.array_equal(store.slot_last.cpu().numpy(), co.slot_last)
    slots = store.slots.cpu().numpy()
    for s in np.nonzero(sk >= 0)[0]:
        assert np.array_equal(slots[s, :src.blob], src.buf[sk[s] % nd]), f"slot {s}"
    assert bad == 0


def test_tier_fills_from_expert_file(tmp_path):
    """The RAM tier filled from a packed expert file (write_expert_file, read back through ExpertFile: O_DIRECT where
    the file system allows it) instead of the seeded source: the same trace as test_cache_multirow_tier, with every
    device record and host decision equal to the oracle's and every output equal to the plain forward on the true
    blobs."""
    from exl3xpu import nvtier
    L, E, S, M, TK, steps, H, I, K = 6, 128, 150, 4, 10, 60, 128, 128, 3
    ids, w = synth.zipf_trace(20261203, steps, L, E, TK, M=M)
    ids = np.ascontiguousarray(ids.reshape(steps, L, M * TK))
    w = np.ascontiguousarray(w.reshape(steps, L, M * TK))
    co = cache.CacheOracle(L, E, S, ring_cap=1 << 12, budget=160, age=4, qmax=64, latency=3)
    orecs, olog = co.run(ids, w)
    src = nvtier.SyntheticExpertSource(H, I, K, 11, n_distinct=16)
    path = str(tmp_path / "experts.bin")
    nvtier.write_expert_file(path, src, L, E, H, I, K)
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L)
    for li in range(L):
        store.add_layer(f"model.layers.{li}.mlp")
    tier = nvtier.NvTierAsync(store, path, ring_cap=1 << 12, budget_records=160, latency=3)
    tier.policy.admit_age, tier.policy.admit_qmax = 4, 64
    tier.log_decisions = True
    print(f"case tier fills from expert file (direct I/O {tier.src.direct})", flush=True)
    blobs = torch.from_numpy(src.buf).cuda()
    ref_ptr = torch.tensor([blobs[r % src.n].data_ptr() for r in range(L * E)], dtype=torch.int64, device="cuda")
    try:
        recs, bad = _run(store, tier, ids, w, H, check_out_every=1, ref_ptr=ref_ptr, M=M)
    finally:
        tier.close()
    mism = np.nonzero((recs != orecs).any(axis=-1))
    assert mism[0].size == 0, f"first mismatch at step/layer {mism[0][0]}/{mism[1][0]}"
    for n, ((a1, e1), (a2, e2)) in enumerate(zip(tier.decisions, olog)):
        assert a1.tolist() == a2.tolist() and e1.tolist() == e2.tolist(), n
    assert bad == 0
    assert tier.src.reads > 0 and recs[:, :, 2 + M * TK].sum() > 0


def test_tier_pool_wallclock_from_expert_file(tmp_path):
    """The record pool with fills from a packed expert file that complete by wall clock (each read on decode-fill
    queue key % 8, resident at the first host step after it finished): the same trace as test_cache_multirow_tier.
    The admissions now follow the disk's timing, so there is no oracle record to compare; instead every output
    equals the plain forward on the true blobs with the post-mask picks, fills and write-backs happened, no
    write-back was dropped, the pool stayed within budget + 3 x queue records and every resident key's record holds
    its own blob."""
    from pool_checks import check_pool
    from exl3xpu import nvtier
    L, E, S, M, TK, steps, H, I, K = 6, 128, 150, 4, 10, 60, 128, 128, 3
    ids, w = synth.zipf_trace(20261203, steps, L, E, TK, M=M)
    ids = np.ascontiguousarray(ids.reshape(steps, L, M * TK))
    w = np.ascontiguousarray(w.reshape(steps, L, M * TK))
    src = nvtier.SyntheticExpertSource(H, I, K, 11, n_distinct=16)
    path = str(tmp_path / "experts.bin")
    nvtier.write_expert_file(path, src, L, E, H, I, K)
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L, pool=True)
    for li in range(L):
        store.add_layer(f"model.layers.{li}.mlp")
    tier = nvtier.NvTierAsync(store, path, ring_cap=1 << 12, budget_records=160, latency=3, completion="wallclock",
                              wb_queue=48)
    tier.policy.admit_age, tier.policy.admit_qmax = 4, 64
    print(f"case tier pool wall-clock fills from expert file (direct I/O {tier.src.direct})", flush=True)
    blobs = torch.from_numpy(src.buf).cuda()
    ref_ptr = torch.tensor([blobs[r % src.n].data_ptr() for r in range(L * E)], dtype=torch.int64, device="cuda")
    try:
        recs, bad = _run(store, tier, ids, w, H, check_out_every=1, ref_ptr=ref_ptr, M=M)
        assert bad == 0
        assert tier.src.reads > 0 and recs[:, :, 2 + M * TK].sum() > 0
        assert tier.stats["wb_taken"] > 0
        check_pool(store, tier, src, 160)
    finally:
        tier.close()


@pytest.mark.parametrize("M", [150, 255])
def test_cache_midsize_rows(M):
    """Cached calls between the decode kernel's limit (1,024 picks) and prefill_min_m (256): M = 150 and 255 rows x
    top-10 at the config-0 shapes (H 2048, I 512, 512 experts), 2 layers, 300 slots, a 600-record RAM tier, Zipf
    routing (reference: the cached op over the align path, kernels/moe-a8/exl3_moe.a8.sycl:1239, 1277-1314). One
    ensure takes all 1,500 / 2,550 picks; victims are written back, fills copied and committed, and the prefill
    kernels read the committed table. Every device record and host decision equals the oracle's (one reference
    ensure per call, Appendix A.1 of the contract), and every output equals the uncached forward on the true blobs
    with the post-mask picks, bit for bit."""
    L, E, S, TK, steps = 2, 512, 300, 10, 8
    print(f"case cache mid-size rows M={M}", flush=True)
    ids, w = synth.zipf_trace(20261210 + M, steps, L, E, TK, M=M)
    ids = np.ascontiguousarray(ids.reshape(steps, L, M * TK))
    w = np.ascontiguousarray(w.reshape(steps, L, M * TK))
    co = cache.CacheOracle(L, E, S, ring_cap=1 << 12, budget=600, age=4, qmax=256, latency=2)
    orecs, olog = co.run(ids, w)
    store, tier, blobs, ref_ptr = _setup(L, E, S, 2048, 512, 3, 600, 256, 4, 2, 1 << 12, 19)
    recs, bad = _run(store, tier, ids, w, 2048, check_out_every=1, ref_ptr=ref_ptr, M=M)
    mism = np.nonzero((recs != orecs).any(axis=-1))
    assert mism[0].size == 0, f"first mismatch at step/layer {mism[0][0]}/{mism[1][0]}"
    for n, ((a1, e1), (a2, e2)) in enumerate(zip(tier.decisions, olog)):
        assert a1.tolist() == a2.tolist() and e1.tolist() == e2.tolist(), n
    assert bad == 0
    P = M * TK
    assert recs[:, :, 1].max() > 0 and recs[:, :, 2 + P].sum() > 0       # masked picks and fills happened
    wb = recs[:, :, 3 + 2 * P:3 + 4 * P:2]
    assert (wb >= 0).any()                                                 # and victims were written back
    tier.close()


@pytest.mark.parametrize("fused", [1, 0])
def test_decision_log_stops_at_its_buffer(fused):
    """A decision log shorter than the run: every call is counted, the records that fit are written, and nothing is
    written past the buffer (a guard region after it keeps its fill value)."""
    from exl3xpu import moe_offload, nvtier
    H, I, K, E, S, P = 128, 128, 3, 16, 4, 4
    print(f"case decision log bound fused={fused}", flush=True)
    store = moe_offload.ExpertStore(H, I, K, E, S, max_layers=1)
    src = nvtier.SyntheticExpertSource(H, I, K, 77, n_distinct=E)
    store.add_layer("layer0", torch.from_numpy(src.buf))
    X = store.X
    rl = cache.rec_len(P)
    fit, calls = 3, 7
    buf = torch.full((1 + fit * rl + 64,), -7, dtype=torch.int32, device="cuda")
    buf[0] = 0
    X.moe_set_fused_ensure(fused)
    X.moe_set_decision_log(buf[:1 + fit * rl])
    rng = np.random.default_rng(5)
    x = torch.randn(1, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).cuda()
    try:
        for _ in range(calls):
            ids = torch.from_numpy(rng.choice(E, P, replace=False).astype(np.int32)).view(1, P).cuda()
            w = torch.full((1, P), 1.0 / P, dtype=torch.float32, device="cuda")
            store.forward_cached("layer0", x, ids, w)
        torch.cuda.synchronize()
    finally:
        X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
        X.moe_set_fused_ensure(1)
    b = buf.cpu().numpy()
    assert b[0] == calls
    recs = b[1:1 + fit * rl].reshape(fit, rl)
    assert (recs[:, 2:2 + P] >= 0).all() and (recs[:, 2:2 + P] < E).all()   # the picks of every record that fits
    assert (b[1 + fit * rl:] == -7).all(), "the log wrote past its buffer"


@pytest.mark.parametrize("fused,pool,K", [(1, False, 96), (0, False, 96), (1, True, 96), (1, False, 4),
                                          (0, True, 4)])
def test_tier_victim_ring(fused, pool, K):
    """The victim ring (experimental/n111-victim-ring): victims go to K ring slots in HBM and the host drains them.
    Every device record (with ring-full drops as write-backs of -1) and every host decision equals the oracle's ring
    mode, the ring's meta equals the oracle's after the run, and every cached output equals the plain forward on the
    true blobs (the reference's own test of this path, n111_test.py). After the ring is drained, every RAM-resident
    key's record holds its true blob. K = 4 overflows on this trace (drops), K = 96 does not."""
    from exl3xpu import nvtier
    L, E, S, M, TK, steps = 4, 96, 90, 2, 8, 60
    print(f"case victim ring K={K} fused={fused} pool={pool}", flush=True)
    ids, w = synth.zipf_trace(20261204, steps, L, E, TK, M=M)
    ids = np.ascontiguousarray(ids.reshape(steps, L, M * TK))
    w = np.ascontiguousarray(w.reshape(steps, L, M * TK))
    co = cache.CacheOracle(L, E, S, ring_cap=1 << 12, budget=120, age=4, qmax=32, latency=3, victim_ring=K)
    orecs, olog = co.run(ids, w)
    store, tier, blobs, ref_ptr = _setup(L, E, S, 128, 128, 3, 120, 32, 4, 3, 1 << 12, 13, pool=pool, wb_queue=48,
                                         victim_ring=K)
    store.X.moe_set_fused_ensure(fused)
    try:
        recs, bad = _run(store, tier, ids, w, 128, check_out_every=1, ref_ptr=ref_ptr, M=M)
    finally:
        store.X.moe_set_fused_ensure(1)
    mism = np.nonzero((recs != orecs).any(axis=-1))
    assert mism[0].size == 0, f"first mismatch at step/layer {mism[0][0]}/{mism[1][0]}"
    for n, ((a1, e1), (a2, e2)) in enumerate(zip(tier.decisions, olog)):
        assert a1.tolist() == a2.tolist() and e1.tolist() == e2.tolist(), n
    assert bad == 0
    ost = co.ring_stats()
    meta = tier.vr_meta.cpu().numpy()
    assert ost["error"] == 0 and ost["claims"] > 0
    assert (ost["drops"] > 0) == (K == 4)
    assert [int(meta[0]), int(meta[1]), int(meta[2])] == [ost["pos"], ost["claims"], ost["drops"]]
    assert np.array_equal(meta[4:4 + K], co.vr_key) and np.array_equal(meta[4 + K:4 + 2 * K], co.vr_seq)
    tier.ring_settle()
    torch.cuda.synchronize()
    assert not tier.policy.inflight[np.nonzero(tier.policy.res)[0]].any()
    for key in np.nonzero(tier.policy.res)[0].tolist():
        want = np.asarray(tier.src.blob_of(tier.rec_index(key)))
        got = np.frombuffer(ctypes_bytes(store.addr(key), want.size), dtype=np.uint8)
        assert np.array_equal(got, want), f"record of key {key}"
    tier.close()


def ctypes_bytes(addr: int, n: int) -> bytes:
    import ctypes
    return ctypes.string_at(addr, n)


def test_tier_victim_ring_wallclock_with_prefill(tmp_path):
    """The victim ring (16 slots, drains landing by wall clock) over the record pool with fills from a packed expert
    file, and every 12 steps a prefill layer whose experts ensure_for_prefill makes RAM-resident (it drains the
    ring first, including the claims the host has not seen yet): every decode output equals the plain forward on the
    true blobs, every prefill output (read zero-copy from the records and slots) equals the all-resident table's,
    and after the last drain every RAM-resident key's record holds its own blob."""
    from pool_checks import check_pool
    from exl3xpu import nvtier
    L, E, S, M, TK, steps, H, I, K = 4, 96, 90, 2, 8, 60, 128, 128, 3
    ids, w = synth.zipf_trace(20261205, steps, L, E, TK, M=M)
    src = nvtier.SyntheticExpertSource(H, I, K, 19, n_distinct=16)
    path = str(tmp_path / "experts.bin")
    nvtier.write_expert_file(path, src, L, E, H, I, K)
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L, pool=True)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    tier = nvtier.NvTierAsync(store, path, ring_cap=1 << 12, budget_records=120, latency=3, completion="wallclock",
                              wb_queue=48, victim_ring=16)
    tier.policy.admit_age, tier.policy.admit_qmax = 4, 32
    print("case victim ring, wall-clock drains, prefill in between", flush=True)
    X = store.X
    blobs = torch.from_numpy(src.buf).cuda()
    ref_ptr = torch.tensor([blobs[r % src.n].data_ptr() for r in range(L * E)], dtype=torch.int64, device="cuda")
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    xp = torch.randn(40, H, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    bad = prefills = 0
    try:
        for n in range(steps):
            for li in range(L):
                it = torch.from_numpy(np.ascontiguousarray(ids[n, li].reshape(M, TK))).cuda()
                wt = torch.from_numpy(np.ascontiguousarray(w[n, li].reshape(M, TK))).cuda()
                out = store.forward_cached(keys[li], x, it, wt)
                ref = X.moe_forward(x, it, wt, ref_ptr[li * E:(li + 1) * E], I, K, E)
                bad += int(not torch.equal(out, ref))
            tier.step()
            if n % 12 == 11:
                li = (n // 12) % L
                pid, pw = synth.softmax_topk(500 + n, 40, E, TK)
                pit, pwt = torch.from_numpy(pid).cuda(), torch.from_numpy(pw).cuda()
                tier.ensure_for_prefill(li, pit)
                out = X.moe_forward(xp, pit, pwt, store.ptrs_all[li * E:(li + 1) * E].clone(), I, K, E)
                ref = X.moe_forward(xp, pit, pwt, ref_ptr[li * E:(li + 1) * E], I, K, E)
                torch.cuda.synchronize()
                assert torch.equal(out, ref), n
                prefills += 1
        assert bad == 0 and prefills == steps // 12
        assert tier.stats["vr_claims"] > 0 and tier.stats["vr_landed"] > 0
        tier.ring_settle()
        check_pool(store, tier, src, 120)
    finally:
        tier.close()
