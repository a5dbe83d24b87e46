"""The named workloads at their full sizes on the GPU.

Config 2: 48 MoE layers x 512 experts at H 2048 / I 512 / K 3 (1,195,008-byte blobs) through the real tier: a
TierStore with 8,000 HBM slots, a pinned RAM arena of every record, NvTierAsync with a budget of 1,075 or 3,763
records (2 GB and 7 GB of 1.86 MB records), AGE 4, QMAX 256, an 8-step fill latency; Zipf(1.1) routing at batch 1, 2
and 4 (each row an independent stream). Every device decision (mask set, misses, victims, slots, ring count) and
every host admission and eviction equals the oracle's; sampled steps check every layer's cached output bit for bit
against the uncached forward on the true blobs with the post-mask picks.

Config 4: hidden 4096, 128 experts of 4096 -> 1536 -> 4096, top-8, K cycling 2, 3, 4 over 48 layers, HBM slots for
30 % of all expert bytes (slot stride = the largest blob), uniform-random routing, batch 4 and 1. The layers' host
records alias three 128-expert arenas, one per bitrate (the decisions do not depend on the bytes, and every output is
checked against its own layer's true blobs), so the host side needs 2.7 GB instead of 58 GB. Plus the top-8 bs=1
output against the oracle for each K (the oracle's outputs are fixtures: about 5 s per expert on a CPU)."""
import os

import numpy as np
import pytest
import torch

from oracle import cache, exl3, synth

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")

C2 = dict(H=2048, I=512, K=3, E=512, L=48, S=8000, topk=10)


@pytest.fixture(scope="module")
def c2_store():
    from exl3xpu import nvtier
    g = C2
    store = nvtier.TierStore(g["H"], g["I"], g["K"], g["E"], g["S"], n_layers=g["L"])
    for li in range(g["L"]):
        store.add_layer(f"model.layers.{li}.mlp")
    src = nvtier.SyntheticExpertSource(g["H"], g["I"], g["K"], 21, n_distinct=64)
    blobs = torch.from_numpy(src.buf).cuda()
    ref_ptr = torch.tensor([blobs[r % src.n].data_ptr() for r in range(g["L"] * g["E"])], dtype=torch.int64,
                           device="cuda")
    yield store, src, ref_ptr, blobs
    del store


@pytest.mark.parametrize("bs,budget,steps,pool", [(1, 1075, 300, False), (2, 1075, 200, False),
                                                  (4, 1075, 150, False), (1, 3763, 300, False),
                                                  (2, 3763, 200, False), (4, 3763, 150, False),
                                                  (1, 1075, 300, True), (4, 1075, 150, True)])
def test_config2_tier_stack(c2_store, bs, budget, steps, pool):
    """pool: the RAM tier pins a RecordPool (budget + 3 x 48 queue records at most, in 32-record chunks) instead of
    the 24,576-record arena; decisions and outputs must not change."""
    from exl3xpu import nvtier
    store, src, ref_ptr, _ = c2_store
    g = C2
    L, E, S, P = g["L"], g["E"], g["S"], bs * g["topk"]
    print(f"case config2 bs={bs} budget={budget} steps={steps} pool={pool}", flush=True)
    if pool:
        store = nvtier.TierStore(g["H"], g["I"], g["K"], g["E"], g["S"], n_layers=g["L"], pool=True)
        for li in range(g["L"]):
            store.add_layer(f"model.layers.{li}.mlp")
    store.reset_cache()
    ids, w = synth.zipf_trace(20261210 + bs, steps, L, E, g["topk"], M=bs)
    ids = np.ascontiguousarray(ids.reshape(steps, L, P))
    w = np.ascontiguousarray(w.reshape(steps, L, P))
    co = cache.CacheOracle(L, E, S, budget=budget, age=4, qmax=256, latency=8)
    orecs, olog = co.run(ids, w)
    tier = nvtier.NvTierAsync(store, src, budget_records=budget, latency=8)
    tier.log_decisions = True
    X = store.X
    rl = cache.rec_len(P)
    logbuf = torch.zeros(1 + steps * L * rl, dtype=torch.int32, device="cuda")
    X.moe_set_decision_log(logbuf)
    x = torch.randn(L, bs, g["H"], generator=torch.Generator().manual_seed(bs)).to(torch.bfloat16).cuda()
    ids_d, w_d = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    keys = list(store.layer_index)
    bad, checked = [], 0
    try:
        for n in range(steps):
            check = n % 37 == 36
            for li in range(L):
                it = ids_d[n, li].view(bs, g["topk"]).clone()
                wt = w_d[n, li].view(bs, g["topk"]).clone()
                out = store.forward_cached(keys[li], x[li], it, wt)
                if check:
                    ref = X.moe_forward(x[li], it, wt, ref_ptr[li * E:(li + 1) * E], g["I"], g["K"], E)
                    if not torch.equal(out, ref):
                        bad.append((n, li))
                    checked += 1
            tier.step()
        torch.cuda.synchronize()
    finally:
        X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
        tier.close()
    lg = logbuf.cpu().numpy()
    assert lg[0] == steps * L
    recs = lg[1:].reshape(steps, L, rl)
    mism = np.nonzero((recs != orecs).any(axis=-1))
    assert mism[0].size == 0, f"first device mismatch at step/layer {mism[0][0]}/{mism[1][0]}"
    assert len(tier.decisions) == len(olog)
    for n, ((a1, e1), (a2, e2)) in enumerate(zip(tier.decisions, olog)):
        assert a1.tolist() == a2.tolist() and e1.tolist() == e2.tolist(), f"host step {n}"
    assert not bad, f"cached != uncached at (step, layer) {bad[:4]}"
    assert checked >= 4 * L
    masked = int(recs[:, :, 1].astype(np.int64).max())       # ring count after the last call of the run
    fills = int((recs[:, :, 2 + P] > 0).sum())
    print(f"config2 bs={bs} budget={budget}: ring count {masked}, calls with fills {fills}", flush=True)
    assert masked > 0 and fills > 0
    if pool:
        from pool_checks import check_pool, write_backs
        check_pool(store, tier, src, budget, int(write_backs(orecs, P)[:-1].sum()))
        full = L * E * store.stride
        print(f"config2 pool: {tier.pinned_bytes() / 2**30:.2f} GiB pinned ({tier.pool.records} records, high-water "
              f"{tier.pool.high}) instead of {full / 2**30:.2f} GiB", flush=True)
        assert tier.pinned_bytes() <= (budget + 3 * tier.wb_cap + tier.pool.chunk) * store.stride


def _c4_case(L, E, K_cycle, nd, seed):
    from exl3xpu import moe_offload, nvtier
    H, I = 4096, 1536
    Ks = [K_cycle[li % len(K_cycle)] for li in range(L)]
    blob = {k: int(moe_offload.ops().blob_bytes(H, I, k)) for k in K_cycle}
    srcs = {k: nvtier.SyntheticExpertSource(H, I, k, seed + k, n_distinct=nd) for k in K_cycle}

    class AliasedStore(moe_offload.ExpertStore):
        """Host records of layer li: the arena of its bitrate (128 records at the largest blob's stride)."""
        arenas = {}

        def _new_records(self, li, blobs):
            k = Ks[li]
            if k not in self.arenas:
                a = self.X.host_alloc(E * self.blob)
                view = a.view(E, self.blob)
                for e in range(E):
                    view[e, :blob[k]].copy_(torch.from_numpy(srcs[k].buf[e % nd]))
                self.arenas[k] = view
            v = self.arenas[k]
            base = v.data_ptr()
            return moe_offload._HostRecords(base, self.blob, base, base + E * self.blob, v)

    total = sum(E * blob[k] for k in Ks)
    S = int(0.3 * total / max(blob.values()))
    store = AliasedStore(H, I, max(K_cycle), E, S, max_layers=L)
    store.mixed_bitrates()
    for li in range(L):
        key = f"model.layers.{li}.mlp"
        store.add_layer(key)
        store.K_of[key] = Ks[li]
    dev = {k: torch.from_numpy(srcs[k].buf).cuda() for k in K_cycle}
    tables = [torch.tensor([dev[Ks[li]][e % nd].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
              for li in range(L)]
    return store, Ks, S, tables, dev


@pytest.mark.parametrize("bs,steps", [(4, 30), (1, 40)])
def test_config4_mixed_bitrate_stack(bs, steps):
    L, E, topk, nd = 48, 128, 8, 8
    print(f"case config4 bs={bs} steps={steps}", flush=True)
    store, Ks, S, tables, keep = _c4_case(L, E, (2, 3, 4), nd, 60)
    P = bs * topk
    ids, w = synth.uniform_trace(61 + bs, steps, L, E, topk, M=bs)
    ids = np.ascontiguousarray(ids.reshape(steps, L, P))
    w = np.ascontiguousarray(w.reshape(steps, L, P))
    co = cache.CacheOracle(L, E, S, tier=False)
    orecs = np.stack([np.stack([co.ensure(li, ids[n, li].copy(), w[n, li].copy()) for li in range(L)])
                      for n in range(steps)])
    X = store.X
    rl = cache.rec_len(P)
    logbuf = torch.zeros(1 + steps * L * rl, dtype=torch.int32, device="cuda")
    X.moe_set_decision_log(logbuf)
    x = torch.randn(L, bs, 4096, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).cuda()
    keys = list(store.layer_index)
    bad = []
    try:
        for n in range(steps):
            for li in range(L):
                it = torch.from_numpy(ids[n, li]).view(bs, topk).cuda()
                wt = torch.from_numpy(w[n, li]).view(bs, topk).cuda()
                out = store.forward_cached(keys[li], x[li], it, wt)
                if n % 5 == 4 or n == 0:
                    ref = X.moe_forward(x[li], it, wt, tables[li], 1536, Ks[li], E)
                    if not torch.equal(out, ref):
                        bad.append((n, li))
        torch.cuda.synchronize()
    finally:
        X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
    lg = logbuf.cpu().numpy()
    assert lg[0] == steps * L
    recs = lg[1:].reshape(steps, L, rl)
    mism = np.nonzero((recs != orecs).any(axis=-1))
    assert mism[0].size == 0, f"first mismatch at step/layer {mism[0][0]}/{mism[1][0]}"
    assert not bad, f"cached != uncached at (step, layer) {bad[:4]}"
    assert recs[:, :, 2 + P].sum() > S                 # more fills than slots: victims were taken


@pytest.mark.parametrize("K", [2, 3, 4])
def test_config4_top8_vs_oracle(K):
    """bs=1, top-8 of 128 experts at H 4096 / I 1536: rel-L2 <= 2e-3 against the oracle's fp32-accumulated output
    (bf16 activations and output: both rounded to bf16 before comparing; fp32 in and out: the kernel's arithmetic)."""
    from exl3xpu.moe_offload import ops
    g = np.load(os.path.join(GOLD, "c4_top8.npz"))
    H, I, E = int(g["H"]), int(g["I"]), int(g["E"])
    ids, w, xb = g[f"ids_{K}"], g[f"w_{K}"], g[f"x_{K}"]
    print(f"case config4 top-8 K={K}", flush=True)
    seed = 5000 + K
    used = sorted(set(ids.reshape(-1).tolist()))
    dev = torch.from_numpy(np.stack([synth.expert_blob(seed, e, H, I, K) for e in used])).cuda()
    table = torch.zeros(E, dtype=torch.int64)
    for i, e in enumerate(used):
        table[e] = dev[i].data_ptr()
    table = table.cuda()
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    xs = torch.from_numpy(exl3.bf16_to_f32(xb))
    ob = ops().moe_forward(xs.to(torch.bfloat16).cuda(), it, wt, table, I, K, E)
    of = ops().moe_forward(xs.cuda(), it, wt, table, I, K, E)
    torch.cuda.synchronize()

    def rel(a, b):
        a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
        return float(np.linalg.norm(a - b) / np.linalg.norm(b))
    rb = rel(ob.float().cpu().numpy(), exl3.bf16_to_f32(g[f"out_bf16_{K}"]))
    rf = rel(of.cpu().numpy(), g[f"out_f32_{K}"])
    print(f"config4 top-8 K={K}: rel-L2 bf16 {rb:.2e} fp32 {rf:.2e}", flush=True)
    assert rb <= 2e-3 and rf <= 2e-3
