"""HIP-graph replay of the cached decode stack (the way a serving engine runs decode: plugin/sglang_plugin.tier.py
captures the MoE layers and replays them, with the host tier step between replays; captured kernels keep the tier
tensors they saw, plugin:525-526).

A graph of every layer's forward_cached is captured once and replayed per decode step; the routing of the step is
copied into the graph's static input buffers before each replay and the host admission step runs eagerly (with its
device synchronisation) between replays. Every replay must reproduce the eager run on an identical store: the same
device decision records, the same host admission/eviction decisions and bit-identical outputs of every layer."""
import os

import numpy as np
import pytest
import torch

from oracle import cache

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _store(g, H, I):
    from exl3xpu import nvtier
    L, E, S = int(g["L"]), int(g["E"]), int(g["S"])
    store = nvtier.TierStore(H, I, 3, E, S, n_layers=L)
    for li in range(L):
        store.add_layer(f"model.layers.{li}.mlp")
    src = nvtier.SyntheticExpertSource(H, I, 3, 3, n_distinct=16)
    tier = nvtier.NvTierAsync(store, src, ring_cap=int(g["ring_cap"]), budget_records=int(g["budget"]),
                              latency=int(g["latency"]))
    tier.policy.admit_age, tier.policy.admit_qmax = int(g["age"]), int(g["qmax"])
    tier.log_decisions = True
    return store, tier


@pytest.mark.parametrize("H,I", [(128, 128), (384, 256)])
def test_graph_replay_matches_eager(H, I):
    g = np.load(os.path.join(GOLD, "cache_small.npz"))
    ids_np, w_np = g["ids"], g["w"]                      # [steps, L, P]
    steps, L, P = ids_np.shape
    print(f"case graph replay H={H} I={I} steps={steps} L={L}", flush=True)
    rl = cache.rec_len(P)
    x = torch.randn(L, 1, H, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).cuda()
    ids_d = torch.from_numpy(ids_np).cuda().view(steps, L, 1, P)
    w_d = torch.from_numpy(w_np).cuda().view(steps, L, 1, P)

    # eager
    store, tier = _store(g, H, I)
    keys = list(store.layer_index)
    log_e = torch.zeros(1 + steps * L * rl, dtype=torch.int32, device="cuda")
    store.X.moe_set_decision_log(log_e)
    outs_e = []
    for n in range(steps):
        it, wt = ids_d[n].clone(), w_d[n].clone()
        outs_e.append([store.forward_cached(keys[li], x[li], it[li], wt[li]).clone() for li in range(L)])
        tier.step()
    torch.cuda.synchronize()
    store.X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
    dec_e = [(a.tolist(), e.tolist()) for a, e in tier.decisions]
    tier.close()
    del store, tier
    torch.cuda.synchronize()

    # graph: step 0 eager (first calls set up the library), steps 1.. replayed
    store, tier = _store(g, H, I)
    log_g = torch.zeros(1 + steps * L * rl, dtype=torch.int32, device="cuda")
    store.X.moe_set_decision_log(log_g)
    ids_s = torch.empty(L, 1, P, dtype=torch.int32, device="cuda")
    w_s = torch.empty(L, 1, P, dtype=torch.float32, device="cuda")
    ids_s.copy_(ids_d[0])
    w_s.copy_(w_d[0])
    first = [store.forward_cached(keys[li], x[li], ids_s[li], w_s[li]).clone() for li in range(L)]
    tier.step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="thread_local"):
        outs_s = [store.forward_cached(keys[li], x[li], ids_s[li], w_s[li]) for li in range(L)]
    bad = [li for li in range(L) if not torch.equal(first[li], outs_e[0][li])]
    assert not bad, f"eager step 0 differs at layers {bad}"
    for n in range(1, steps):
        ids_s.copy_(ids_d[n])
        w_s.copy_(w_d[n])
        graph.replay()
        got = [o.clone() for o in outs_s]
        tier.step()                                      # eager host step + device synchronisation between replays
        torch.cuda.synchronize()
        bad = [li for li in range(L) if not torch.equal(got[li], outs_e[n][li])]
        assert not bad, f"replay {n}: outputs differ from eager at layers {bad}"
    store.X.moe_set_decision_log(torch.zeros(0, dtype=torch.int32, device="cuda"))
    rec_e = log_e.cpu().numpy()
    rec_g = log_g.cpu().numpy()
    assert rec_e[0] == rec_g[0] == steps * L
    assert np.array_equal(rec_e, rec_g)
    assert [(a.tolist(), e.tolist()) for a, e in tier.decisions] == dec_e
    tier.close()


def test_graph_replay_after_exchange_growth():
    """A graph captured at bs=1 keeps the address of the decode exchange buffer in its kernel arguments. An eager call
    large enough to grow that buffer afterwards (100 rows x top-10, 1,000 pairs) must leave the captured buffer
    allocated: replays before and after the growth equal the eager bs=1 output bit for bit."""
    from exl3xpu.moe_offload import ops
    from oracle import exl3, synth
    H, I, K, E, topk = 2048, 512, 3, 16, 10
    print("case graph replay after exchange growth", flush=True)
    blobs = torch.from_numpy(np.stack([synth.expert_blob(41, e, H, I, K) for e in range(E)])).cuda()
    table = torch.tensor([blobs[e].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
    X = ops()

    def inputs(M, seed):
        ids, w = synth.softmax_topk(seed, M, E, topk)
        x = torch.from_numpy(exl3.bf16_to_f32(synth.activations(seed, M, H))).to(torch.bfloat16).cuda()
        return x, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()

    x1, i1, w1 = inputs(1, 42)
    ref = X.moe_forward(x1, i1, w1, table, I, K, E).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, capture_error_mode="thread_local"):
        out = X.moe_forward(x1, i1, w1, table, I, K, E)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    xb, ib, wb = inputs(100, 43)
    big = X.moe_forward(xb, ib, wb, table, I, K, E)
    torch.cuda.synchronize()
    assert torch.isfinite(big.float()).all()
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
