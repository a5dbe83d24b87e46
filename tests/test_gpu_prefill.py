"""GPU parity of the prefill path (M >= prefill_min_m): the token sort (moe_align) bit for bit against the oracle's
canonical stable counting sort, and the grouped MFMA GEMMs against the oracle's prefill rounding points (y stored in
fp16 like the reference's DownDpasKernel<.., fp16>, a8:802) within rel-L2 2e-3. At the full prefill size (8,192
tokens x 512 experts, top-10) the oracle is too slow, so there the prefill output is checked against the decode
kernel on the same inputs (itself checked against the oracle in test_gpu_decode.py)."""
import numpy as np
import pytest
import torch

from oracle import exl3, synth

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ops():
    from exl3xpu.moe_offload import ops
    return ops()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


class _PrefillFrom:
    """Route calls with M >= m to the prefill path for the duration of a test."""

    def __init__(self, m):
        self.m = m

    def __enter__(self):
        _ops().moe_set_prefill_min_m(self.m)

    def __exit__(self, *exc):
        _ops().moe_set_prefill_min_m(256)


@pytest.mark.parametrize("M,topk,E,pad", [(300, 10, 64, 32), (1000, 8, 1024, 1), (3, 2, 16, 32), (257, 10, 512, 32)])
def test_align_matches_oracle(M, topk, E, pad):
    print(f"case align M={M} topk={topk} E={E} pad={pad}", flush=True)
    ids, w = synth.softmax_topk(900 + M, M, E, topk)
    ib, fb = _ops().moe_align(torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), E, pad)
    torch.cuda.synchronize()
    ib, fb = ib.cpu().numpy(), fb.cpu().numpy()
    ref = exl3.align(ids, w, E, pad)
    npairs, A = M * topk, min(M * topk, E)
    na = int(ib[4 * A])
    assert na == ref["n_act"]
    for i, key in enumerate(("act_expert", "act_start", "act_cnt", "act_pstart")):
        assert np.array_equal(ib[i * A:i * A + na], ref[key]), key
    p0 = 4 * A + 1
    assert np.array_equal(ib[p0:p0 + npairs], ref["pair_tok"])
    assert np.array_equal(ib[p0 + npairs:p0 + 2 * npairs], ref["pair_of"])
    assert np.array_equal(fb, ref["pair_w"])


def test_align_empty():
    ib, fb = _ops().moe_align(torch.zeros((0, 4), dtype=torch.int32, device="cuda"),
                              torch.zeros((0, 4), dtype=torch.float32, device="cuda"), 16, 32)
    torch.cuda.synchronize()
    assert int(ib[0]) == 0 and fb.numel() == 0


def _case(H, I, K, E, M, topk, seed, n_distinct=None):
    ids, w = synth.softmax_topk(seed, M, E, topk)
    used = sorted(set(ids.reshape(-1).tolist()))
    nd = n_distinct or E
    made = {}
    for e in used:
        if e % nd not in made:
            made[e % nd] = synth.expert_blob(seed, e % nd, H, I, K)
    blobs = {e: made[e % nd] for e in used}
    dev = torch.from_numpy(np.stack([blobs[e] for e in used])).cuda()
    table = np.zeros(E, dtype=np.int64)
    for i, e in enumerate(used):
        table[e] = dev[i].data_ptr()
    x = synth.activations(seed, M, H)
    return x, ids, w, blobs, torch.from_numpy(table).cuda(), dev


def _run(x_bits, ids, w, table, I, K, E, fp32=False):
    xs = torch.from_numpy(exl3.bf16_to_f32(x_bits)).cuda()
    if not fp32:
        xs = xs.to(torch.bfloat16)
    out = _ops().moe_forward(xs, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), table, I, K, E)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _check_vs_oracle(H, I, K, E, M, topk, seed, min_m):
    x, ids, w, blobs, table, keep = _case(H, I, K, E, M, topk, seed)
    ews = {e: exl3.ExpertWeights(b, H, I, K) for e, b in blobs.items()}
    ob, of = exl3.moe_forward(x, ids, w, ews, variant="prefill")
    with _PrefillFrom(min_m):
        gb = _run(x, ids, w, table, I, K, E)
        gf = _run(x, ids, w, table, I, K, E, fp32=True)
    rb, rf = rel_l2(gb, exl3.bf16_to_f32(ob)), rel_l2(gf, of)
    print(f"prefill H={H} I={I} K={K} E={E} M={M} top-{topk}: rel-L2 bf16 {rb:.2e} fp32 {rf:.2e}", flush=True)
    assert np.isfinite(gb).all() and np.isfinite(gf).all()
    assert rb <= TOL and rf <= TOL


def test_prefill_golden():
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "moe_small.npz"))
    H, I, K = int(g["H"]), int(g["I"]), int(g["K"])
    print(f"case prefill golden H={H} I={I} K={K}", flush=True)
    blobs = torch.from_numpy(g["blobs"]).cuda()
    E = blobs.shape[0]
    table = torch.tensor([blobs[e].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
    with _PrefillFrom(1):
        gf = _run(g["x"], g["ids"], g["w"], table, I, K, E, fp32=True)
    r = rel_l2(gf, g["out_prefill_f32"])
    print(f"prefill golden rel-L2 fp32 {r:.2e}", flush=True)
    assert r <= TOL


@pytest.mark.parametrize("K", [2, 3, 4])
def test_prefill_c0_shapes(K):
    """H 2048 / I 512 experts; 256 rows (the default prefill threshold) x top-4 over 32 experts."""
    print(f"case prefill c0 K={K}", flush=True)
    _check_vs_oracle(2048, 512, K, 32, 256, 4, 7000 + K, 256)


def test_prefill_expert_with_more_than_256_rows():
    """Every row picks both of 2 experts: 300 rows per expert, two row passes of the GEMM workgroups."""
    print("case prefill 300 rows per expert", flush=True)
    _check_vs_oracle(256, 256, 3, 2, 300, 2, 7100, 1)


def test_prefill_fp16_activations():
    """fp16 activations and output (the combine's 16-byte stores of fp16 values) against the oracle's fp32 result; the
    synthetic bf16 inputs are exact in fp16, so the difference is the prefill's own rounding."""
    print("case prefill fp16 activations", flush=True)
    H, I, K, E, M, topk, seed = 2048, 512, 3, 32, 256, 4, 7400
    x, ids, w, blobs, table, keep = _case(H, I, K, E, M, topk, seed)
    ews = {e: exl3.ExpertWeights(b, H, I, K) for e, b in blobs.items()}
    _, of = exl3.moe_forward(x, ids, w, ews, variant="prefill")
    xs = torch.from_numpy(exl3.bf16_to_f32(x)).cuda().half()
    with _PrefillFrom(256):
        out = _ops().moe_forward(xs, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), table, I, K, E)
        torch.cuda.synchronize()
    assert out.dtype == torch.float16
    got = out.float().cpu().numpy()
    r = rel_l2(got, of)
    print(f"prefill fp16 rel-L2 {r:.2e}", flush=True)
    assert np.isfinite(got).all() and r <= TOL


@pytest.mark.parametrize("K", [2, 3, 4])
def test_prefill_large_expert_shapes(K):
    """H 4096 / I 1536 (12 column blocks of I, 16 column tiles of H), each bitrate."""
    print(f"case prefill c4 K={K}", flush=True)
    _check_vs_oracle(4096, 1536, K, 8, 32, 2, 7200 + K, 1)


def test_prefill_full_chunk_vs_decode():
    """8,192 tokens x 512 experts (H 2048, I 512, K=3), top-10: the prefill output against the decode kernel run on
    64-row slices of the same inputs (fp32 activations and outputs: the only difference is the prefill's fp16 y), and
    32 seeded rows of it against the oracle's prefill rounding points (expert_pair, variant "prefill")."""
    H, I, K, E, M, topk = 2048, 512, 3, 512, 8192, 10
    print("case prefill full chunk vs decode", flush=True)
    x, ids, w, blobs, table, keep = _case(H, I, K, E, M, topk, 7300, n_distinct=64)
    pf = _run(x, ids, w, table, I, K, E, fp32=True)
    rows_o = np.sort(np.random.default_rng(7301).choice(M, size=32, replace=False))
    ews = {}
    ref = np.zeros((rows_o.size, H), dtype=np.float32)
    for i, m in enumerate(rows_o):
        xf = exl3.bf16_to_f32(x[m])
        acc = np.zeros(H, dtype=np.float32)
        for k in range(topk):
            e = int(ids[m, k])
            if e % 64 not in ews:
                ews[e % 64] = exl3.ExpertWeights(blobs[e], H, I, K)
            acc = (acc + exl3.expert_pair(xf, ews[e % 64], float(w[m, k]), "prefill")).astype(np.float32)
        ref[i] = acc
    ro = rel_l2(pf[rows_o], ref)
    worst = (np.linalg.norm(pf[rows_o] - ref, axis=1) / np.linalg.norm(ref, axis=1)).max()
    print(f"full chunk: rel-L2 prefill vs oracle on {rows_o.size} rows {ro:.2e}, worst row {worst:.2e}", flush=True)
    assert ro <= TOL and worst <= 2 * TOL
    xs = torch.from_numpy(exl3.bf16_to_f32(x)).cuda()
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    dec = []
    for m0 in range(0, M, 64):
        dec.append(_ops().moe_forward(xs[m0:m0 + 64], it[m0:m0 + 64].contiguous(), wt[m0:m0 + 64].contiguous(),
                                      table, I, K, E))
    torch.cuda.synchronize()
    dc = torch.cat(dec).cpu().numpy()
    r = rel_l2(pf, dc)
    rows = np.linalg.norm(pf - dc, axis=1) / np.linalg.norm(dc, axis=1)
    print(f"full chunk: rel-L2 prefill vs decode {r:.2e}, worst row {rows.max():.2e}", flush=True)
    assert np.isfinite(pf).all()
    assert r <= TOL and rows.max() <= 4 * TOL


def test_prefill_staged_matches_resident():
    """ExpertStore.forward_prefill_staged (non-resident experts copied from the pinned RAM arena into a staging buffer
    on a copy stream, double-buffered across layers) gives the same bits as the prefill on an all-resident table."""
    import ctypes
    from exl3xpu import nvtier
    H, I, K, E, S, L, M, topk = 256, 128, 3, 16, 20, 3, 300, 4
    print("case prefill staged vs resident", flush=True)
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    src = nvtier.SyntheticExpertSource(H, I, K, 11, n_distinct=L * E)
    for key in range(L * E):
        ctypes.memmove(store.addr(key), src.buf[key].ctypes.data, store.blob)
    rng = np.random.default_rng(5)
    for li in range(L):
        store.make_resident(keys[li], sorted(rng.choice(E, size=6, replace=False).tolist()))
    blobs = torch.from_numpy(src.buf).cuda()
    xs, outs, refs = [], [], []
    for rep in range(2):                           # the second pass reuses the buffers staged at the end of the first
        for li in range(L):
            ids, w = synth.softmax_topk(40 + li, M, E, topk)
            x = torch.from_numpy(exl3.bf16_to_f32(synth.activations(50 + li, M, H))).to(torch.bfloat16).cuda()
            it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
            outs.append(store.forward_prefill_staged(keys[li], x, it, wt))
            table = torch.tensor([blobs[li * E + e].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
            refs.append(_ops().moe_forward(x, it, wt, table, I, K, E))
    torch.cuda.synchronize()
    for n, (o, r) in enumerate(zip(outs, refs)):
        assert torch.equal(o, r), n


def test_tier_stage_forward_matches_resident():
    """NvTier.stage_forward (non-HBM experts read from the fill source into a pinned host ring, copied to an HBM
    staging buffer on a side stream, read-ahead across layers) gives the same bits as the all-resident table; two
    passes over the layers so the host ring and both staging buffers are reused."""
    import ctypes
    from exl3xpu import nvtier
    H, I, K, E, S, L, M, topk = 256, 128, 3, 16, 20, 3, 300, 4
    print("case tier stage_forward vs resident", flush=True)
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    src = nvtier.SyntheticExpertSource(H, I, K, 13, n_distinct=L * E)
    for key in range(L * E):                       # RAM copies, the source of make_resident
        ctypes.memmove(store.addr(key), src.buf[key].ctypes.data, store.blob)
    tier = nvtier.NvTier(store, src, budget_records=L * E)
    try:
        rng = np.random.default_rng(6)
        for li in range(L):
            store.make_resident(keys[li], sorted(rng.choice(np.arange(1, E), size=5, replace=False).tolist()))
        blobs = torch.from_numpy(src.buf).cuda()
        outs, refs = [], []
        for rep in range(2):
            for li in range(L):
                ids, w = synth.softmax_topk(60 + li + 7 * rep, M, E, topk)
                x = torch.from_numpy(exl3.bf16_to_f32(synth.activations(70 + li, M, H))).to(torch.bfloat16).cuda()
                it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
                outs.append(tier.stage_forward(store, keys[li], li, x, it, wt))
                table = torch.tensor([blobs[li * E + e].data_ptr() for e in range(E)], dtype=torch.int64,
                                     device="cuda")
                refs.append(_ops().moe_forward(x, it, wt, table, I, K, E))
        torch.cuda.synchronize()
        for n, (o, r) in enumerate(zip(outs, refs)):
            assert torch.equal(o, r), n
        assert tier.stats["stage_bytes"] == 2 * L * (E - 5) * store.stride     # every non-HBM expert, each pass
    finally:
        tier.close()


def test_tier_ensure_for_prefill():
    """NvTier.ensure_for_prefill (nvtier.py:389-457): before a prefill layer, every expert of the batch is made
    RAM-resident (filled from the source) and flagged on the device within the record budget, evicting first the
    transient fills of other layers, then RAM copies of HBM-resident experts, then the rest, oldest first with ties by
    ascending key; never the layer's own keys or pinned keys. The eviction set below is derived by hand from that
    rule for this state; the prefill kernels then read the batch zero-copy from the RAM arena and give the same bits
    as an all-resident table."""
    from exl3xpu import nvtier
    H, I, K, E, S, L, M, topk = 256, 128, 3, 16, 20, 3, 300, 4
    print("case tier ensure_for_prefill", flush=True)
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    src = nvtier.SyntheticExpertSource(H, I, K, 17, n_distinct=L * E)
    tier = nvtier.NvTier(store, src, budget_records=20)           # pinned safe experts 0, 16, 32 filled at init
    try:
        ram = list(range(1, 7)) + list(range(17, 23)) + list(range(33, 37))
        tier.fill_many(ram)
        store.make_resident(keys[1], [1, 2, 3])                    # keys 17, 18, 19 also in HBM
        store.make_resident(keys[2], [1])                          # key 33
        tier.transient = np.zeros(L * E, dtype=bool)
        tier.transient[[21, 22]] = True                            # fills of an earlier prefill of layer 1
        tier.res_dev.copy_(torch.from_numpy(tier.res))
        assert int(tier.res.sum()) == 19
        ids, w = synth.softmax_topk(81, M, E, topk)
        assert len(np.unique(ids)) == E                            # the batch uses every expert of layer 0
        it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
        n_fill = tier.ensure_for_prefill(0, it)
        torch.cuda.synchronize()
        # 9 misses (keys 7..15) over a budget of 20 with 19 resident: 8 evictions, by class then (age, key)
        evicted = {21, 22, 17, 18, 19, 33, 20, 34}
        assert n_fill == 9
        want = set([0, 16, 32] + list(range(1, 16)) + list(range(17, 23)) + list(range(33, 37))) - evicted
        assert set(np.nonzero(tier.res)[0].tolist()) == want
        assert int(tier.res.sum()) == 20
        assert np.array_equal(tier.res_dev.cpu().numpy(), tier.res)
        assert set(np.nonzero(tier.transient)[0].tolist()) == set(range(7, 16))
        x = torch.from_numpy(exl3.bf16_to_f32(synth.activations(82, M, H))).to(torch.bfloat16).cuda()
        table = store.ptrs_all[0:E].clone()                         # layer 0: host copies, read zero-copy
        out = _ops().moe_forward(x, it, wt, table, I, K, E)
        blobs = torch.from_numpy(src.buf).cuda()
        ref_t = torch.tensor([blobs[e].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
        ref = _ops().moe_forward(x, it, wt, ref_t, I, K, E)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    finally:
        tier.close()


def test_prefill_zero_copy_config0_shapes():
    """The prefill kernels at the config-0 expert shape (H 2048, I 512, 512 experts, top-10) on a table that mixes HBM
    slots (100 experts) and records of the pinned RAM-tier arena read over PCIe (the other 412, all routed to by
    2,048 tokens): the same bits as a table of HBM copies of the same blobs."""
    from exl3xpu import nvtier
    H, I, K, E, M, topk = 2048, 512, 3, 512, 2048, 10
    print("case prefill zero-copy config-0 shapes", flush=True)
    store = nvtier.TierStore(H, I, K, E, 100, n_layers=2)
    src = nvtier.SyntheticExpertSource(H, I, K, 23, n_distinct=32)
    blobs = torch.from_numpy(src.buf[np.arange(E) % src.n])
    keys = ["model.layers.0.mlp", "model.layers.1.mlp"]
    for k in keys:
        store.add_layer(k, blobs)
    resident = np.random.default_rng(5).choice(E, 100, replace=False)
    store.make_resident(keys[0], resident)
    ids, w = synth.softmax_topk(83, M, E, topk)
    assert len(np.unique(ids)) == E
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    x = torch.from_numpy(exl3.bf16_to_f32(synth.activations(84, M, H))).to(torch.bfloat16).cuda()
    out = store.forward(keys[0], x, it, wt)
    dblobs = torch.from_numpy(src.buf).cuda()
    ref_t = torch.tensor([dblobs[e % src.n].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
    ref = _ops().moe_forward(x, it, wt, ref_t, I, K, E)
    torch.cuda.synchronize()
    assert int((store.slot_of[keys[0]] >= 0).sum()) == 100
    assert torch.equal(out, ref)


def _plugin_sequence(H, I, K, E, S, L, topk, dsteps, budget, n_distinct, prompts, seed, pool=False, tail=(),
                     dsteps2=0):
    """The tier plugin's call sequence (plugin/sglang_plugin.tier.py:531-561 `apply`, 944-956 the host step after every
    model step) over this API, tier mode: the prompts of `prompts` ((tokens, staged?) pairs; staged prompts of at
    least 256 tokens go through stage_forward, the others through ensure_for_prefill and the zero-copy forward), then
    decode steps through forward_cached (tier mask, RAM hits written through), then the prompts of `tail` and dsteps2
    more decode steps, NvTierAsync.step after every model step. Every prompt output equals the all-resident output
    bit for bit; every decode output equals the uncached forward on the true blobs with the post-mask picks. pool:
    the RAM tier in a RecordPool (its invariants checked at the end)."""
    from exl3xpu import nvtier
    store = nvtier.TierStore(H, I, K, E, S, n_layers=L, pool=pool)
    keys = [f"model.layers.{li}.mlp" for li in range(L)]
    for k in keys:
        store.add_layer(k)
    src = nvtier.SyntheticExpertSource(H, I, K, seed, n_distinct=n_distinct)
    tier = nvtier.NvTierAsync(store, src, budget_records=budget, latency=2)
    blobs = torch.from_numpy(src.buf).cuda()
    tables = [torch.tensor([blobs[(li * E + e) % n_distinct].data_ptr() for e in range(E)], dtype=torch.int64,
                           device="cuda") for li in range(L)]

    def apply(li, x, it, wt, stage):            # the plugin's dispatch in tier mode
        if x.shape[0] >= 3:
            if stage and x.shape[0] >= 256:
                return tier.stage_forward(store, keys[li], li, x, it, wt)
            tier.ensure_for_prefill(li, it)
            return store.forward(keys[li], x, it, wt)
        store.prefill_reset()
        return store.forward_cached(keys[li], x, it, wt)

    bad, masked = [], 0
    try:
        steps = [(M, st, seed * 10 + 90 + n) for n, (M, st) in enumerate(prompts)]
        steps += [(1, False, seed * 10 + 100 + n) for n in range(dsteps)]
        steps += [(M, st, seed * 10 + 70 + n) for n, (M, st) in enumerate(tail)]
        steps += [(1, False, seed * 10 + 300 + n) for n in range(dsteps2)]
        for M, stage, sd in steps:
            for li in range(L):
                ids, w = synth.softmax_topk(sd * 7 + li, M, E, topk)
                x = torch.from_numpy(exl3.bf16_to_f32(synth.activations(sd + li, M, H))).to(torch.bfloat16).cuda()
                it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
                out = apply(li, x, it, wt, stage)
                if M == 1:
                    masked += int((wt == 0).sum().item())
                ref = _ops().moe_forward(x, it, wt, tables[li], I, K, E)     # it / wt after the tier mask
                torch.cuda.synchronize()
                if not torch.equal(out, ref):
                    bad.append((M, sd, li))
            tier.step()                            # the host step hook after every model step
        torch.cuda.synchronize()
        if pool:
            from pool_checks import check_pool
            check_pool(store, tier, src, budget)
    finally:
        tier.close()
    assert not bad, f"outputs differ at (M, seed, layer) {bad[:4]}"
    assert masked > 0                              # the decode steps exercised the tier mask
    return tier


def test_plugin_caller_sequence():
    """The plugin's tier-mode call sequence at small expert shapes (H 256, I 128, 32 experts, top-4): a 300-token
    prompt streamed through stage_forward (staging buffers within the verified size), a 24-token prompt, 40 decode
    steps."""
    print("case plugin caller sequence", flush=True)
    _plugin_sequence(256, 128, 3, 32, 24, 3, 4, 40, 40, 3 * 32, [(300, True), (24, False)], 23)


def test_plugin_caller_sequence_record_pool():
    """The plugin's sequence with the RAM tier in a RecordPool (H 256, I 128, 32 experts, top-4, 3 layers, 24 HBM
    slots, a 40-record budget, write-back queue 48): a staged 300-token prompt, a 24-token prompt, 40 decode steps,
    then a 24-token and a staged 300-token prompt while fills are in flight and write-backs unsettled (the prefill
    path finishes those fills and patches the snapshot the next host step reads), then 30 more decode steps. Outputs
    as in the other sequences; at the end the pool's invariants hold (no dropped write-back, within budget +
    3 x queue records, every resident key's record holds its blob)."""
    print("case plugin caller sequence record pool", flush=True)
    tier = _plugin_sequence(256, 128, 3, 32, 24, 3, 4, 40, 40, 3 * 32, [(300, True), (24, False)], 31, pool=True,
                            tail=[(24, False), (300, True)], dsteps2=30)
    assert tier.stats["wb_taken"] > 0 and tier.stats.get("prefill_evicts", 0) > 0


def test_plugin_caller_sequence_config0_shapes():
    """The same sequence at the config-0 expert shapes (H 2048, I 512, 512 experts of 1.2 MB, top-10; 2 layers, 300
    HBM slots, a 700-record RAM tier): the 300-token prompt through stage_forward needs a 612 MB staging buffer, above
    the verified size, so it takes the zero-copy route (ensure_for_prefill, then the prefill kernels read the non-HBM
    experts from their pinned records); its output equals the all-resident output bit for bit, as do the 24-token
    prompt's and the decode steps'."""
    from exl3xpu.moe_offload import staging_fits
    print("case plugin caller sequence config-0 shapes", flush=True)
    assert not staging_fits(512, 1196032)
    _plugin_sequence(2048, 512, 3, 512, 300, 2, 10, 12, 700, 64, [(300, True), (24, False)], 29)


@pytest.mark.parametrize("M", [150, 255])
def test_midsize_rows_uncached_vs_oracle(M):
    """Uncached calls with more picks than the decode kernel takes (1,500 and 2,550 at top-10) below prefill_min_m
    (256, unchanged) run the prefill kernels (the reference's align path, kernels/moe-a8/exl3_moe.a8.sycl:1277-1314):
    config-0 shapes, against the oracle's prefill rounding points within rel-L2 2e-3 (16 distinct blobs over the 512
    experts keep the oracle to seconds)."""
    H, I, K, E, TK, nd = 2048, 512, 3, 512, 10, 16
    print(f"case mid-size rows uncached M={M}", flush=True)
    ids, w = synth.softmax_topk(700 + M, M, E, TK)
    made = [synth.expert_blob(31, j, H, I, K) for j in range(nd)]
    dev = torch.from_numpy(np.stack(made)).cuda()
    table = torch.tensor([dev[e % nd].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
    x = synth.activations(800 + M, M, H)
    gb = _run(x, ids, w, table, I, K, E)
    ews = [exl3.ExpertWeights(b, H, I, K) for b in made]
    ob, _ = exl3.moe_forward(x, ids, w, lambda e: ews[e % nd], variant="prefill")
    r = rel_l2(gb, exl3.bf16_to_f32(ob))
    print(f"mid-size M={M}: rel-L2 bf16 {r:.2e}", flush=True)
    assert np.isfinite(gb).all() and r <= TOL
