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

