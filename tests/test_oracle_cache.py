"""Pins the cache oracle (oracle/cache_oracle.c) with a from-scratch pure-Python brute force on tiny configurations,
and checks the cache invariants over a long Zipf trace."""
import numpy as np
import pytest

from oracle import cache, synth


class Brute:
    """Direct restatement of the device ensure (a8:864-1039) and the admission host step (nvtier.py:708-806), written
    with explicit sorts and Python sets instead of selection/compaction."""

    def __init__(self, L, E, S, R, budget, age, qmax, latency, tier=True):
        self.L, self.E, self.S, self.R = L, E, S, R
        self.budget, self.agemin, self.qmax, self.lat, self.tier = budget, age, qmax, latency, tier
        n = L * E
        self.slot_of = [-1] * n
        self.slot_key = [-1] * S
        self.slot_last = [-1] * S
        self.tick = 0
        self.ram = [0] * n
        self.ring = [0] * (1 + R)
        self.res = [0] * n
        self.pin = set()
        if tier:
            for li in range(L):
                self.res[li * E] = self.ram[li * E] = 1
                self.pin.add(li * E)
        self.age = [0] * n
        self.inflight = set()
        self.htick = 1
        self.snaps = []
        self.last = {}
        self.seen = 0
        self.pending = {}
        self.hstep = 0

    def ensure(self, li, ids, w):
        E = self.E
        self.tick += 1
        T = self.tick
        if self.tier:
            for i in range(len(ids)):
                key = li * E + ids[i]
                if self.slot_of[key] < 0 and not self.ram[key]:
                    c = self.ring[0]
                    self.ring[0] += 1
                    self.ring[1 + c % self.R] = key
                    ids[i], w[i] = 0, 0.0
        need = sorted(set(ids))
        miss = []
        for e in need:
            s = self.slot_of[li * E + e]
            if s >= 0:
                if self.slot_last[s] != 0x7FFFFFFF:
                    self.slot_last[s] = T
            else:
                miss.append(e)
        elig = [(self.slot_last[s] + 1, s) for s in range(self.S) if self.slot_last[s] < T]
        nm = min(len(miss), len(elig)) if self.S else 0
        chosen = sorted(elig)[:nm]                        # exact LRU, ties by slot
        tau = chosen[-1][0] if nm else None
        V = sorted(s for u, s in chosen if u < tau) + [s for u, s in chosen if u == tau]
        vict = []
        for mi in range(nm):
            s, e = V[mi], miss[mi]
            old = self.slot_key[s]
            wb = -1 if (self.tier and old >= 0 and self.ram[old]) else old
            if old >= 0:
                self.slot_of[old] = -1
            key = li * E + e
            self.slot_key[s], self.slot_of[key], self.slot_last[s] = key, s, T
            vict.append((wb, s))
            if self.tier and wb >= 0:
                self.ram[wb] = 1
        return T, list(ids), nm, miss[:nm], vict

    def host_step(self):
        n = self.L * self.E
        self.htick += 1
        snap = (list(self.ram), list(self.ring), [s >= 0 for s in self.slot_of])
        self.snaps.append(snap)
        hs = self.hstep
        self.hstep += 1
        if len(self.snaps) < 2:
            return [], []
        prev = self.snaps[-2]
        view = list(prev[0])
        for k, v in self.last.items():
            view[k] = v
        ring, vram = prev[1], prev[2]
        res = list(self.res)
        for k in range(n):
            if view[k] == 1 and self.res[k] == 0:
                self.age[k] = self.htick
                res[k] = 1
        for k in self.pending.pop(hs, []):
            res[k] = 1
            self.age[k] = self.htick
            self.inflight.discard(k)
        cnt = ring[0]
        newm = min(cnt - self.seen, self.R)
        keys = [ring[1 + (p % self.R)] for p in range(cnt - newm, cnt)] if newm > 0 else []
        counts = {}
        for k in keys:
            counts[k] = counts.get(k, 0) + 1
        want = [k for k in sorted(counts) if res[k] == 0 and k not in self.inflight]
        want.sort(key=lambda k: -counts[k])               # Python sort is stable
        self.seen = cnt
        inflight_n = len(self.inflight)
        over = sum(res) + inflight_n + len(want) - self.budget
        ev = []
        if over > 0:
            c1 = sorted((k for k in range(n) if res[k] and vram[k] and k not in self.pin), key=lambda k: (self.age[k], k))
            ev = c1[:over]
            over -= len(ev)
            if over > 0:
                c2 = sorted((k for k in range(n) if res[k] and k not in self.pin and self.age[k] <= self.htick - self.agemin
                             and k not in ev), key=lambda k: (self.age[k], k))
                ev += c2[:over]
            for k in ev:
                res[k] = 0
        free = max(0, min(self.budget - sum(res) - inflight_n, self.qmax - inflight_n))
        adm = want[:free]
        for k in adm:
            self.inflight.add(k)
        self.pending.setdefault(hs + self.lat, []).extend(adm)
        self.last = {k: res[k] for k in range(n) if res[k] != view[k]}
        for k, v in self.last.items():
            self.ram[k] = v
        self.res = res
        return adm, ev


@pytest.mark.parametrize("seed,tier", [(1, True), (2, True), (3, False), (4, True)])
def test_cache_oracle_vs_bruteforce(seed, tier):
    L, E, S, R, P = 3, 8, 5, 16, 3
    budget, age, qmax, lat = 7, 2, 3, 2
    rng = np.random.default_rng(seed)
    steps = 120
    ids = np.stack([np.stack([rng.choice(E, P, replace=False) for _ in range(L)]) for _ in range(steps)]).astype(np.int32)
    w = rng.random((steps, L, P)).astype(np.float32)
    co = cache.CacheOracle(L, E, S, ring_cap=R, tier=tier, budget=budget, age=age, qmax=qmax, latency=lat)
    br = Brute(L, E, S, R, budget, age, qmax, lat, tier=tier)
    for n in range(steps):
        for li in range(L):
            a_ids, a_w = ids[n, li].copy(), w[n, li].copy()
            rec = co.ensure(li, a_ids, a_w)
            T, post, nm, miss, vict = br.ensure(li, list(ids[n, li]), list(w[n, li]))
            assert rec[0] == T and list(rec[2:2 + P]) == post and rec[2 + P] == nm
            assert list(rec[3 + P:3 + P + nm]) == miss
            assert [tuple(rec[3 + 2 * P + 2 * i:5 + 2 * P + 2 * i]) for i in range(nm)] == vict
            assert np.array_equal(a_ids, np.array(post, np.int32))
        if tier:
            adm, ev = co.host_step()
            badm, bev = br.host_step()
            assert adm.tolist() == badm and ev.tolist() == bev, n
            assert co.ram_res.tolist() == br.ram
        assert co.slot_of.tolist() == br.slot_of and co.slot_last.tolist() == br.slot_last


def test_cache_invariants_zipf():
    L, E, S = 8, 64, 120
    steps, P = 600, 6
    ids, w = synth.zipf_trace(99, steps, L, E, P)
    co = cache.CacheOracle(L, E, S, budget=60, qmax=16, latency=3)
    qmax = 16
    for n in range(steps):
        for li in range(L):
            a, b = ids[n, li, 0].copy(), w[n, li, 0].copy()
            rec = co.ensure(li, a, b)
            T, nm = rec[0], rec[2 + P]
            slots = rec[3 + 2 * P + 1:3 + 4 * P:2][:nm]
            assert len(set(slots.tolist())) == nm
            # every assigned slot is now stamped T and owned by a key of this layer
            assert all(co.slot_last[s] == T and co.slot_key[s] // E == li for s in slots)
        adm, ev = co.host_step()
        assert len(adm) <= qmax and int(co.inflight.sum()) <= qmax
        sk = co.slot_key
        own = sk[sk >= 0]
        assert len(set(own.tolist())) == own.size                          # one slot per key
        assert all(co.slot_of[k] == s for s, k in enumerate(sk) if k >= 0)  # slot_of / slot_key bijection
        assert int((co.slot_of >= 0).sum()) == own.size <= S
        # budget holds after eviction, except for device write-backs flagged during the step
        assert int(co.res.sum()) + int(co.inflight.sum()) <= 60 + 2 * L * P


def test_cache_oracle_prefetch_hand_case():
    """Prefetch mode (moe_prefetch, a8:846-851, 1194-1222) on a case derived by hand: 4 slots, 8 experts, no tier.
    The tick is not advanced, so slots stamped by the last MoE call stay protected; hits are re-stamped with the
    current tick; misses take exact-LRU slots among those older than the tick."""
    L, E, S, P = 1, 8, 4, 2
    co = cache.CacheOracle(L, E, S, tier=False)
    k = cache.rec_len
    # MoE call 1 (T = 1): experts 0, 1 miss and take the empty slots 0, 1 (u = 0, ascending slot)
    r = co.ensure(0, np.array([0, 1], np.int32), np.ones(2, np.float32))
    assert r[0] == 1 and r[2 + P] == 2 and r[3 + P:3 + 2 * P].tolist() == [0, 1]
    assert r[3 + 2 * P:].tolist() == [-1, 0, -1, 1]
    # prefetch of [2, 3, 1] (T stays 1): 1 hits; 2, 3 take the empty slots 2, 3; nothing is advanced
    r = co.prefetch(0, np.array([2, 3, 1], np.int32))
    assert len(r) == k(3) and r[0] == 1 and r[2 + 3] == 2
    assert r[3 + 3:3 + 6].tolist() == [2, 3, -1] and r[3 + 6:3 + 10].tolist() == [-1, 2, -1, 3]
    assert co.tick[0] == 1 and co.slot_last.tolist() == [1, 1, 1, 1] and co.slot_key.tolist() == [0, 1, 2, 3]
    # prefetch of [4]: every slot was stamped by the current tick, so none is eligible
    r = co.prefetch(0, np.array([4], np.int32))
    assert r[2 + 1] == 0 and co.slot_of[4] == -1 and co.slot_key.tolist() == [0, 1, 2, 3]
    # MoE call 2 (T = 2) with [3, 4]: 3 hits (stamped 2); 4 misses; eligible slots 0, 1, 2 all hold u = 2 -> slot 0,
    # whose owner (expert 0) goes back to host
    r = co.ensure(0, np.array([3, 4], np.int32), np.ones(2, np.float32))
    assert r[0] == 2 and r[2 + P] == 1 and r[3 + P] == 4 and r[3 + 2 * P:3 + 2 * P + 2].tolist() == [0, 0]
    assert co.slot_of[0] == -1 and co.slot_of[4] == 0 and co.slot_last.tolist() == [2, 1, 1, 2]
    # prefetch of [0, 5, 6] with max_fill 2 (T stays 2): misses 0, 5 (ascending, capped at 2) take the LRU slots 1, 2
    r = co.prefetch(0, np.array([0, 5, 6], np.int32), max_fill=2)
    assert r[0] == 2 and r[2 + 3] == 2 and r[3 + 3:3 + 5].tolist() == [0, 5]
    assert r[3 + 6:3 + 10].tolist() == [1, 1, 2, 2]          # (old key 1, slot 1), (old key 2, slot 2)
    assert co.slot_key.tolist() == [4, 0, 5, 3] and co.slot_last.tolist() == [2, 2, 2, 2] and co.tick[0] == 2


def test_cache_oracle_plan_hand_case():
    """Copy-engine plan mode (moe_prefetch_plan, a8:853-901, 1013-1038, 1127-1142) on a case derived by hand: claimed
    slots are pinned (never victims, hits do not re-stamp them) until the next call commits them with the plan's
    tick; at most 16 misses per plan."""
    L, E, S = 1, 8, 4
    co = cache.CacheOracle(L, E, S, tier=False)
    co.ensure(0, np.array([0, 1], np.int32), np.ones(2, np.float32))           # T = 1: experts 0, 1 -> slots 0, 1
    r = co.plan(0, np.array([2, 3], np.int32))                                  # T stays 1: 2, 3 -> slots 2, 3
    assert r[0] == 1 and r[2 + 2] == 2 and r[3 + 2:3 + 4].tolist() == [2, 3]
    assert co.slot_last.tolist() == [1, 1, 0x7FFFFFFF, 0x7FFFFFFF] and co.tick[0] == 1
    # next decode call (T = 2): the plan is committed first (slots 2, 3 -> tick 1); 2 hits (stamped 2); 5 misses and
    # takes the lowest slot among the eligible u = 2 (slots 0, 1, 3): slot 0, evicting expert 0
    r = co.ensure(0, np.array([2, 5], np.int32), np.ones(2, np.float32))
    assert r[0] == 2 and r[2 + 2] == 1 and r[3 + 2] == 5 and r[3 + 4:3 + 6].tolist() == [0, 0]
    assert co.slot_last.tolist() == [2, 1, 2, 1] and co.slot_key.tolist() == [5, 1, 2, 3]
    r = co.plan(0, np.array([4], np.int32))                                     # T = 2: 4 -> slot 1, pinned
    assert r[2 + 1] == 1 and r[3 + 2 * 1 + 1] == 1 and co.slot_last[1] == 0x7FFFFFFF
    # a second plan commits the first (slot 1 -> 2), so only slot 3 (last 1 < 2) is eligible: 6 -> slot 3
    r = co.plan(0, np.array([6, 7], np.int32))
    assert r[2 + 2] == 1 and r[3 + 2] == 6 and r[3 + 4:3 + 6].tolist() == [3, 3]
    assert co.slot_last.tolist() == [2, 2, 2, 0x7FFFFFFF] and co.slot_key.tolist() == [5, 4, 2, 6]
    # a prefetch call does not commit pending plans: slot 3 stays pinned and is not a victim
    r = co.prefetch(0, np.array([7], np.int32))
    assert r[2 + 1] == 0 and co.slot_last[3] == 0x7FFFFFFF
    # the cap: a plan claims at most 16 slots whatever max_fill says
    co2 = cache.CacheOracle(1, 64, 40, tier=False)
    r = co2.plan(0, np.arange(30, dtype=np.int32), max_fill=30)
    assert r[2 + 30] == 16 and int((co2.slot_last == 0x7FFFFFFF).sum()) == 16


@pytest.mark.parametrize("K", [3, 96])
def test_cache_oracle_victim_ring_claims_and_drains(K):
    """The victim ring (co_set_ring) against a closed form of the reference's serial claim loop and the drain
    protocol, call by call: the slots a call claims are the first min(write-backs, free) free slots in circular order
    from the search position before it, taken by the call's written-back victims in victim order with consecutive
    claim numbers; the rest are dropped; the position moves past the last slot claimed. Every key the host takes into
    flight at step h is RAM-resident at step h + 1 with age h + 1, its slot free again before the next call; a ring
    key is never RAM-resident and in flight at once."""
    L, E, S, P, steps = 3, 48, 30, 6, 160
    ids, w = synth.zipf_trace(77 + K, steps, L, E, P)
    ids, w = ids[:, :, 0], w[:, :, 0]
    co = cache.CacheOracle(L, E, S, budget=90, age=4, qmax=24, latency=2, victim_ring=K)
    flying_prev = set()
    total_claims = total_drops = 0
    for n in range(steps):
        for li in range(L):
            key0, seq0, st0 = co.vr_key.copy(), co.vr_seq.copy(), co.ring_stats()
            rec = co.ensure(li, ids[n, li].copy(), w[n, li].copy())
            st1 = co.ring_stats()
            nc, nd = st1["claims"] - st0["claims"], st1["drops"] - st0["drops"]
            total_claims, total_drops = total_claims + nc, total_drops + nd
            nm = int(rec[2 + P])
            wbs = [int(rec[3 + 2 * P + 2 * mi]) for mi in range(nm)]
            claimed_keys = [k for k in wbs if k >= 0]
            assert len(claimed_keys) == nc
            free = [(st0["pos"] + t) % K for t in range(K) if key0[(st0["pos"] + t) % K] < 0]
            want = free[:nc]
            assert nd == 0 or nc == len(free), "dropped while a slot was free"
            got = [r for r in range(K) if co.vr_seq[r] != seq0[r]]
            assert sorted(got) == sorted(want)
            assert [int(co.vr_key[r]) for r in want] == claimed_keys
            assert [int(co.vr_seq[r]) for r in want] == list(range(st0["claims"] + 1, st1["claims"] + 1))
            if nc:
                assert st1["pos"] == (want[-1] + 1) % K
            else:
                assert st1["pos"] == st0["pos"]
            for k in claimed_keys:                     # the device never flags a ring victim RAM-resident
                assert co.ram_res[k] == 0
        infl0 = co.inflight.copy()
        co.host_step()
        t = co.host_tick
        for k in flying_prev:                          # drains taken into flight last step have landed
            assert co.res[k] == 1 and co.age[k] == t and co.inflight[k] == 0
            assert k not in set(co.vr_key.tolist())      # and its slot is free again
        # the ring keys taken into flight by this step (fills admitted now are not in the ring)
        flying_prev = {int(k) for k in np.nonzero(co.inflight & ~infl0)[0]}
        flying_prev &= {int(k) for k in co.vr_key.tolist() if k >= 0}
        assert not (co.inflight.astype(bool) & (co.res == 1)).any()
        assert co.ring_stats()["error"] == 0
    assert total_claims > 0
    if K == 3:
        assert total_drops > 0                         # a small ring overflows on this trace
    else:
        assert total_drops == 0
