"""Pins the EXL3 oracle (oracle/exl3.py) against independent checks: closed forms computed another way, brute force,
invariants and a float64 dense reconstruction. A plausible slip (wrong byte, wrong shift, transposed tile, dropped
rounding) fails at least one of these."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

from oracle import exl3, synth

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _half_bits(v: float) -> int:
    return struct.unpack("<H", struct.pack("<e", v))[0]


def test_codebook_exhaustive_vs_python_ints():
    """Every state: pure-Python integer arithmetic + IEEE half rounding from the struct module (independent of numpy's
    float16 cast)."""
    tab = exl3.codebook_table().view(np.uint16)
    c1 = struct.unpack("<e", struct.pack("<H", 0x1EEE))[0]
    c2 = struct.unpack("<e", struct.pack("<H", 0xC931))[0]
    assert (c1, c2) == (exl3.C1, exl3.C2)
    for s in range(65536):
        x = (s * 0x83DCD12D) & 0xFFFFFFFF
        h = 1024 + sum((x >> (8 * i)) & 0xFF for i in range(4))
        assert 1024 <= h <= 2044
        assert tab[s] == _half_bits(h * c1 + c2), s


def test_codebook_known_answers_and_range():
    cb = exl3.codebook_table().astype(np.float64)
    assert cb[0] == -3.453125                       # x = 0: h = 1024, 1024*c1 + c2 exactly
    # state 1: x = 0x83DCD12D, bytes 0x83+0xDC+0xD1+0x2D = 131+220+209+45 = 605 -> h = 1629
    assert exl3.codebook_raw_h(np.array([1]))[0] == 1629
    assert cb[1] == float(np.float16(1629 * exl3.C1 + exl3.C2))
    assert cb.min() >= -3.4532 and cb.max() <= 3.4532     # exl3_ops.sycl:522 range
    assert abs(cb.mean()) < 0.05 and 0.9 < cb.std() < 1.1
    h = json.load(open(os.path.join(GOLD, "codebook.json")))
    assert hashlib.sha256(exl3.codebook_table().tobytes()).hexdigest() == h["sha256"]
    assert [int(v) for v in exl3.codebook_table().view(np.uint16)[h["probe_states"]]] == h["probe_bits"]


@pytest.mark.parametrize("cb", [0, 1])
def test_codebook_lcg_exhaustive_vs_python_ints(cb):
    """3inst / mcg, every state: pure-Python integer arithmetic, both halves decoded by the struct module and summed
    exactly (Python floats hold the sum of two halves exactly), then one IEEE half rounding (struct 'e' packs
    half-to-even): independent of numpy's float16 arithmetic."""
    tab = exl3.codebook_table(cb).view(np.uint16)
    a, b = ((89226354, 64248484), (0xCBAC1FED, 0))[cb]
    for s in range(65536):
        x = (s * a + b) & 0xFFFFFFFF
        m = (x & 0x8FFF8FFF) ^ 0x3B603B60
        lo = struct.unpack("<e", struct.pack("<H", m & 0xFFFF))[0]
        hi = struct.unpack("<e", struct.pack("<H", m >> 16))[0]
        assert tab[s] == _half_bits(lo + hi), (cb, s)


def test_codebook_lcg_known_answers_and_invariants():
    """Hand-computed values, the exponent range the mask / xor step forces on both halves (fields 12..15, so every
    half is normal with magnitude in [1/8, 2) and every weight in (-4, 4)), and a zero mean over all states."""
    t3, tm = exl3.codebook_table(0), exl3.codebook_table(1)
    # 3inst, state 0: x = 64248484 = 0x03D45AA4 -> m = 0x38B431C4: 0.587890625 + 0.18017578125 = 0.76806640625
    assert t3.view(np.uint16)[0] == 0x3A25 and float(t3[0]) == 0.76806640625
    # mcg, state 0: m = 0x3B603B60: 0.921875 + 0.921875 = 1.84375; state 1: x = 0xCBAC1FED -> m = 0xB0CC348D:
    # -0.14990234375 + 0.284423828125 = 0.134521484375
    assert tm.view(np.uint16)[0] == 0x3F60 and tm.view(np.uint16)[1] == 0x304E
    st = np.arange(65536, dtype=np.uint64)
    for cb, tab in ((0, t3), (1, tm)):
        a, b = exl3.LCG[cb]
        m = (((st * np.uint64(a) + np.uint64(b)) & np.uint64(0xFFFFFFFF)) & np.uint64(0x8FFF8FFF)) ^ np.uint64(0x3B603B60)
        for half in (m & np.uint64(0xFFFF), m >> np.uint64(16)):
            e = (half >> np.uint64(10)) & np.uint64(0x1F)
            assert e.min() == 12 and e.max() == 15
        w = tab.astype(np.float64)
        assert np.isfinite(w).all() and np.abs(w).max() < 4.0
        assert abs(w.mean()) < 0.01 and 1.2 < w.std() < 1.3


def _brute_states(words, K):
    """Bit-by-bit: bit b of the tile stream is bit 31 - b%32 of word b//32 (MSB first); state t = the 16 bits
    ending (exclusive) at (t+1)K, circular."""
    nb = 32 * words.size
    bits = [(int(words[b // 32]) >> (31 - b % 32)) & 1 for b in range(nb)]
    out = []
    for t in range(256):
        e = (t + 1) * K
        v = 0
        for b in range(e - 16, e):
            v = (v << 1) | bits[b % nb]
        out.append(v)
    return np.array(out)


@pytest.mark.parametrize("K", [2, 3, 4])
def test_tile_states_bruteforce(K):
    rng = np.random.default_rng(K)
    for _ in range(3):
        w = rng.integers(0, 1 << 32, size=8 * K, dtype=np.uint64).astype(np.uint32)
        assert np.array_equal(exl3.tile_states(w[None], K)[0], _brute_states(w, K))


@pytest.mark.parametrize("K", [2, 3, 4])
def test_trellis_symbol_invariants(K):
    """Encode 256 random K-bit symbols MSB-first: state t's low K bits are symbol t and state t >> K equals the low
    16-K bits of state t-1 (the trellis shift)."""
    rng = np.random.default_rng(10 + K)
    sym = rng.integers(0, 1 << K, size=256)
    bits = []
    for s in sym:
        bits += [(int(s) >> (K - 1 - i)) & 1 for i in range(K)]
    words = np.array([int("".join(map(str, bits[32 * i:32 * i + 32])), 2) for i in range(8 * K)], dtype=np.uint32)
    st = exl3.tile_states(words[None], K)[0].astype(np.int64)
    assert np.array_equal(st & ((1 << K) - 1), sym)
    mask = (1 << (16 - K)) - 1
    assert np.array_equal(st >> K, np.roll(st, 1) & mask)


def test_tile_pos_bijection():
    r, c = exl3.tile_pos(np.arange(256))
    assert len(set(zip(r.tolist(), c.tolist()))) == 256 and r.max() == 15 and c.max() == 15
    assert (r[0], c[0]) == (0, 0) and (r[1], c[1]) == (1, 0) and (r[4], c[4]) == (0, 8) and (r[32], c[32]) == (0, 1)


def test_planar4_index_map():
    K, G, D = 3, 8, 3
    rows, n = 2, 8
    nat = np.arange(rows * n * 24, dtype=np.uint32).reshape(rows, n, 24)
    pl = exl3.planar4(nat, K)
    for r in range(rows):
        flat_in, flat_out = nat[r].reshape(-1), pl[r].reshape(-1)
        for q in range(n // 4):
            for t in range(4):
                for g in range(G):
                    for i in range(D):
                        assert flat_out[q * 96 + i * 32 + t * 8 + g] == flat_in[(q * 4 + t) * 24 + 3 * g + i]
    assert np.array_equal(exl3.unplanar4(pl, K), nat)
    nat2 = np.arange(64, dtype=np.uint32).reshape(1, 4, 16)
    assert np.array_equal(exl3.planar4(nat2, 2), nat2)


def test_trellis_words_little_endian():
    tr = np.array([[[0x1234, 0x5678, -1, 0]]], dtype=np.int16)
    assert exl3.trellis_words(tr).tolist() == [[[0x56781234, 0x0000FFFF]]]


def test_fwht128_vs_scipy():
    from scipy.linalg import hadamard
    Hm = hadamard(128)
    v = np.random.default_rng(0).standard_normal((5, 128)).astype(np.float32)
    ref = v.astype(np.float64) @ Hm.T
    assert np.allclose(exl3.fwht128(v), ref, rtol=1e-5, atol=1e-4)
    assert np.array_equal(Hm @ Hm, 128 * np.eye(128, dtype=Hm.dtype))
    e = np.zeros(128, np.float32)
    e[5] = 1.0
    assert np.array_equal(exl3.fwht128(e), Hm[:, 5].astype(np.float32))


def test_blob_layout():
    o = exl3.blob_layout(2048, 512, 3)
    assert o["blob"] == 1_195_008 and o["d"] == 786_432 and o["suh_g"] == 786_432 + 393_216
    assert exl3.blob_bytes(2560, 640, 3) == 1_862_400           # reference value (moe_offload.py:8)
    assert [exl3.blob_bytes(4096, 1536, k) for k in (2, 3, 4)] == [4_752_384, 7_111_680, 9_470_976]


def test_pack_unpack_roundtrip():
    H, I, K = 256, 128, 3
    g, u, d = synth.expert_checkpoint(np.random.default_rng(1), H, I, K)
    blob = exl3.pack_expert(g, u, d, K)
    assert blob.size == exl3.blob_bytes(H, I, K)
    up = exl3.unpack_blob(blob, H, I, K)
    gu = exl3.trellis_words(np.concatenate([g["trellis"], u["trellis"]], axis=1))
    assert np.array_equal(up["gu"], gu) and np.array_equal(up["d"], exl3.trellis_words(d["trellis"]))
    assert np.array_equal(up["svh_d"], d["svh"]) and np.array_equal(up["suh_u"], u["suh"])


@pytest.mark.parametrize("K", [2, 3, 4])
def test_expert_forward_vs_dense_float64(K):
    """The rounded oracle pipeline stays close to an independent float64 dense computation; a dropped scale, a
    transposed tile or a sign error would move it by O(1)."""
    H, I = 256, 256
    blob = synth.expert_blob(7, K, H, I, K)
    ew = exl3.ExpertWeights(blob, H, I, K)
    x = exl3.bf16_to_f32(synth.activations(7, 3, H))
    for m in range(3):
        y = exl3.expert_pair(x[m], ew, 0.37)
        ref = exl3.dense_reference(x[m], ew, 0.37)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 3e-3
        yp = exl3.expert_pair(x[m], ew, 0.37, "prefill")
        assert np.linalg.norm(yp - ref) / np.linalg.norm(ref) < 3e-3


def test_moe_forward_combine_order():
    H, I, K = 256, 128, 3
    ews = {e: exl3.ExpertWeights(synth.expert_blob(3, e, H, I, K), H, I, K) for e in range(4)}
    x = synth.activations(3, 2, H)
    ids = np.array([[0, 2], [3, 1]], np.int32)
    w = np.array([[0.6, 0.4], [0.5, 0.5]], np.float32)
    out, of = exl3.moe_forward(x, ids, w, ews)
    y = exl3.expert_pair(exl3.bf16_to_f32(x[1]), ews[3], 0.5) + exl3.expert_pair(exl3.bf16_to_f32(x[1]), ews[1], 0.5)
    assert np.allclose(of[1], y, rtol=0, atol=1e-7)
    assert np.array_equal(out, exl3.f32_to_bf16(of))


def test_bf16_rne():
    f = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e-3], np.float32)    # 1 + 2^-8 ties to even (1.0)
    b = exl3.f32_to_bf16(f)
    assert b[0] == 0x3F80 and b[1] == 0x3F80 and b[2] == 0x3F82 and exl3.bf16_to_f32(b)[3] == -2.5


def test_align_stable_counting_sort():
    rng = np.random.default_rng(5)
    ids = rng.integers(0, 16, size=(37, 4)).astype(np.int32)
    w = rng.random((37, 4)).astype(np.float32)
    a = exl3.align(ids, w, 16, pad=8)
    order = np.argsort(ids.reshape(-1), kind="stable")
    assert np.array_equal(a["pair_tok"], order // 4)
    assert np.array_equal(np.sort(a["act_expert"]), np.unique(ids))
    assert np.array_equal(ids.reshape(-1)[order][a["pair_of"]], ids.reshape(-1))
    assert a["n_blk"] == sum(-(-c // 8) for c in np.bincount(ids.reshape(-1)) if c)


def _f32_nudge(x, k):
    """x (float32 array) moved by k in {-1, 0, 1} ulps."""
    if k == 0:
        return x
    return np.nextafter(x, np.float32(np.inf) if k > 0 else np.float32(-np.inf)).astype(np.float32)


def test_silu_device_formula_bound():
    """The SiLU of both expert kernels (silu_mul, csrc/exl3_common.cuh): g * rcp(1 + exp2(fp32(-g * log2e_f32))) with
    v_exp_f32 and v_rcp_f32 each within one fp32 ulp. For every finite fp16 g and every combination of those ulp
    errors, the fp32 SiLU stays within 4e-6 relative of g / (1 + exp(-g)) in float64 (results below 1e-30 in
    magnitude: both below 1e-30), and its fp16 rounding is at most one fp16 ulp from that of the exact value. A
    formula with exp(+g), or a lost factor g, fails both bounds by orders of magnitude."""
    g16 = np.arange(65536, dtype=np.uint16).view(np.float16)
    g16 = g16[np.isfinite(g16)]
    g32, g = g16.astype(np.float32), g16.astype(np.float64)
    with np.errstate(over="ignore"):
        exact = g / (1.0 + np.exp(-g))
        e32 = np.exp2(((-g32) * np.float32(float.fromhex("0x1.715476p+0"))).astype(np.float64)).astype(np.float32)

    def order(h):                      # fp16 values -> integers in value order (one step = one fp16 ulp)
        b = h.view(np.int16).astype(np.int32)
        return np.where(b < 0, -(b & 0x7FFF), b)
    big = np.abs(exact) > 1e-30
    worst_rel, worst_ulp = 0.0, 0
    for de in (-1, 0, 1):
        d = np.float32(1) + _f32_nudge(e32, de)
        with np.errstate(divide="ignore", over="ignore"):
            r = (1.0 / d.astype(np.float64)).astype(np.float32)
        for dr in (-1, 0, 1):
            s = g32 * _f32_nudge(r, dr)
            rel = np.abs(s[big].astype(np.float64) - exact[big]) / np.abs(exact[big])
            worst_rel = max(worst_rel, float(rel.max()))
            assert (np.abs(s[~big]) <= 1e-30).all()
            worst_ulp = max(worst_ulp, int(np.abs(order(s.astype(np.float16)) - order(exact.astype(np.float16))).max()))
    assert worst_rel <= 4e-6 and worst_ulp <= 1, (worst_rel, worst_ulp)
