"""NumPy restatement of the EXL3 (mul1 trellis) expert format and the routed-expert forward.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the checker, never the product.

Reference files restated here (paths relative to the reference repository root):
  kernels/moe-a8/exl3_esimd.h            Geo (4-35), decode_cb_h mul1 (40-68) and 3inst / mcg (69-79),
                                         tile_states (120-149),
                                         fwht128 + kRsqrt128 (210-223), ReconstructKernel (869-936)
  kernels/moe-a8/exl3_moe.a8.sycl        blob layout (1-22, 42-54), GateUpKernel (121-260), DownKernel (264-368),
                                         CombineKernel (371-395), GateUpDpasKernel/DownDpasKernel (422-635),
                                         launch_align (639-680)
  plugin/exl3xpu/moe_offload.py          planar4 / pack_expert (68-89)

Parity pinning (what fixes each function independently of this file; tests/test_oracle_exl3.py):
  codebook_mul1   exhaustive closed form checked against pure-Python integer arithmetic + struct 'e' (IEEE half)
                  rounding, hand-computed known answers, range and h-range invariants, committed table hash.
  codebook_lcg    (3inst, mcg) exhaustive check against pure-Python integer arithmetic + struct 'e' (IEEE half)
                  decoding of both halves and an exact-rational sum rounded half-to-even; hand-computed known answers;
                  the exponent-range invariant of the mask/xor step; a zero mean over the 65,536 states (a wrong
                  mask gives 0.70). The generator constants themselves rest on the reference's source text only: the
                  reference holds no vectors for these codebooks (parity of the constants unpinned).
  tile_states     bit-by-bit brute force on random tiles; trellis invariants (low K bits of state t are symbol t,
                  consecutive states overlap by 16-K bits); tail-biting wrap.
  tile_pos        bijection onto the 16x16 tile.
  planar4         hand-built index tensors; round trip with unplanar4.
  fwht128         scipy.linalg.hadamard(128) product; H.H = 128 I.
  expert_forward  float64 dense reconstruction W_eff = diag(suh) Hb W_inner Hb diag(svh) / 128 (independent path).
  align           stable counting sort vs numpy argsort(kind="stable").
"""
from __future__ import annotations

import numpy as np

MUL1 = 0x83DCD12D                       # exl3_esimd.h:54 (st * 0x83DCD12D)
C1 = 0.00676727294921875                # fp16 0x1eee, exl3_esimd.h:64
C2 = -10.3828125                        # fp16 0xc931, exl3_esimd.h:64
RSQRT128 = np.float32(0.08838834764831845)   # exl3_esimd.h:223


# ------------------------------------------------------------------------------------------------
# geometry

def geo(K: int) -> dict:
    """Geo<K> (exl3_esimd.h:28-35): words per period D, values per period V, periods per tile G, words per tile."""
    g = int(np.gcd(K, 32))
    D, V = K // g, 32 // g
    return dict(g=g, D=D, V=V, G=256 // V, WORDS=8 * K)


def blob_layout(H: int, I: int, K: int) -> dict:
    """Byte offsets inside one expert blob (a8:42-54): gate|up trellis, down trellis, then six fp16 vectors."""
    W = 8 * K
    gu = (H // 16) * (2 * I // 16) * W * 4
    d = (I // 16) * (H // 16) * W * 4
    o = dict(gu=0, d=gu)
    off = gu + d
    for name, n in (("suh_g", H), ("suh_u", H), ("svh_g", I), ("svh_u", I), ("suh_d", I), ("svh_d", H)):
        o[name] = off
        off += 2 * n
    o["blob"] = off
    return o


def blob_bytes(H: int, I: int, K: int) -> int:
    return blob_layout(H, I, K)["blob"]


# ------------------------------------------------------------------------------------------------
# codebook (mul1)

def codebook_raw_h(states: np.ndarray) -> np.ndarray:
    """h = 1024 + bytesum(state * 0x83DCD12D mod 2^32), an exact integer in [1024, 2044] (exl3_esimd.h:52-62)."""
    x = (np.asarray(states, dtype=np.uint64) * np.uint64(MUL1)) & np.uint64(0xFFFFFFFF)
    bs = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + ((x >> 24) & 0xFF)
    return (1024 + bs).astype(np.int64)


def codebook_mul1(states: np.ndarray) -> np.ndarray:
    """16-bit trellis state -> fp16 weight: RNE_fp16(h * c1 + c2) with one rounding (exl3_esimd.h:64-67).
    h * c1 + c2 is exact in float64 (and in fp32), so the single rounding is the float64 -> float16 cast."""
    h = codebook_raw_h(states).astype(np.float64)
    return (h * C1 + C2).astype(np.float16)


# codebooks 3inst (id 0) and mcg (id 1): x = state * a + b mod 2^32 (exl3_esimd.h:72-73), then
# m = (x & 0x8FFF8FFF) ^ 0x3B603B60 and w = RNE_fp16(half(m & 0xFFFF) + half(m >> 16)) (exl3_esimd.h:74-78)
LCG = {0: (89226354, 64248484), 1: (0xCBAC1FED, 0)}
LCG_MASK, LCG_XOR = 0x8FFF8FFF, 0x3B603B60


def codebook_lcg(states: np.ndarray, cb: int) -> np.ndarray:
    """16-bit trellis state -> fp16 weight for codebook 0 (3inst) or 1 (mcg). numpy's float16 add converts both
    halves to float32, adds (exact: both are normal halves within a factor 16 of each other) and rounds once to
    float16 (RNE), which is the IEEE half addition."""
    a, b = LCG[cb]
    x = (np.asarray(states, dtype=np.uint64) * np.uint64(a) + np.uint64(b)) & np.uint64(0xFFFFFFFF)
    m = ((x & np.uint64(LCG_MASK)) ^ np.uint64(LCG_XOR)).astype(np.uint32)
    lo = (m & 0xFFFF).astype(np.uint16).view(np.float16)
    hi = (m >> 16).astype(np.uint16).view(np.float16)
    return lo + hi


_CB_TABLES: dict = {}


def codebook_table(cb: int = 2) -> np.ndarray:
    """All 65,536 values of codebook cb (2 = mul1, 1 = mcg, 0 = 3inst), fp16."""
    t = _CB_TABLES.get(cb)
    if t is None:
        st = np.arange(65536, dtype=np.uint32)
        t = _CB_TABLES[cb] = codebook_mul1(st) if cb == 2 else codebook_lcg(st, cb)
    return t


# ------------------------------------------------------------------------------------------------
# trellis tiles

def tile_pos(t):
    """Value t of a 16x16 tile lands at (row = input/k, col = output/n) (exl3_esimd.h:6-8)."""
    t = np.asarray(t)
    row = 8 * ((t >> 1) & 1) + 2 * ((t >> 3) & 3) + (t & 1)
    col = (t >> 5) + 8 * ((t >> 2) & 1)
    return row, col


def tile_states(words: np.ndarray, K: int) -> np.ndarray:
    """words uint32 [..., 8K] in natural (tile-major, MSB-first) order -> 16-bit states uint32 [..., 256].
    Value t is the 16-bit window ending at bit (t+1)*K of the tile's 256*K-bit stream, circular (tail-biting):
    exl3_esimd.h:120-149 (per-period form) restated over the whole tile."""
    w = np.asarray(words, dtype=np.uint64)
    nw = 8 * K
    assert w.shape[-1] == nw
    out = np.empty(w.shape[:-1] + (256,), dtype=np.uint32)
    for t in range(256):
        e = (t + 1) * K                      # end bit (exclusive)
        i1 = (e - 1) // 32                   # word holding the last bit
        s = (i1 + 1) * 32 - e                # right shift that aligns the window end
        B = w[..., i1]
        if e - 16 >= 32 * i1:                # window inside word i1
            st = B >> np.uint64(s)
        else:                                # window spans word i1-1 (circular) and word i1
            A = w[..., (i1 - 1) % nw]
            st = (((A << np.uint64(32)) | B) >> np.uint64(s))
        out[..., t] = (st & np.uint64(0xFFFF)).astype(np.uint32)
    return out


def decode_tiles(words: np.ndarray, K: int, cb: int = 2) -> np.ndarray:
    """words uint32 [..., 8K] -> fp16 tiles [..., 16, 16] (W_inner, row = k, col = n) of codebook cb.
    ReconstructKernel (exl3_esimd.h:869-936) restated: bit-exact dequantization."""
    st = tile_states(words, K)
    vals = codebook_table(cb)[st]
    row, col = tile_pos(np.arange(256))
    tiles = np.empty(st.shape[:-1] + (16, 16), dtype=np.float16)
    tiles[..., row, col] = vals
    return tiles


def tiles_to_matrix(tiles: np.ndarray) -> np.ndarray:
    """[R, C, 16, 16] -> [16R, 16C]."""
    R, C = tiles.shape[:2]
    return tiles.transpose(0, 2, 1, 3).reshape(R * 16, C * 16)


# ------------------------------------------------------------------------------------------------
# PLANAR4 word order and the blob

def planar4(words: np.ndarray, K: int) -> np.ndarray:
    """words uint32 [rows, tiles, 8K] (natural) -> PLANAR4 order, same shape semantics flattened per row:
    [row, group of 4 tiles, plane i, tile, period g] (moe_offload.py:68-73). For D = 1 (even K) the order is
    unchanged."""
    gm = geo(K)
    r, n, nw = words.shape
    if gm["D"] == 1:
        return words.copy()
    assert n % 4 == 0
    w = words.reshape(r, n // 4, 4, gm["G"], gm["D"])        # [row, group, tile, g, plane]
    return np.ascontiguousarray(w.transpose(0, 1, 4, 2, 3)).reshape(r, n, nw)


def unplanar4(words: np.ndarray, K: int) -> np.ndarray:
    gm = geo(K)
    r, n, nw = words.shape
    if gm["D"] == 1:
        return words.copy()
    w = words.reshape(r, n // 4, gm["D"], 4, gm["G"])        # [row, group, plane, tile, g]
    return np.ascontiguousarray(w.transpose(0, 1, 3, 4, 2)).reshape(r, n, nw)


def trellis_words(tr_i16: np.ndarray) -> np.ndarray:
    """Checkpoint trellis int16 [rows, tiles, 16K] -> uint32 words [rows, tiles, 8K] (little-endian int16 pairs,
    the `.view(torch.int32)` of moe_offload.py:71)."""
    a = np.ascontiguousarray(tr_i16).view(np.uint16).astype(np.uint32)
    return a[..., 0::2] | (a[..., 1::2] << 16)


def pack_expert(gate: dict, up: dict, down: dict, K: int) -> np.ndarray:
    """Checkpoint tensors {trellis int16, suh, svh} of one expert -> blob uint8 (moe_offload.py:76-89)."""
    gu = np.concatenate([gate["trellis"], up["trellis"]], axis=1)
    parts = [planar4(trellis_words(gu), K), planar4(trellis_words(down["trellis"]), K),
             gate["suh"], up["suh"], gate["svh"], up["svh"], down["suh"], down["svh"]]
    out = []
    for p in parts:
        if p.dtype != np.uint32:
            p = np.asarray(p).astype(np.float16)
        out.append(np.ascontiguousarray(p).view(np.uint8).reshape(-1))
    return np.concatenate(out)


def unpack_blob(blob: np.ndarray, H: int, I: int, K: int) -> dict:
    """blob uint8 -> natural-order words and fp16 vectors."""
    o = blob_layout(H, I, K)
    b = np.asarray(blob, dtype=np.uint8)
    assert b.size == o["blob"], (b.size, o["blob"])
    W = 8 * K
    gu = b[o["gu"]:o["d"]].view(np.uint32).reshape(H // 16, 2 * I // 16, W)
    d = b[o["d"]:o["suh_g"]].view(np.uint32).reshape(I // 16, H // 16, W)
    r = dict(gu=unplanar4(gu, K), d=unplanar4(d, K))
    for name, n in (("suh_g", H), ("suh_u", H), ("svh_g", I), ("svh_u", I), ("suh_d", I), ("svh_d", H)):
        r[name] = b[o[name]:o[name] + 2 * n].view(np.float16).copy()
    return r


def dequant_blob(blob: np.ndarray, H: int, I: int, K: int):
    """-> (W_gu fp16 [H, 2I] = [gate | up], W_d fp16 [I, H]), Hadamard-domain W_inner."""
    u = unpack_blob(blob, H, I, K)
    return tiles_to_matrix(decode_tiles(u["gu"], K)), tiles_to_matrix(decode_tiles(u["d"], K)), u


# ------------------------------------------------------------------------------------------------
# Hadamard

def fwht128(v: np.ndarray) -> np.ndarray:
    """Unnormalised Sylvester-order Walsh-Hadamard over the last axis (128), float32 butterflies h = 1..64 in the
    order of exl3_esimd.h:210-220 (a + b, a - b)."""
    v = np.asarray(v, dtype=np.float32)
    lead = v.shape[:-1]
    assert v.shape[-1] == 128
    x = v.reshape(-1, 128)
    h = 1
    while h < 128:
        m = x.reshape(x.shape[0], 128 // (2 * h), 2, h)
        a, b = m[:, :, 0, :], m[:, :, 1, :]
        x = np.stack([a + b, a - b], axis=2).reshape(x.shape[0], 128)
        h *= 2
    return x.reshape(lead + (128,))


def had_blocks(v: np.ndarray) -> np.ndarray:
    """fwht128 over consecutive 128-blocks of the last axis."""
    n = v.shape[-1]
    return fwht128(v.reshape(v.shape[:-1] + (n // 128, 128))).reshape(v.shape)


# ------------------------------------------------------------------------------------------------
# bf16 helpers (numpy has no bf16 dtype: bf16 travels as uint16 bit patterns)

def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """round-to-nearest-even float32 -> bf16 bits (finite inputs)."""
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


# ------------------------------------------------------------------------------------------------
# expert forward

class ExpertWeights:
    """Dequantized view of one blob (cached fp16 W_inner + vectors)."""

    def __init__(self, blob, H, I, K):
        self.W_gu, self.W_d, u = dequant_blob(blob, H, I, K)
        self.H, self.I = H, I
        for k in ("suh_g", "suh_u", "svh_g", "svh_u", "suh_d", "svh_d"):
            setattr(self, k, u[k])


def _input_had(xf: np.ndarray, suh: np.ndarray) -> np.ndarray:
    """fp16(H(fp16(x * suh)) / sqrt(128)) per 128-block (a8:188-191)."""
    v = (xf * suh.astype(np.float32)).astype(np.float16).astype(np.float32)
    return (had_blocks(v) * RSQRT128).astype(np.float16)


def expert_pair(xf: np.ndarray, ew: ExpertWeights, w: float, variant: str = "decode") -> np.ndarray:
    """One (token, expert) pair: x fp32 [H] (from bf16) -> y fp32 [H] scaled by routing weight w.
    Rounding points of GateUpKernel (a8:188-255) and DownKernel (a8:352-361) / the DPAS prefill epilogues
    (a8:520-541, 625-631), with fp32-exact accumulation of the GEMVs (float64 dot products rounded to fp32).
    variant "prefill" stores y in fp16 like DownDpasKernel<.., fp16> (a8:802, 630)."""
    I = ew.I
    xg = _input_had(xf, ew.suh_g).astype(np.float64)
    xu = _input_had(xf, ew.suh_u).astype(np.float64)
    g_raw = (xg @ ew.W_gu[:, :I].astype(np.float64)).astype(np.float32)
    u_raw = (xu @ ew.W_gu[:, I:].astype(np.float64)).astype(np.float32)
    g = (had_blocks(g_raw) * RSQRT128 * ew.svh_g.astype(np.float32)).astype(np.float16).astype(np.float32)
    u = (had_blocks(u_raw) * RSQRT128 * ew.svh_u.astype(np.float32)).astype(np.float16).astype(np.float32)
    with np.errstate(over="ignore"):
        act = g / (np.float32(1.0) + np.exp(-g)) * u
    act = act.astype(np.float32).astype(np.float16).astype(np.float32)
    act = (act * ew.suh_d.astype(np.float32)).astype(np.float16).astype(np.float32)
    abuf = (had_blocks(act) * RSQRT128).astype(np.float16)
    v_raw = (abuf.astype(np.float64) @ ew.W_d.astype(np.float64)).astype(np.float32)
    y = had_blocks(v_raw) * (RSQRT128 * np.float32(w)) * ew.svh_d.astype(np.float32)
    y = y.astype(np.float32)
    if variant == "prefill":
        y = y.astype(np.float16).astype(np.float32)
    return y


def moe_forward(x_bf16: np.ndarray, ids: np.ndarray, w: np.ndarray, experts, variant: str = "decode"):
    """Routed MoE: out[m] = bf16(sum_k y(m, ids[m, k], w[m, k])) summed in k order (CombineKernel a8:371-395).
    experts: callable or mapping e -> ExpertWeights. Returns (out bf16 bits [M, H], out fp32 [M, H])."""
    get = experts if callable(experts) else experts.__getitem__
    M = x_bf16.shape[0]
    H = x_bf16.shape[1]
    out = np.zeros((M, H), dtype=np.float32)
    for m in range(M):
        xf = bf16_to_f32(x_bf16[m])
        acc = np.zeros(H, dtype=np.float32)
        for k in range(ids.shape[1]):
            acc = (acc + expert_pair(xf, get(int(ids[m, k])), float(w[m, k]), variant)).astype(np.float32)
        out[m] = acc
    return f32_to_bf16(out), out


def dense_reference(xf: np.ndarray, ew: ExpertWeights, w: float) -> np.ndarray:
    """Independent float64 path (no intermediate roundings): W_eff = diag(suh) Hb W_inner Hb diag(svh) / 128,
    y = w * (silu(x W_g) * (x W_u)) W_d. Used to pin expert_pair within a tolerance."""
    from scipy.linalg import hadamard
    Hm = hadamard(128).astype(np.float64)

    def eff(W, suh, svh):
        k, n = W.shape
        A = W.astype(np.float64)
        A = np.einsum("ab,kbn->kan", Hm, A.reshape(k // 128, 128, n)).reshape(k, n)       # Hb on the left
        A = np.einsum("knb,bc->knc", A.reshape(k, n // 128, 128), Hm).reshape(k, n)       # Hb on the right
        return suh.astype(np.float64)[:, None] * A * svh.astype(np.float64)[None, :] / 128.0

    I = ew.I
    Wg = eff(ew.W_gu[:, :I], ew.suh_g, ew.svh_g)
    Wu = eff(ew.W_gu[:, I:], ew.suh_u, ew.svh_u)
    Wd = eff(ew.W_d, ew.suh_d, ew.svh_d)
    x = xf.astype(np.float64)
    g, u = x @ Wg, x @ Wu
    return w * ((g / (1.0 + np.exp(-g)) * u) @ Wd)


# ------------------------------------------------------------------------------------------------
# token alignment (prefill routing)

def align(ids: np.ndarray, w: np.ndarray, E: int, pad: int) -> dict:
    """launch_align (a8:639-680) in canonical order: pairs sorted by expert, ascending pair index inside an expert
    (the reference's SLM-atomic order inside an expert is arbitrary; results do not depend on it)."""
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    topk = ids.shape[1]
    npairs = flat.size
    cnt = np.bincount(flat, minlength=E)[:E]
    start = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    act = np.nonzero(cnt)[0]
    pc = (cnt + pad - 1) // pad * pad
    pstart = np.concatenate([[0], np.cumsum(pc)[:-1]])
    order = np.argsort(flat, kind="stable")
    pair_of = np.empty(npairs, dtype=np.int64)
    pair_of[order] = np.arange(npairs)
    blk_a = np.concatenate([np.full(pc[e] // pad, ai) for ai, e in enumerate(act)]) if len(act) else np.zeros(0)
    return dict(act_expert=act, act_start=start[act], act_cnt=cnt[act], act_pstart=pstart[act], n_act=len(act),
                pair_tok=order // topk, pair_w=np.asarray(w, np.float32).reshape(-1)[order], pair_of=pair_of,
                blk_a=blk_a.astype(np.int64), n_blk=int(pc.sum() // pad))
