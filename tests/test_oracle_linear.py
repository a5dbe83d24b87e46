"""Pins oracle/linear.py: the dense EXL3 linear against a float64 reconstruction of the same matrix built by an
independent path (scipy's Hadamard matrix instead of the butterflies, the effective weight diag(suh_g) Hb W Hb
diag(svh) / 128 per shard); the only difference is the fp16 rounding of x * suh and xh inside the restatement."""
import numpy as np
import pytest
from scipy.linalg import hadamard

from oracle import exl3, linear, synth


def _dense(xf, ck):
    W = linear.weight(ck["trellis"], ck["K"], ck["cb"]).astype(np.float64)
    k, n = W.shape
    Hb = np.kron(np.eye(k // 128), hadamard(128)).astype(np.float64)
    Hn = np.kron(np.eye(n // 128), hadamard(128)).astype(np.float64)
    core = Hb @ W @ Hn / 128.0                                    # Hb W Hb / 128 (blocks of the output side: n)
    out = np.empty((xf.shape[0], n))
    for g in range(ck["suh"].shape[0]):
        cols = np.nonzero(np.repeat(ck["shard_of_nb"] == g, 128))[0]
        out[:, cols] = (xf.astype(np.float64) * ck["suh"][g].astype(np.float64)) @ core[:, cols]
    return out * ck["svh"].astype(np.float64)


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


@pytest.mark.parametrize("K,cb", [(2, 2), (3, 2), (4, 2), (5, 2), (6, 2), (4, 0), (4, 1), (6, 0), (6, 1)])
def test_linear_vs_dense_float64(K, cb):
    ck = linear.checkpoint(30 + K, 256, [128, 256, 128], K, cb)    # three shards (q, k, v style)
    xf = exl3.bf16_to_f32(synth.activations(40 + K, 3, 256))
    ref = _dense(xf, ck)
    for variant, tol in (("small", 2e-3), ("large", 3e-3)):
        r = _rel(linear.linear(xf, ck, variant), ref)
        assert r < tol, (variant, r)


def test_linear_shards_use_their_own_suh():
    """Swapping the shards' suh rows changes exactly the columns of those shards (the shard map is honoured)."""
    ck = linear.checkpoint(5, 128, [128, 128], 3)
    xf = exl3.bf16_to_f32(synth.activations(6, 2, 128))
    a = linear.linear(xf, ck)
    ck2 = dict(ck, suh=ck["suh"][::-1].copy())
    b = linear.linear(xf, ck2)
    assert not np.allclose(a[:, :128], b[:, :128]) and not np.allclose(a[:, 128:], b[:, 128:])
    ck3 = dict(ck2, shard_of_nb=ck["shard_of_nb"][::-1].copy())
    assert np.array_equal(linear.linear(xf, ck3), a)


def test_weight_natural_order_matches_tile_decode():
    """W_inner: tile (r, c) of the matrix is the decode of trellis tile [r, c] (no PLANAR4 reordering)."""
    ck = linear.checkpoint(9, 128, [256], 3)
    W = linear.weight(ck["trellis"], 3)
    words = exl3.trellis_words(ck["trellis"])
    for r, c in ((0, 0), (3, 7), (7, 15)):
        t = exl3.decode_tiles(words[r, c], 3)
        assert np.array_equal(W[16 * r:16 * r + 16, 16 * c:16 * c + 16], t)


@pytest.mark.parametrize("K", [4, 6])
def test_linear_q8_vs_dense_float64(K):
    """The W8A8 route against the float64 reconstruction: within the int8 quantization error (a wrong or missing
    scale is off by orders of magnitude), and its integer GEMM equals float64 products of the int8 operands."""
    ck = linear.checkpoint(60 + K, 512, [256, 128, 128], K)
    xf = exl3.bf16_to_f32(synth.activations(70 + K, 24, 512))
    ref = _dense(xf, ck)
    r8 = _rel(linear.linear_q8(xf, ck), ref)
    r16 = _rel(linear.linear(xf, ck, "large"), ref)
    assert r8 < 2e-2 and r16 < 3e-3, (r8, r16)
    xq, sx = linear.q8_act(xf, ck["suh"])
    wq = linear.q8_weight(ck["trellis"], K)
    y = xq[1].astype(np.int64) @ wq[:, 256:384].astype(np.int64)
    assert np.array_equal(y, np.rint(xq[1].astype(np.float64) @ wq[:, 256:384].astype(np.float64)).astype(np.int64))


def test_q8_scale_invariants():
    """Each row's largest |xq| is 127 and |xh - xq sc| <= sc / 2 (round to nearest); an all-zero row gets scale 1 and
    zeros; the codebook's largest magnitude (its minimum, -3.453125 at h = 1024) maps to -127 and every weight stays
    within [-127, 127]."""
    ck = linear.checkpoint(80, 256, [128, 128], 4)
    xf = exl3.bf16_to_f32(synth.activations(81, 20, 256))
    xf[3] = 0.0
    xq, sx = linear.q8_act(xf, ck["suh"])
    xh = linear.had_in(xf, ck["suh"]).astype(np.float64)
    live = np.ones(20, bool)
    live[3] = False
    assert (np.abs(xq[:, live].astype(np.int64)).max(axis=2) == 127).all()
    assert (sx[:, 3] == 1.0).all() and not xq[:, 3].any()
    err = np.abs(xh - xq.astype(np.float64) * sx[:, :, None].astype(np.float64))
    assert (err <= sx[:, :, None].astype(np.float64) * (0.5 + 1e-6)).all()
    cbv = exl3.codebook_table(2).astype(np.float32)
    q = np.rint(cbv * linear.Q8_WINV)
    assert cbv.min() == -3.453125 and np.abs(cbv).max() == 3.453125 and q.min() == -127 and q.max() <= 127
    wq = linear.q8_weight(ck["trellis"], 4)
    assert np.abs(wq.astype(np.int64)).max() <= 127
