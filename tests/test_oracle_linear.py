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
