"""Seeded synthetic inputs for every workload (weights, activations, routing, decode traces).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference has no quantizer (EXL3 quantization lives in exllamav3, which is absent), and any bitstream is a valid
EXL3 trellis encoding, so synthetic experts are uniform random trellis words with +-1 suh and +-0.02 svh sign/scale
vectors. The product package carries its own copy of the blob generator (exl3xpu.synth) so that GPU runs do not
depend on this directory; tests check that both produce the same bytes.

Seeds: workload index c uses 20261201 + c; per-tensor streams come from numpy SeedSequence.spawn.
"""
from __future__ import annotations

import numpy as np

from . import exl3

SEED0 = 20261201


def rng_for(*key) -> np.random.Generator:
    """Generator keyed by a tuple of non-negative ints (SeedSequence entropy)."""
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([int(k) for k in key])))


def expert_checkpoint(rng: np.random.Generator, H: int, I: int, K: int) -> tuple:
    """Checkpoint-form tensors of one expert: trellis int16 [k/16, n/16, 16K], suh fp16 [k] (+-1), svh fp16 [n]
    (+-0.02) for gate (k=H, n=I), up (k=H, n=I), down (k=I, n=H)."""
    def proj(k, n):
        tr = rng.integers(0, 1 << 16, size=(k // 16, n // 16, 16 * K), dtype=np.uint16).view(np.int16)
        suh = np.where(rng.integers(0, 2, size=k) == 1, 1.0, -1.0).astype(np.float16)
        svh = (np.where(rng.integers(0, 2, size=n) == 1, 1.0, -1.0) * 0.02).astype(np.float16)
        return dict(trellis=tr, suh=suh, svh=svh)
    return proj(H, I), proj(H, I), proj(I, H)


def expert_blob(seed: int, index: int, H: int, I: int, K: int) -> np.ndarray:
    """Blob of synthetic expert `index` of a workload seeded by `seed` (packed by the oracle's pack_expert)."""
    g, u, d = expert_checkpoint(rng_for(seed, 1, index), H, I, K)
    return exl3.pack_expert(g, u, d, K)


def activations(seed: int, M: int, H: int) -> np.ndarray:
    """x ~ N(0, 1) as bf16 bits [M, H]."""
    return exl3.f32_to_bf16(rng_for(seed, 2).standard_normal((M, H)).astype(np.float32))


def softmax_topk(seed: int, M: int, E: int, topk: int, stream: int = 3):
    """Router: logits N(0,1) [M, E] -> softmax -> top-k -> renormalised weights (norm_topk_prob)."""
    logits = rng_for(seed, stream).standard_normal((M, E))
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    w = np.take_along_axis(p, ids, axis=1)
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids.astype(np.int32), w


def zipf_trace(seed: int, steps: int, L: int, E: int, topk: int, M: int = 1, s: float = 1.1, step0: int = 0):
    """Decode routing trace: ids int32 [steps, L, M, topk], w fp32 [steps, L, M, topk].
    Per layer a seeded permutation pi_l of the E experts; each (step, layer, row) draws `topk` distinct ranks with
    P(rank r) ~ r^-s (Gumbel-top-k, i.e. sampling without replacement) mapped through pi_l; weights are the
    renormalised softmax of N(0,1) logits over the picks. Step n of a trace depends only on (seed, n), so a trace
    can be generated in pieces (step0)."""
    perm = np.stack([rng_for(seed, 4, l).permutation(E) for l in range(L)])            # [L, E]
    logp = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    ids = np.empty((steps, L, M, topk), dtype=np.int32)
    w = np.empty((steps, L, M, topk), dtype=np.float32)
    for i in range(steps):
        r = rng_for(seed, 5, step0 + i)
        g = logp + r.gumbel(size=(L, M, E))
        ranks = np.argpartition(-g, topk, axis=-1)[..., :topk]
        # order the picks by key (descending) for a stable, documented pick order
        kk = np.take_along_axis(g, ranks, axis=-1)
        ranks = np.take_along_axis(ranks, np.argsort(-kk, axis=-1, kind="stable"), axis=-1)
        ids[i] = perm[np.arange(L)[:, None, None], ranks]
        lg = r.standard_normal((L, M, topk))
        pw = np.exp(lg - lg.max(axis=-1, keepdims=True))
        w[i] = (pw / pw.sum(axis=-1, keepdims=True)).astype(np.float32)
    return ids, w


def uniform_trace(seed: int, steps: int, L: int, E: int, topk: int, M: int = 1):
    """Worst-case routing for the cache: uniform-random distinct top-k per (step, layer, row)."""
    ids = np.empty((steps, L, M, topk), dtype=np.int32)
    w = np.empty((steps, L, M, topk), dtype=np.float32)
    for i in range(steps):
        r = rng_for(seed, 6, i)
        ids[i] = np.argsort(r.random((L, M, E)), axis=-1)[..., :topk]
        lg = r.standard_normal((L, M, topk))
        pw = np.exp(lg - lg.max(axis=-1, keepdims=True))
        w[i] = (pw / pw.sum(axis=-1, keepdims=True)).astype(np.float32)
    return ids, w
