"""Seeded synthetic EXL3 experts (uniform random trellis words, +-1 suh, +-0.02 svh) and routing traces.

Any bitstream is a valid EXL3 trellis encoding, so random words are valid weights; the checkpoint-form tensors are
packed with `moe_offload.pack_expert`. Generator streams are keyed by numpy SeedSequence([...]) so a blob or a trace
step can be regenerated independently. The oracle carries its own copy of these generators (oracle/synth.py); tests
check that both give the same bytes.
"""
from __future__ import annotations

import numpy as np
import torch

from .moe_offload import pack_expert


def rng_for(*key) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([int(k) for k in key])))


def expert_checkpoint(rng: np.random.Generator, H: int, I: int, K: int):
    def proj(k, n):
        tr = rng.integers(0, 1 << 16, size=(k // 16, n // 16, 16 * K), dtype=np.uint16).view(np.int16)
        suh = np.where(rng.integers(0, 2, size=k) == 1, 1.0, -1.0).astype(np.float16)
        svh = (np.where(rng.integers(0, 2, size=n) == 1, 1.0, -1.0) * 0.02).astype(np.float16)
        return dict(trellis=torch.from_numpy(tr), suh=torch.from_numpy(suh), svh=torch.from_numpy(svh))
    return proj(H, I), proj(H, I), proj(I, H)


def expert_blob(seed: int, index: int, H: int, I: int, K: int) -> torch.Tensor:
    """uint8 CPU blob of synthetic expert `index` of a workload seeded by `seed`."""
    g, u, d = expert_checkpoint(rng_for(seed, 1, index), H, I, K)
    return pack_expert(g, u, d, K)


def zipf_trace(seed: int, steps: int, L: int, E: int, topk: int, M: int = 1, s: float = 1.1, step0: int = 0):
    """ids int32 / w fp32 [steps, L, M, topk]: per-layer seeded permutation, `topk` distinct Zipf(s) ranks per
    (step, layer, row) by Gumbel-top-k, renormalised softmax weights of N(0,1) logits."""
    perm = np.stack([rng_for(seed, 4, l).permutation(E) for l in range(L)])
    logp = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    ids = np.empty((steps, L, M, topk), dtype=np.int32)
    w = np.empty((steps, L, M, topk), dtype=np.float32)
    for i in range(steps):
        r = rng_for(seed, 5, step0 + i)
        g = logp + r.gumbel(size=(L, M, E))
        ranks = np.argpartition(-g, topk, axis=-1)[..., :topk]
        kk = np.take_along_axis(g, ranks, axis=-1)
        ranks = np.take_along_axis(ranks, np.argsort(-kk, axis=-1, kind="stable"), axis=-1)
        ids[i] = perm[np.arange(L)[:, None, None], ranks]
        lg = r.standard_normal((L, M, topk))
        pw = np.exp(lg - lg.max(axis=-1, keepdims=True))
        w[i] = (pw / pw.sum(axis=-1, keepdims=True)).astype(np.float32)
    return ids, w


def uniform_trace(seed: int, steps: int, L: int, E: int, topk: int, M: int = 1):
    ids = np.empty((steps, L, M, topk), dtype=np.int32)
    w = np.empty((steps, L, M, topk), dtype=np.float32)
    for i in range(steps):
        r = rng_for(seed, 6, i)
        ids[i] = np.argsort(r.random((L, M, E)), axis=-1)[..., :topk]
        lg = r.standard_normal((L, M, topk))
        pw = np.exp(lg - lg.max(axis=-1, keepdims=True))
        w[i] = (pw / pw.sum(axis=-1, keepdims=True)).astype(np.float32)
    return ids, w
