"""Writes the small golden fixtures under tests/golden/ from the oracle.

The reference commits no golden vectors for this path (its exactness test compares two of its own kernels on data
that is not in the repository), so these fixtures are the oracle's outputs, pinned by tests/test_oracle_*.py.
Run: python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import cache, exl3, synth  # noqa: E402


def main():
    tab = exl3.codebook_table()
    probes = [0, 1, 2, 255, 256, 4095, 12345, 32768, 54321, 65535]
    json.dump(dict(sha256=hashlib.sha256(tab.tobytes()).hexdigest(), probe_states=probes,
                   probe_bits=[int(v) for v in tab.view(np.uint16)[probes]]),
              open(os.path.join(HERE, "codebook.json"), "w"), indent=1)
    # one small MoE layer: H=256, I=128, K=3, 6 experts, M=2 rows, top-3
    H, I, K, E, M, topk = 256, 128, 3, 6, 2, 3
    blobs = np.stack([synth.expert_blob(11, e, H, I, K) for e in range(E)])
    x = synth.activations(11, M, H)
    ids, w = synth.softmax_topk(11, M, E, topk)
    ews = {e: exl3.ExpertWeights(blobs[e], H, I, K) for e in range(E)}
    out, outf = exl3.moe_forward(x, ids, w, ews)
    outp, outpf = exl3.moe_forward(x, ids, w, ews, "prefill")
    W_gu, W_d, _ = exl3.dequant_blob(blobs[0], H, I, K)
    np.savez_compressed(os.path.join(HERE, "moe_small.npz"), H=H, I=I, K=K, blobs=blobs, x=x, ids=ids, w=w,
                        out_bf16=out, out_f32=outf, out_prefill_f32=outpf, W_gu0=W_gu.view(np.uint16),
                        W_d0=W_d.view(np.uint16))
    # device cache + host tier on a tiny config
    L, E2, S, P, steps = 4, 16, 12, 4, 200
    tid, tw = synth.zipf_trace(12, steps, L, E2, P)
    co = cache.CacheOracle(L, E2, S, ring_cap=64, budget=14, age=4, qmax=6, latency=3)
    recs, log = co.run(tid[:, :, 0], tw[:, :, 0])
    flat = np.concatenate([np.concatenate([[len(a), len(e)], a, e]) for a, e in log]).astype(np.int32)
    np.savez_compressed(os.path.join(HERE, "cache_small.npz"), L=L, E=E2, S=S, P=P, ring_cap=64, budget=14, age=4,
                        qmax=6, latency=3, ids=tid[:, :, 0], w=tw[:, :, 0], recs=recs, host_log=flat)
    print("written")


def c4_top8():
    """Config-4 expert shape (H 4096, I 1536, 128 experts) at top-8, bs=1, for K = 2, 3, 4: the oracle's outputs for
    seeded inputs that the GPU test regenerates (blobs and activations from synth with seed 5000 + K). The oracle
    needs about 5 s per expert at this shape, too slow to run inside a GPU test."""
    H, I, E, topk = 4096, 1536, 128, 8
    out = {}
    for K in (2, 3, 4):
        seed = 5000 + K
        ids, w = synth.softmax_topk(seed, 1, E, topk)
        x = synth.activations(seed, 1, H)
        ews = {int(e): exl3.ExpertWeights(synth.expert_blob(seed, int(e), H, I, K), H, I, K) for e in ids[0]}
        ob, of = exl3.moe_forward(x, ids, w, ews)
        out.update({f"ids_{K}": ids, f"w_{K}": w, f"x_{K}": x, f"out_bf16_{K}": ob, f"out_f32_{K}": of})
        print(f"c4 top-8 K={K} done", flush=True)
    np.savez_compressed(os.path.join(HERE, "c4_top8.npz"), H=H, I=I, E=E, topk=topk, **out)


if __name__ == "__main__":
    if "c4" in sys.argv[1:]:
        c4_top8()
    else:
        main()
