"""PyTorch CPU restatement of the routed-expert decode path: the CPU baseline timed by bench.py.

TEST INFRASTRUCTURE / BASELINE ONLY (see oracle/__init__.py). The reference has no CPU implementation of this path
(every store and tier call runs XPU ops, plugin/exl3xpu/moe_offload.py:44-61, 235-249), so the baseline is this
restatement of its math (kernels/moe-a8/exl3_moe.a8.sycl:121-395): dequantization through a 65,536-entry fp16
codebook table with vectorised bit-window extraction from the PLANAR4 words, then fp32 matmuls with the reference's
fp16 rounding points (input Hadamard, gate/up outputs, SiLU product, down input).
"""
from __future__ import annotations

import numpy as np
import torch

from . import exl3


class CpuExperts:
    """Blobs of one layer (uint8 [n, BLOB]) -> dequantize on demand with torch ops."""

    def __init__(self, H, I, K):
        self.H, self.I, self.K = H, I, K
        self.o = exl3.blob_layout(H, I, K)
        self.cb = torch.from_numpy(exl3.codebook_table().astype(np.float32))
        t = np.arange(256)
        self.row, self.col = (torch.from_numpy(a.astype(np.int64)) for a in exl3.tile_pos(t))
        e = (t + 1) * K
        i1 = (e - 1) // 32
        self.i1 = torch.from_numpy(i1.astype(np.int64))
        self.i0 = torch.from_numpy(((i1 - 1) % (8 * K)).astype(np.int64))
        self.s = torch.from_numpy(((i1 + 1) * 32 - e).astype(np.int64))
        gm = exl3.geo(K)
        self.D, self.G = gm["D"], gm["G"]
        self.Hm = torch.from_numpy(self._had())

    @staticmethod
    def _had():
        h = np.array([[1.0]], dtype=np.float32)
        while h.shape[0] < 128:
            h = np.block([[h, h], [h, -h]])
        return h

    def _decode(self, words_planar: torch.Tensor, kt: int, nt: int, planar: bool = True) -> torch.Tensor:
        K, D, G = self.K, self.D, self.G
        w = words_planar.view(kt, nt, 8 * K).to(torch.int64) & 0xFFFFFFFF
        if planar and D > 1:      # PLANAR4 -> natural: [row, group, plane, tile, g] -> [row, tile, g, plane]
            w = w.view(kt, nt // 4, D, 4, G).permute(0, 1, 3, 4, 2).reshape(kt, nt, 8 * K)
        B = w[..., self.i1]
        A = w[..., self.i0]
        st = (((A << 32) | B) >> self.s) & 0xFFFF
        vals = self.cb[st]                                                      # [kt, nt, 256]
        tiles = torch.empty(kt, nt, 16, 16)
        tiles[:, :, self.row, self.col] = vals
        return tiles.permute(0, 2, 1, 3).reshape(kt * 16, nt * 16)

    def weights(self, blob: torch.Tensor):
        H, I, o = self.H, self.I, self.o
        gu = blob[o["gu"]:o["d"]].view(torch.int32)
        d = blob[o["d"]:o["suh_g"]].view(torch.int32)
        W_gu = self._decode(gu, H // 16, 2 * I // 16)
        W_d = self._decode(d, I // 16, H // 16)
        vec = {k: blob[o[k]:o[k] + 2 * n].view(torch.float16).float()
               for k, n in (("suh_g", H), ("suh_u", H), ("svh_g", I), ("svh_u", I), ("suh_d", I), ("svh_d", H))}
        return W_gu, W_d, vec

    def had(self, v: torch.Tensor) -> torch.Tensor:
        n = v.shape[-1]
        return (v.reshape(-1, n // 128, 128) @ self.Hm).reshape(v.shape)

    def pair(self, x: torch.Tensor, blob: torch.Tensor, w: float) -> torch.Tensor:
        I = self.I
        W_gu, W_d, v = self.weights(blob)
        r = float(exl3.RSQRT128)
        xg = (self.had((x * v["suh_g"]).half().float()) * r).half().float()
        xu = (self.had((x * v["suh_u"]).half().float()) * r).half().float()
        g = (self.had(xg @ W_gu[:, :I]) * r * v["svh_g"]).half().float()
        u = (self.had(xu @ W_gu[:, I:]) * r * v["svh_u"]).half().float()
        a = (torch.nn.functional.silu(g) * u).half().float()
        a = (a * v["suh_d"]).half().float()
        a = (self.had(a) * r).half().float()
        return self.had(a @ W_d) * (r * w) * v["svh_d"]

    def layer(self, x: torch.Tensor, ids, w, blobs) -> torch.Tensor:
        """x fp32 [M, H]; ids/w [M, topk]; blobs: mapping expert -> uint8 torch blob."""
        out = torch.zeros_like(x)
        for m in range(x.shape[0]):
            for k in range(len(ids[m])):
                out[m] += self.pair(x[m], blobs[int(ids[m][k])], float(w[m][k]))
        return out.to(torch.bfloat16)


class CpuLinear(CpuExperts):
    """The dense EXL3 linear (experimental/n111-victim-ring/csrc/exl3_ops.sycl:651-757) on the CPU: the checkpoint
    trellis (natural word order) decoded through the codebook table on every call, then the input Hadamards per shard,
    fp32 matmuls of each shard's columns, and the output Hadamard x svh."""

    def __init__(self, K, cb: int = 2):
        super().__init__(128, 128, K)
        self.cb = torch.from_numpy(exl3.codebook_table(cb).astype(np.float32))

    def __call__(self, x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, bounds):
        """x fp32 [M, k]; trellis int16 [k/16, n/16, 16K]; suh fp16 [S, k]; svh fp16 [n]; bounds [0, ..., n]."""
        kt, nt = trellis.shape[:2]
        W = self._decode(trellis.contiguous().view(torch.int32), kt, nt, planar=False)
        r = float(exl3.RSQRT128)
        y = torch.empty(x.shape[0], nt * 16)
        for g in range(len(bounds) - 1):
            xh = (self.had((x * suh[g].float()).half().float()) * r).half().float()
            y[:, bounds[g]:bounds[g + 1]] = xh @ W[:, bounds[g]:bounds[g + 1]]
        return self.had(y) * r * svh.float()
