"""GPU parity of the decode path: bit-exact dequantization and the routed-expert MoE forward against the oracle:
rel-L2 <= 2e-3 (the bound the north star sets for MoE outputs) between the GPU output and the oracle's
fp32-accumulated result rounded to the output dtype (bf16 rounding alone is ~1.1e-3 rel-L2, so both sides are
compared after the same final rounding)."""
import os

import numpy as np
import pytest
import torch

from oracle import exl3, synth

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
TOL = 2e-3


def _ops():
    from exl3xpu.moe_offload import ops
    return ops()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def _bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


def _bf16_to_f32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


@pytest.mark.parametrize("K", [2, 3, 4])
def test_dequant_bitexact_capi(K):
    """exl3_dequant through the C-ABI == oracle ReconstructKernel restatement, bit for bit."""
    from exl3xpu import capi
    print(f"case dequant K={K}", flush=True)
    rng = np.random.default_rng(K)
    kt, nt = 8, 24
    nat = rng.integers(0, 1 << 32, size=(kt, nt, 8 * K), dtype=np.uint64).astype(np.uint32)
    ref = exl3.tiles_to_matrix(exl3.decode_tiles(nat, K)).view(np.uint16)
    d = torch.from_numpy(exl3.planar4(nat, K).view(np.int32)).cuda()
    out = torch.empty((16 * kt, 16 * nt), dtype=torch.int16, device="cuda")
    L = capi.lib()
    capi.check(L.exl3_dequant(d.data_ptr(), kt, nt, K, out.data_ptr(), capi.stream_handle()), "dequant")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref)


def test_dequant_exhaustive_states():
    """Nearly every 16-bit state through the GPU decoder: 4,096 random K=2 tiles (1M values) cover > 60,000 of the
    65,536 states; every decoded value must equal the oracle's."""
    K = 2
    rng = np.random.default_rng(77)
    nat = rng.integers(0, 1 << 32, size=(64, 64, 16), dtype=np.uint64).astype(np.uint32)
    st = exl3.tile_states(nat, K)
    ref = exl3.tiles_to_matrix(exl3.decode_tiles(nat, K)).view(np.uint16)
    got = _ops().dequant(torch.from_numpy(nat.view(np.int32)).cuda(), 64, 64, K)
    torch.cuda.synchronize()
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), ref)
    assert len(np.unique(st)) > 60000          # the sample covers nearly every state


def test_moe_forward_golden():
    g = np.load(os.path.join(GOLD, "moe_small.npz"))
    H, I, K = int(g["H"]), int(g["I"]), int(g["K"])
    print(f"case golden H={H} I={I} K={K}", flush=True)
    blobs = torch.from_numpy(g["blobs"]).cuda()
    E = blobs.shape[0]
    ptrs = torch.tensor([blobs[e].data_ptr() for e in range(E)], dtype=torch.int64, device="cuda")
    x = _bf16_tensor(g["x"]).cuda()
    ids = torch.from_numpy(g["ids"]).cuda()
    w = torch.from_numpy(g["w"]).cuda()
    out = _ops().moe_forward(x, ids, w, ptrs, I, K, E)
    torch.cuda.synchronize()
    o = _bf16_to_f32(out)
    assert rel_l2(o, exl3.bf16_to_f32(g["out_bf16"])) <= TOL
    assert rel_l2(o, g["out_f32"]) <= 3e-3
    # fp32 activations in and out: the kernel's own arithmetic against the oracle's fp32 result
    xf = torch.from_numpy(exl3.bf16_to_f32(g["x"])).cuda()
    of = _ops().moe_forward(xf, ids, w, ptrs, I, K, E)
    torch.cuda.synchronize()
    r32 = rel_l2(of.cpu().numpy(), g["out_f32"])
    print(f"golden rel-L2 bf16 {rel_l2(o, exl3.bf16_to_f32(g['out_bf16'])):.2e} fp32 {r32:.2e}")
    assert r32 <= TOL


def _moe_case(H, I, K, E, M, topk, seed, host=False):
    ids, w = synth.softmax_topk(seed, M, E, topk)
    used = sorted(set(ids.reshape(-1).tolist()))
    blobs = {e: synth.expert_blob(seed, e, H, I, K) for e in used}
    nb = exl3.blob_bytes(H, I, K)
    if host:
        from exl3xpu.moe_offload import ops
        arena = ops().host_alloc(len(used) * nb)
        for i, e in enumerate(used):
            arena[i * nb:(i + 1) * nb].copy_(torch.from_numpy(blobs[e]))
        addr = {e: arena.data_ptr() + i * nb for i, e in enumerate(used)}
        keep = arena
    else:
        dev = torch.from_numpy(np.stack([blobs[e] for e in used])).cuda()
        addr = {e: dev[i].data_ptr() for i, e in enumerate(used)}
        keep = dev
    table = np.zeros(E, dtype=np.int64)
    for e in used:
        table[e] = addr[e]
    x = synth.activations(seed, M, H)
    ews = {e: exl3.ExpertWeights(blobs[e], H, I, K) for e in used}
    ob, of = exl3.moe_forward(x, ids, w, ews)
    return x, ids, w, torch.from_numpy(table).cuda(), exl3.bf16_to_f32(ob), keep, of


@pytest.mark.parametrize("M", [1, 2, 4])
def test_moe_forward_c0_shapes(M):
    """One MoE layer at the config-0 shapes (H 2048, I 512, 512 experts, top-10, K=3), bs 1/2/4."""
    H, I, K, E, topk = 2048, 512, 3, 512, 10
    print(f"case c0 M={M}", flush=True)
    x, ids, w, table, ref, keep, ref32 = _moe_case(H, I, K, E, M, topk, 20261201 + M)
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    out = _ops().moe_forward(_bf16_tensor(x).cuda(), it, wt, table, I, K, E)
    of = _ops().moe_forward(torch.from_numpy(exl3.bf16_to_f32(x)).cuda(), it, wt, table, I, K, E)
    torch.cuda.synchronize()
    rb, rf = rel_l2(_bf16_to_f32(out), ref), rel_l2(of.cpu().numpy(), ref32)
    print(f"c0 M={M}: rel-L2 bf16 {rb:.2e} fp32 {rf:.2e}")
    assert rb <= TOL and rf <= TOL


def test_moe_forward_host_resident_experts():
    """Experts read zero-copy from pinned host memory give the same output bits as HBM-resident ones."""
    H, I, K, E, topk, M = 2048, 512, 3, 512, 10, 1
    x, ids, w, t_dev, ref, k1, _ = _moe_case(H, I, K, E, M, topk, 31)
    _, _, _, t_host, _, k2, _ = _moe_case(H, I, K, E, M, topk, 31, host=True)
    xs, it, wt = _bf16_tensor(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    o1 = _ops().moe_forward(xs, it, wt, t_dev, I, K, E)
    o2 = _ops().moe_forward(xs, it, wt, t_host, I, K, E)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert rel_l2(_bf16_to_f32(o1), ref) <= TOL


@pytest.mark.parametrize("K", [2, 3, 4])
def test_moe_forward_large_expert_shapes(K):
    """Larger-expert geometry (H 4096, I 1536, 128 experts) at each bitrate; top-2 keeps the oracle fast."""
    H, I, E, topk, M = 4096, 1536, 128, 2, 1
    print(f"case c4 K={K}", flush=True)
    x, ids, w, table, ref, keep, ref32 = _moe_case(H, I, K, E, M, topk, 4000 + K)
    it, wt = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    out = _ops().moe_forward(_bf16_tensor(x).cuda(), it, wt, table, I, K, E)
    of = _ops().moe_forward(torch.from_numpy(exl3.bf16_to_f32(x)).cuda(), it, wt, table, I, K, E)
    torch.cuda.synchronize()
    rb, rf = rel_l2(_bf16_to_f32(out), ref), rel_l2(of.cpu().numpy(), ref32)
    print(f"c4 K={K}: rel-L2 bf16 {rb:.2e} fp32 {rf:.2e}")
    assert rb <= TOL and rf <= TOL


def test_moe_forward_fp16_activations():
    H, I, K, E, topk, M = 2048, 512, 3, 512, 10, 2
    x, ids, w, table, ref, keep, ref32 = _moe_case(H, I, K, E, M, topk, 55)
    xf = torch.from_numpy(exl3.bf16_to_f32(x)).half().cuda()
    out = _ops().moe_forward(xf, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), table, I, K, E)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    assert rel_l2(out.float().cpu().numpy(), ref) <= 3e-3     # ref is bf16-rounded, the output fp16


def test_moe_forward_repeatable():
    """Fixed-order reductions: two runs give identical bits."""
    H, I, K, E, topk, M = 2048, 512, 3, 512, 10, 4
    x, ids, w, table, ref, keep, ref32 = _moe_case(H, I, K, E, M, topk, 66)
    args = (_bf16_tensor(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), table, I, K, E)
    o1 = _ops().moe_forward(*args)
    o2 = _ops().moe_forward(*args)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
