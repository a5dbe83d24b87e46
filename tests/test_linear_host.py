"""Host side of the dense EXL3 linear without a GPU: the fused-group packing (plugin/sglang_plugin.tier.py:345-372),
the sign unpacking (115-117), the op's shape function on meta tensors and the K / codebook support query."""
import numpy as np
import pytest
import torch

from oracle import linear as olin


def _shards(ck):
    tr = torch.from_numpy(ck["trellis"])
    b = ck["bounds"]
    return [(tr[:, b[g] // 16:b[g + 1] // 16].contiguous(), torch.from_numpy(ck["suh"][g]),
             torch.from_numpy(ck["svh"][b[g]:b[g + 1]])) for g in range(len(b) - 1)]


def test_fused_group_packs_like_the_oracle_checkpoint():
    from exl3xpu.linear import FusedGroup
    ck = olin.checkpoint(3, 256, [256, 128, 384], 4)
    g = FusedGroup(_shards(ck), "cpu")
    assert (g.k, g.n, g.K, g.cb, g.bounds) == (256, 768, 4, 2, [0, 256, 384, 768])
    assert np.array_equal(g.trellis.numpy(), ck["trellis"])
    assert np.array_equal(g.suh.numpy(), ck["suh"]) and np.array_equal(g.svh.numpy(), ck["svh"])
    assert g.shard_of_nb.tolist() == [0, 0, 1, 2, 2, 2]


def test_fused_group_codebook_id():
    from exl3xpu.linear import FusedGroup
    sh = _shards(olin.checkpoint(6, 256, [128], 4))
    assert FusedGroup(sh, "cpu", cb=1).cb == 1 and FusedGroup(sh, "cpu", cb=0).cb == 0
    with pytest.raises(ValueError):
        FusedGroup(sh, "cpu", cb=3)


def test_fused_group_rejects_mixed_or_unaligned_shards():
    from exl3xpu.linear import FusedGroup
    a = _shards(olin.checkpoint(4, 256, [128], 3))[0]
    b = _shards(olin.checkpoint(5, 256, [128], 4))[0]
    with pytest.raises(ValueError, match="bitrates"):
        FusedGroup([a, b], "cpu")
    t = torch.zeros((16, 5, 48), dtype=torch.int16)               # n = 80: not a multiple of 128
    with pytest.raises(ValueError, match="multiples of 128"):
        FusedGroup([(t, torch.ones(256), torch.ones(80))], "cpu")
    with pytest.raises(ValueError, match="scale vectors"):
        FusedGroup([(a[0], a[1][:128], a[2])], "cpu")


def test_unpack_signs():
    from exl3xpu.linear import unpack_signs
    packed = torch.tensor([0b1, -1, 0], dtype=torch.int16)       # bit i of word j -> element 16 j + i
    s = unpack_signs(packed)
    assert s.dtype == torch.float16 and s.numel() == 48
    assert s[0] == -1 and (s[1:16] == 1).all() and (s[16:32] == -1).all() and (s[32:] == 1).all()


def test_linear_meta_shape_and_support():
    from exl3xpu.linear import C
    c = C()
    x = torch.empty(2, 3, 512, device="meta", dtype=torch.bfloat16)
    y = c.linear(x, torch.empty(32, 48, 48, device="meta", dtype=torch.int16),
                 torch.empty(2, 512, device="meta", dtype=torch.float16),
                 torch.empty(768, device="meta", dtype=torch.float16), torch.empty(6, device="meta", dtype=torch.int32),
                 [0, 512, 768], 3, 2, 8, 4096)
    assert tuple(y.shape) == (2, 3, 768) and y.dtype == torch.bfloat16
    assert [c.exl3_supported(k, 2) for k in range(1, 8)] == [False, True, True, True, True, True, False]
    for cb in (0, 1):       # 3inst / mcg: K = 4 and 6, as the reference's EXL3_ALL_CODEBOOKS build
        assert [c.exl3_supported(k, cb) for k in range(1, 8)] == [False, False, False, True, False, True, False]
    assert not c.exl3_supported(4, 3)


@pytest.mark.parametrize("K", [2, 4, 6])
def test_cpu_linear_baseline_matches_oracle(K):
    """The torch CPU linear that bench.py times as its CPU baseline computes what oracle/linear.py computes."""
    from oracle import cpu_path, exl3, synth
    ck = olin.checkpoint(60 + K, 256, [128, 256], K)
    xf = exl3.bf16_to_f32(synth.activations(61 + K, 2, 256))
    y = cpu_path.CpuLinear(K)(torch.from_numpy(xf), torch.from_numpy(ck["trellis"]), torch.from_numpy(ck["suh"]),
                              torch.from_numpy(ck["svh"]), ck["bounds"]).numpy()
    ref = olin.linear(xf, ck)
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-5
