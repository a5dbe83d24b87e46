"""C-ABI library: loads, exports every function include/exl3moe.h declares, validates arguments on the host (no
compute calls: this runs without a GPU)."""
import ctypes

import pytest

from exl3xpu import capi


def test_exports_every_declared_symbol():
    names = capi.declared_functions()
    assert len(names) >= 20
    L = ctypes.CDLL(capi.LIB_PATH)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(capi.SIGNATURES), set(names) ^ set(capi.SIGNATURES)


def test_blob_bytes():
    L = capi.lib()
    assert L.exl3_blob_bytes(2048, 512, 3) == 1_195_008
    assert L.exl3_blob_bytes(2560, 640, 3) == 1_862_400
    assert [L.exl3_blob_bytes(4096, 1536, k) for k in (2, 3, 4)] == [4_752_384, 7_111_680, 9_470_976]


@pytest.mark.parametrize("H,I,K,E,code", [(100, 512, 3, 512, 1), (2048, 500, 3, 512, 1), (2048, 512, 5, 512, 2),
                                          (2048, 512, 3, 2048, 1)])
def test_forward_rejects_bad_geometry(H, I, K, E, code):
    L = capi.lib()
    rc = L.exl3_moe_forward(None, 0, 0, 1, H, None, None, 10, None, I, K, E, None, 0, None, 0, None)
    assert rc == code
    assert L.exl3_last_error()


def test_forward_rejects_bad_dtype_and_workspace():
    L = capi.lib()
    assert L.exl3_moe_forward(None, 7, 0, 1, 2048, None, None, 10, None, 512, 3, 512, None, 0, None, 0, None) == 1
    assert L.exl3_moe_forward(None, 1, 0, 0, 2048, None, None, 10, None, 512, 3, 512, None, 0, None, 0, None) == 0
    assert L.exl3_moe_forward_workspace(1, 2048, 512, 10, 512) > 0
    assert L.exl3_moe_forward_workspace(8192, 2048, 512, 10, 512) > L.exl3_moe_forward_workspace(4, 2048, 512, 10, 512)
    assert L.exl3_moe_align_workspace(8192, 10, 512) == 80 * 512 * 4


def test_setters():
    L = capi.lib()
    assert L.exl3_set_host_stride(7) == 1
    assert L.exl3_set_host_stride(0) == 0
    assert L.exl3_set_tier(None, None, 0, None) == 0
    assert L.exl3_set_pair_max_m(4) == 0 and L.exl3_set_prefill_min_m(256) == 0
    # the victim ring: K in 1..256 with meta, sel and a buffer (pointers are only stored, never touched here)
    fake = 0x1000
    assert L.exl3_set_victim_ring(fake, fake, fake, 1 << 20, 257) == 1
    assert L.exl3_set_victim_ring(fake, None, fake, 1 << 20, 8) == 1
    assert L.exl3_set_victim_ring(fake, fake, fake, 0, 8) == 1
    assert L.exl3_set_victim_ring(fake, fake, fake, 1 << 20, 8) == 0
    assert L.exl3_set_victim_ring(None, None, None, 0, 0) == 0


def test_linear_entry_points_validate_without_a_gpu():
    L = capi.lib()
    assert [L.exl3_linear_supported(k, 2) for k in range(1, 8)] == [0, 1, 1, 1, 1, 1, 0]
    assert L.exl3_linear_supported(3, 1) == 0
    assert [L.exl3_linear_supported(k, cb) for cb in (0, 1) for k in (2, 3, 4, 5, 6)] == [0, 0, 1, 0, 1] * 2
    # tagged 64-bit parts [ceil(k / 512), M, n], 256-byte aligned
    assert L.exl3_linear_workspace(1, 2048, 4096) == 4 * 4096 * 8
    assert L.exl3_linear_workspace(8, 2560, 12288) == 5 * 8 * 12288 * 8
    assert L.exl3_linear_workspace(1, 128, 128) == 1024
    assert L.exl3_linear_small(None, 0, 0, 1, 100, 256, None, 3, 2, None, 1, None, None, None, 0, 0, None, 0,
                               None) == 1                       # k not a multiple of 128
    assert L.exl3_linear_small(None, 0, 0, 9, 128, 256, None, 3, 2, None, 1, None, None, None, 0, 0, None, 0,
                               None) == 2                       # more rows than the fused path takes
    assert L.exl3_linear_small(None, 0, 0, 1, 128, 256, None, 7, 2, None, 1, None, None, None, 0, 0, None, 0,
                               None) == 2                       # K outside 2..6
    assert L.exl3_linear_small(None, 0, 0, 0, 128, 256, None, 3, 2, None, 1, None, None, None, 0, 0, None, 0,
                               None) == 0                       # no rows: nothing to do
    assert L.exl3_reconstruct(None, 128, 256, 16, 8, 3, 2, None, None) == 1
    assert L.exl3_had_in(None, 0, 0, 0, 256, None, 1, None, None) == 0
    assert L.exl3_had_out(None, 1, 100, None, None, 0, 100, None) == 1
