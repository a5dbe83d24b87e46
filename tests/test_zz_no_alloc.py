"""exl3_moe_forward_cached_static (the entry point that allocates nothing: decode scratch in a static device array)
against exl3_moe_forward_cached (caller workspace + library exchange buffer), both through the C-ABI on two stores
that start identical: every call's output is bit-identical and every cache decision (slot map, slot owners, LRU
stamps, tick, fill list, the routing after the call) is the same. Two calls in a row, the second smaller, then a
longer mixed sequence; calls beyond the static array, or that would take the uncached path, are refused."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import exl3, synth

pytestmark = pytest.mark.gpu
H, I, K, E, L, S, TOPK = 2048, 512, 3, 32, 2, 24, 10


def _stores():
    from exl3xpu.moe_offload import ExpertStore
    distinct = [synth.expert_blob(71, e, H, I, K) for e in range(8)]
    stores = []
    for _ in range(2):
        st = ExpertStore(H, I, K, E, S, max_layers=L)
        for li in range(L):
            st.add_layer(f"layer{li}", torch.from_numpy(np.stack([distinct[(li * E + e) % 8] for e in range(E)])))
        stores.append(st)
    return stores


def _call(lib, st, li, x, ids, w, out, static, ws=None):
    args = [x.data_ptr(), 1, x.stride(0), x.shape[0], H, ids.data_ptr(), w.data_ptr(), TOPK, st.ptrs_all.data_ptr(), li,
            st.slot_of_dev.data_ptr(), st.slot_key.data_ptr(), st.slot_last.data_ptr(), st.tick.data_ptr(), S,
            st.host_base.data_ptr(), st.slot_base, st.fill_all.data_ptr(), st.fill_list.data_ptr(), E, I, K, E,
            out.data_ptr(), out.stride(0)]
    sh = torch.cuda.current_stream().cuda_stream
    if static:
        return lib.exl3_moe_forward_cached_static(*args, sh)
    return lib.exl3_moe_forward_cached(*args, ws.data_ptr(), ws.numel(), sh)


def _inputs(M, seed):
    rng = np.random.default_rng(seed)
    pr = 1.0 / np.arange(1, E + 1) ** 1.1
    pr /= pr.sum()
    ids = np.stack([rng.choice(E, TOPK, replace=False, p=pr) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, TOPK), dtype=np.float32)
    x = torch.from_numpy(exl3.bf16_to_f32(synth.activations(seed, M, H))).to(torch.bfloat16).cuda()
    return x, torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()


@pytest.mark.parametrize("fused", [1, 0])
def test_static_entry_matches_cached(fused):
    from exl3xpu import capi
    lib = capi.lib()
    print(f"case no-alloc entry fused={fused}", flush=True)
    stores = _stores()
    stores[0]._bind_strides()                      # both stores: blob-strided slots and host records
    for rc in (lib.exl3_set_tier(None, None, 0, None), lib.exl3_set_victims(None),
               lib.exl3_set_prefetch_commit(None, None, 0), lib.exl3_set_decision_log(None, 0),
               lib.exl3_set_fused_ensure(fused)):
        assert rc == 0
    try:
        # two calls in a row, the second smaller; then a longer sequence over both layers with hits and misses
        seq = [(4, 0), (1, 1)] + [((1, 2, 4)[n % 3], n % 2) for n in range(12)]
        for n, (M, li) in enumerate(seq):
            x, ids, w = _inputs(M, 100 + n)
            outs = []
            for s, st in enumerate(stores):
                out = torch.empty_like(x)
                ws = torch.empty(lib.exl3_moe_forward_workspace(M, H, I, TOPK, E), dtype=torch.uint8, device="cuda")
                it, wt = ids.clone(), w.clone()
                rc = _call(lib, st, li, x, it, wt, out, static=(s == 1), ws=ws)
                assert rc == 0, lib.exl3_last_error().decode()
                outs.append((out, it, wt))
            torch.cuda.synchronize()
            (oa, ia, wa), (ob, ib, wb) = outs
            assert torch.equal(oa, ob), f"call {n}: outputs differ"
            assert torch.equal(ia, ib) and torch.equal(wa, wb)
            a, b = stores
            for t in ("slot_of_dev", "slot_key", "slot_last", "tick", "fill_list", "fill_all"):
                ta, tb = getattr(a, t), getattr(b, t)
                if t == "fill_all":                # pending fill targets: slot addresses of each store
                    ta, tb = (ta != 0), (tb != 0)
                assert torch.equal(ta, tb), f"call {n}: {t} differs"
        assert int(stores[1].tick.item()) == len(seq) and int((stores[1].slot_key >= 0).sum().item()) == S
        # refused without enqueueing anything: more scratch than the static array holds, and the uncached path
        x, ids, w = _inputs(26, 900)
        out = torch.empty_like(x)
        assert _call(lib, stores[1], 0, x, ids, w, out, static=True) == 2     # EXL3_EUNSUPPORTED
        assert b"static scratch" in lib.exl3_last_error()
        x, ids, w = _inputs(1, 901)
        args_no_slots = stores[1]
        rc = lib.exl3_moe_forward_cached_static(x.data_ptr(), 1, x.stride(0), 1, H, ids.data_ptr(), w.data_ptr(), TOPK,
                                                 args_no_slots.ptrs_all.data_ptr(), 0, args_no_slots.slot_of_dev.data_ptr(),
                                                 args_no_slots.slot_key.data_ptr(), args_no_slots.slot_last.data_ptr(),
                                                 args_no_slots.tick.data_ptr(), 0, args_no_slots.host_base.data_ptr(),
                                                 args_no_slots.slot_base, args_no_slots.fill_all.data_ptr(),
                                                 args_no_slots.fill_list.data_ptr(), E, I, K, E, out.data_ptr(),
                                                 out.stride(0), torch.cuda.current_stream().cuda_stream)
        assert rc == 2 and b"uncached path" in lib.exl3_last_error()
        # M = 0: nothing to do
        e0 = torch.empty((0, H), dtype=torch.bfloat16, device="cuda")
        assert _call(lib, stores[1], 0, e0, ids, w, e0, static=True) == 0
        torch.cuda.synchronize()
    finally:
        lib.exl3_set_fused_ensure(1)
