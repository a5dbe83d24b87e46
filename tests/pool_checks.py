"""Invariants of the RAM tier's record pool after a run (shared by the GPU tests of the cache and the workloads)."""
import numpy as np
import torch


def write_backs(recs: np.ndarray, P: int) -> np.ndarray:
    """Write-backs per step from decision records [steps, L, 3 + 4P] (victim lanes with a key >= 0)."""
    return (recs[:, :, 3 + 2 * P::2] >= 0).sum(axis=(1, 2))


def check_pool(store, tier, src, budget: int, expect_taken: int | None = None) -> None:
    """No write-back dropped; the pool within budget + 3 x queue records (its chunks: the records rounded up);
    every key the tier holds in RAM owns a distinct record that holds its own true blob, and the device's host
    address table (and, for keys outside HBM, the pointer table) points at it. expect_taken: the write-backs the
    host steps settled (all but the last decode step's)."""
    pool = tier.pool
    assert tier.stats["wb_dropped"] == 0, f"{tier.stats['wb_dropped']} write-backs dropped"
    if expect_taken is not None:
        assert tier.stats["wb_taken"] == expect_taken, (tier.stats["wb_taken"], expect_taken)
    bound = budget + 3 * tier.wb_cap
    assert pool.high <= bound, f"pool high-water {pool.high} records > {bound}"
    assert pool.records <= -(-bound // pool.chunk) * pool.chunk
    assert tier.pinned_bytes() == pool.records * store.stride
    torch.cuda.synchronize()
    keys = np.nonzero(tier.res)[0]
    rec = store.rec_of[keys]
    assert (rec != 0).all(), "a RAM-resident key without a record"
    assert np.unique(rec).size == rec.size, "two keys share a record"
    ha = store.host_addr_dev.cpu().numpy()
    assert np.array_equal(ha[keys], rec)
    so = store.slot_of_dev[:ha.size].cpu().numpy()
    pa = store.ptrs_all[:ha.size].cpu().numpy()
    out = keys[so[keys] < 0]
    assert np.array_equal(pa[out], store.rec_of[out])
    for key, r in zip(keys.tolist(), rec.tolist()):
        want = np.asarray(src.blob_of(tier.rec_index(key)))
        got = pool.view(int(r), want.size).numpy()
        assert np.array_equal(got, want), f"record of key {key} does not hold its blob"
