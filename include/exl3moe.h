/* C-ABI of the MI355X EXL3 expert-offload hot path (libexl3moe.so).
 *
 * Plain pointers, sizes and a hipStream_t (passed as void*); every entry point returns 0 on success or an EXL3_E*
 * code, with a message available from exl3_last_error() (thread-local). Device pointers are HIP device (or pinned,
 * device-mapped host) addresses. Work is enqueued on `stream`; nothing synchronises the host except where noted.
 *
 * Each function replaces one op of the reference's torch library TORCH_LIBRARY(exl3xpu_moe)
 * (kernels/moe-a8/exl3_moe.a8.sycl:1555-1592); the reference file:line of the implementation it replaces is given on
 * every declaration. The torch custom-op library _moe.so registers the same schemas and calls these functions.
 *
 * Process-wide configuration (tier flags, victim list, host stride, thresholds) mirrors the reference's moe_set_*
 * globals (a8:682-789): it is read when a call is enqueued, so a captured HIP graph keeps the pointers it saw.
 * Calls that use the expert cache on one device must be stream-ordered: the device-side cache state and the
 * reduction counters of the decode kernels are shared by all calls on that device.
 */
#ifndef EXL3MOE_H
#define EXL3MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    EXL3_OK = 0,
    EXL3_EINVAL = 1,        /* bad argument / shape / dtype (the reference's TORCH_CHECK failures) */
    EXL3_EUNSUPPORTED = 2,  /* geometry outside what the kernels implement */
    EXL3_EHIP = 3,          /* HIP runtime error */
    EXL3_EWORKSPACE = 4,    /* workspace smaller than exl3_*_workspace() */
    EXL3_ENOMEM = 5
};

/* activation / output dtypes (the reference accepts fp16 and bf16; fp32 is an extension for exact checks) */
enum { EXL3_DT_F16 = 0, EXL3_DT_BF16 = 1, EXL3_DT_F32 = 2 };

/* last error message of the calling thread ("" if none) */
const char* exl3_last_error(void);

/* bytes of one expert blob. Replaces blob_bytes (a8:1551; Geom a8:42-54). */
int64_t exl3_blob_bytes(int H, int I, int K);

/* ---- process-wide configuration (a8:682-789) ---------------------------------------------------------------------- */

/* moe_set_tier (a8:768-774): ram_res uint8 [L*E] (1 = RAM-tier copy valid), miss ring int32 [1 + cap]
 * ([0] = count of masked picks modulo 2^32; entry c at position 1 + (c mod 2^32) % cap, cap a power of two so that
 * positions stay continuous across the wrap of the count; EXL3_EINVAL otherwise), safe int32 [L].
 * ram_res == NULL turns the tier (masking) off. */
int exl3_set_tier(uint8_t* ram_res, int32_t* miss_ring, int64_t ring_numel, const int32_t* safe);
/* moe_set_victims (a8:757): device int32 [1 + 2E] victim list, NULL = no victim write-back */
int exl3_set_victims(int32_t* vict);
/* Write-back target of each victim of a cached call (replaces the fixed-address write-back of
 * plugin/exl3xpu/nvtier.py:22-53, where every key owns a page of a sparse memfd): device int64 [E], written by the
 * ensure beside the victim list and read by the copies; NULL = the fixed record host_base[layer] + e * host_stride. */
int exl3_set_victim_addrs(int64_t* vict_addr);
/* The RAM tier's record pool (replaces the sparse memfd and the hole punches of plugin/exl3xpu/nvtier.py:19-53 and
 * 109-126 that hold RAM to the budget): the host record of every key is host_addr[key] (device int64 [L*E]) instead of
 * a fixed address, and a victim whose RAM copy is not valid is written back into the next free record of the step's
 * queue wbq (device int64 [wbq_cap], installed by exl3_tier_exchange_pool). wbq_state (device int32 [2 + wbq_cap]):
 * [0] = records taken, [1 + i] = the key written into wbq[i], [1 + wbq_cap] = write-backs dropped because the queue
 * was used up (the victim then leaves HBM without a copy and stays masked until a fill brings it back). Needs the
 * victim list and exl3_set_victim_addrs; the fixed-record paths (exl3_moe_prefetch, exl3_moe_prefetch_plan, the
 * copy-engine worker) return EXL3_EUNSUPPORTED while it is set. host_addr == NULL turns it off. */
int exl3_set_record_pool(int64_t* host_addr, const int64_t* wbq, int32_t* wbq_state, int64_t wbq_cap);
/* moe_set_victim_ring (experimental/n111-victim-ring/a9.patch:17-30): victims are written back into a ring of K slots
 * in device memory (buf, at least K x the slot stride bytes) instead of into their RAM records, and the host drains
 * the ring. meta (device int32 [4 + 2K]): [0] next search position, [1] claims made, [2] write-backs dropped because
 * no ring slot was free, [3] K, then key[K] (-1 = free, else the key whose bytes the slot holds) and seq[K] (the claim
 * number of that key); the ensure claims free slots in circular order from [0], in victim order (a9.patch:46-65).
 * sel (device int32 [E]): the ring slot of victim i of the last call (-1 = none). The device never flags a ring
 * victim RAM-resident and never frees a slot: the host does both once the slot's copy to RAM has completed. Needs the
 * victim list and exl3_set_victim_addrs; works with fixed records and with the record pool; the prefetch paths
 * return EXL3_EUNSUPPORTED while it is set. meta == NULL turns it off. K <= 256. */
int exl3_set_victim_ring(int32_t* meta, int32_t* sel, void* buf, int64_t buf_bytes, int64_t K);
/* moe_set_host_stride (a8:765): stride of a key's RAM-tier address, 0 = the slot stride */
int exl3_set_host_stride(int64_t stride);
/* Bytes between HBM slots, 0 = the blob size of the call (no reference counterpart: the reference assumes one expert
 * geometry per store, plugin/sglang_plugin.tier.py:166-167). Set to the largest blob when layers of one store use
 * different bitrates K; victims are then written back as whole slots. */
int exl3_set_slot_stride(int64_t stride);
/* 1 (default): a cached decode call within the fused limits (<= 512 experts, <= 64 picks, <= 16384 slots, K <= 3)
 * runs the ensure as the first workgroup of the layer kernel, so pairs that hit start streaming at once; 0: the
 * ensure is a separate launch before the layer kernel. The decisions are the same either way (no reference
 * counterpart: the reference always launches its ensure kernel first, kernels/moe-a8/exl3_moe.a8.sycl:1040). */
int exl3_set_fused_ensure(int64_t enable);
/* moe_set_prefill_min_m (a8:775), moe_set_pair_max_m (a8:727), moe_set_splits (a8:685), moe_set_mr (a8:729) */
int exl3_set_prefill_min_m(int64_t m);
int exl3_set_pair_max_m(int64_t m);
int exl3_set_splits(int64_t gu_p, int64_t dn_p);
int exl3_set_mr(int64_t mr);
/* moe_set_debug (a8:728): accepted for API compatibility; kernel skipping for timing probes is not provided */
int exl3_set_debug(int64_t v);
/* Decision log of the device cache (no reference counterpart; test hook): int32 buffer [1 + cap_words],
 * buf[0] = ensure calls counted; one record per ensure call of 3 + 4P int32 (P picks of the call; one P per log):
 * [T, ring count, P post-mask ids, misses nm, P filled experts (-1 pad), P (write-back key or -1, slot) pairs (-2
 * pad)], record i at buf + 1 + i (3 + 4P), written only if it ends within the cap_words words. NULL = off. */
int exl3_set_decision_log(int32_t* buf, int64_t cap_words);

/* ---- routed-expert MoE --------------------------------------------------------------------------------------------- */

/* workspace bytes of an exl3_moe_forward call with these sizes (decode kernels for M < prefill_min_m: the blob
 * pointer of every pick; the prefill path otherwise: sorted routing, input Hadamards [M topk][2][H] fp16, abuf
 * [M topk][I] fp16, y [M topk][H] fp16). The decode kernel's cross-workgroup exchange is not in the workspace: the
 * library owns one zeroed device buffer per device and grows it when a call needs more (hipMalloc + hipMemset, after
 * a device synchronisation; the replaced buffer stays allocated, since graphs captured earlier still address it); a
 * call that would grow it while its stream is being captured fails with EXL3_EUNSUPPORTED, so run one call of the
 * largest size before capturing. */
size_t exl3_moe_forward_workspace(int M, int H, int I, int topk, int n_experts);

/* moe_forward (a8:1221-1225 -> moe_forward_impl a8:1263-1314): out[m] = sum_k w[m,k] * expert(ids[m,k])(x[m]).
 * x, out: [M, H] with row strides, dtype EXL3_DT_*; ids int32 / w fp32 [M, topk] contiguous; ptrs int64 [n_experts]
 * blob addresses (device slots or device-mapped pinned host memory). M < prefill_min_m runs the fused decode kernel
 * (M <= 256 rows, M * topk <= 1024 pairs); M >= prefill_min_m the prefill path (moe_prefill a8:792-828): token sort,
 * grouped MFMA GEMMs with the trellis decoded into LDS, y in fp16, combine (needs H % 256 == 0). */
int exl3_moe_forward(const void* x, int x_dtype, int64_t x_stride, int M, int H, const int32_t* topk_ids,
                     const float* topk_w, int topk, const int64_t* ptrs, int I, int K, int n_experts, void* out,
                     int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);

/* moe_forward_cached (a8:1229-1261): the same through the device-managed expert cache of layer `layer`:
 * ensure (tier mask, hits, exact-LRU victims, assignment) -> victim write-back -> GEMVs with write-through of misses
 * -> combine + commit. topk_ids / topk_w are rewritten in place by the tier mask (the reference does the same).
 * M == 0, M >= prefill_min_m or n_slots == 0 fall back to exl3_moe_forward on the layer's pointer table. */
int exl3_moe_forward_cached(const void* x, int x_dtype, int64_t x_stride, int M, int H, int32_t* topk_ids,
                            float* topk_w, int topk, int64_t* ptrs_all, int layer, int32_t* slot_of, int32_t* slot_key,
                            int32_t* slot_last, int32_t* tick, int n_slots, const int64_t* host_base,
                            int64_t slot_base, int64_t* fill_all, int32_t* fill_list, int max_fill, int I, int K,
                            int n_experts, void* out, int64_t out_stride, void* workspace, size_t workspace_bytes,
                            void* stream);

/* The same call without any allocation (no reference counterpart: the reference always passes a workspace that
 * torch allocates, a8:1229-1261). For callers that cannot allocate device memory: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. The decode scratch (the blob pointer of every pick and the
 * cross-workgroup exchange words) comes from one static device array of EXL3_STATIC_SCRATCH_BYTES per device, held
 * until the process ends; its address is looked up on the first call on a device and the array is cleared then (one
 * fill kernel on `stream`). Limit: calls whose scratch exceeds the array (8 MiB: config-0 shapes up to 25 rows x
 * top-10, config-4 shapes up to 7 rows x top-8) and calls that would take the uncached path (M >= prefill_min_m, or
 * n_slots == 0) fail with EXL3_EUNSUPPORTED before anything is enqueued. Every call on one device shares the array
 * and it keeps the last call's contents: calls that overlap on one device (other streams) race; stream-ordered calls
 * are safe. Decisions and outputs are those of exl3_moe_forward_cached. */
#define EXL3_STATIC_SCRATCH_BYTES ((size_t)8 << 20)
int exl3_moe_forward_cached_static(const void* x, int x_dtype, int64_t x_stride, int M, int H, int32_t* topk_ids,
                                   float* topk_w, int topk, int64_t* ptrs_all, int layer, int32_t* slot_of,
                                   int32_t* slot_key, int32_t* slot_last, int32_t* tick, int n_slots,
                                   const int64_t* host_base, int64_t slot_base, int64_t* fill_all, int32_t* fill_list,
                                   int max_fill, int I, int K, int n_experts, void* out, int64_t out_stride,
                                   void* stream);

/* moe_prefetch (a8:1194-1222): claim slots for the (predicted) experts `ids` of layer `layer` with the ensure in
 * prefetch mode (launch_ensure a8:846-851: the tick is not advanced, so slots stamped by the last MoE call stay
 * protected; hits re-stamped, misses up to max_fill get exact-LRU slots older than the tick, old owners repointed to
 * their host records; no tier mask, no write-back), copy each assigned expert from its host record into its slot
 * (PrefetchCopyKernel), then repoint ptrs_all. pf_list int32 [1 + n_experts] = [n, e...], pf_slot int32
 * [n_experts]. Enqueued on `stream`: run it on a side stream that waited for the previous MoE call and make the
 * compute stream wait for it before the next one. n_slots == 0 or n_ids == 0: nothing is done. */
int exl3_moe_prefetch(const int32_t* ids, int n_ids, int64_t* ptrs_all, int layer, int32_t* slot_of,
                      int32_t* slot_key, int32_t* slot_last, int32_t* tick, int n_slots, const int64_t* host_base,
                      int64_t slot_base, int32_t* pf_list, int32_t* pf_slot, int max_fill, int n_experts, int64_t blob,
                      void* stream);

/* Copy-engine prefetch (a8:1047-1142; moe_offload.py:264-302). moe_prefetch_plan: the ensure in plan mode on the
 * compute stream: claims up to 16 exact-LRU slots (tick not advanced) for predicted experts of `layer`, pins them
 * (slot_last = INT_MAX), records them in pend[layer] (int32 [n_layers][35]: n, seq, T, e[16], s[16]) and publishes
 * the plan in pinned host memory (plans int32 [n_layers][4 + 2 n_experts]: seq, n, T, layer, e[], s[]); a layer whose
 * previous plan is pending is skipped. Every plan call, and every moe_forward_cached call while
 * exl3_set_prefetch_commit is set, first commits the plans with done_seq[layer] >= their seq (ptrs_all -> slot,
 * slot_last = the plan's tick; the fused ensure is off meanwhile). */
int exl3_moe_prefetch_plan(const int32_t* ids, int n_ids, int64_t* ptrs_all, int layer, int32_t* slot_of,
                           int32_t* slot_key, int32_t* slot_last, int32_t* tick, int n_slots,
                           const int64_t* host_base, int64_t slot_base, int32_t* pf_list, int32_t* pf_slot,
                           int32_t* plans, int32_t* plan_seq, int32_t* pend, const int32_t* done_seq, int n_layers,
                           int max_fill, int n_experts, int64_t blob, void* stream);
/* moe_prefetch_worker_start / _stop: a host thread polls `plans`; per new plan it copies each claimed expert from
 * host_base_host[layer] + e * host stride into its slot on `stream` (a dedicated stream), then copies the plan's seq
 * (from seq_host, pinned int32 [n_layers][2]) into done_seq[layer] on the same stream. Stop drains the stream and
 * returns [plans handled, experts copied] in counts. */
int exl3_prefetch_worker_start(int32_t* plans, const int64_t* host_base_host, int64_t slot_base, int64_t blob,
                               int32_t* done_seq, int32_t* seq_host, int n_layers, int n_experts, void* stream);
int exl3_prefetch_worker_stop(int64_t* counts);
/* the pending-plan tables that moe_forward_cached commits from (n_layers 0: off); moe_forward_cached's pend /
 * done_seq arguments (a8:1229-1261) set it per call */
int exl3_set_prefetch_commit(int32_t* pend, const int32_t* done_seq, int n_layers);

/* moe_align (a8:1316-1323 -> launch_align a8:639-680): token sort by expert into the reference's packed buffers:
 * ib int32 [4A + 1 + 2*npairs + 16] = act_expert[A] act_start[A] act_cnt[A] act_pstart[A] n_act pair_tok[npairs]
 * pair_of[npairs] ..., fb fp32 [npairs] = pair_w, A = min(npairs, n_experts); active experts ascending, act_pstart the
 * starts padded to multiples of `pad`. Canonical order: pairs of an expert in ascending pair index (the reference's
 * order inside an expert depends on atomics). Ids outside [0, n_experts) are clamped. The workspace (device,
 * exl3_moe_align_workspace bytes) holds per-chunk counts. */
size_t exl3_moe_align_workspace(int M, int topk, int n_experts);
int exl3_moe_align(const int32_t* topk_ids, const float* topk_w, int M, int topk, int n_experts, int pad, int32_t* ib,
                   float* fb, void* workspace, size_t workspace_bytes, void* stream);

/* Flag upload of the host tier step (replaces the index_copy_ of plugin/exl3xpu/nvtier.py:791-793):
 * flags[packed[i] >> 1] = packed[i] & 1 for i < n. `packed` may be pinned, device-mapped host memory (read in place,
 * no staging copy): the caller keeps it unchanged until the work queued on `stream` so far has run. Keys outside
 * [0, n_flags) are skipped. */
int exl3_scatter_flags(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n, void* stream);

/* The device side of one host tier step as one launch (replaces the snapshot .to("cpu") copies and the flag
 * index_copy_ of plugin/exl3xpu/nvtier.py:282-386 and 791-793): applies the diff as exl3_scatter_flags; mirrors the
 * miss ring (int32 [1 + ring_cap], [0] = count) into ring_mirror (same layout, device-mapped pinned): the entries at
 * counts [ring_from, count) modulo 2^32 (the last ring_cap of them at most) and the count; then copies src[k] -> dst[k]
 * (nbytes[k] bytes, k < n_copies <= 4; dst device-mapped pinned host memory, both 16-byte aligned). ring may be NULL;
 * ring_cap is a power of two (as exl3_set_tier requires).
 * A flag the diff sets may be snapshotted before or after its update. */
int exl3_tier_exchange(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n_diff, const int32_t* ring,
                       int64_t ring_cap, int64_t ring_from, int32_t* ring_mirror, const void* const* src,
                       void* const* dst, const int64_t* nbytes, int n_copies, void* stream);

/* exl3_tier_exchange with the record pool (replaces the evict/punch bookkeeping of plugin/exl3xpu/nvtier.py:282-386):
 * first upd (pinned int64 [2 n_upd], (key, record address) pairs, keys outside [0, n_flags) skipped) sets
 * host_addr[key] and, for a key not in an HBM slot (slot_of[key] < 0), ptrs_all[key]; then, when wbq is not NULL, one
 * workgroup copies wbq_state [2 + wbq_cap] into wbq_mirror (pinned), installs next (pinned int64 [wbq_cap]) as the
 * queue of the following decode step and clears the taken and dropped counts; then the diff, ring and copies as
 * exl3_tier_exchange. upd and next are read in place: the caller keeps them unchanged until the launch has run. */
int exl3_tier_exchange_pool(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n_diff,
                            const int32_t* ring, int64_t ring_cap, int64_t ring_from, int32_t* ring_mirror,
                            const void* const* src, void* const* dst, const int64_t* nbytes, int n_copies,
                            const int64_t* upd, int64_t n_upd, int64_t* host_addr, int64_t* ptrs_all,
                            const int32_t* slot_of, const int64_t* next, int64_t* wbq, int32_t* wbq_state,
                            int32_t* wbq_mirror, int64_t wbq_cap, void* stream);

/* Device health flags (no reference counterpart): flags4[0] = bounded waits of the fused decode kernel that timed
 * out since load (0 in a healthy run; a timeout means an output was computed from an incomplete intermediate, so
 * callers must treat a non-zero value as fatal). Synchronises `stream`. */
int exl3_device_status(int32_t* flags4, void* stream);

/* Device address (current device) of those four status words, 16-byte aligned, so that a caller can copy them
 * without a synchronisation of its own: the host tier step adds them to the snapshot copies of exl3_tier_exchange
 * and raises when flags4[0] != 0 (no reference counterpart). */
int exl3_device_status_address(void** dev_ptr);

/* Mirror of flags4[0] in host memory (no reference counterpart): host_word points into pinned host memory
 * (exl3_host_alloc) and is raised by one, with a system-scope atomic, by every bounded wait that times out on the
 * current device, from then on (NULL: no mirror). A caller notices a timeout by reading that word, with no copy and
 * no synchronisation, so graph-captured decode loops stay sync-free; the ExpertStore wrappers raise RuntimeError at
 * their next call when it moved. Synchronous (sets a device symbol); call it outside graph capture. */
int exl3_set_status_mirror(int32_t* host_word);

/* Bit-exact dequantization (ReconstructKernel, exl3_esimd.h:869-936): PLANAR4 trellis words
 * [k_tiles][n_tiles][8K] -> fp16 bits [16 k_tiles][16 n_tiles] (W_inner, Hadamard domain). */
int exl3_dequant(const uint32_t* trellis, int k_tiles, int n_tiles, int K, uint16_t* out, void* stream);

/* ---- the dense EXL3 linear (exl3xpu_C.linear, experimental/n111-victim-ring/csrc/exl3_ops.sycl:651-757; the
 * plugin's Exl3XpuLinearMethod.apply, plugin/sglang_plugin.tier.py:380-388) -------------------------------------
 * out[M, n] = svh * H(sum_k xh[g][m][k] W[k][n]) / sqrt 128 with xh[g] = fp16(H(fp16(x * suh[g])) / sqrt 128), g the
 * shard of output block n / 128 (shard_of_nb int32 [n/128]), W the codebook values of the checkpoint trellis (int16
 * [k/16][n/16][16K] read as little-endian uint32 words, natural order); suh fp16 [S][k], svh fp16 [n]; k, n multiples
 * of 128. Codebooks: cb = 2 (mul1) with K = 2..6, and cb = 0 (3inst) and 1 (mcg) with K = 4 and 6 (the reference's
 * set when built with EXL3_ALL_CODEBOOKS, exl3_esimd.h:69-79). */

/* exl3_supported (exl3_ops.sycl:767-773): 1 when (K, cb) is implemented, else 0 */
int exl3_linear_supported(int K, int cb);
/* workspace bytes of exl3_linear_small: the tagged partial sums over K-slices of 512 rows [ceil(k/512)][M][n], 64-bit
 * words ((1 << 32) | fp32 bits), rounded up to 256 bytes */
size_t exl3_linear_workspace(int M, int k, int n);
/* the small-M path (exl3_gemm_small, exl3_ops.sycl:258-321): M <= 8 rows, x and out dtype EXL3_DT_* with row
 * strides; one launch on `stream` (input Hadamards, dequant-GEMV, and the output Hadamard by the last workgroup of
 * each 128-column block, which polls the other workgroups' tagged partials and clears them). The workspace must be
 * zero before the first call (e.g. memset once at allocation); every call leaves it zero. Calls that share a
 * workspace must not run concurrently. */
int exl3_linear_small(const void* x, int x_dtype, int64_t x_stride, int M, int k, int n, const void* trellis, int K,
                      int cb, const void* suh, int S, const void* svh, const int32_t* shard_of_nb, void* out,
                      int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream);
/* exl3_had_in_rm (exl3_ops.sycl:602-608): xh fp16 [S][M][k] = fp16(H(fp16(x * suh[g])) / sqrt 128) */
int exl3_had_in(const void* x, int x_dtype, int64_t x_stride, int M, int k, const void* suh, int S, void* xh,
                void* stream);
/* exl3_had_out_h (exl3_ops.sycl:610-616): out[M, n] = svh * H(y) / sqrt 128 for y fp16 [M][n] */
int exl3_had_out(const void* y, int M, int n, const void* svh, void* out, int out_dtype, int64_t out_stride,
                 void* stream);
/* exl3_reconstruct (ReconstructKernel, exl3_esimd.h:869-936): w fp16 [k][n1 - n0] = the codebook weights of
 * columns [n0, n1) (multiples of 16) of a natural-order trellis of k x n, bit-exact */
int exl3_reconstruct(const void* trellis, int k, int n, int n0, int n1, int K, int cb, void* w, void* stream);

/* ---- the W8A8 route of the large-M linear (exl3_ops.sycl:520-537, 668-740: opt-in through exl3_set_int8, mul1 at
 * K = 4 and 6, more than 16 rows): int8 activations with one scale per (shard, row), int8 weights at the static
 * scale 127 / 3.453125, an int8 GEMM with int32 sums (the caller's library GEMM), then the output Hadamard. ---- */
/* HadInQ8Kernel (exl3_esimd.h:341-421): xq int8 [S][ms][k] = rne(xh * inv) and sx fp32 [S][ms] = sc, with xh the
 * fp16 input Hadamard of exl3_had_in, amax its largest magnitude over the row, sc = amax / 127 (1 for a zero row) and
 * inv = 1 / sc; ms >= M is the row stride of xq and sx */
int exl3_had_in_q8(const void* x, int x_dtype, int64_t x_stride, int M, int k, const void* suh, int S, void* xq,
                   void* sx, int64_t ms, void* stream);
/* launch_reconstruct_q8 (exl3_ops.sycl:528-537): w int8 [k][n1 - n0] = rne(W * 127 / 3.453125) of the mul1 weights
 * of columns [n0, n1), K = 2..6 */
int exl3_reconstruct_q8(const void* trellis, int k, int n, int n0, int n1, int K, void* w, void* stream);
/* HadOutQ8Kernel (exl3_esimd.h:423-440): out[M, n] = svh * H(y * (sx[m] * sw)) / sqrt 128 for y int32 [M][n] (one
 * shard group's columns, n a multiple of 128), sx fp32 [M], sw the weight scale (3.453125 / 127) */
int exl3_had_out_q8(const int32_t* y, int M, int n, const float* sx, float sw, const void* svh, void* out,
                    int out_dtype, int64_t out_stride, void* stream);

/* ---- RAM-tier admission (host) ---------------------------------------------------------------------------------- */

/* Books of the admission step besides the per-key arrays; the counters accumulate over calls. */
typedef struct {
    int64_t n;              /* keys (layers x experts) */
    int64_t budget;         /* RAM records */
    int64_t admit_age;      /* evict non-HBM RAM copies only when older than this many steps (AGE) */
    int64_t admit_qmax;     /* at most this many fills in flight (QMAX) */
    int64_t ring_cap;       /* capacity of the device miss ring */
    int64_t tick;           /* current host step (set by the caller) */
    int64_t ring_seen;      /* miss-ring count consumed so far */
    int64_t masked, evicts, admit_dropped, ring_overflow;
} exl3_admit_state;

/* One admission decision (_async_step_admit, plugin/exl3xpu/nvtier.py:708-806), host only, no allocation after the
 * first call of a thread. res u8 [n] / age i64 [n] / inflight u8 [n]: the host's books, updated in place; pin u8 [n];
 * view u8 [n]: previous step's device flags with the previous upload overlaid; ring i32 [1 + ring_cap] and slot_of
 * i32 [n]: previous step's snapshots; done [n_done]: fills completed now. Outputs (capacity n each): admitted keys
 * (misses by descending count, ties ascending key), evicted keys (HBM-duplicated RAM copies first, then entries older
 * than admit_age, each by ascending age, ties ascending key), and the flag diff (keys ascending, new values). */
int exl3_admit_decide(exl3_admit_state* st, uint8_t* res, int64_t* age, uint8_t* inflight, const uint8_t* pin,
                      const uint8_t* view, const int32_t* ring, const int32_t* slot_of, const int64_t* done,
                      int64_t n_done, int64_t* adm, int64_t* n_adm, int64_t* ev, int64_t* n_ev, int64_t* diff,
                      uint8_t* vals, int64_t* n_diff);

/* ---- host memory and copies (a8:1527-1549) --------------------------------------------------------------------------- */

/* host_alloc (a8:1529-1537): pinned, device-mapped host memory (hipHostMalloc); NULL on failure */
void* exl3_host_alloc(int64_t nbytes);
int exl3_host_free(void* p);
/* usm_kind (a8:1540-1544): 0 unknown/pageable, 1 pinned host, 2 device, 3 managed */
int exl3_usm_kind(const void* p);
/* memcpy_async (a8:1546-1549): async copy of raw bytes on `stream` */
int exl3_memcpy_async(void* dst, const void* src, int64_t nbytes, void* stream);

/* A batch of memcpy_async calls on one stream (replaces the Python loops of memcpy_async over expert runs in
 * ExpertStore.make_resident / stage_layer, plugin/exl3xpu/moe_offload.py:173, 315-323, and NvTier._stage_forward,
 * plugin/exl3xpu/nvtier.py:598-607). Every copy i must lie inside [dst_lo, dst_hi) and [src_lo, src_hi); the whole
 * batch is checked first and nothing is enqueued when one copy is out of bounds (EXL3_EINVAL). */
int exl3_copy_batch(void* const* dst, const void* const* src, const int64_t* nbytes, int64_t n, int64_t dst_lo,
                    int64_t dst_hi, int64_t src_lo, int64_t src_hi, void* stream);

/* Device tables of static placement in one launch (replaces the index_copy_ / index_fill_ sequences of
 * ExpertStore.make_resident and evict, plugin/exl3xpu/moe_offload.py:178-184, 204-211). rec: device int64 [n][3] =
 * (key, slot, ptr) on distinct keys and slots. slot >= 0: key -> slot (slot_key[slot] = key, slot_last[slot] = 0);
 * slot < 0: key leaves slot -1 - slot (its slot_key and slot_last become -1). ptrs_all[key] = ptr, slot_of[key] =
 * the new slot or -1. */
int exl3_table_update(int64_t* ptrs_all, int32_t* slot_of, int32_t* slot_key, int32_t* slot_last, const int64_t* rec,
                      int64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* EXL3MOE_H */
