// C-ABI entry points of libexl3moe.so (declarations and reference citations: include/exl3moe.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/exl3moe.h"
#include "exl3_kernels.h"

using namespace exl3;

namespace {

thread_local std::string g_err;

struct Config {
    uint8_t* ram_res = nullptr;
    int32_t* ring = nullptr;
    int ring_cap = 0;
    const int32_t* safe = nullptr;
    int32_t* vict = nullptr;
    int64_t host_stride = 0;
    int64_t slot_stride = 0;                      // bytes between HBM slots (0: the blob size of the call)
    int fused_ensure = 1;                         // ensure inside the layer kernel when the call fits
    int prefill_min_m = 256;
    int pair_max_m = 4;
    int gu_p = 0, dn_p = 0, mr = 0, debug = 0;
    int32_t* log = nullptr;
    int64_t log_cap = 0;
    int32_t* pend = nullptr;                      // copy-engine prefetch: pending plans committed by every ensure
    const int32_t* done_seq = nullptr;
    int n_layers = 0;
    int64_t* vict_addr = nullptr;                 // write-back target of each victim of a call [E]
    int64_t* host_addr = nullptr;                 // record pool of the RAM tier: host record of every key [L * E]
    const int64_t* wbq = nullptr;                 // the step's free records for write-backs [wbq_cap]
    int32_t* wbq_state = nullptr;                 // [0] taken, [1 + i] key written into wbq[i], [1 + cap] dropped
    int wbq_cap = 0;
    int32_t* vr_meta = nullptr;                   // victim ring: [4 + 2K] search position, claims, drops, K, keys, seqs
    int32_t* vr_sel = nullptr;                    // ring slot of each victim of a call [E]
    uint8_t* vr_buf = nullptr;                    // K ring slots in device memory
    int64_t vr_bytes = 0;
    int vr_K = 0;
};
Config g_cfg;

// Copy-engine prefetch worker (reference PfWorker a8:1047-1090): a host thread that polls the plans the plan-mode
// ensure publishes in pinned host memory and, per new plan, copies each claimed expert from its host record into its
// slot on the worker's stream, then copies the plan's sequence number into done_seq[layer] on the same stream (after
// the data). The device commits a plan in the first ensure that sees done_seq >= its sequence number.
struct PrefetchWorker {
    std::thread th;
    std::atomic<bool> stop{false};
    int32_t* plans = nullptr;                     // [L][4 + 2E]: seq, n, T, layer, e[E], s[E]
    int L = 0, E = 0, dev = 0;
    std::vector<int64_t> host_base;               // per layer
    int64_t slot_base = 0, sstride = 0, hstride = 0, blob = 0;
    int32_t* done_seq = nullptr;                  // device [L]
    int32_t* seqv = nullptr;                      // pinned host [L][2]: stable sources of the done_seq copies
    hipStream_t s = nullptr;
    std::vector<int> last_seq;
    std::atomic<int64_t> n_plans{0}, n_copies{0};
    hipError_t err = hipSuccess;

    void run() {
        (void)hipSetDevice(dev);
        const int stride = 4 + 2 * E;
        while (!stop.load(std::memory_order_relaxed)) {
            bool any = false;
            for (int li = 0; li < L; ++li) {
                int32_t* pl = plans + (size_t)li * stride;
                const int seq = __atomic_load_n(pl, __ATOMIC_ACQUIRE);
                if (seq == last_seq[li]) continue;
                any = true;
                const int n = __atomic_load_n(pl + 1, __ATOMIC_ACQUIRE);
                for (int i = 0; i < n && err == hipSuccess; ++i) {
                    const int e = pl[4 + i], sl = pl[4 + E + i];
                    err = hipMemcpyAsync((void*)(slot_base + (int64_t)sl * sstride),
                                         (const void*)(host_base[li] + (int64_t)e * hstride), (size_t)blob,
                                         hipMemcpyHostToDevice, s);
                }
                // one plan per layer is in flight at a time (the plan-mode ensure skips a pending layer), so the two
                // parity slots keep the source of the previous copy intact
                int32_t* sv = seqv + li * 2 + (seq & 1);
                *sv = seq;
                if (err == hipSuccess) err = hipMemcpyAsync(done_seq + li, sv, 4, hipMemcpyHostToDevice, s);
                last_seq[li] = seq;
                n_plans++;
                n_copies += n;
            }
            if (!any) std::this_thread::yield();
        }
        const hipError_t e = hipStreamSynchronize(s);
        if (err == hipSuccess) err = e;
    }
};
std::unique_ptr<PrefetchWorker> g_pfw;
std::mutex g_pfw_mu;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(EXL3_EHIP, "%s: %s", what, hipGetErrorString(e));
}

int check_geometry(int H, int I, int K, int E) {
    if (H <= 0 || I <= 0 || H % 128 || I % 128) return fail(EXL3_EINVAL, "moe: H (%d) and I (%d) must be multiples of 128", H, I);
    if (K < 2 || K > 4) return fail(EXL3_EUNSUPPORTED, "moe: K=%d not supported (K in 2..4)", K);
    if (E <= 0 || E > kMaxExperts) return fail(EXL3_EINVAL, "moe: n_experts=%d must be in 1..%d", E, kMaxExperts);
    if (H > 64 * 128 || I > kMaxI) return fail(EXL3_EUNSUPPORTED, "moe: H up to 8192, I up to %d (got %d, %d)", kMaxI, H, I);
    return EXL3_OK;
}

}  // namespace

extern "C" {

const char* exl3_last_error(void) { return g_err.c_str(); }

int64_t exl3_blob_bytes(int H, int I, int K) { return blob_geom(H, I, K).blob; }

int exl3_set_tier(uint8_t* ram_res, int32_t* miss_ring, int64_t ring_numel, const int32_t* safe) {
    if (!ram_res) {
        g_cfg.ram_res = nullptr;
        g_cfg.ring = nullptr;
        g_cfg.ring_cap = 0;
        g_cfg.safe = nullptr;
        return EXL3_OK;
    }
    if (!miss_ring || ring_numel < 2 || !safe) return fail(EXL3_EINVAL, "moe_set_tier: ring [1 + cap] and safe [L] required");
    // entry c sits at 1 + (c mod 2^32) % cap: with a power-of-two cap the position is continuous across the 2^32 wrap
    // of the count (any other cap maps counts on either side of the wrap to the same entry)
    const int64_t cap = ring_numel - 1;
    if (cap > INT32_MAX || (cap & (cap - 1)))
        return fail(EXL3_EINVAL, "moe_set_tier: ring capacity %lld must be a power of two <= 2^30", (long long)cap);
    g_cfg.ram_res = ram_res;
    g_cfg.ring = miss_ring;
    g_cfg.ring_cap = (int)(ring_numel - 1);
    g_cfg.safe = safe;
    return EXL3_OK;
}

int exl3_set_victims(int32_t* vict) {
    g_cfg.vict = vict;
    return EXL3_OK;
}

int exl3_set_victim_addrs(int64_t* vict_addr) {
    g_cfg.vict_addr = vict_addr;
    return EXL3_OK;
}

int exl3_set_victim_ring(int32_t* meta, int32_t* sel, void* buf, int64_t buf_bytes, int64_t K) {
    if (!meta) {
        g_cfg.vr_meta = nullptr;
        g_cfg.vr_sel = nullptr;
        g_cfg.vr_buf = nullptr;
        g_cfg.vr_bytes = 0;
        g_cfg.vr_K = 0;
        return EXL3_OK;
    }
    if (!sel || !buf || K <= 0 || K > kVictimRingMax || buf_bytes <= 0)
        return fail(EXL3_EINVAL, "set_victim_ring: K=%lld (1..%d) with meta, sel and a buffer", (long long)K,
                    kVictimRingMax);
    g_cfg.vr_meta = meta;
    g_cfg.vr_sel = sel;
    g_cfg.vr_buf = (uint8_t*)buf;
    g_cfg.vr_bytes = buf_bytes;
    g_cfg.vr_K = (int)K;
    return EXL3_OK;
}

int exl3_set_record_pool(int64_t* host_addr, const int64_t* wbq, int32_t* wbq_state, int64_t wbq_cap) {
    if (!host_addr) {
        g_cfg.host_addr = nullptr;
        g_cfg.wbq = nullptr;
        g_cfg.wbq_state = nullptr;
        g_cfg.wbq_cap = 0;
        return EXL3_OK;
    }
    if (!wbq || !wbq_state || wbq_cap <= 0 || wbq_cap > (1 << 20))
        return fail(EXL3_EINVAL, "set_record_pool: queue [cap] and state [2 + cap] required (cap=%lld)",
                    (long long)wbq_cap);
    g_cfg.host_addr = host_addr;
    g_cfg.wbq = wbq;
    g_cfg.wbq_state = wbq_state;
    g_cfg.wbq_cap = (int)wbq_cap;
    return EXL3_OK;
}

int exl3_set_slot_stride(int64_t stride) {
    if (stride < 0 || stride % 16) return fail(EXL3_EINVAL, "moe_set_slot_stride: stride must be a non-negative multiple of 16");
    g_cfg.slot_stride = stride;
    return EXL3_OK;
}

int exl3_set_fused_ensure(int64_t enable) {
    g_cfg.fused_ensure = enable != 0;
    return EXL3_OK;
}

int exl3_set_host_stride(int64_t stride) {
    if (stride < 0 || stride % 16) return fail(EXL3_EINVAL, "moe_set_host_stride: stride must be a non-negative multiple of 16");
    g_cfg.host_stride = stride;
    return EXL3_OK;
}

int exl3_set_prefill_min_m(int64_t m) {
    g_cfg.prefill_min_m = (int)std::max<int64_t>(1, m);
    return EXL3_OK;
}

int exl3_set_pair_max_m(int64_t m) {
    g_cfg.pair_max_m = (int)std::max<int64_t>(0, m);
    return EXL3_OK;
}

int exl3_set_splits(int64_t gu_p, int64_t dn_p) {
    g_cfg.gu_p = (int)gu_p;
    g_cfg.dn_p = (int)dn_p;
    return EXL3_OK;
}

int exl3_set_mr(int64_t mr) {
    g_cfg.mr = (int)mr;
    return EXL3_OK;
}

int exl3_set_debug(int64_t v) {
    g_cfg.debug = (int)v;
    return EXL3_OK;
}

int exl3_set_decision_log(int32_t* buf, int64_t cap_words) {
    if (buf && cap_words < 0) return fail(EXL3_EINVAL, "set_decision_log: cap_words=%lld", (long long)cap_words);
    g_cfg.log = buf;
    g_cfg.log_cap = buf ? cap_words : 0;
    return EXL3_OK;
}

// the prefill kernels serve a call from prefill_min_m rows on, and also below it when the call has more picks or rows
// than the fused decode kernel takes (the reference's align path covers pair_max_m < M < prefill_min_m, a8:1277-1314;
// the prefill kernels here are exact from M = 1 on)
static bool exceeds_decode(int M, int topk) { return (int64_t)M * topk > kMaxPairs || M > kMaxRows; }
static bool use_prefill(int M, int topk) { return M >= g_cfg.prefill_min_m || exceeds_decode(M, topk); }

size_t exl3_moe_forward_workspace(int M, int H, int I, int topk, int n_experts) {
    if (M <= 0 || topk <= 0 || H <= 0 || I <= 0) return 0;
    const int E = std::min(std::max(n_experts, 1), kMaxExperts);
    return use_prefill(M, topk) ? prefill_workspace_bytes(M, H, I, topk, E) : decode_workspace_bytes(M * topk, H, I);
}

static int64_t* pair_ptr_area(void* ws, int npairs, int H, int I) {
    (void)npairs;
    (void)H;
    (void)I;
    return (int64_t*)ws;
}

// The decode kernel's cross-workgroup exchange buffer: library-owned, one per device, zeroed when (re)allocated so that
// no word carries a live tag before the kernel writes it. It grows to the largest call seen; growing synchronizes the
// device and cannot happen while the stream is being captured into a graph. A replaced buffer is never freed: a graph
// captured before the growth keeps its address in its kernel arguments and replays into it (the sizes double, so the
// retired buffers together are at most the size of the current one).
struct Exchange {
    uint64_t* p = nullptr;
    size_t words = 0;
    std::vector<uint64_t*> retired;
};
static constexpr int kMaxDevices = 64;
static std::mutex g_exch_mu;
static Exchange g_exch[kMaxDevices];

static int exchange_buffer(size_t words, hipStream_t st, uint64_t** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_EUNSUPPORTED, "device %d >= %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_exch_mu);
    Exchange& x = g_exch[dev];
    if (words <= x.words) {
        *out = x.p;
        return EXL3_OK;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone)
        return fail(EXL3_EUNSUPPORTED, "moe decode: exchange buffer of %zu words needed inside a graph capture (have "
                    "%zu): run one call of this size before capturing", words, x.words);
    const size_t n = std::max(words, std::max((size_t)1 << 16, 2 * x.words));
    uint64_t* p = nullptr;
    if ((e = hipDeviceSynchronize()) != hipSuccess) return hip_fail(e, "exchange buffer: synchronize");
    if ((e = hipMalloc((void**)&p, n * 8)) != hipSuccess) return hip_fail(e, "exchange buffer: hipMalloc");
    if ((e = hipMemset(p, 0, n * 8)) != hipSuccess || (e = hipDeviceSynchronize()) != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(e, "exchange buffer: zero fill");
    }
    if (x.p) x.retired.push_back(x.p);
    x.p = p;
    x.words = n;
    *out = p;
    return EXL3_OK;
}

static int forward_impl(const void* x, int x_dtype, int64_t x_stride, int M, int H, const int32_t* ids, const float* w,
                        int topk, const int64_t* ptrs, int I, int K, int E, void* out, int64_t out_stride, void* ws,
                        size_t ws_bytes, hipStream_t st, const int64_t* fill, int64_t* commit_ptrs, int64_t* commit_fill,
                        const int32_t* fill_list, const int64_t* pair_ptr, const VictimArgs* va = nullptr,
                        int max_victims = 0, const EnsureArgs* fused_ens = nullptr, bool vict_inline = false,
                        uint64_t* xb_given = nullptr) {
    if (!fill && use_prefill(M, topk)) {
        if (H % 256) return fail(EXL3_EUNSUPPORTED, "moe prefill: H %% 256 == 0 required (H=%d)", H);
        if ((int64_t)M * topk > (1 << 28)) return fail(EXL3_EUNSUPPORTED, "moe prefill: %d x %d pairs", M, topk);
        const size_t need = prefill_workspace_bytes(M, H, I, topk, E);
        if (!ws || ws_bytes < need)
            return fail(EXL3_EWORKSPACE, "moe_forward (prefill): workspace %zu < %zu bytes", ws_bytes, need);
        PrefillArgs pa{};
        pa.x = x;
        pa.x_dt = x_dtype;
        pa.x_stride = x_stride;
        pa.ids = ids;
        pa.w = w;
        pa.M = M;
        pa.topk = topk;
        pa.npairs = M * topk;
        pa.ptrs = ptrs;
        pa.out = out;
        pa.out_stride = out_stride;
        pa.g = blob_geom(H, I, K);
        hipError_t e = launch_prefill(pa, E, ws, st);
        return e == hipSuccess ? EXL3_OK : hip_fail(e, "moe prefill launch");
    }
    const int npairs = M * topk;
    if (npairs > kMaxPairs || M > kMaxRows)
        return fail(EXL3_EUNSUPPORTED, "moe_forward: M=%d x topk=%d exceeds the decode kernels (%d pairs, %d rows)", M,
                    topk, kMaxPairs, kMaxRows);
    const size_t need = decode_workspace_bytes(npairs, H, I);
    if (!ws || ws_bytes < need) return fail(EXL3_EWORKSPACE, "moe_forward: workspace %zu < %zu bytes", ws_bytes, need);
    uint64_t* xb = xb_given;                      // the static scratch's exchange words, or the library buffer
    if (!xb) {
        const int rx = exchange_buffer(decode_exchange_words(npairs, H, I), st, &xb);
        if (rx) return rx;
    }
    DecodeArgs a{};
    a.x = x;
    a.x_dt = x_dtype;
    a.x_stride = x_stride;
    a.ids = ids;
    a.w = w;
    a.M = M;
    a.topk = topk;
    a.npairs = npairs;
    a.E = E;
    a.ptrs = ptrs;
    a.pair_ptr = pair_ptr;
    a.fill = fill;
    a.commit_ptrs = commit_ptrs;
    a.commit_fill = commit_fill;
    a.fill_list = fill_list;
    a.xpart = xb;
    a.xy = xb + (size_t)npairs * gu_kslices(H) * 2 * I;
    a.xstart = a.xy + (size_t)npairs * H;
    a.n_gu = decode_gu_workgroups(npairs, H, I);
    a.out = out;
    a.out_stride = out_stride;
    a.g = blob_geom(H, I, K);
    if (va && max_victims > 0) {
        a.va = *va;
        if (vict_inline) {                        // victim write-back by the writers of each miss
            a.vict_inline = 1;
        } else {                                  // victim write-back: the first workgroups of the layer kernel
            a.vict_chunks = (int)((a.g.blob + va->chunk_bytes - 1) / va->chunk_bytes);
            a.n_vict_wg = max_victims * a.vict_chunks;
        }
    }
    if (fused_ens) {                              // the ensure runs as workgroup 0 of the layer kernel
        a.fused = 1;
        a.ens = *fused_ens;
    }
    hipError_t e = launch_moe_layer(K, a, st);
    if (e != hipSuccess) return hip_fail(e, "moe layer launch");
    return EXL3_OK;
}

int exl3_moe_forward(const void* x, int x_dtype, int64_t x_stride, int M, int H, const int32_t* topk_ids,
                     const float* topk_w, int topk, const int64_t* ptrs, int I, int K, int n_experts, void* out,
                     int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream) {
    if (M < 0 || topk <= 0) return fail(EXL3_EINVAL, "moe_forward: M=%d topk=%d", M, topk);
    if (x_dtype < EXL3_DT_F16 || x_dtype > EXL3_DT_F32) return fail(EXL3_EINVAL, "moe_forward: x dtype");
    int r = check_geometry(H, I, K, n_experts);
    if (r) return r;
    if (M == 0) return EXL3_OK;
    if (!x || !topk_ids || !topk_w || !ptrs || !out) return fail(EXL3_EINVAL, "moe_forward: null pointer");
    return forward_impl(x, x_dtype, x_stride, M, H, topk_ids, topk_w, topk, ptrs, I, K, n_experts, out, out_stride,
                        workspace, workspace_bytes, (hipStream_t)stream, nullptr, nullptr, nullptr, nullptr, nullptr);
}

int exl3_moe_prefetch(const int32_t* ids, int n_ids, int64_t* ptrs_all, int layer, int32_t* slot_of,
                      int32_t* slot_key, int32_t* slot_last, int32_t* tick, int n_slots, const int64_t* host_base,
                      int64_t slot_base, int32_t* pf_list, int32_t* pf_slot, int max_fill, int n_experts, int64_t blob,
                      void* stream) {
    if (g_cfg.host_addr)                          // its copies address fixed host records
        return fail(EXL3_EUNSUPPORTED, "moe_prefetch: not with the RAM tier's record pool");
    if (g_cfg.vr_meta)                            // its victims would bypass the ring
        return fail(EXL3_EUNSUPPORTED, "moe_prefetch: not with the victim ring");
    const int E = n_experts;
    if (n_ids < 0 || layer < 0 || max_fill < 0 || blob <= 0)
        return fail(EXL3_EINVAL, "moe_prefetch: n_ids=%d layer=%d max_fill=%d blob=%lld", n_ids, layer, max_fill,
                    (long long)blob);
    if (E <= 0 || E > kMaxExperts) return fail(EXL3_EINVAL, "moe_prefetch: n_experts=%d must be in 1..%d", E, kMaxExperts);
    if (n_slots <= 0 || n_ids == 0) return EXL3_OK;            // as the reference: nothing to claim
    if (!ids || !ptrs_all || !slot_of || !slot_key || !slot_last || !tick || !host_base || !pf_list || !pf_slot)
        return fail(EXL3_EINVAL, "moe_prefetch: null argument");
    const int64_t sstride = g_cfg.slot_stride ? g_cfg.slot_stride : blob;
    const int64_t hstride = g_cfg.host_stride ? g_cfg.host_stride : sstride;
    if (sstride < blob) return fail(EXL3_EINVAL, "moe_prefetch: slot stride %lld < blob %lld", (long long)sstride,
                                    (long long)blob);
    if (blob % 16 || sstride % 16 || hstride % 16 || slot_base % 16)
        return fail(EXL3_EUNSUPPORTED, "moe_prefetch: blob, strides and slot base must be multiples of 16 bytes");
    EnsureArgs ea{};
    ea.ids = const_cast<int32_t*>(ids);           // never written: prefetch mode has no tier mask
    ea.P = n_ids;
    ea.layer = layer;
    ea.E = E;
    ea.S = n_slots;
    ea.ptrs_all = ptrs_all;
    ea.slot_of = slot_of;
    ea.slot_key = slot_key;
    ea.slot_last = slot_last;
    ea.tick = tick;
    ea.host_base = host_base;
    ea.slot_base = slot_base;
    ea.blob = sstride;
    ea.hstride = hstride;
    ea.fill_list = pf_list;
    ea.max_fill = std::min(max_fill, E);
    ea.log = g_cfg.log;
    ea.log_cap = g_cfg.log_cap;
    ea.pf_slot = pf_slot;
    hipError_t e = launch_prefetch(ea, sstride, blob, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return fail(EXL3_EUNSUPPORTED, "moe_prefetch: ensure state does not fit in LDS");
    if (e != hipSuccess) return hip_fail(e, "prefetch launch");
    return EXL3_OK;
}

int exl3_set_prefetch_commit(int32_t* pend, const int32_t* done_seq, int n_layers) {
    if (n_layers < 0 || (n_layers > 0 && (!pend || !done_seq)))
        return fail(EXL3_EINVAL, "set_prefetch_commit: n_layers=%d with null tables", n_layers);
    g_cfg.pend = pend;
    g_cfg.done_seq = done_seq;
    g_cfg.n_layers = n_layers;
    return EXL3_OK;
}

int exl3_moe_prefetch_plan(const int32_t* ids, int n_ids, int64_t* ptrs_all, int layer, int32_t* slot_of,
                           int32_t* slot_key, int32_t* slot_last, int32_t* tick, int n_slots,
                           const int64_t* host_base, int64_t slot_base, int32_t* pf_list, int32_t* pf_slot,
                           int32_t* plans, int32_t* plan_seq, int32_t* pend, const int32_t* done_seq, int n_layers,
                           int max_fill, int n_experts, int64_t blob, void* stream) {
    if (g_cfg.host_addr)                          // its copies address fixed host records
        return fail(EXL3_EUNSUPPORTED, "moe_prefetch_plan: not with the RAM tier's record pool");
    if (g_cfg.vr_meta)                            // its victims would bypass the ring
        return fail(EXL3_EUNSUPPORTED, "moe_prefetch_plan: not with the victim ring");
    const int E = n_experts;
    if (n_ids < 0 || layer < 0 || max_fill < 0 || blob <= 0 || n_layers <= layer)
        return fail(EXL3_EINVAL, "moe_prefetch_plan: n_ids=%d layer=%d n_layers=%d max_fill=%d", n_ids, layer,
                    n_layers, max_fill);
    if (E <= 0 || E > kMaxExperts)
        return fail(EXL3_EINVAL, "moe_prefetch_plan: n_experts=%d must be in 1..%d", E, kMaxExperts);
    if (n_slots <= 0 || n_ids == 0) return EXL3_OK;
    if (!ids || !ptrs_all || !slot_of || !slot_key || !slot_last || !tick || !host_base || !pf_list || !pf_slot ||
        !plans || !plan_seq || !pend || !done_seq)
        return fail(EXL3_EINVAL, "moe_prefetch_plan: null argument");
    const int64_t sstride = g_cfg.slot_stride ? g_cfg.slot_stride : blob;
    if (sstride < blob) return fail(EXL3_EINVAL, "moe_prefetch_plan: slot stride < blob");
    EnsureArgs ea{};
    ea.ids = const_cast<int32_t*>(ids);           // never written: no tier mask in plan mode
    ea.P = n_ids;
    ea.layer = layer;
    ea.E = E;
    ea.S = n_slots;
    ea.ptrs_all = ptrs_all;
    ea.slot_of = slot_of;
    ea.slot_key = slot_key;
    ea.slot_last = slot_last;
    ea.tick = tick;
    ea.host_base = host_base;
    ea.slot_base = slot_base;
    ea.blob = sstride;
    ea.hstride = g_cfg.host_stride ? g_cfg.host_stride : sstride;
    ea.fill_list = pf_list;
    ea.max_fill = std::min(std::min(max_fill, E), kPlanMax);
    ea.log = g_cfg.log;
    ea.log_cap = g_cfg.log_cap;
    ea.pf_slot = pf_slot;
    ea.host_plan = plans + (size_t)layer * (4 + 2 * E);
    ea.plan_seq = plan_seq;
    ea.pend = pend;
    ea.done_seq = done_seq;
    ea.n_layers = n_layers;
    const hipError_t e = launch_ensure(ea, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return fail(EXL3_EUNSUPPORTED, "moe_prefetch_plan: ensure state does not fit in LDS");
    if (e != hipSuccess) return hip_fail(e, "prefetch plan launch");
    return EXL3_OK;
}

int exl3_prefetch_worker_start(int32_t* plans, const int64_t* host_base_host, int64_t slot_base, int64_t blob,
                               int32_t* done_seq, int32_t* seq_host, int n_layers, int n_experts, void* stream) {
    if (g_cfg.host_addr)                          // its copies address fixed host records
        return fail(EXL3_EUNSUPPORTED, "prefetch_worker_start: not with the RAM tier's record pool");
    if (g_cfg.vr_meta)                            // its victims would bypass the ring
        return fail(EXL3_EUNSUPPORTED, "prefetch_worker_start: not with the victim ring");
    std::lock_guard<std::mutex> lk(g_pfw_mu);
    if (g_pfw) return fail(EXL3_EINVAL, "prefetch worker already running");
    if (!plans || !host_base_host || !done_seq || !seq_host || n_layers <= 0 || n_experts <= 0 || blob <= 0)
        return fail(EXL3_EINVAL, "prefetch_worker_start: bad arguments");
    auto w = std::make_unique<PrefetchWorker>();
    hipError_t e = hipGetDevice(&w->dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    w->plans = plans;
    w->L = n_layers;
    w->E = n_experts;
    w->host_base.assign(host_base_host, host_base_host + n_layers);
    w->slot_base = slot_base;
    w->blob = blob;
    w->sstride = g_cfg.slot_stride ? g_cfg.slot_stride : blob;
    w->hstride = g_cfg.host_stride ? g_cfg.host_stride : w->sstride;
    w->done_seq = done_seq;
    w->seqv = seq_host;
    w->s = (hipStream_t)stream;
    w->last_seq.resize(n_layers);
    for (int li = 0; li < n_layers; ++li)
        w->last_seq[li] = __atomic_load_n(plans + (size_t)li * (4 + 2 * n_experts), __ATOMIC_ACQUIRE);
    PrefetchWorker* raw = w.get();
    w->th = std::thread([raw] { raw->run(); });
    g_pfw = std::move(w);
    return EXL3_OK;
}

int exl3_prefetch_worker_stop(int64_t* counts) {
    std::lock_guard<std::mutex> lk(g_pfw_mu);
    if (counts) counts[0] = counts[1] = 0;
    if (!g_pfw) return EXL3_OK;
    g_pfw->stop = true;
    g_pfw->th.join();
    if (counts) {
        counts[0] = g_pfw->n_plans.load();
        counts[1] = g_pfw->n_copies.load();
    }
    const hipError_t e = g_pfw->err;
    g_pfw.reset();
    if (e != hipSuccess) return hip_fail(e, "prefetch worker copies");
    return EXL3_OK;
}

}  // extern "C"

// moe_forward_cached with the decode scratch either from the caller's workspace and the library's exchange buffer
// (xb == nullptr) or both from the static scratch (xb given: calls that fall back to another path are refused)
static int cached_impl(const void* x, int x_dtype, int64_t x_stride, int M, int H, int32_t* topk_ids, float* topk_w,
                       int topk, int64_t* ptrs_all, int layer, int32_t* slot_of, int32_t* slot_key, int32_t* slot_last,
                       int32_t* tick, int n_slots, const int64_t* host_base, int64_t slot_base, int64_t* fill_all,
                       int32_t* fill_list, int max_fill, int I, int K, int n_experts, void* out, int64_t out_stride,
                       void* workspace, size_t workspace_bytes, void* stream, uint64_t* xb) {
    const int E = n_experts;
    if (M < 0 || topk <= 0 || layer < 0) return fail(EXL3_EINVAL, "moe_forward_cached: M=%d topk=%d layer=%d", M, topk, layer);
    if (x_dtype < EXL3_DT_F16 || x_dtype > EXL3_DT_F32) return fail(EXL3_EINVAL, "moe_forward_cached: x dtype");
    int r = check_geometry(H, I, K, E);
    if (r) return r;
    if (M == 0) return EXL3_OK;
    hipStream_t st = (hipStream_t)stream;
    if (!ptrs_all) return fail(EXL3_EINVAL, "moe_forward_cached: null ptrs_all");
    if (M >= g_cfg.prefill_min_m || n_slots == 0) {
        if (xb) return fail(EXL3_EUNSUPPORTED, "moe_forward_cached_static: M=%d n_slots=%d takes the uncached path, "
                            "which needs a workspace (use exl3_moe_forward_cached)", M, n_slots);
        return exl3_moe_forward(x, x_dtype, x_stride, M, H, topk_ids, topk_w, topk, ptrs_all + (int64_t)layer * E, I, K,
                                E, out, out_stride, workspace, workspace_bytes, stream);
    }
    if (!slot_of || !slot_key || !slot_last || !tick || !host_base || !fill_all || !fill_list)
        return fail(EXL3_EINVAL, "moe_forward_cached: null cache state");
    const BlobGeom g = blob_geom(H, I, K);
    const int P = M * topk;
    if (exceeds_decode(M, topk) && xb)
        return fail(EXL3_EUNSUPPORTED, "moe_forward_cached_static: %d x %d picks take the prefill kernels, which need "
                    "a workspace (use exl3_moe_forward_cached)", M, topk);
    EnsureArgs ea{};
    ea.ids = topk_ids;
    ea.w = topk_w;
    ea.P = P;
    ea.layer = layer;
    ea.E = E;
    ea.S = n_slots;
    ea.ptrs_all = ptrs_all;
    ea.slot_of = slot_of;
    ea.slot_key = slot_key;
    ea.slot_last = slot_last;
    ea.tick = tick;
    ea.host_base = host_base;
    ea.slot_base = slot_base;
    ea.blob = g_cfg.slot_stride ? g_cfg.slot_stride : g.blob;        // slot stride (slot s at slot_base + s * stride)
    if (ea.blob < g.blob) return fail(EXL3_EINVAL, "moe_forward_cached: slot stride %lld < blob %lld",
                                      (long long)ea.blob, (long long)g.blob);
    ea.hstride = g_cfg.host_stride ? g_cfg.host_stride : ea.blob;
    ea.fill_all = fill_all;
    ea.fill_list = fill_list;
    ea.max_fill = std::min(max_fill, E);
    ea.ram_res = g_cfg.ram_res;
    ea.ring = g_cfg.ring;
    ea.ring_cap = g_cfg.ring_cap;
    ea.safe = g_cfg.safe;
    ea.vict = g_cfg.vict;
    ea.vict_addr = g_cfg.vict ? g_cfg.vict_addr : nullptr;
    ea.host_addr = g_cfg.host_addr;
    ea.wbq = g_cfg.wbq;
    ea.wbq_state = g_cfg.wbq_state;
    ea.wbq_cap = g_cfg.wbq_cap;
    if (ea.host_addr && (!ea.vict || !ea.vict_addr))
        return fail(EXL3_EINVAL, "moe_forward_cached: the record pool needs the victim list and its addresses "
                                 "(exl3_set_victims, exl3_set_victim_addrs)");
    if (g_cfg.vr_meta && ea.vict) {              // victim ring: write-backs into ring slots of the slot stride
        if (!ea.vict_addr)
            return fail(EXL3_EINVAL, "moe_forward_cached: the victim ring needs the victim addresses "
                                     "(exl3_set_victim_addrs)");
        if ((int64_t)g_cfg.vr_K * ea.blob > g_cfg.vr_bytes)
            return fail(EXL3_EINVAL, "moe_forward_cached: victim ring of %lld bytes < %d slots of %lld",
                        (long long)g_cfg.vr_bytes, g_cfg.vr_K, (long long)ea.blob);
        ea.vr_meta = g_cfg.vr_meta;
        ea.vr_sel = g_cfg.vr_sel;
        ea.vr_base = (int64_t)g_cfg.vr_buf;
        ea.vr_K = g_cfg.vr_K;
    }
    // with the ring the host flags a victim RAM-resident once its drain has landed, never the device
    uint8_t* vict_res = ea.vr_meta ? nullptr : g_cfg.ram_res;
    ea.log = g_cfg.log;
    ea.log_cap = g_cfg.log_cap;
    if (exceeds_decode(M, topk)) {
        // more picks than the decode kernel takes: one ensure over all of them, victim write-back, fill copies and
        // the commit, then the prefill kernels over the committed table (the caller's ids and w carry the tier mask)
        if (H % 256) return fail(EXL3_EUNSUPPORTED, "moe_forward_cached: %d picks need the prefill kernels (H %% 256)", P);
        const size_t need = prefill_workspace_bytes(M, H, I, topk, E);
        if (!workspace || workspace_bytes < need)
            return fail(EXL3_EWORKSPACE, "moe_forward_cached: workspace %zu < %zu bytes", workspace_bytes, need);
        ea.pend = g_cfg.n_layers > 0 ? g_cfg.pend : nullptr;   // commit finished copy-engine plans first
        ea.done_seq = g_cfg.done_seq;
        ea.n_layers = g_cfg.n_layers;
        hipError_t e = launch_ensure(ea, st);
        if (e == hipErrorInvalidValue) return fail(EXL3_EUNSUPPORTED, "moe_forward_cached: ensure state does not fit in LDS");
        if (e != hipSuccess) return hip_fail(e, "ensure launch");
        e = launch_cached_fills(ea, g.blob, std::min(std::min(ea.max_fill, E), P), vict_res, st);
        if (e != hipSuccess) return hip_fail(e, "cached fills launch");
        return forward_impl(x, x_dtype, x_stride, M, H, topk_ids, topk_w, topk, ptrs_all + (int64_t)layer * E, I, K, E,
                            out, out_stride, workspace, workspace_bytes, st, nullptr, nullptr, nullptr, nullptr, nullptr);
    }
    const size_t need = decode_workspace_bytes(P, H, I);
    if (!workspace || workspace_bytes < need)
        return fail(EXL3_EWORKSPACE, "moe_forward_cached: workspace %zu < %zu bytes", workspace_bytes, need);
    // the ensure inside the layer kernel needs one thread per expert, one lane per pick and the slot stamps in
    // registers; K = 4 kernels run one workgroup per CU, too few to let the victim workgroups wait for it
    ea.pend = g_cfg.n_layers > 0 ? g_cfg.pend : nullptr;       // commit finished copy-engine plans first
    ea.done_seq = g_cfg.done_seq;
    ea.n_layers = g_cfg.n_layers;
    // the ensure inside the layer kernel has no plan commit: calls with plans in use run the ensure kernel
    const bool fused = g_cfg.fused_ensure && E <= kEnsMaxE && P <= kEnsMaxP && n_slots <= kEnsMaxE * kEnsRegSlots &&
                       K <= 3 && !ea.pend;
    if (!fused) {
        ea.pair_ptr = pair_ptr_area(workspace, P, H, I);
        hipError_t e = launch_ensure(ea, st);
        if (e != hipSuccess) return hip_fail(e, "ensure launch");
    }
    // with the ensure inside the layer kernel and slots at the blob size (one layout for victim and miss), the writers
    // of each miss copy the victim's old bytes before overwriting them: no victim workgroups in the launch
    const bool vict_inline = fused && g_cfg.vict && ea.blob == g.blob;
    if (vict_inline) ea.pair_own = (int32_t*)pair_ptr_area(workspace, P, H, I);
    VictimArgs va{};
    int mv = 0;
    if (g_cfg.vict) {
        va.vict = g_cfg.vict;
        va.host_base = host_base;
        va.slot_base = slot_base;
        va.blob = ea.blob;                        // a victim may be an expert of another bitrate: copy the slot
        va.hstride = ea.hstride;
        va.E = E;
        va.ram_res = vict_res;
        va.chunk_bytes = kVictimChunkBytes;
        va.vaddr = ea.vict_addr;
        mv = std::min(std::min(ea.max_fill, E), P);
    }
    int64_t* pl = ptrs_all + (int64_t)layer * E;
    int64_t* fl = fill_all + (int64_t)layer * E;
    return forward_impl(x, x_dtype, x_stride, M, H, topk_ids, topk_w, topk, pl, I, K, E, out, out_stride, workspace,
                        workspace_bytes, st, fl, pl, fl, fill_list, ea.pair_ptr, &va, mv, fused ? &ea : nullptr,
                        vict_inline, xb);
}

// ---- the entry point that allocates nothing ------------------------------------------------------------------------
// Decode scratch in static device memory: a pointer area sized for the largest call (the blob pointer or the
// first-pick flag of every pick, kMaxPairs entries), then the exchange words. Both start at fixed offsets whatever
// the call's size: the exchange words are validated only by their tag (call epoch + 1 in the high half), so they
// must never share an address with pointers or flags of an earlier call, whose high halves could pass as a tag.
// Every device holds its own copy for the life of the process; its address on a device is looked up once
// (hipGetSymbolAddress, that device current) and kept: host code never uses the array's name as an address.
constexpr size_t kStaticScratchBytes = EXL3_STATIC_SCRATCH_BYTES;
constexpr size_t kStaticPtrBytes = align256((size_t)kMaxPairs * 8);      // offset of the exchange words
static_assert(decode_workspace_bytes(kMaxPairs, 0, 0) <= kStaticPtrBytes,
              "the pointer area of the static scratch must hold the workspace of the largest decode call");
static_assert(kStaticPtrBytes % 256 == 0 && kStaticPtrBytes < kStaticScratchBytes, "static scratch layout");
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_ptr[kMaxDevices];

__global__ void zero_fill_kernel(uint4* p, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// this device's scratch, set up on first use: its address, then one clear by a kernel on `st` (no memset node if the
// first call is being captured; the exchange words only need to carry no live tag, which zero never is)
static int static_scratch(hipStream_t st, uint8_t** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(EXL3_EUNSUPPORTED, "device %d >= %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e, "static scratch: hipGetSymbolAddress");
        hipLaunchKernelGGL(zero_fill_kernel, dim3(256), dim3(256), 0, st, (uint4*)p, kStaticScratchBytes / 16);
        if ((e = hipGetLastError()) != hipSuccess) return hip_fail(e, "static scratch: clear");
        g_scratch_ptr[dev] = (uint8_t*)p;
    }
    *out = g_scratch_ptr[dev];
    return EXL3_OK;
}

extern "C" {

int exl3_moe_forward_cached(const void* x, int x_dtype, int64_t x_stride, int M, int H, int32_t* topk_ids,
                            float* topk_w, int topk, int64_t* ptrs_all, int layer, int32_t* slot_of, int32_t* slot_key,
                            int32_t* slot_last, int32_t* tick, int n_slots, const int64_t* host_base,
                            int64_t slot_base, int64_t* fill_all, int32_t* fill_list, int max_fill, int I, int K,
                            int n_experts, void* out, int64_t out_stride, void* workspace, size_t workspace_bytes,
                            void* stream) {
    return cached_impl(x, x_dtype, x_stride, M, H, topk_ids, topk_w, topk, ptrs_all, layer, slot_of, slot_key,
                       slot_last, tick, n_slots, host_base, slot_base, fill_all, fill_list, max_fill, I, K, n_experts,
                       out, out_stride, workspace, workspace_bytes, stream, nullptr);
}

int exl3_moe_forward_cached_static(const void* x, int x_dtype, int64_t x_stride, int M, int H, int32_t* topk_ids,
                                   float* topk_w, int topk, int64_t* ptrs_all, int layer, int32_t* slot_of,
                                   int32_t* slot_key, int32_t* slot_last, int32_t* tick, int n_slots,
                                   const int64_t* host_base, int64_t slot_base, int64_t* fill_all, int32_t* fill_list,
                                   int max_fill, int I, int K, int n_experts, void* out, int64_t out_stride,
                                   void* stream) {
    if (M < 0 || topk <= 0 || H <= 0 || I <= 0) return fail(EXL3_EINVAL, "moe_forward_cached_static: M=%d topk=%d", M, topk);
    if (M == 0)                                   // nothing to do; validated like any call, no scratch needed
        return cached_impl(x, x_dtype, x_stride, 0, H, topk_ids, topk_w, topk, ptrs_all, layer, slot_of, slot_key,
                           slot_last, tick, n_slots, host_base, slot_base, fill_all, fill_list, max_fill, I, K,
                           n_experts, out, out_stride, nullptr, 0, stream, nullptr);
    if ((int64_t)M * topk > kMaxPairs) return fail(EXL3_EUNSUPPORTED, "moe_forward_cached_static: %d picks > %d", M * topk, kMaxPairs);
    const size_t ws = decode_workspace_bytes(M * topk, H, I);
    if (ws > kStaticPtrBytes) return fail(EXL3_EUNSUPPORTED, "moe_forward_cached_static: pointer area");
    const size_t need = kStaticPtrBytes + decode_exchange_words(M * topk, H, I) * 8;
    if (need > kStaticScratchBytes)
        return fail(EXL3_EUNSUPPORTED, "moe_forward_cached_static: the call needs %zu bytes of scratch, the static "
                    "scratch holds %zu (fewer rows, or exl3_moe_forward_cached)", need, kStaticScratchBytes);
    uint8_t* sp = nullptr;
    const int r = static_scratch((hipStream_t)stream, &sp);
    if (r) return r;
    return cached_impl(x, x_dtype, x_stride, M, H, topk_ids, topk_w, topk, ptrs_all, layer, slot_of, slot_key,
                       slot_last, tick, n_slots, host_base, slot_base, fill_all, fill_list, max_fill, I, K, n_experts,
                       out, out_stride, sp, ws, stream, (uint64_t*)(sp + kStaticPtrBytes));
}

size_t exl3_moe_align_workspace(int M, int topk, int n_experts) {
    if (M <= 0 || topk <= 0 || n_experts <= 0) return 0;
    return align_scratch_bytes(M * topk, std::min(n_experts, kMaxExperts));
}

int exl3_moe_align(const int32_t* topk_ids, const float* topk_w, int M, int topk, int n_experts, int pad, int32_t* ib,
                   float* fb, void* workspace, size_t workspace_bytes, void* stream) {
    if (M < 0 || topk <= 0 || n_experts <= 0 || n_experts > kMaxExperts || pad <= 0)
        return fail(EXL3_EINVAL, "moe_align: M=%d topk=%d n_experts=%d pad=%d", M, topk, n_experts, pad);
    const int npairs = M * topk, A = std::min(npairs, n_experts);
    if (npairs > 0 && (!topk_ids || !topk_w)) return fail(EXL3_EINVAL, "moe_align: null ids / w");
    if (!ib || (npairs > 0 && !fb)) return fail(EXL3_EINVAL, "moe_align: null outputs");
    const size_t need = exl3_moe_align_workspace(M, topk, n_experts);
    if (need && (!workspace || workspace_bytes < need))
        return fail(EXL3_EWORKSPACE, "moe_align: workspace %zu < %zu bytes", workspace_bytes, need);
    AlignOut o{};
    o.act_expert = ib;
    o.act_start = ib + A;
    o.act_cnt = ib + 2 * A;
    o.act_pstart = ib + 3 * A;
    o.n_act = ib + 4 * A;
    o.pair_tok = ib + 4 * A + 1;
    o.pair_of = o.pair_tok + npairs;
    o.pair_w = fb;
    o.pair_exp = nullptr;
    hipError_t e = launch_align(topk_ids, topk_w, npairs, topk, n_experts, pad, (int*)workspace, o, (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "moe_align launch");
}

int exl3_scatter_flags(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n, void* stream) {
    if (n < 0 || n_flags < 0 || n > (int64_t)1 << 31) return fail(EXL3_EINVAL, "scatter_flags: n=%lld", (long long)n);
    if (n == 0) return EXL3_OK;
    if (!flags || !packed) return fail(EXL3_EINVAL, "scatter_flags: null pointer");
    hipError_t e = launch_scatter_flags(flags, n_flags, packed, n, (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "scatter_flags");
}

static int tier_exchange_impl(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n_diff,
                              const int32_t* ring, int64_t ring_cap, int64_t ring_from, int32_t* ring_mirror,
                              const void* const* src, void* const* dst, const int64_t* nbytes, int n_copies,
                              const TierPool& pl, void* stream) {
    if (n_diff < 0 || n_flags < 0 || n_diff > (int64_t)1 << 31 || n_copies < 0 || n_copies > 4)
        return fail(EXL3_EINVAL, "tier_exchange: n_diff=%lld n_copies=%d", (long long)n_diff, n_copies);
    if (n_diff && (!flags || !packed)) return fail(EXL3_EINVAL, "tier_exchange: null flags / diff");
    // ring_from is a ring count (modulo 2^32, as the device keeps it): 0 <= ring_from < 2^32; the capacity is a power
    // of two, as exl3_set_tier requires, so that positions stay continuous across the wrap of the count
    if (ring && (!ring_mirror || ring_cap <= 0 || ring_cap > INT32_MAX || (ring_cap & (ring_cap - 1)) || ring_from < 0 ||
                 ring_from > (int64_t)UINT32_MAX))
        return fail(EXL3_EINVAL, "tier_exchange: ring cap=%lld (a power of two) from=%lld", (long long)ring_cap,
                    (long long)ring_from);
    const TierRing rg{ring, ring_cap, ring_from, ring_mirror};
    TierCopies cp{};
    for (int k = 0; k < n_copies; ++k) {
        if (!src || !dst || !nbytes || nbytes[k] < 0 || (nbytes[k] && (!src[k] || !dst[k])))
            return fail(EXL3_EINVAL, "tier_exchange: copy %d", k);
        if (((uintptr_t)src[k] | (uintptr_t)dst[k]) & 15)
            return fail(EXL3_EINVAL, "tier_exchange: copy %d not 16-byte aligned", k);
        cp.c[cp.n++] = TierCopy{(const uint8_t*)src[k], (uint8_t*)dst[k], nbytes[k]};
    }
    hipError_t e = launch_tier_exchange(flags, n_flags, packed, n_diff, rg, cp, pl, (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "tier_exchange");
}

int exl3_tier_exchange(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n_diff, const int32_t* ring,
                       int64_t ring_cap, int64_t ring_from, int32_t* ring_mirror, const void* const* src,
                       void* const* dst, const int64_t* nbytes, int n_copies, void* stream) {
    return tier_exchange_impl(flags, n_flags, packed, n_diff, ring, ring_cap, ring_from, ring_mirror, src, dst, nbytes,
                              n_copies, TierPool{}, stream);
}

int exl3_tier_exchange_pool(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n_diff,
                            const int32_t* ring, int64_t ring_cap, int64_t ring_from, int32_t* ring_mirror,
                            const void* const* src, void* const* dst, const int64_t* nbytes, int n_copies,
                            const int64_t* upd, int64_t n_upd, int64_t* host_addr, int64_t* ptrs_all,
                            const int32_t* slot_of, const int64_t* next, int64_t* wbq, int32_t* wbq_state,
                            int32_t* wbq_mirror, int64_t wbq_cap, void* stream) {
    if (n_upd < 0 || (n_upd && (!upd || !host_addr || !ptrs_all || !slot_of)))
        return fail(EXL3_EINVAL, "tier_exchange_pool: %lld address updates with null tables", (long long)n_upd);
    if (wbq && (!next || !wbq_state || !wbq_mirror || wbq_cap <= 0 || wbq_cap > (1 << 20)))
        return fail(EXL3_EINVAL, "tier_exchange_pool: queue cap=%lld with null arrays", (long long)wbq_cap);
    TierPool pl{};
    pl.upd = upd;
    pl.n_upd = n_upd;
    pl.host_addr = host_addr;
    pl.ptrs_all = ptrs_all;
    pl.slot_of = slot_of;
    pl.next = next;
    pl.wbq = wbq;
    pl.state = wbq_state;
    pl.mirror = wbq_mirror;
    pl.cap = wbq ? (int)wbq_cap : 0;
    return tier_exchange_impl(flags, n_flags, packed, n_diff, ring, ring_cap, ring_from, ring_mirror, src, dst, nbytes,
                              n_copies, pl, stream);
}

int exl3_device_status(int32_t* flags4, void* stream) {
    if (!flags4) return fail(EXL3_EINVAL, "device_status: null output");
    hipError_t e = (hipError_t)read_status(flags4, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "device_status");
    e = hipStreamSynchronize((hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "device_status sync");
}

int exl3_set_status_mirror(int32_t* host_word) {
    const hipError_t e = set_status_mirror((int*)host_word);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "set_status_mirror");
}

int exl3_device_status_address(void** dev_ptr) {
    if (!dev_ptr) return fail(EXL3_EINVAL, "device_status_address: null output");
    const hipError_t e = status_address(dev_ptr);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "device_status_address");
}

int exl3_dequant(const uint32_t* trellis, int k_tiles, int n_tiles, int K, uint16_t* out, void* stream) {
    if (K < 2 || K > 4) return fail(EXL3_EUNSUPPORTED, "dequant: K=%d", K);
    if (!trellis || !out || k_tiles <= 0 || n_tiles <= 0) return fail(EXL3_EINVAL, "dequant: bad arguments");
    if ((K & 1) && n_tiles % 4) return fail(EXL3_EINVAL, "dequant: PLANAR4 needs n_tiles %% 4 == 0");
    hipError_t e = launch_dequant(K, trellis, (_Float16*)out, k_tiles, n_tiles, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return EXL3_OK;
}

// ---- the dense EXL3 linear ---------------------------------------------------------------------------------------

// mul1 at K = 2..6; 3inst and mcg at K = 4 and 6 (the reference's set with EXL3_ALL_CODEBOOKS, exl3_ops.sycl:767-773)
int exl3_linear_supported(int K, int cb) {
    if (cb == 2) return K >= 2 && K <= 6 ? 1 : 0;
    if (cb == 0 || cb == 1) return K == 4 || K == 6 ? 1 : 0;
    return 0;
}

size_t exl3_linear_workspace(int M, int k, int n) {
    if (M < 0 || k <= 0 || n <= 0) return 0;
    return linear_workspace_bytes(M, k, n);
}

// this device's status words and the word holding their host mirror's address, looked up once per device
static std::mutex g_lin_status_mu;
static void* g_lin_status[kMaxDevices][2];
static hipError_t linear_status(int** st, int* const** sh) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_lin_status_mu);
    if (!g_lin_status[dev][0]) {
        void* a = nullptr;
        void* b = nullptr;
        if ((e = status_address(&a)) != hipSuccess) return e;
        if ((e = status_host_slot(&b)) != hipSuccess) return e;
        g_lin_status[dev][1] = b;
        g_lin_status[dev][0] = a;
    }
    *st = (int*)g_lin_status[dev][0];
    *sh = (int* const*)g_lin_status[dev][1];
    return hipSuccess;
}

static int linear_dims(const char* what, int M, int k, int n, int S) {
    if (M < 0 || k <= 0 || n <= 0 || S <= 0 || k % 128 || n % 128)
        return fail(EXL3_EINVAL, "%s: M=%d k=%d n=%d S=%d (k, n multiples of 128)", what, M, k, n, S);
    return EXL3_OK;
}

int exl3_linear_small(const void* x, int x_dtype, int64_t x_stride, int M, int k, int n, const void* trellis, int K,
                      int cb, const void* suh, int S, const void* svh, const int32_t* shard_of_nb, void* out,
                      int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream) {
    if (int r = linear_dims("linear_small", M, k, n, S)) return r;
    if (!exl3_linear_supported(K, cb)) return fail(EXL3_EUNSUPPORTED, "linear_small: K=%d cb=%d", K, cb);
    if (M > kLinMaxRows) return fail(EXL3_EUNSUPPORTED, "linear_small: M=%d > %d rows", M, kLinMaxRows);
    if (x_dtype < EXL3_DT_F16 || x_dtype > EXL3_DT_F32 || out_dtype < EXL3_DT_F16 || out_dtype > EXL3_DT_F32)
        return fail(EXL3_EINVAL, "linear_small: dtype");
    if (M == 0) return EXL3_OK;
    if (!x || !trellis || !suh || !svh || !shard_of_nb || !out) return fail(EXL3_EINVAL, "linear_small: null pointer");
    if (x_stride < k || out_stride < n) return fail(EXL3_EINVAL, "linear_small: row strides");
    const size_t need = linear_workspace_bytes(M, k, n);
    if (!workspace || workspace_bytes < need)
        return fail(EXL3_EWORKSPACE, "linear_small: workspace %zu < %zu bytes", workspace_bytes, need);
    LinearArgs a{};
    a.x = x;
    a.x_dt = x_dtype;
    a.x_stride = x_stride;
    a.M = M;
    a.k = k;
    a.n = n;
    a.S = S;
    a.tr = (const uint32_t*)trellis;
    a.suh = (const _Float16*)suh;
    a.svh = (const _Float16*)svh;
    a.shard_of_nb = shard_of_nb;
    a.part = (uint64_t*)workspace;
    a.P = linear_kslices(k);
    hipError_t e = linear_status(&a.status, &a.status_host);
    if (e != hipSuccess) return hip_fail(e, "linear_small: status words");
    e = launch_linear_small(K, cb, a, out, out_dtype, out_stride, (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "linear_small launch");
}

int exl3_had_in(const void* x, int x_dtype, int64_t x_stride, int M, int k, const void* suh, int S, void* xh,
                void* stream) {
    if (int r = linear_dims("had_in", M, k, 128, S)) return r;
    if (x_dtype < EXL3_DT_F16 || x_dtype > EXL3_DT_F32) return fail(EXL3_EINVAL, "had_in: x dtype");
    if (M == 0) return EXL3_OK;
    if (!x || !suh || !xh || x_stride < k) return fail(EXL3_EINVAL, "had_in: bad arguments");
    LinearArgs a{};
    a.x = x;
    a.x_dt = x_dtype;
    a.x_stride = x_stride;
    a.M = M;
    a.k = k;
    a.S = S;
    a.suh = (const _Float16*)suh;
    a.xh = (_Float16*)xh;
    const hipError_t e = launch_linear_had_in(a, (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "had_in launch");
}

int exl3_had_out(const void* y, int M, int n, const void* svh, void* out, int out_dtype, int64_t out_stride,
                 void* stream) {
    if (int r = linear_dims("had_out", M, 128, n, 1)) return r;
    if (out_dtype < EXL3_DT_F16 || out_dtype > EXL3_DT_F32) return fail(EXL3_EINVAL, "had_out: out dtype");
    if (M == 0) return EXL3_OK;
    if (!y || !svh || !out || out_stride < n) return fail(EXL3_EINVAL, "had_out: bad arguments");
    const hipError_t e = launch_linear_had_out(y, 1, 1, M, n, (const _Float16*)svh, out, out_dtype, out_stride,
                                               (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "had_out launch");
}

int exl3_reconstruct(const void* trellis, int k, int n, int n0, int n1, int K, int cb, void* w, void* stream) {
    if (!exl3_linear_supported(K, cb)) return fail(EXL3_EUNSUPPORTED, "reconstruct: K=%d cb=%d", K, cb);
    if (k <= 0 || n <= 0 || k % 16 || n % 16 || n0 < 0 || n1 > n || n0 >= n1 || n0 % 16 || n1 % 16)
        return fail(EXL3_EINVAL, "reconstruct: k=%d n=%d columns [%d, %d)", k, n, n0, n1);
    if (!trellis || !w) return fail(EXL3_EINVAL, "reconstruct: null pointer");
    const hipError_t e = launch_linear_reconstruct(K, cb, (const uint32_t*)trellis, k, n, n0, n1, (_Float16*)w,
                                                   (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "reconstruct launch");
}

int exl3_had_in_q8(const void* x, int x_dtype, int64_t x_stride, int M, int k, const void* suh, int S, void* xq,
                   void* sx, int64_t ms, void* stream) {
    if (int r = linear_dims("had_in_q8", M, k, 128, S)) return r;
    if (x_dtype < EXL3_DT_F16 || x_dtype > EXL3_DT_F32) return fail(EXL3_EINVAL, "had_in_q8: x dtype");
    if (ms < M) return fail(EXL3_EINVAL, "had_in_q8: row stride %lld < M=%d", (long long)ms, M);
    if (M == 0) return EXL3_OK;
    if (!x || !suh || !xq || !sx || x_stride < k) return fail(EXL3_EINVAL, "had_in_q8: bad arguments");
    LinearArgs a{};
    a.x = x;
    a.x_dt = x_dtype;
    a.x_stride = x_stride;
    a.M = M;
    a.k = k;
    a.S = S;
    a.suh = (const _Float16*)suh;
    const hipError_t e = launch_linear_had_in_q8(a, (int8_t*)xq, (float*)sx, ms, (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "had_in_q8 launch");
}

int exl3_reconstruct_q8(const void* trellis, int k, int n, int n0, int n1, int K, void* w, void* stream) {
    if (K < 2 || K > 6) return fail(EXL3_EUNSUPPORTED, "reconstruct_q8: K=%d (mul1, K = 2..6)", K);
    if (k <= 0 || n <= 0 || k % 16 || n % 16 || n0 < 0 || n1 > n || n0 >= n1 || n0 % 16 || n1 % 16)
        return fail(EXL3_EINVAL, "reconstruct_q8: k=%d n=%d columns [%d, %d)", k, n, n0, n1);
    if (!trellis || !w) return fail(EXL3_EINVAL, "reconstruct_q8: null pointer");
    const hipError_t e = launch_linear_reconstruct_q8(K, (const uint32_t*)trellis, k, n, n0, n1, (int8_t*)w,
                                                      (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "reconstruct_q8 launch");
}

int exl3_had_out_q8(const int32_t* y, int M, int n, const float* sx, float sw, const void* svh, void* out,
                    int out_dtype, int64_t out_stride, void* stream) {
    if (int r = linear_dims("had_out_q8", M, 128, n, 1)) return r;
    if (out_dtype < EXL3_DT_F16 || out_dtype > EXL3_DT_F32) return fail(EXL3_EINVAL, "had_out_q8: out dtype");
    if (M == 0) return EXL3_OK;
    if (!y || !sx || !svh || !out || out_stride < n) return fail(EXL3_EINVAL, "had_out_q8: bad arguments");
    const hipError_t e = launch_linear_had_out_q8(y, sx, sw, M, n, (const _Float16*)svh, out, out_dtype, out_stride,
                                                  (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "had_out_q8 launch");
}

void* exl3_host_alloc(int64_t nbytes) {
    void* p = nullptr;
    if (nbytes <= 0) {
        fail(EXL3_EINVAL, "host_alloc: %lld bytes", (long long)nbytes);
        return nullptr;
    }
    hipError_t e = hipHostMalloc(&p, (size_t)nbytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        hip_fail(e, "hipHostMalloc");
        return nullptr;
    }
    return p;
}

int exl3_host_free(void* p) {
    if (!p) return EXL3_OK;
    hipError_t e = hipHostFree(p);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "hipHostFree");
}

int exl3_usm_kind(const void* p) {
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    switch (at.type) {
        case hipMemoryTypeHost: return 1;
        case hipMemoryTypeDevice: return 2;
        case hipMemoryTypeManaged: return 3;
        default: return 0;
    }
}

int exl3_copy_batch(void* const* dst, const void* const* src, const int64_t* nbytes, int64_t n, int64_t dst_lo,
                    int64_t dst_hi, int64_t src_lo, int64_t src_hi, void* stream) {
    if (n < 0 || (n > 0 && (!dst || !src || !nbytes))) return fail(EXL3_EINVAL, "copy_batch: n=%lld", (long long)n);
    // every range is checked against the caller's bounds before anything is enqueued: a batch is all or nothing
    for (int64_t i = 0; i < n; ++i) {
        const int64_t d = (int64_t)(uintptr_t)dst[i], s = (int64_t)(uintptr_t)src[i], b = nbytes[i];
        if (b < 0 || (b > 0 && (d < dst_lo || d > dst_hi - b || s < src_lo || s > src_hi - b)))
            return fail(EXL3_EINVAL, "copy_batch: copy %lld (%lld bytes) outside its bounds", (long long)i, (long long)b);
    }
    for (int64_t i = 0; i < n; ++i) {
        if (!nbytes[i]) continue;
        const hipError_t e = hipMemcpyAsync(dst[i], src[i], (size_t)nbytes[i], hipMemcpyDefault, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "copy_batch: hipMemcpyAsync");
    }
    return EXL3_OK;
}

int exl3_table_update(int64_t* ptrs_all, int32_t* slot_of, int32_t* slot_key, int32_t* slot_last, const int64_t* rec,
                      int64_t n, void* stream) {
    if (n < 0 || (n > 0 && (!ptrs_all || !slot_of || !slot_key || !slot_last || !rec)))
        return fail(EXL3_EINVAL, "table_update: n=%lld", (long long)n);
    const hipError_t e = launch_table_update(ptrs_all, slot_of, slot_key, slot_last, rec, n, (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "table_update");
}

int exl3_memcpy_async(void* dst, const void* src, int64_t nbytes, void* stream) {
    if (nbytes < 0 || (nbytes && (!dst || !src))) return fail(EXL3_EINVAL, "memcpy_async: bad arguments");
    if (!nbytes) return EXL3_OK;
    hipError_t e = hipMemcpyAsync(dst, src, (size_t)nbytes, hipMemcpyDefault, (hipStream_t)stream);
    return e == hipSuccess ? EXL3_OK : hip_fail(e, "hipMemcpyAsync");
}

}  // extern "C"
