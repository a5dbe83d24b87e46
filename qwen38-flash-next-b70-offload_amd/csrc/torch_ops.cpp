// torch.ops.exl3xpu_moe: the reference's op schemas (kernels/moe-a8/exl3_moe.a8.sycl:1555-1592) implemented on the HIP
// dispatch key (DispatchKey::CUDA under PyTorch-ROCm) as thin wrappers over the C-ABI of libexl3moe.so.
// Shape/dtype checks raise RuntimeError like the reference's TORCH_CHECKs (a8:1266-1271).
#include <ATen/hip/HIPContext.h>
#include <c10/hip/HIPStream.h>
#include <torch/all.h>
#include <torch/library.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "../../include/exl3moe.h"

namespace {

void* cur_stream(const at::Tensor& like) {
    return (void*)c10::hip::getCurrentHIPStream(like.device().index()).stream();
}

void check(int rc, const char* what) { TORCH_CHECK(rc == EXL3_OK, what, ": ", exl3_last_error()); }

int dtype_code(const at::Tensor& x) {
    if (x.scalar_type() == at::kBFloat16) return EXL3_DT_BF16;
    if (x.scalar_type() == at::kHalf) return EXL3_DT_F16;
    if (x.scalar_type() == at::kFloat) return EXL3_DT_F32;
    TORCH_CHECK(false, "x dtype: bf16, fp16 or fp32 expected, got ", x.scalar_type());
}

at::Tensor moe_forward(at::Tensor x, at::Tensor topk_ids, at::Tensor topk_w, at::Tensor ptrs, int64_t I, int64_t K,
                       int64_t n_experts) {
    TORCH_CHECK(x.dim() == 2 && x.stride(1) == 1, "moe_forward: x must be [M, H] with unit column stride");
    TORCH_CHECK(topk_ids.scalar_type() == at::kInt && topk_ids.is_contiguous(), "moe_forward: topk_ids int32 contiguous");
    TORCH_CHECK(topk_w.scalar_type() == at::kFloat && topk_w.is_contiguous(), "moe_forward: topk_w fp32 contiguous");
    TORCH_CHECK(ptrs.scalar_type() == at::kLong && ptrs.is_contiguous(), "moe_forward: ptrs int64 contiguous");
    const int M = (int)x.size(0), H = (int)x.size(1), topk = (int)topk_ids.size(-1);
    TORCH_CHECK(topk_ids.numel() == (int64_t)M * topk && topk_w.numel() == topk_ids.numel(), "moe_forward: ids/w [M, topk]");
    TORCH_CHECK(ptrs.numel() >= n_experts, "moe_forward: ptrs [n_experts]");
    auto out = at::empty_like(x);
    if (M == 0) return out;
    const size_t ws = exl3_moe_forward_workspace(M, H, (int)I, topk, (int)n_experts);
    auto w = at::empty({(int64_t)ws}, x.options().dtype(at::kByte));
    check(exl3_moe_forward(x.data_ptr(), dtype_code(x), x.stride(0), M, H, topk_ids.data_ptr<int>(),
                           topk_w.data_ptr<float>(), topk, ptrs.data_ptr<int64_t>(), (int)I, (int)K, (int)n_experts,
                           out.data_ptr(), out.stride(0), w.data_ptr(), ws, cur_stream(x)),
          "moe_forward");
    return out;
}

// moe_prefetch (a8:1194-1222): claim slots for predicted experts of `layer`, copy them from host, repoint the table,
// on the current stream (use a side stream; make the compute stream wait before the next MoE call)
void moe_prefetch(at::Tensor ids, at::Tensor ptrs_all, int64_t layer, at::Tensor slot_of, at::Tensor slot_key,
                  at::Tensor slot_last, at::Tensor tick, at::Tensor host_base, int64_t slot_base, at::Tensor pf_list,
                  at::Tensor pf_slot, int64_t max_fill, int64_t n_experts, int64_t blob) {
    TORCH_CHECK(ids.scalar_type() == at::kInt && ids.is_contiguous(), "moe_prefetch: ids int32 contiguous");
    TORCH_CHECK(ptrs_all.scalar_type() == at::kLong && slot_of.scalar_type() == at::kInt &&
                    pf_list.scalar_type() == at::kInt && pf_slot.scalar_type() == at::kInt,
                "moe_prefetch: ptrs_all int64, slot_of / pf_list / pf_slot int32");
    TORCH_CHECK(ptrs_all.numel() >= (layer + 1) * n_experts && slot_of.numel() == ptrs_all.numel() &&
                    host_base.numel() > layer && pf_list.numel() >= 1 + n_experts &&
                    slot_last.numel() == slot_key.numel(),
                "moe_prefetch: cache state sizes");
    const int64_t mf = std::min<int64_t>(max_fill, pf_slot.numel());
    check(exl3_moe_prefetch(ids.data_ptr<int>(), (int)ids.numel(), ptrs_all.data_ptr<int64_t>(), (int)layer,
                            slot_of.data_ptr<int>(), slot_key.data_ptr<int>(), slot_last.data_ptr<int>(),
                            tick.data_ptr<int>(), (int)slot_key.numel(), host_base.data_ptr<int64_t>(), slot_base,
                            pf_list.data_ptr<int>(), pf_slot.data_ptr<int>(), (int)mf, (int)n_experts, blob,
                            cur_stream(ids)),
          "moe_prefetch");
}

// copy-engine prefetch (a8:1047-1142): plan on the current (compute) stream; the worker copies on the stream that is
// current when it starts
void moe_prefetch_plan(at::Tensor ids, at::Tensor ptrs_all, int64_t layer, at::Tensor slot_of, at::Tensor slot_key,
                       at::Tensor slot_last, at::Tensor tick, at::Tensor host_base, int64_t slot_base, at::Tensor pf_list,
                       at::Tensor pf_slot, at::Tensor plans, at::Tensor plan_seq, at::Tensor pend, at::Tensor done_seq,
                       int64_t max_fill, int64_t n_experts, int64_t blob) {
    TORCH_CHECK(ids.scalar_type() == at::kInt && ids.is_contiguous(), "moe_prefetch_plan: ids int32 contiguous");
    const int64_t L = done_seq.numel();
    TORCH_CHECK(L > layer && plan_seq.numel() >= L && pend.numel() >= L * 35 &&
                    plans.nbytes() >= (size_t)(L * (4 + 2 * n_experts) * 4) && pf_list.numel() >= 1 + n_experts,
                "moe_prefetch_plan: plan state sizes (start_copy_prefetch first)");
    check(exl3_moe_prefetch_plan(ids.data_ptr<int>(), (int)ids.numel(), ptrs_all.data_ptr<int64_t>(), (int)layer,
                                 slot_of.data_ptr<int>(), slot_key.data_ptr<int>(), slot_last.data_ptr<int>(),
                                 tick.data_ptr<int>(), (int)slot_key.numel(), host_base.data_ptr<int64_t>(), slot_base,
                                 pf_list.data_ptr<int>(), pf_slot.data_ptr<int>(), (int32_t*)plans.data_ptr(),
                                 plan_seq.data_ptr<int>(), pend.data_ptr<int>(), done_seq.data_ptr<int>(), (int)L,
                                 (int)std::min<int64_t>(max_fill, pf_slot.numel()), (int)n_experts, blob,
                                 cur_stream(ids)),
          "moe_prefetch_plan");
}

void moe_prefetch_worker_start(at::Tensor plans, at::Tensor host_base_cpu, int64_t slot_base, int64_t blob,
                               at::Tensor ptrs_all, at::Tensor slot_last, at::Tensor commit_host, at::Tensor done_seq,
                               int64_t n_layers, int64_t n_experts) {
    (void)ptrs_all;
    (void)slot_last;       // the commit runs on the device (ensure); the worker only publishes done_seq
    TORCH_CHECK(host_base_cpu.device().is_cpu() && host_base_cpu.scalar_type() == at::kLong &&
                    host_base_cpu.numel() >= n_layers && commit_host.nbytes() >= (size_t)(n_layers * 2 * 4),
                "moe_prefetch_worker_start: host_base_cpu int64 [n_layers] on the CPU, commit_host pinned");
    auto hb = host_base_cpu.contiguous();
    check(exl3_prefetch_worker_start((int32_t*)plans.data_ptr(), hb.data_ptr<int64_t>(), slot_base, blob,
                                     done_seq.data_ptr<int>(), (int32_t*)commit_host.data_ptr(), (int)n_layers,
                                     (int)n_experts, cur_stream(done_seq)),
          "moe_prefetch_worker_start");
}

std::vector<int64_t> moe_prefetch_worker_stop() {
    int64_t c[2] = {0, 0};
    check(exl3_prefetch_worker_stop(c), "moe_prefetch_worker_stop");
    return {c[0], c[1]};
}

at::Tensor moe_forward_cached(at::Tensor x, at::Tensor topk_ids, at::Tensor topk_w, at::Tensor ptrs_all, int64_t layer,
                              at::Tensor slot_of, at::Tensor slot_key, at::Tensor slot_last, at::Tensor tick,
                              at::Tensor host_base, int64_t slot_base, at::Tensor fill_all, at::Tensor fill_list,
                              int64_t max_fill, int64_t I, int64_t K, int64_t n_experts, at::Tensor pend,
                              at::Tensor done_seq) {
    // plans of the copy-engine prefetch are committed by this call's ensure when done_seq is in use
    if (done_seq.numel() > 0) {
        TORCH_CHECK(pend.numel() >= done_seq.numel() * 35, "moe_forward_cached: pend [n_layers * 35]");
        check(exl3_set_prefetch_commit(pend.data_ptr<int>(), done_seq.data_ptr<int>(), (int)done_seq.numel()),
              "moe_forward_cached");
    } else {
        check(exl3_set_prefetch_commit(nullptr, nullptr, 0), "moe_forward_cached");
    }
    TORCH_CHECK(x.dim() == 2 && x.stride(1) == 1, "moe_forward_cached: x must be [M, H] with unit column stride");
    TORCH_CHECK(ptrs_all.scalar_type() == at::kLong && fill_all.scalar_type() == at::kLong &&
                    slot_of.scalar_type() == at::kInt,
                "moe_forward_cached: ptrs_all/fill_all int64, slot_of int32");
    TORCH_CHECK(topk_ids.scalar_type() == at::kInt && topk_ids.is_contiguous() && topk_w.scalar_type() == at::kFloat &&
                    topk_w.is_contiguous(),
                "tier mask: int32 ids, fp32 w");
    const int M = (int)x.size(0), H = (int)x.size(1), topk = (int)topk_ids.size(-1);
    TORCH_CHECK(topk_ids.numel() == (int64_t)M * topk && topk_w.numel() == topk_ids.numel(), "moe_forward_cached: ids/w [M, topk]");
    TORCH_CHECK(ptrs_all.numel() >= (layer + 1) * n_experts && slot_of.numel() == ptrs_all.numel() &&
                    fill_all.numel() == ptrs_all.numel() && host_base.numel() > layer &&
                    fill_list.numel() >= 1 + n_experts && slot_last.numel() == slot_key.numel(),
                "moe_forward_cached: cache state sizes");
    auto out = at::empty_like(x);
    if (M == 0) return out;
    const size_t ws = exl3_moe_forward_workspace(M, H, (int)I, topk, (int)n_experts);
    auto w = at::empty({(int64_t)ws}, x.options().dtype(at::kByte));
    check(exl3_moe_forward_cached(x.data_ptr(), dtype_code(x), x.stride(0), M, H, topk_ids.data_ptr<int>(),
                                  topk_w.data_ptr<float>(), topk, ptrs_all.data_ptr<int64_t>(), (int)layer,
                                  slot_of.data_ptr<int>(), slot_key.data_ptr<int>(), slot_last.data_ptr<int>(),
                                  tick.data_ptr<int>(), (int)slot_key.numel(), host_base.data_ptr<int64_t>(), slot_base,
                                  fill_all.data_ptr<int64_t>(), fill_list.data_ptr<int>(), (int)max_fill, (int)I,
                                  (int)K, (int)n_experts, out.data_ptr(), out.stride(0), w.data_ptr(), ws,
                                  cur_stream(x)),
          "moe_forward_cached");
    return out;
}

std::vector<at::Tensor> moe_align(at::Tensor topk_ids, at::Tensor topk_w, int64_t n_experts, int64_t pad) {
    TORCH_CHECK(topk_ids.scalar_type() == at::kInt && topk_ids.is_contiguous() && topk_ids.dim() == 2, "moe_align: ids");
    TORCH_CHECK(topk_w.scalar_type() == at::kFloat && topk_w.is_contiguous(), "moe_align: w");
    const int M = (int)topk_ids.size(0), topk = (int)topk_ids.size(1), npairs = M * topk;
    const int A = std::min(npairs, (int)n_experts);
    auto ib = at::empty({4 * A + 1 + 2 * npairs + 16}, topk_ids.options());
    auto fb = at::empty({npairs}, topk_w.options());
    const size_t wsb = exl3_moe_align_workspace(M, topk, (int)n_experts);
    auto ws = at::empty({(int64_t)std::max<size_t>(wsb, 1)}, topk_ids.options().dtype(at::kByte));
    check(exl3_moe_align(topk_ids.data_ptr<int>(), topk_w.data_ptr<float>(), M, topk, (int)n_experts, (int)pad,
                         ib.data_ptr<int>(), fb.data_ptr<float>(), ws.data_ptr(), wsb, cur_stream(topk_ids)),
          "moe_align");
    return {ib, fb};
}

at::Tensor host_alloc(int64_t nbytes) {
    void* p = exl3_host_alloc(nbytes);
    TORCH_CHECK(p, "host_alloc failed for ", nbytes, " bytes: ", exl3_last_error());
    return at::from_blob(p, {nbytes}, [](void* q) { exl3_host_free(q); },
                         at::TensorOptions().dtype(at::kByte).device(at::kCPU));
}

int64_t usm_kind(int64_t ptr) { return exl3_usm_kind(reinterpret_cast<const void*>(ptr)); }

void memcpy_async(int64_t dst, int64_t src, int64_t nbytes) {
    void* s = (void*)c10::hip::getCurrentHIPStream().stream();
    check(exl3_memcpy_async(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), nbytes, s), "memcpy_async");
}

int64_t blob_bytes(int64_t H, int64_t I, int64_t K) { return exl3_blob_bytes((int)H, (int)I, (int)K); }

void moe_set_splits(int64_t gu_p, int64_t dn_p) { check(exl3_set_splits(gu_p, dn_p), "moe_set_splits"); }
void moe_set_mr(int64_t mr) { check(exl3_set_mr(mr), "moe_set_mr"); }
void moe_set_debug(int64_t v) { check(exl3_set_debug(v), "moe_set_debug"); }
void moe_set_pair_max_m(int64_t v) { check(exl3_set_pair_max_m(v), "moe_set_pair_max_m"); }
void moe_set_prefill_min_m(int64_t v) { check(exl3_set_prefill_min_m(v), "moe_set_prefill_min_m"); }
// moe_set_victim_ring (experimental/n111-victim-ring/a9.patch:17-30): meta int32 [4 + 2K], sel int32 [E], buf the
// K ring slots; an empty meta turns the ring off
void moe_set_victim_ring(at::Tensor meta, at::Tensor sel, at::Tensor buf) {
    if (!meta.numel()) return check(exl3_set_victim_ring(nullptr, nullptr, nullptr, 0, 0), "moe_set_victim_ring");
    TORCH_CHECK(meta.scalar_type() == at::kInt && sel.scalar_type() == at::kInt && meta.is_contiguous() &&
                    sel.is_contiguous() && meta.is_cuda() && sel.is_cuda() && buf.is_cuda(),
                "moe_set_victim_ring: device int32 meta and sel");
    const int64_t K = (meta.numel() - 4) / 2;
    TORCH_CHECK(K > 0 && meta.numel() == 4 + 2 * K && buf.numel() > 0, "victim ring: meta [4 + 2K], buf [K * blob]");
    check(exl3_set_victim_ring(meta.data_ptr<int>(), sel.data_ptr<int>(), buf.data_ptr(),
                               (int64_t)buf.numel() * (int64_t)buf.element_size(), K),
          "moe_set_victim_ring");
}

void moe_set_victims(at::Tensor v) {
    if (!v.numel()) return check(exl3_set_victims(nullptr), "moe_set_victims");
    TORCH_CHECK(v.scalar_type() == at::kInt && v.is_cuda(), "moe_set_victims: device int32 tensor");
    check(exl3_set_victims(v.data_ptr<int>()), "moe_set_victims");
}
void moe_set_tier(at::Tensor ram_res, at::Tensor miss, at::Tensor safe) {
    if (!ram_res.numel()) return check(exl3_set_tier(nullptr, nullptr, 0, nullptr), "moe_set_tier");
    TORCH_CHECK(ram_res.scalar_type() == at::kByte && miss.scalar_type() == at::kInt && safe.scalar_type() == at::kInt,
                "moe_set_tier: uint8 ram_res, int32 miss ring, int32 safe");
    check(exl3_set_tier(ram_res.data_ptr<uint8_t>(), miss.data_ptr<int>(), miss.numel(), safe.data_ptr<int>()),
          "moe_set_tier");
}
void moe_set_host_stride(int64_t s) { check(exl3_set_host_stride(s), "moe_set_host_stride"); }
void moe_set_slot_stride(int64_t s) { check(exl3_set_slot_stride(s), "moe_set_slot_stride"); }
void moe_set_fused_ensure(int64_t v) { check(exl3_set_fused_ensure(v), "moe_set_fused_ensure"); }
// pinned host memory is device-mapped on MI355X: nothing to prefetch (the reference maps xe-SVM pages, a8:777-781)
void moe_svm_prefetch(at::Tensor ptrs, int64_t nbytes, at::Tensor like) {
    (void)ptrs;
    (void)nbytes;
    (void)like;
}
void moe_set_decision_log(at::Tensor buf) {
    if (!buf.numel()) return check(exl3_set_decision_log(nullptr, 0), "moe_set_decision_log");
    TORCH_CHECK(buf.scalar_type() == at::kInt && buf.is_cuda() && buf.is_contiguous(), "decision log: device int32");
    check(exl3_set_decision_log(buf.data_ptr<int>(), buf.numel() - 1), "moe_set_decision_log");
}
at::Tensor dequant(at::Tensor trellis, int64_t k_tiles, int64_t n_tiles, int64_t K) {
    TORCH_CHECK(trellis.is_cuda() && trellis.is_contiguous(), "dequant: contiguous device words");
    auto out = at::empty({16 * k_tiles, 16 * n_tiles}, trellis.options().dtype(at::kHalf));
    check(exl3_dequant(reinterpret_cast<const uint32_t*>(trellis.data_ptr()), (int)k_tiles, (int)n_tiles, (int)K,
                       reinterpret_cast<uint16_t*>(out.data_ptr()), cur_stream(trellis)),
          "dequant");
    return out;
}

// ---- torch.ops.exl3xpu_C: the dense EXL3 linear (experimental/n111-victim-ring/csrc/exl3_ops.sycl:639-781, 784-815)

void linear_checks(const at::Tensor& trellis, const at::Tensor& suh, const at::Tensor& svh, const at::Tensor& sonb,
                   int64_t k, int64_t K, int64_t cb) {
    TORCH_CHECK(exl3_linear_supported((int)K, (int)cb), "exl3xpu_C.linear: K=", K, " cb=", cb, " not built");
    TORCH_CHECK(trellis.is_cuda() && trellis.is_contiguous() && trellis.dim() == 3 && trellis.size(0) * 16 == k &&
                    trellis.size(2) == 16 * K,
                "exl3xpu_C.linear: trellis [k/16, n/16, 16K] contiguous on the device");
    TORCH_CHECK(suh.scalar_type() == at::kHalf && suh.is_contiguous() && suh.dim() == 2 && suh.size(1) == k,
                "exl3xpu_C.linear: suh fp16 [S, k]");
    TORCH_CHECK(svh.scalar_type() == at::kHalf && svh.is_contiguous() && svh.size(0) == trellis.size(1) * 16,
                "exl3xpu_C.linear: svh fp16 [n]");
    TORCH_CHECK(sonb.scalar_type() == at::kInt && sonb.is_contiguous() && sonb.numel() * 128 == svh.size(0),
                "exl3xpu_C.linear: shard_of_nb int32 [n / 128]");
}

// The small-M workspace. Its tagged partials must be zero when a call starts; every call leaves them zero.
// Eager calls on one (device, stream) share one buffer, zeroed when it is allocated, and run in stream order. A call
// made while its stream is being captured into a HIP graph gets a buffer of that capture alone (keyed by the capture
// id), allocated and zeroed inside the capture: the zero fill (a fill kernel, not a memset node) is then a node of
// that graph, so each replay starts from zero whatever ran on the buffer of another graph or of eager calls, and
// graphs captured one after another on the same stream can be replayed in any order. Sized for 8 rows; a larger one
// replaces it when a call needs more. Buffers are kept until the process ends: a captured graph holds their
// addresses.
at::Tensor& small_workspace(const at::Tensor& x, size_t bytes) {
    static std::mutex mu;
    static auto* cache = new std::map<std::tuple<int, void*, unsigned long long>, at::Tensor>();
    static auto* retired = new std::vector<at::Tensor>();
    void* st = cur_stream(x);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    TORCH_CHECK(hipStreamGetCaptureInfo((hipStream_t)st, &cs, &cid) == hipSuccess, "exl3_gemm_small: capture status");
    if (cs != hipStreamCaptureStatusActive) cid = 0;            // eager: the stream's own buffer
    else if (cid == 0) cid = ~0ull;                             // (capture ids start at 1; keep 0 for eager calls)
    std::lock_guard<std::mutex> lock(mu);
    auto& t = (*cache)[{(int)x.device().index(), st, cid}];
    if (!t.defined() || (size_t)t.numel() < bytes) {
        if (t.defined()) retired->push_back(t);
        t = at::zeros({(int64_t)bytes}, x.options().dtype(at::kByte));
    }
    return t;
}

void gemm_small(at::Tensor x2, at::Tensor trellis, at::Tensor suh, at::Tensor svh, at::Tensor shard_of_nb, at::Tensor out,
                int64_t K, int64_t cb) {
    const int64_t M = x2.size(0), k = x2.size(1), n = svh.size(0);
    linear_checks(trellis, suh, svh, shard_of_nb, k, K, cb);
    TORCH_CHECK(x2.stride(1) == 1 && out.dim() == 2 && out.size(0) == M && out.size(1) == n && out.stride(1) == 1,
                "exl3_gemm_small: x [M, k], out [M, n] with unit column strides");
    TORCH_CHECK(M <= 8, "exl3_gemm_small: at most 8 rows, got ", M);
    const size_t ws_bytes = exl3_linear_workspace(8, (int)k, (int)n);
    auto& ws = small_workspace(x2, ws_bytes);
    check(exl3_linear_small(x2.data_ptr(), dtype_code(x2), x2.stride(0), (int)M, (int)k, (int)n, trellis.data_ptr(),
                            (int)K, (int)cb, suh.data_ptr(), (int)suh.size(0), svh.data_ptr(),
                            shard_of_nb.data_ptr<int>(), out.data_ptr(), dtype_code(out), out.stride(0), ws.data_ptr(),
                            ws_bytes, cur_stream(x2)),
          "exl3xpu_C.exl3_gemm_small");
}

void had_in_rm(at::Tensor x, at::Tensor suh, at::Tensor xh) {
    TORCH_CHECK(x.dim() == 2 && x.stride(1) == 1, "exl3_had_in_rm: x [M, k]");
    TORCH_CHECK(xh.scalar_type() == at::kHalf && xh.is_contiguous() && xh.dim() == 3 && xh.size(1) == x.size(0) &&
                    xh.size(2) == x.size(1) && suh.scalar_type() == at::kHalf && suh.dim() == 2 &&
                    suh.size(0) == xh.size(0) && suh.is_contiguous(),
                "exl3_had_in_rm: xh fp16 [S, M, k], suh fp16 [S, k]");
    check(exl3_had_in(x.data_ptr(), dtype_code(x), x.stride(0), (int)x.size(0), (int)x.size(1), suh.data_ptr(),
                      (int)suh.size(0), xh.data_ptr(), cur_stream(x)),
          "exl3xpu_C.exl3_had_in_rm");
}

void had_out_h(at::Tensor y, at::Tensor svh, at::Tensor out) {
    TORCH_CHECK(y.scalar_type() == at::kHalf && y.is_contiguous() && y.sizes() == out.sizes() && y.dim() == 2 &&
                    out.stride(1) == 1 && svh.scalar_type() == at::kHalf && svh.numel() == y.size(1),
                "exl3_had_out_h: y fp16 [M, n] contiguous, out [M, n], svh fp16 [n]");
    check(exl3_had_out(y.data_ptr(), (int)y.size(0), (int)y.size(1), svh.data_ptr(), out.data_ptr(), dtype_code(out),
                       out.stride(0), cur_stream(y)),
          "exl3xpu_C.exl3_had_out_h");
}

void reconstruct(at::Tensor trellis, at::Tensor w, int64_t n0, int64_t K, int64_t cb) {
    TORCH_CHECK(trellis.is_cuda() && trellis.is_contiguous() && trellis.dim() == 3, "exl3_reconstruct: trellis");
    TORCH_CHECK(w.scalar_type() == at::kHalf && w.is_contiguous() && w.dim() == 2 && w.size(0) == trellis.size(0) * 16,
                "exl3_reconstruct: w fp16 [k, width] contiguous");
    check(exl3_reconstruct(trellis.data_ptr(), (int)w.size(0), (int)trellis.size(1) * 16, (int)n0,
                           (int)(n0 + w.size(1)), (int)K, (int)cb, w.data_ptr(), cur_stream(w)),
          "exl3xpu_C.exl3_reconstruct");
}

// the W8A8 route's switch (exl3_set_int8, exl3_ops.sycl:524): off unless the caller turns it on
std::atomic<bool> g_int8{false};
void set_int8(int64_t on) { g_int8.store(on != 0); }

// the W8A8 route (exl3_ops.sycl:668-740, the path without oneDNN): int8 xh with one scale per (shard, row), then per
// shard group the int8 weights at the static scale, the library's int8 GEMM (int32 sums) and the output Hadamard of
// y * sx * sw into the group's columns of out
void linear_q8(const at::Tensor& x2, const at::Tensor& trellis, const at::Tensor& suh, const at::Tensor& svh,
               at::IntArrayRef group_bounds, int64_t K, at::Tensor& out) {
    const int64_t M = x2.size(0), k = x2.size(1), n = svh.size(0), S = suh.size(0);
    void* st = cur_stream(x2);
    auto xq = at::empty({S, M, k}, x2.options().dtype(at::kChar));
    auto sx = at::empty({S, M}, x2.options().dtype(at::kFloat));
    check(exl3_had_in_q8(x2.data_ptr(), dtype_code(x2), x2.stride(0), (int)M, (int)k, suh.data_ptr(), (int)S,
                         xq.data_ptr(), sx.data_ptr(), M, st),
          "exl3xpu_C.linear (int8 had_in)");
    const float sw = 3.453125f / 127.0f;
    for (int64_t g = 0; g < S; ++g) {
        const int64_t g0 = group_bounds[g], g1 = group_bounds[g + 1], ng = g1 - g0;
        TORCH_CHECK(g0 <= g1 && g1 <= n && g0 % 128 == 0 && ng % 128 == 0,
                    "exl3xpu_C.linear: int8 route needs shard groups of whole 128-column blocks");
        if (ng == 0) continue;
        auto w = at::empty({k, ng}, x2.options().dtype(at::kChar));
        check(exl3_reconstruct_q8(trellis.data_ptr(), (int)k, (int)n, (int)g0, (int)g1, (int)K, w.data_ptr(), st),
              "exl3xpu_C.linear (int8 weights)");
        auto y = at::_int_mm(xq[g], w);                               // [M, ng] int32
        auto og = out.narrow(1, g0, ng);
        check(exl3_had_out_q8(y.data_ptr<int32_t>(), (int)M, (int)ng, sx.data_ptr<float>() + g * M, sw,
                              svh.narrow(0, g0, ng).data_ptr(), og.data_ptr(), dtype_code(out), out.stride(0), st),
              "exl3xpu_C.linear (int8 had_out)");
    }
}

// exl3_linear (exl3_ops.sycl:651-757): M <= small_m_max (at most 8 rows here) -> the fused path; otherwise the input
// Hadamards, per shard group the reconstructed fp16 weights in slices of slice_n columns times xh[g] (a library
// GEMM, fp16 output), then the output Hadamard
at::Tensor linear(at::Tensor x, at::Tensor trellis, at::Tensor suh, at::Tensor svh, at::Tensor shard_of_nb,
                  at::IntArrayRef group_bounds, int64_t K, int64_t cb, int64_t small_m_max, int64_t slice_n) {
    auto shape = x.sizes().vec();
    const int64_t k = shape.back(), n = svh.size(0);
    auto x2 = x.reshape({-1, k});
    if (!x2.is_contiguous()) x2 = x2.contiguous();
    const int64_t M = x2.size(0);
    shape.back() = n;
    auto out = at::empty({M, n}, x.options());
    if (M == 0) return out.view(shape);
    linear_checks(trellis, suh, svh, shard_of_nb, k, K, cb);
    if (M <= std::min<int64_t>(small_m_max, 8)) {
        gemm_small(x2, trellis, suh, svh, shard_of_nb, out, K, cb);
        return out.view(shape);
    }
    const int64_t S = suh.size(0);
    TORCH_CHECK((int64_t)group_bounds.size() == S + 1 && group_bounds[0] == 0 && group_bounds[S] == n,
                "exl3xpu_C.linear: group_bounds [0, ..., n] with one group per suh row");
    if (g_int8.load() && cb == 2 && (K == 4 || K == 6) && M > 16) {     // exl3_ops.sycl:668
        linear_q8(x2, trellis, suh, svh, group_bounds, K, out);
        return out.view(shape);
    }
    auto xh = at::empty({S, M, k}, x.options().dtype(at::kHalf));
    had_in_rm(x2, suh, xh);
    auto y = at::empty({M, n}, x.options().dtype(at::kHalf));
    const int64_t step = slice_n > 0 ? std::max<int64_t>(16, slice_n / 16 * 16) : n;
    // one reconstructed slice at a time, from the caching allocator (stream-ordered reuse across slices and calls)
    auto wbuf = at::empty({k * std::min(step, n)}, x.options().dtype(at::kHalf));
    for (int64_t g = 0; g < S; ++g) {
        const int64_t g0 = group_bounds[g], g1 = group_bounds[g + 1];
        TORCH_CHECK(g0 <= g1 && g1 <= n, "exl3xpu_C.linear: group_bounds not ascending");
        for (int64_t n0 = g0; n0 < g1; n0 += step) {
            const int64_t n1 = std::min(n0 + step, g1);
            auto w = wbuf.narrow(0, 0, k * (n1 - n0)).view({k, n1 - n0});
            reconstruct(trellis, w, n0, K, cb);
            auto ys = y.narrow(1, n0, n1 - n0);
            at::matmul_out(ys, xh[g], w);
        }
    }
    had_out_h(y, svh, out);
    return out.view(shape);
}

at::Tensor linear_meta(at::Tensor x, at::Tensor trellis, at::Tensor suh, at::Tensor svh, at::Tensor shard_of_nb,
                       at::IntArrayRef group_bounds, int64_t K, int64_t cb, int64_t small_m_max, int64_t slice_n) {
    auto shape = x.sizes().vec();
    shape.back() = svh.size(0);
    return at::empty(shape, x.options());
}

bool linear_supported(int64_t K, int64_t cb) { return exl3_linear_supported((int)K, (int)cb) != 0; }

}  // namespace

TORCH_LIBRARY(exl3xpu_C, m) {
    m.def("linear(Tensor x, Tensor trellis, Tensor suh, Tensor svh, Tensor shard_of_nb, int[] group_bounds, int K, "
          "int cb, int small_m_max, int slice_n) -> Tensor");
    m.impl("linear", c10::DispatchKey::CUDA, &linear);
    m.impl("linear", c10::DispatchKey::Meta, &linear_meta);
    m.def("exl3_gemm_small(Tensor x, Tensor trellis, Tensor suh, Tensor svh, Tensor shard_of_nb, Tensor(a!) out, "
          "int K, int cb) -> ()");
    m.impl("exl3_gemm_small", c10::DispatchKey::CUDA, &gemm_small);
    m.def("exl3_supported(int K, int cb) -> bool", &linear_supported);
    m.def("exl3_set_int8(int on) -> ()", &set_int8);
    m.def("exl3_had_in_rm(Tensor x, Tensor suh, Tensor(a!) xh) -> ()");
    m.impl("exl3_had_in_rm", c10::DispatchKey::CUDA, &had_in_rm);
    m.def("exl3_had_out_h(Tensor y, Tensor svh, Tensor(a!) out) -> ()");
    m.impl("exl3_had_out_h", c10::DispatchKey::CUDA, &had_out_h);
    m.def("exl3_reconstruct(Tensor trellis, Tensor(a!) w, int n0, int K, int cb) -> ()");
    m.impl("exl3_reconstruct", c10::DispatchKey::CUDA, &reconstruct);
}

TORCH_LIBRARY(exl3xpu_moe, m) {
    m.def("moe_forward(Tensor x, Tensor topk_ids, Tensor topk_w, Tensor ptrs, int I, int K, int n_experts) -> Tensor");
    m.impl("moe_forward", c10::DispatchKey::CUDA, &moe_forward);
    m.def("moe_forward_cached(Tensor x, Tensor(i!) topk_ids, Tensor(j!) topk_w, Tensor(a!) ptrs_all, int layer, "
          "Tensor(b!) slot_of, Tensor(c!) slot_key, Tensor(d!) slot_last, Tensor(e!) tick, Tensor host_base, "
          "int slot_base, Tensor(f!) fill_all, Tensor(g!) fill_list, int max_fill, int I, int K, int n_experts, "
          "Tensor(h!) pend, Tensor done_seq) -> Tensor");
    m.impl("moe_forward_cached", c10::DispatchKey::CUDA, &moe_forward_cached);
    m.def("moe_prefetch(Tensor ids, Tensor(a!) ptrs_all, int layer, Tensor(b!) slot_of, Tensor(c!) slot_key, "
          "Tensor(d!) slot_last, Tensor tick, Tensor host_base, int slot_base, Tensor(e!) pf_list, Tensor(f!) pf_slot, "
          "int max_fill, int n_experts, int blob) -> ()");
    m.impl("moe_prefetch", c10::DispatchKey::CUDA, &moe_prefetch);
    m.def("moe_prefetch_plan(Tensor ids, Tensor(a!) ptrs_all, int layer, Tensor(b!) slot_of, Tensor(c!) slot_key, "
          "Tensor(d!) slot_last, Tensor tick, Tensor host_base, int slot_base, Tensor(e!) pf_list, Tensor(f!) pf_slot, "
          "Tensor(g!) plans, Tensor(h!) plan_seq, Tensor(i!) pend, Tensor done_seq, int max_fill, int n_experts, "
          "int blob) -> ()");
    m.impl("moe_prefetch_plan", c10::DispatchKey::CUDA, &moe_prefetch_plan);
    m.def("moe_prefetch_worker_start(Tensor plans, Tensor host_base_cpu, int slot_base, int blob, Tensor ptrs_all, "
          "Tensor slot_last, Tensor commit_host, Tensor done_seq, int n_layers, int n_experts) -> ()",
          &moe_prefetch_worker_start);
    m.def("moe_prefetch_worker_stop() -> int[]", &moe_prefetch_worker_stop);
    m.def("moe_align(Tensor topk_ids, Tensor topk_w, int n_experts, int pad) -> Tensor[]");
    m.impl("moe_align", c10::DispatchKey::CUDA, &moe_align);
    m.def("host_alloc(int nbytes) -> Tensor", &host_alloc);
    m.def("usm_kind(int ptr) -> int", &usm_kind);
    m.def("memcpy_async(int dst, int src, int nbytes) -> ()", &memcpy_async);
    m.def("blob_bytes(int H, int I, int K) -> int", &blob_bytes);
    m.def("moe_set_splits(int gu_p, int dn_p) -> ()", &moe_set_splits);
    m.def("moe_set_mr(int mr) -> ()", &moe_set_mr);
    m.def("moe_set_debug(int v) -> ()", &moe_set_debug);
    m.def("moe_set_pair_max_m(int v) -> ()", &moe_set_pair_max_m);
    m.def("moe_set_prefill_min_m(int v) -> ()", &moe_set_prefill_min_m);
    m.def("moe_set_victims(Tensor v) -> ()", &moe_set_victims);
    m.def("moe_set_victim_ring(Tensor meta, Tensor sel, Tensor buf) -> ()", &moe_set_victim_ring);
    m.def("moe_set_tier(Tensor ram_res, Tensor miss, Tensor safe) -> ()", &moe_set_tier);
    m.def("moe_set_host_stride(int s) -> ()", &moe_set_host_stride);
    m.def("moe_set_slot_stride(int s) -> ()", &moe_set_slot_stride);
    m.def("moe_set_fused_ensure(int v) -> ()", &moe_set_fused_ensure);
    m.def("moe_svm_prefetch(Tensor ptrs, int nbytes, Tensor like) -> ()", &moe_svm_prefetch);
    m.def("moe_set_decision_log(Tensor buf) -> ()", &moe_set_decision_log);
    m.def("dequant(Tensor trellis, int k_tiles, int n_tiles, int K) -> Tensor");
    m.impl("dequant", c10::DispatchKey::CUDA, &dequant);
}
