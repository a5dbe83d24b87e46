// Device-managed expert slot cache for CDNA4: one 1024-thread workgroup per MoE layer call.
//
// ensure_kernel, decode mode (reference kernels/moe-a8/exl3_moe.a8.sycl:831-1040, canonical order):
//   1. T = ++tick
//   2. tier mask: picks whose expert is in neither VRAM (slot_of < 0) nor RAM (ram_res == 0) are logged to the miss
//      ring in ascending pick order (wave ballot + prefix popcount) and replaced in place by (safe expert, weight 0)
//   3. need = set of post-mask picks; hits (ascending expert) stamp slot_last = T unless pinned; misses are compacted in
//      ascending expert id (block exclusive scan)
//   4. nm = min(misses, max_fill, slots with slot_last < T); tau = nm-th smallest u = slot_last + 1 among those slots,
//      found by 8-bit radix passes over LDS histograms starting at the highest byte where the keys differ
//   5. victims = ascending-slot({u < tau}) ++ first `want` of ascending-slot({u == tau}) (ordered compaction over
//      per-thread contiguous slot chunks), paired with misses in order; the old owner is repointed to its host copy,
//      the miss gets the slot and a write-through target fill_all[key]
// Calls of at most 64 picks whose post-mask picks all hold a slot finish in wave 0 after step 2 (stamps, pair pointers,
// empty lists): the same decisions without the slot-table staging, the block scans and their barriers.
// Prefetch mode (pf_slot set; reference moe_prefetch a8:1194-1222 and the prefetch branch of launch_ensure a8:846-851,
// 884, 1019-1021): T = tick (not advanced, so slots stamped by the last MoE call stay protected), no tier mask, no
// victims or write-through targets; the assigned slots go to pf_slot for prefetch_copy_kernel and the commit.
// Plan mode (host_plan set as well; moe_prefetch_plan a8:1127-1142, launch_ensure a8:853-901, 1013-1038): at most 16
// claims, pinned (slot_last = INT_MAX) and recorded in pend; the plan goes to pinned host memory for the copy worker
// (entries, a system-scope fence, then the sequence number). A layer whose previous plan is pending is skipped. With
// pend set, every call first commits the plans whose copies the worker has finished (done_seq >= the plan's sequence
// number): ptrs_all -> slot, slot_last = the plan's tick.
// The reference builds the miss and victim lists with SLM fetch_add, so its pairing is not deterministic; here every
// list is produced by prefix sums in work-item order, which defines the canonical decisions the oracle restates.
//
// The victim write-back (reference VictimCopyKernel a8:1168-1189) runs as the first workgroups of the layer kernel
// (moe_decode.hip).
#include <algorithm>
#include <climits>

#include "exl3_common.cuh"
#include "exl3_kernels.h"

namespace exl3 {

constexpr int kEnsureThreads = 1024;
constexpr int kEnsureLdsSlots = 24576;     // slot_last is staged in LDS up to this many slots

// exclusive scan over the 1024 threads of the block; `total` = block sum. Contains barriers: call uniformly.
__device__ __forceinline__ int block_excl_scan(int v, int* sw, int& total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
    }
    if (lane == 63) sw[wv] = incl;
    __syncthreads();
    int wbase = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = sw[i];
        wbase += i < wv ? t : 0;
        tot += t;
    }
    __syncthreads();
    total = tot;
    return wbase + incl - v;
}

__device__ __forceinline__ int block_sum(int v, int* sw) {
    int t;
    block_excl_scan(v, sw, t);
    return t;
}

__device__ __forceinline__ uint32_t block_min_u32(uint32_t v, uint32_t* su) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
    if (lane == 0) su[wv] = v;
    __syncthreads();
    uint32_t r = su[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) r = min(r, su[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* su) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
    if (lane == 0) su[wv] = v;
    __syncthreads();
    uint32_t r = su[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) r = max(r, su[i]);
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(kEnsureThreads) ensure_kernel(EnsureArgs A) {
    extern __shared__ int dyn[];
    __shared__ int sw[16];
    __shared__ uint32_t su[16];
    __shared__ int sh[8];
    __shared__ int hist[256];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int E = A.E, S = A.S, P = A.P;
    int* need = dyn;                  // [E]
    int* miss = need + E;             // [E]
    int* vslot = miss + E;            // [E]
    int* vwb = vslot + E;             // [E]
    int* pid = vwb + E;               // [P]
    int* sl = pid + P;                // [S] when staged
    const bool sl_lds = S <= kEnsureLdsSlots;
    const int32_t* slg = A.slot_last;
    if (A.pend && A.n_layers > 0) {                           // commit finished copy-engine plans first
        int* vflag = sl + (sl_lds ? S : 0);                   // [n_layers]
        for (int li = tid; li < A.n_layers; li += kEnsureThreads) {
            const int32_t* pl = A.pend + li * kPendStride;
            const int dn = __hip_atomic_load(A.done_seq + li, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            vflag[li] = (pl[0] > 0 && dn >= pl[1]) ? 1 : 0;
        }
        __syncthreads();
        for (int t = tid; t < A.n_layers * kPlanMax; t += kEnsureThreads) {
            const int li = t / kPlanMax, i = t % kPlanMax;
            const int32_t* pl = A.pend + li * kPendStride;
            if (vflag[li] && i < pl[0]) {
                const int e = pl[3 + i], s = pl[3 + kPlanMax + i];
                A.ptrs_all[(int64_t)li * E + e] = A.slot_base + (int64_t)s * A.blob;
                A.slot_last[s] = pl[2];
            }
        }
        __syncthreads();
        for (int li = tid; li < A.n_layers; li += kEnsureThreads)
            if (vflag[li]) A.pend[li * kPendStride] = 0;
        __syncthreads();
    }
    if (A.host_plan && A.pend[A.layer * kPendStride] > 0) {  // this layer's previous plan is still being copied
        if (tid == 0) A.fill_list[0] = 0;
        return;
    }

    // Calls of at most 64 picks keep pick `lane`'s post-mask slot and blob pointer in wave 0's registers: loaded in the
    // same round as the tier mask, they serve the fast path, the slow path's hit stamps and the pair pointers.
    const bool small = P <= 64;
    int pslot = -1;
    if (wv == 0) {                                            // tier mask, ascending pick order
        const int kb = A.layer * E;
        uint32_t cnt = A.ram_res ? (uint32_t)A.ring[0] : 0u;      // modulo 2^32, as the host reads it
        const int safe = A.ram_res ? A.safe[A.layer] : 0;
        const int safe_slot = A.ram_res ? A.slot_of[kb + safe] : -1;
        const int64_t safe_ptr = A.ram_res && small ? A.ptrs_all[kb + safe] : 0;
        int T = 0;
        if (lane == 0) {
            T = A.pf_slot ? A.tick[0] : A.tick[0] + 1;    // prefetch mode: the tick is not advanced
            if (!A.pf_slot) A.tick[0] = T;
            sh[0] = T;
        }
        T = __shfl(T, 0, 64);
        int64_t pptr = 0;
        for (int b = 0; b < P; b += 64) {
            const int i = b + lane;
            int id = i < P ? min(max(A.ids[i], 0), E - 1) : 0;
            int so = i < P ? A.slot_of[kb + id] : -1;
            if (small && i < P) pptr = A.ptrs_all[kb + id];
            const bool msk = A.ram_res && i < P && so < 0 && !A.ram_res[kb + id];
            const uint64_t bal = __ballot(msk);
            if (msk) {
                const uint32_t pos = cnt + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
                A.ring[1 + (int)(pos % (uint32_t)A.ring_cap)] = kb + id;
                id = safe;
                so = safe_slot;
                pptr = safe_ptr;
                A.ids[i] = id;
                A.w[i] = 0.0f;
            }
            if (i < P) pid[i] = id;
            pslot = so;
            cnt += (uint32_t)__popcll(bal);
        }
        if (A.ram_res && lane == 0) A.ring[0] = (int32_t)cnt;
        if (lane == 0) sh[5] = (int)cnt;
        // blob pointer of every post-mask pick (read by the GEMV workgroups). Assignments below never touch it: a
        // victim slot's owner is not a pick of this call (hits are stamped T, so their slots are not eligible), and
        // a miss keeps its host copy's pointer until the fill is committed at the end of the call.
        if (small && lane < P && A.pair_ptr) A.pair_ptr[lane] = pptr;
        // no-miss fast path: every post-mask pick holds a slot, so the call's only decisions are the hit stamps;
        // fills, victims and the LRU scan are empty. The stamp rule "slot_last = T unless pinned (INT_MAX)" is an
        // atomic max here: every other slot_last value is a tick of an earlier call, 0 (loaded by the host) or -1
        // (empty), all below T, and the max needs no read round trip.
        const bool fast = small && __ballot(lane < P && pslot < 0) == 0ull;
        if (fast) {
            if (lane < P) atomicMax(A.slot_last + pslot, T);
            if (lane == 0) {
                A.fill_list[0] = 0;
                if (A.vict) A.vict[0] = 0;
            }
            if (A.log) {
                const int idx = A.log[0];
                if ((int64_t)(idx + 1) * (3 + 4 * P) <= A.log_cap) {   // the record fits the buffer
                    int32_t* r = A.log + 1 + (int64_t)idx * (3 + 4 * P);
                    if (lane == 0) {
                        r[0] = T;
                        r[1] = cnt;
                        r[2 + P] = 0;
                    }
                    if (lane < P) {
                        r[2 + lane] = pid[lane];
                        r[3 + P + lane] = -1;
                        r[3 + 2 * P + 2 * lane] = -2;
                        r[4 + 2 * P + 2 * lane] = -2;
                    }
                }
                if (lane == 0) A.log[0] = idx + 1;
            }
        }
        if (lane == 0) sh[6] = fast ? 1 : 0;
    }
    for (int e = tid; e < E; e += kEnsureThreads) need[e] = 0;
    if (sl_lds)
        for (int s = tid; s < S; s += kEnsureThreads) sl[s] = slg[s];
    __syncthreads();
    if (sh[6]) return;                                         // uniform: the fast path finished the call
    const int T = sh[0];
    if (small) {
        // need[e] = 1 hit, 2 miss; hits stamp slot_last = T unless pinned (duplicate picks write the same value)
        if (tid < P) {
            need[pid[tid]] = pslot >= 0 ? 1 : 2;
            if (pslot >= 0) {
                const int la = sl_lds ? sl[pslot] : slg[pslot];
                if (la != INT_MAX) {
                    A.slot_last[pslot] = T;
                    if (sl_lds) sl[pslot] = T;
                }
            }
        }
    } else {
        for (int i = tid; i < P; i += kEnsureThreads) need[pid[i]] = 1;
    }
    __syncthreads();
    // hits and misses: work-item e = expert e (E <= 1024)
    bool is_miss = false;
    if (small) {
        is_miss = tid < E && need[tid] == 2;
    } else if (tid < E && need[tid]) {
        const int s = A.slot_of[A.layer * E + tid];
        if (s >= 0) {
            const int la = sl_lds ? sl[s] : slg[s];
            if (la != INT_MAX) {
                A.slot_last[s] = T;
                if (sl_lds) sl[s] = T;
            }
        } else {
            is_miss = true;
        }
    }
    int nmiss;
    const int mpos = block_excl_scan(is_miss ? 1 : 0, sw, nmiss);
    if (is_miss) miss[mpos] = tid;
    int nm = S > 0 ? min(nmiss, A.max_fill) : 0;
    __syncthreads();

    if (nm > 0) {
        const int C = (S + kEnsureThreads - 1) / kEnsureThreads;
        const int s0 = min(S, tid * C), s1 = min(S, s0 + C);
        int elig = 0, empty = 0;
        uint32_t umin = 0xFFFFFFFFu, umax = 0u;
        for (int s = s0; s < s1; ++s) {
            const int la = sl_lds ? sl[s] : slg[s];
            if (la >= T) continue;
            const uint32_t u = (uint32_t)(la + 1);
            ++elig;
            empty += la == -1;
            umin = min(umin, u);
            umax = max(umax, u);
        }
        elig = block_sum(elig, sw);
        empty = block_sum(empty, sw);
        umin = block_min_u32(umin, su);
        umax = block_max_u32(umax, su);
        nm = min(nm, elig);
        if (nm > 0) {
            int top = 24;
            while (top > 0 && ((umin ^ umax) >> top) == 0) top -= 8;
            uint32_t prefix = top == 24 ? 0u : (umin & (0xFFFFFFFFu << (top + 8)));
            int want = nm;
            if (empty >= nm) {
                prefix = 0u;
                top = -8;
            }
            for (int shift = top; shift >= 0; shift -= 8) {
                if (tid < 256) hist[tid] = 0;
                __syncthreads();
                const uint32_t hmask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
                for (int s = s0; s < s1; ++s) {
                    const int la = sl_lds ? sl[s] : slg[s];
                    if (la >= T) continue;
                    const uint32_t u = (uint32_t)(la + 1);
                    if ((u & hmask) != (prefix & hmask)) continue;
                    atomicAdd(&hist[(u >> shift) & 255u], 1);
                }
                __syncthreads();
                if (wv == 0) {
                    int c[4], loc = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        c[k] = hist[lane * 4 + k];
                        loc += c[k];
                    }
                    int incl = loc;
#pragma unroll
                    for (int o = 1; o < 64; o <<= 1) {
                        const int t = __shfl_up(incl, o, 64);
                        if (lane >= o) incl += t;
                    }
                    int cum = incl - loc;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        if (cum < want && want <= cum + c[k]) {
                            sh[2] = lane * 4 + k;
                            sh[3] = want - cum;
                        }
                        cum += c[k];
                    }
                }
                __syncthreads();
                prefix |= (uint32_t)sh[2] << shift;
                want = sh[3];
                __syncthreads();
            }
            const uint32_t tau = prefix;
            int n_lt = 0, n_eq = 0;
            for (int s = s0; s < s1; ++s) {
                const int la = sl_lds ? sl[s] : slg[s];
                if (la >= T) continue;
                const uint32_t u = (uint32_t)(la + 1);
                n_lt += u < tau;
                n_eq += u == tau;
            }
            int tot_lt, tot_eq;
            int blt = block_excl_scan(n_lt, sw, tot_lt);
            const int beq = block_excl_scan(n_eq, sw, tot_eq);
            const int take_eq = max(0, min(n_eq, want - beq));
            int ieq = 0;
            for (int s = s0; s < s1; ++s) {
                const int la = sl_lds ? sl[s] : slg[s];
                if (la >= T) continue;
                const uint32_t u = (uint32_t)(la + 1);
                if (u < tau) vslot[blt++] = s;
                else if (u == tau && ieq < take_eq) vslot[tot_lt + beq + ieq++] = s;
            }
            __syncthreads();
            // one miss per thread (nm <= E <= kEnsureThreads); victims as in ensure_wg: the old owner of the slot is
            // written back into its fixed record or, with the record pool, into the next free record of the step
            const int mi = tid;
            int s = 0, e = 0, old = -1, wb = -1;
            if (mi < nm) {
                s = vslot[mi];
                e = miss[mi];
                old = A.slot_key[s];
                wb = (old >= 0 && A.ram_res && A.ram_res[old]) ? -1 : old;
            }
            int64_t waddr = 0;
            const bool ring = A.vr_meta && A.vict;
            if (ring) {                          // victim ring: a free ring slot or dropped
                const int r = ring_claim<kEnsureThreads>(A.vr_meta, A.vr_K, wb, hist,
                                                         [&](int v, int& t) { return block_excl_scan(v, sw, t); });
                if (mi < nm) A.vr_sel[mi] = r;
                if (r >= 0) waddr = A.vr_base + (int64_t)r * A.blob;
                else wb = -1;
            } else if (A.host_addr && A.vict) {  // write-backs on: each takes a record of the step's queue
                int tot;
                const int rank = block_excl_scan(wb >= 0 ? 1 : 0, sw, tot);
                const int used0 = A.wbq_state[0];
                if (wb >= 0) {
                    const int q = used0 + rank;
                    if (q < A.wbq_cap) {
                        waddr = A.wbq[q];
                        A.wbq_state[1 + q] = wb;
                    } else {
                        wb = -1;
                    }
                }
                __syncthreads();
                if (tid == 0) {
                    const int taken = min(tot, max(0, A.wbq_cap - used0));
                    A.wbq_state[0] = used0 + taken;
                    A.wbq_state[1 + A.wbq_cap] += tot - taken;
                }
            } else if (wb >= 0) {
                waddr = A.host_base[wb / E] + (int64_t)(wb % E) * A.hstride;
            }
            if (mi < nm) {
                vwb[mi] = wb;
                if (A.vict) {
                    A.vict[1 + 2 * mi] = wb;
                    A.vict[2 + 2 * mi] = s;
                    if (A.vict_addr) A.vict_addr[mi] = waddr;
                }
                if (old >= 0) {
                    A.slot_of[old] = -1;
                    // the victim's blob is read from its RAM record from now on: the write-back target, else the
                    // record it already has (a dropped write-back leaves the key masked until a fill brings it back).
                    // A ring slot is no record: the key stays masked until the host has drained it into one.
                    int64_t hp = waddr;
                    if (A.host_addr) {
                        if (waddr && !ring) A.host_addr[old] = waddr;
                        else hp = A.host_addr[old];
                    } else if (wb < 0 || ring) {
                        hp = A.host_base[old / E] + (int64_t)(old % E) * A.hstride;
                    }
                    A.ptrs_all[old] = hp;
                }
                const int key = A.layer * E + e;
                A.slot_key[s] = key;
                A.slot_of[key] = s;
                A.slot_last[s] = A.host_plan ? INT_MAX : T;
                if (A.pf_slot) A.pf_slot[mi] = s;
                else A.fill_all[key] = A.slot_base + (int64_t)s * A.blob;
                A.fill_list[1 + mi] = e;
                if (A.host_plan) {
                    A.host_plan[4 + mi] = e;
                    A.host_plan[4 + E + mi] = s;
                    A.pend[A.layer * kPendStride + 3 + mi] = e;
                    A.pend[A.layer * kPendStride + 3 + kPlanMax + mi] = s;
                    __threadfence_system();                   // the entries reach host memory before the seq below
                }
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        A.fill_list[0] = nm;
        if (A.vict) A.vict[0] = nm;
        if (A.host_plan && nm > 0) {                          // publish the plan: header, fence, then the seq
            A.host_plan[1] = nm;
            A.host_plan[2] = T;
            A.host_plan[3] = A.layer;
            __threadfence_system();
            const int sq = A.plan_seq[A.layer] + 1;
            A.plan_seq[A.layer] = sq;
            int32_t* pl = A.pend + A.layer * kPendStride;
            pl[1] = sq;
            pl[2] = T;
            pl[0] = nm;
            __hip_atomic_store(A.host_plan, sq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    // blob pointer of every post-mask pick (calls of more than 64 picks; see the wave-0 block for the others)
    if (A.pair_ptr && !small)
        for (int i = tid; i < P; i += kEnsureThreads) A.pair_ptr[i] = A.ptrs_all[A.layer * E + pid[i]];
    if (A.log && wv == 0) {                                   // decision record, same layout as the oracle's
        const int idx = A.log[0];
        if ((int64_t)(idx + 1) * (3 + 4 * P) <= A.log_cap) {   // the record fits the buffer
            int32_t* r = A.log + 1 + (int64_t)idx * (3 + 4 * P);
            if (lane == 0) {
                r[0] = T;
                r[1] = sh[5];
                r[2 + P] = nm;
            }
            for (int i = lane; i < P; i += 64) {
                r[2 + i] = pid[i];
                r[3 + P + i] = i < nm ? miss[i] : -1;
                r[3 + 2 * P + 2 * i] = i < nm ? vwb[i] : -2;
                r[4 + 2 * P + 2 * i] = i < nm ? vslot[i] : -2;
            }
        }
        if (lane == 0) A.log[0] = idx + 1;
    }
}

// ---- host launchers ------------------------------------------------------------------------------------------------

hipError_t launch_ensure(const EnsureArgs& a, hipStream_t s) {
    const size_t lds =
        (size_t)(4 * a.E + a.P + (a.S <= kEnsureLdsSlots ? a.S : 0) + (a.pend ? a.n_layers : 0)) * sizeof(int);
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)ensure_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           120 * 1024);
        if (e != hipSuccess) return e;
        attr = true;
    }
    if (lds > 120 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(ensure_kernel, dim3(1), dim3(kEnsureThreads), lds, s, a);
    return hipGetLastError();
}

// ---- prefetch copy and commit ------------------------------------------------------------------------------------------
// (reference PrefetchCopyKernel and the commit task of moe_prefetch a8:1208-1221) workgroup (mi, chunk) copies 64 KiB of
// the mi-th assigned expert from its host record (device-mapped pinned memory) into its slot with 16-byte accesses;
// workgroups past the call's count return. The commit runs after the copy on the same stream, so a reader of ptrs_all
// that is ordered after it sees the whole blob.
constexpr int kPrefetchChunk = 64 * 1024;

__global__ void __launch_bounds__(256) prefetch_copy_kernel(const int32_t* fill_list, const int32_t* pf_slot,
                                                            const int64_t* host_base, int64_t hstride,
                                                            int64_t slot_base, int64_t sstride, int64_t bytes,
                                                            int layer, int chunks) {
    const int mi = blockIdx.x / chunks, ch = blockIdx.x % chunks;
    if (mi >= fill_list[0]) return;
    const int e = fill_list[1 + mi], s = pf_slot[mi];
    const uint8_t* src = (const uint8_t*)(host_base[layer] + (int64_t)e * hstride);
    uint8_t* dst = (uint8_t*)(slot_base + (int64_t)s * sstride);
    const int64_t b1 = min(bytes, (int64_t)(ch + 1) * kPrefetchChunk);
    for (int64_t o = (int64_t)ch * kPrefetchChunk + threadIdx.x * 16; o < b1; o += 256 * 16)
        *(uint4*)(dst + o) = *(const uint4*)(src + o);
}

__global__ void __launch_bounds__(256) prefetch_commit_kernel(const int32_t* fill_list, const int32_t* pf_slot,
                                                              int64_t* ptrs_all, int layer, int E, int64_t slot_base,
                                                              int64_t sstride) {
    const int n = fill_list[0];
    for (int mi = threadIdx.x; mi < n; mi += 256)
        ptrs_all[(int64_t)layer * E + fill_list[1 + mi]] = slot_base + (int64_t)pf_slot[mi] * sstride;
}

hipError_t launch_prefetch(const EnsureArgs& a, int64_t sstride, int64_t copy_bytes, hipStream_t s) {
    hipError_t e = launch_ensure(a, s);
    if (e != hipSuccess) return e;
    const int chunks = (int)((copy_bytes + kPrefetchChunk - 1) / kPrefetchChunk);
    if (a.max_fill > 0 && chunks > 0)
        hipLaunchKernelGGL(prefetch_copy_kernel, dim3((unsigned)(a.max_fill * chunks)), dim3(256), 0, s, a.fill_list,
                           a.pf_slot, a.host_base, a.hstride, a.slot_base, sstride, copy_bytes, a.layer, chunks);
    hipLaunchKernelGGL(prefetch_commit_kernel, dim3(1), dim3(256), 0, s, a.fill_list, a.pf_slot, a.ptrs_all, a.layer,
                       a.E, a.slot_base, sstride);
    return hipGetLastError();
}

// ---- cached calls larger than the decode kernel takes --------------------------------------------------------------
// A cached call with more picks (or rows) than the fused decode kernel takes, below prefill_min_m, runs the ensure over
// all its picks (one launch, the decode-mode decisions), then these three kernels, then the prefill kernels over the
// committed table: victim write-back (each victim with a write-back key copies its slot to that key's host record and
// flags it RAM-resident; a8:1168-1189), the fills (each assigned miss copied from the host record its table entry
// still names into its new slot), and the commit (ptrs_all = fill_all, fill_all = 0; a8:371-395). The reference
// reads such misses zero-copy and writes them through inside its align-path GEMV (a8:1239, 1277-1314): the decisions,
// the final cache state and the slot bytes are the same, and the outputs too (the same blob bytes are read).
// Workgroup (i, chunk) copies 64 KiB of the i-th entry with 16-byte accesses; entries past the call's count return.
__device__ __forceinline__ void copy_chunk(const uint8_t* src, uint8_t* dst, int64_t bytes, int ch) {
    const int64_t b1 = min(bytes, (int64_t)(ch + 1) * kPrefetchChunk);
    for (int64_t o = (int64_t)ch * kPrefetchChunk + threadIdx.x * 16; o < b1; o += 256 * 16)
        *(uint4*)(dst + o) = *(const uint4*)(src + o);
}

__global__ void __launch_bounds__(256) cached_victim_kernel(const int32_t* vict, const int64_t* vaddr,
                                                            const int64_t* host_base, int64_t hstride, int E,
                                                            int64_t slot_base, int64_t sstride, uint8_t* ram_res,
                                                            int chunks) {
    const int mi = blockIdx.x / chunks, ch = blockIdx.x % chunks;
    if (mi >= vict[0]) return;
    const int old = vict[1 + 2 * mi], s = vict[2 + 2 * mi];
    if (old < 0) return;                                       // no write-back (empty slot, or a valid RAM copy)
    if (ram_res && ch == 0 && threadIdx.x == 0) ram_res[old] = 1;
    copy_chunk((const uint8_t*)(slot_base + (int64_t)s * sstride),
               (uint8_t*)(vaddr ? vaddr[mi] : host_base[old / E] + (int64_t)(old % E) * hstride), sstride, ch);
}

__global__ void __launch_bounds__(256) cached_fill_kernel(const int32_t* fill_list, const int64_t* ptrs_all,
                                                          const int64_t* fill_all, int layer, int E, int64_t bytes,
                                                          int chunks) {
    const int mi = blockIdx.x / chunks, ch = blockIdx.x % chunks;
    if (mi >= fill_list[0]) return;
    const int64_t key = (int64_t)layer * E + fill_list[1 + mi];
    copy_chunk((const uint8_t*)ptrs_all[key], (uint8_t*)fill_all[key], bytes, ch);
}

__global__ void __launch_bounds__(256) cached_commit_kernel(const int32_t* fill_list, int64_t* ptrs_all,
                                                            int64_t* fill_all, int layer, int E) {
    const int n = fill_list[0];
    for (int mi = threadIdx.x; mi < n; mi += 256) {
        const int64_t key = (int64_t)layer * E + fill_list[1 + mi];
        ptrs_all[key] = fill_all[key];
        fill_all[key] = 0;
    }
}

hipError_t launch_cached_fills(const EnsureArgs& a, int64_t blob, int max_n, uint8_t* ram_res, hipStream_t s) {
    if (max_n <= 0) return hipSuccess;
    if (a.vict) {
        const int vchunks = (int)((a.blob + kPrefetchChunk - 1) / kPrefetchChunk);     // whole slots (a.blob: stride)
        hipLaunchKernelGGL(cached_victim_kernel, dim3((unsigned)(max_n * vchunks)), dim3(256), 0, s, a.vict,
                           a.vict_addr, a.host_base, a.hstride, a.E, a.slot_base, a.blob, ram_res, vchunks);
    }
    const int chunks = (int)((blob + kPrefetchChunk - 1) / kPrefetchChunk);
    hipLaunchKernelGGL(cached_fill_kernel, dim3((unsigned)(max_n * chunks)), dim3(256), 0, s, a.fill_list, a.ptrs_all,
                       a.fill_all, a.layer, a.E, blob, chunks);
    hipLaunchKernelGGL(cached_commit_kernel, dim3(1), dim3(256), 0, s, a.fill_list, a.ptrs_all, a.fill_all, a.layer,
                       a.E);
    return hipGetLastError();
}

// flag upload of the host tier step: packed[i] = key << 1 | value, read in place (pinned host memory is device-mapped)
__global__ void scatter_flags_kernel(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t p = packed[i];
    const int64_t key = p >> 1;
    if (p >= 0 && key < n_flags) flags[key] = (uint8_t)(p & 1);
}

hipError_t launch_scatter_flags(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(scatter_flags_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, flags, n_flags, packed, n);
    return hipGetLastError();
}

// Residency records of static placement (make_resident / evict): record i = (key, slot, ptr) as three int64.
// slot >= 0: the key now lives in that slot (slot_key[slot] = key, slot_last[slot] = 0: never used by a cached call
// yet); slot < 0: the key left slot -1 - slot (slot_key and slot_last of that slot to -1). Either way
// ptrs_all[key] = ptr and slot_of[key] = the new slot or -1. Records touch distinct keys and distinct slots.
__global__ void table_update_kernel(int64_t* ptrs_all, int32_t* slot_of, int32_t* slot_key, int32_t* slot_last,
                                    const int64_t* rec, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t key = rec[3 * i], slot = rec[3 * i + 1], ptr = rec[3 * i + 2];
    ptrs_all[key] = ptr;
    if (slot >= 0) {
        slot_of[key] = (int32_t)slot;
        slot_key[slot] = (int32_t)key;
        slot_last[slot] = 0;
    } else {
        slot_of[key] = -1;
        slot_key[-1 - slot] = -1;
        slot_last[-1 - slot] = -1;
    }
}

hipError_t launch_table_update(int64_t* ptrs_all, int32_t* slot_of, int32_t* slot_key, int32_t* slot_last,
                               const int64_t* rec, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(table_update_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ptrs_all, slot_of,
                       slot_key, slot_last, rec, n);
    return hipGetLastError();
}

// The whole device side of one host tier step in one launch: the flag diff of the step (as scatter_flags_kernel), the
// miss-ring entries appended since position `from` (the count the host last read) into a pinned mirror of the ring,
// with the count itself, and the snapshot copies of the device state into device-mapped pinned host buffers (16-byte
// words, then the tail bytes). A flag being set by the diff may be copied before or after its update; the host
// overlays the diff on the snapshot, so either is fine. More than ring_cap entries since `from` keeps the last
// ring_cap, as the ring itself does.
__device__ __forceinline__ void copy_part(const TierCopy& c, int64_t t, int64_t nt) {
    const int64_t n16 = c.n >> 4;
    const uint4* s16 = (const uint4*)c.src;
    uint4* d16 = (uint4*)c.dst;
    for (int64_t i = t; i < n16; i += nt) d16[i] = s16[i];
    for (int64_t i = (n16 << 4) + t; i < c.n; i += nt) c.dst[i] = c.src[i];
}

__global__ void __launch_bounds__(256) tier_exchange_kernel(uint8_t* flags, int64_t n_flags, const int32_t* packed,
                                                            int64_t n_diff, TierRing rg, TierCopies cp, TierPool pl) {
    const int64_t nt = (int64_t)gridDim.x * blockDim.x;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    // record pool: the records of keys that become RAM-resident with this diff (their flag rises in the same launch,
    // so the next decode step sees both); a key in an HBM slot keeps the slot in its table entry; keys outside
    // [0, n_flags) are ignored
    for (int64_t i = t; i < pl.n_upd; i += nt) {
        const int64_t key = pl.upd[2 * i], addr = pl.upd[2 * i + 1];
        if (key >= 0 && key < n_flags) {
            pl.host_addr[key] = addr;
            if (pl.slot_of[key] < 0) pl.ptrs_all[key] = addr;
        }
    }
    if (pl.wbq && blockIdx.x == 0) {             // the write-back queue, in order, by one workgroup
        for (int i = threadIdx.x; i < 2 + pl.cap; i += blockDim.x) pl.mirror[i] = pl.state[i];
        __syncthreads();
        for (int i = threadIdx.x; i < pl.cap; i += blockDim.x) pl.wbq[i] = pl.next[i];
        if (threadIdx.x == 0) {
            pl.state[0] = 0;
            pl.state[1 + pl.cap] = 0;
        }
    }
    for (int64_t i = t; i < n_diff; i += nt) {
        const int32_t p = packed[i];
        const int64_t key = p >> 1;
        if (p >= 0 && key < n_flags) flags[key] = (uint8_t)(p & 1);
    }
    if (rg.ring) {                               // the count and `from` are taken modulo 2^32
        const uint32_t cnt = (uint32_t)rg.ring[0];
        const int64_t n = min((int64_t)(uint32_t)(cnt - (uint32_t)rg.from), rg.cap);
        for (int64_t i = t; i < n; i += nt) {
            const int64_t q = 1 + (int64_t)((uint32_t)(cnt - (uint32_t)(n - i)) % (uint32_t)rg.cap);
            rg.mirror[q] = rg.ring[q];
        }
        if (t == 0) rg.mirror[0] = (int32_t)cnt;
    }
    for (int k = 0; k < cp.n; ++k) copy_part(cp.c[k], t, nt);
}

hipError_t launch_tier_exchange(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n_diff,
                                const TierRing& rg, const TierCopies& cp, const TierPool& pl, hipStream_t s) {
    int64_t work = std::max<int64_t>(n_diff, rg.ring ? 256 : 0);
    work = std::max(work, std::max<int64_t>(pl.n_upd, pl.wbq ? 256 : 0));
    for (int k = 0; k < cp.n; ++k) work = std::max(work, cp.c[k].n >> 4);
    if (work <= 0) return hipSuccess;
    const unsigned blocks = (unsigned)std::min<int64_t>(128, (work + 255) / 256);
    hipLaunchKernelGGL(tier_exchange_kernel, dim3(blocks), dim3(256), 0, s, flags, n_flags, packed, n_diff, rg, cp, pl);
    return hipGetLastError();
}

}  // namespace exl3
