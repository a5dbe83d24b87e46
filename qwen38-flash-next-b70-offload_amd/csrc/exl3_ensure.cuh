// The expert-cache ensure as one workgroup of the decode layer kernel (moe_decode.hip): the same canonical decisions
// as ensure_kernel (moe_cache.hip; reference kernels/moe-a8/exl3_moe.a8.sycl:831-1040), made by NT = 512 work-items
// while the gate/up and down workgroups of the same launch already stream their experts.
//
// Differences from ensure_kernel, none of which changes a decision:
//   - every thread holds its contiguous chunk of slot_last in registers (S <= NT * kEnsRegSlots), loaded at the start
//     while wave 0 applies the tier mask; the hit stamps reach the registers through an LDS bitmap of stamped slots
//   - the picks' ids / weights are NOT rewritten here (the GEMV workgroups read them during the call and apply the
//     mask rule themselves); the last workgroup of the call rewrites them
//   - what other workgroups of the launch read (fill targets, the fill list, the victim list) is written with
//     agent-scope stores, and the workgroup then raises `done` (after its stores completed)
// Limits checked by the host: E <= NT, P <= 64, S <= NT * kEnsRegSlots.
#pragma once
#include <climits>

#include "exl3_common.cuh"
#include "exl3_kernels.h"

namespace exl3 {

struct EnsureShared {
    int need[kEnsMaxE];                          // [E]: 0 not picked, 1 hit, 2 miss
    int miss[kEnsMaxE];                          // misses, ascending expert
    int vslot[kEnsMaxE];                         // victim slots, canonical order
    int vwb[kEnsMaxE];                           // write-back owner per victim (-1: none)
    int pid[kEnsMaxP];                           // post-mask expert of every pick
    uint32_t stm[kEnsMaxE * kEnsRegSlots / 32];  // stamped-slot bitmap
    int hist[256];
    int sw[16];
    uint32_t su[16];
    int sh[8];
};

__device__ __forceinline__ void st_agent_i32(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_i64(int64_t* p, int64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_agent_i32(const int32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int64_t ld_agent_i64(const int64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// exclusive scan / sum / min / max over the NW waves of the workgroup. Contain barriers: call uniformly.
template <int NW>
__device__ __forceinline__ int wg_excl_scan(int v, int* sw, int& total) {
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
    for (int i = 0; i < NW; ++i) {
        const int t = sw[i];
        wbase += i < wv ? t : 0;
        tot += t;
    }
    __syncthreads();
    total = tot;
    return wbase + incl - v;
}

template <int NW>
__device__ __forceinline__ int wg_sum(int v, int* sw) {
    int t;
    wg_excl_scan<NW>(v, sw, t);
    return t;
}

template <int NW, bool MAX>
__device__ __forceinline__ uint32_t wg_minmax(uint32_t v, uint32_t* su) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t t = (uint32_t)__shfl_xor((int)v, o, 64);
        v = MAX ? max(v, t) : min(v, t);
    }
    if (lane == 0) su[wv] = v;
    __syncthreads();
    uint32_t r = su[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) r = MAX ? max(r, su[i]) : min(r, su[i]);
    __syncthreads();
    return r;
}

template <int NT>
__device__ void ensure_wg(const EnsureArgs& A, EnsureShared& Z, int* done) {
    constexpr int NW = NT / 64;
    static_assert(NT == kEnsMaxE, "one thread per expert");
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int E = A.E, S = A.S, P = A.P;
    const int kb = A.layer * E;
    const int nwords = (S + 31) >> 5;

    // this thread's contiguous slot chunk [s0, s0 + n_own) of the stamps, loaded only once the call is known to
    // miss: a call without misses never reads them, and its done signal (after a store fence, which on this
    // architecture also waits for outstanding loads) is not held up by S stamps read beside the layer's weights
    const int C = (S + NT - 1) / NT;
    const int s0 = min(S, tid * C);
    const int n_own = min(S, s0 + C) - s0;
    for (int i = tid; i < nwords; i += NT) Z.stm[i] = 0u;
    for (int e = tid; e < E; e += NT) Z.need[e] = 0;

    int pslot = -1;                              // wave 0: post-mask slot of pick `lane`
    if (wv == 0) {                               // tier mask, ascending pick order
        // the ring count is taken modulo 2^32 (it wraps after 2^32 masked picks; the host reads it the same way)
        uint32_t cnt = A.ram_res ? (uint32_t)A.ring[0] : 0u;
        const int safe = A.ram_res ? A.safe[A.layer] : 0;
        const int safe_slot = A.ram_res ? A.slot_of[kb + safe] : -1;
        int T = 0;
        if (lane == 0) {
            T = A.tick[0] + 1;
            A.tick[0] = T;
            Z.sh[0] = T;
        }
        T = __shfl(T, 0, 64);
        int id = lane < P ? min(max(A.ids[lane], 0), E - 1) : 0;
        int so = lane < P ? A.slot_of[kb + id] : -1;
        const bool msk = A.ram_res && lane < P && so < 0 && !A.ram_res[kb + id];
        const uint64_t bal = __ballot(msk);
        if (msk) {
            const uint32_t pos = cnt + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull));
            A.ring[1 + (int)(pos % (uint32_t)A.ring_cap)] = kb + id;
            id = safe;
            so = safe_slot;
        }
        if (lane < P) Z.pid[lane] = id;
        pslot = so;
        if (A.pair_own && lane < P) {            // the first pick of each post-mask expert writes it through
            int own = 1;
            for (int j = 0; j < lane; ++j)
                if (Z.pid[j] == id) {
                    own = 0;
                    break;
                }
            st_agent_i32(A.pair_own + lane, own);
        }
        cnt += (uint32_t)__popcll(bal);
        if (A.ram_res && lane == 0) A.ring[0] = (int32_t)cnt;
        if (lane == 0) Z.sh[5] = (int)cnt;
        // no-miss call: the hit stamps are the only decisions (atomic max = "T unless pinned": every unpinned stamp
        // is an earlier tick, 0 or -1)
        const bool fast = __ballot(lane < P && pslot < 0) == 0ull;
        if (fast) {
            if (lane < P) atomicMax(A.slot_last + pslot, T);
            if (lane == 0) {
                st_agent_i32(A.fill_list, 0);
                if (A.vict) st_agent_i32(A.vict, 0);
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
                        r[2 + lane] = id;
                        r[3 + P + lane] = -1;
                        r[3 + 2 * P + 2 * lane] = -2;
                        r[4 + 2 * P + 2 * lane] = -2;
                    }
                }
                if (lane == 0) A.log[0] = idx + 1;
            }
        }
        if (lane == 0) Z.sh[6] = fast ? 1 : 0;
    }
    wait_stores();
    __syncthreads();
    if (Z.sh[6]) {                               // uniform
        if (tid == 0) counter_add(done, 1);
        return;
    }
    int slr[kEnsRegSlots];
#pragma unroll
    for (int j = 0; j < kEnsRegSlots; ++j) slr[j] = j < n_own ? A.slot_last[s0 + j] : INT_MAX;
    const int T = Z.sh[0];
    // need[e] = 1 hit / 2 miss; hits stamp slot_last = T unless pinned, and mark the slot in the bitmap
    if (tid < P) {
        Z.need[Z.pid[tid]] = pslot >= 0 ? 1 : 2;
        if (pslot >= 0) {
            atomicMax(A.slot_last + pslot, T);
            atomicOr(&Z.stm[pslot >> 5], 1u << (pslot & 31));
        }
    }
    __syncthreads();
    if (n_own > 0) {                             // fold the stamps into the register chunk (n_own <= 32)
        const int w0 = s0 >> 5;
        uint64_t m = (uint64_t)Z.stm[w0] | ((uint64_t)(w0 + 1 < nwords ? Z.stm[w0 + 1] : 0u) << 32);
        m >>= (s0 & 31);
#pragma unroll
        for (int j = 0; j < kEnsRegSlots; ++j)
            if (j < n_own && ((m >> j) & 1ull) && slr[j] != INT_MAX) slr[j] = T;
    }
    // misses in ascending expert order: work-item e = expert e
    const bool is_miss = tid < E && Z.need[tid] == 2;
    int nmiss;
    const int mpos = wg_excl_scan<NW>(is_miss ? 1 : 0, Z.sw, nmiss);
    if (is_miss) Z.miss[mpos] = tid;
    int nm = S > 0 ? min(nmiss, A.max_fill) : 0;
    __syncthreads();

    if (nm > 0) {
        int elig = 0, empty = 0;
        uint32_t umin = 0xFFFFFFFFu, umax = 0u;
#pragma unroll
        for (int j = 0; j < kEnsRegSlots; ++j) {
            const int la = slr[j];
            if (j < n_own && la < T) {
                const uint32_t u = (uint32_t)(la + 1);
                ++elig;
                empty += la == -1;
                umin = min(umin, u);
                umax = max(umax, u);
            }
        }
        elig = wg_sum<NW>(elig, Z.sw);
        empty = wg_sum<NW>(empty, Z.sw);
        umin = wg_minmax<NW, false>(umin, Z.su);
        umax = wg_minmax<NW, true>(umax, Z.su);
        nm = min(nm, elig);
        if (nm > 0) {                            // tau = nm-th smallest u: 8-bit radix passes over LDS histograms
            int top = 24;
            while (top > 0 && ((umin ^ umax) >> top) == 0) top -= 8;
            uint32_t prefix = top == 24 ? 0u : (umin & (0xFFFFFFFFu << (top + 8)));
            int want = nm;
            if (empty >= nm) {
                prefix = 0u;
                top = -8;
            }
            for (int shift = top; shift >= 0; shift -= 8) {
                if (tid < 256) Z.hist[tid] = 0;
                __syncthreads();
                const uint32_t hmask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
#pragma unroll
                for (int j = 0; j < kEnsRegSlots; ++j) {
                    const int la = slr[j];
                    const uint32_t u = (uint32_t)(la + 1);
                    if (j < n_own && la < T && (u & hmask) == (prefix & hmask)) atomicAdd(&Z.hist[(u >> shift) & 255u], 1);
                }
                __syncthreads();
                if (wv == 0) {
                    int c[4], loc = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        c[k] = Z.hist[lane * 4 + k];
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
                            Z.sh[2] = lane * 4 + k;
                            Z.sh[3] = want - cum;
                        }
                        cum += c[k];
                    }
                }
                __syncthreads();
                prefix |= (uint32_t)Z.sh[2] << shift;
                want = Z.sh[3];
                __syncthreads();
            }
            const uint32_t tau = prefix;
            int n_lt = 0, n_eq = 0;
#pragma unroll
            for (int j = 0; j < kEnsRegSlots; ++j) {
                const int la = slr[j];
                const uint32_t u = (uint32_t)(la + 1);
                if (j < n_own && la < T) {
                    n_lt += u < tau;
                    n_eq += u == tau;
                }
            }
            int tot_lt, tot_eq;
            int blt = wg_excl_scan<NW>(n_lt, Z.sw, tot_lt);
            const int beq = wg_excl_scan<NW>(n_eq, Z.sw, tot_eq);
            const int take_eq = max(0, min(n_eq, want - beq));
            int ieq = 0;
#pragma unroll
            for (int j = 0; j < kEnsRegSlots; ++j) {
                const int la = slr[j];
                const uint32_t u = (uint32_t)(la + 1);
                if (j < n_own && la < T) {
                    if (u < tau) Z.vslot[blt++] = s0 + j;
                    else if (u == tau && ieq < take_eq) Z.vslot[tot_lt + beq + ieq++] = s0 + j;
                }
            }
            __syncthreads();
            // one miss per thread (nm <= E <= NT): its slot's old owner is the victim; an owner whose RAM copy is not
            // valid is written back (wb = its key) into a record: its fixed record, or with the record pool the
            // next free record the host queued for this step (none left: the write-back is dropped and counted)
            const int mi = tid;
            int s = 0, e = 0, old = -1, wb = -1;
            if (mi < nm) {
                s = Z.vslot[mi];
                e = Z.miss[mi];
                old = A.slot_key[s];
                wb = (old >= 0 && A.ram_res && A.ram_res[old]) ? -1 : old;
            }
            int64_t waddr = 0;
            const bool ring = A.vr_meta && A.vict;
            if (ring) {                          // victim ring: a free ring slot or dropped
                const int r = ring_claim<NT>(A.vr_meta, A.vr_K, wb, Z.hist,
                                             [&](int v, int& t) { return wg_excl_scan<NW>(v, Z.sw, t); });
                if (mi < nm) A.vr_sel[mi] = r;
                if (r >= 0) waddr = A.vr_base + (int64_t)r * A.blob;
                else wb = -1;
            } else if (A.host_addr && A.vict) {  // write-backs on: each takes a record of the step's queue
                int tot;
                const int rank = wg_excl_scan<NW>(wb >= 0 ? 1 : 0, Z.sw, tot);
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
                __syncthreads();                 // every thread has read the count before it moves
                if (tid == 0) {
                    const int taken = min(tot, max(0, A.wbq_cap - used0));
                    A.wbq_state[0] = used0 + taken;
                    A.wbq_state[1 + A.wbq_cap] += tot - taken;
                }
            } else if (wb >= 0) {
                waddr = A.host_base[wb / E] + (int64_t)(wb % E) * A.hstride;
            }
            if (mi < nm) {
                Z.vwb[mi] = wb;
                if (A.vict) {
                    st_agent_i32(A.vict + 1 + 2 * mi, wb);
                    st_agent_i32(A.vict + 2 + 2 * mi, s);
                    if (A.vict_addr) st_agent_i64(A.vict_addr + mi, waddr);
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
                const int key = kb + e;
                A.slot_key[s] = key;
                A.slot_of[key] = s;
                A.slot_last[s] = T;
                st_agent_i64(A.fill_all + key, A.slot_base + (int64_t)s * A.blob);
                st_agent_i32(A.fill_list + 1 + mi, e);
            }
        }
    }
    __syncthreads();
    if (tid == 0) {
        st_agent_i32(A.fill_list, nm);
        if (A.vict) st_agent_i32(A.vict, nm);
    }
    if (A.log && wv == 0) {                      // decision record, same layout as the oracle's
        const int idx = A.log[0];
        if ((int64_t)(idx + 1) * (3 + 4 * P) <= A.log_cap) {   // the record fits the buffer
            int32_t* r = A.log + 1 + (int64_t)idx * (3 + 4 * P);
            if (lane == 0) {
                r[0] = T;
                r[1] = Z.sh[5];
                r[2 + P] = nm;
            }
            if (lane < P) {
                r[2 + lane] = Z.pid[lane];
                r[3 + P + lane] = lane < nm ? Z.miss[lane] : -1;
                r[3 + 2 * P + 2 * lane] = lane < nm ? Z.vwb[lane] : -2;
                r[4 + 2 * P + 2 * lane] = lane < nm ? Z.vslot[lane] : -2;
            }
        }
        if (lane == 0) A.log[0] = idx + 1;
    }
    wait_stores();
    __syncthreads();
    if (tid == 0) counter_add(done, 1);
}

}  // namespace exl3
